"""GPU: the runner's Step as a sequence (gollmgo_amd/runner.py, the twin of
internal/backend/rocm/runner.go Runner.Step), driven by an engine twin that does what the
reference engine does around it (internal/engine/serving.go): the decode batch of the current
token plus NGramDrafter drafts with slots from the block tables (:376-417), then
emitSpeculative over the returned LogitsPerPosition (:496-593) and BlockTable.Truncate of the
rejected drafts' slots before the next step.

The model is synthetic (random bf16 projections, no RoPE, and a bigram bias on the logits so
that the n-gram drafts are often right). Over several consecutive steps, every step checks:
  - the device decision equals the oracle's on the step's own device logits and uniforms
    (ora_accept_greedy_sample / ora_accept_greedy / ora_accept_rejection), bit for bit;
  - layer 0's attention output equals the fp64 oracle over the pool as the step left it
    (appended rows included, rejected rows of earlier steps overwritten), within 2e-3 plus the
    bf16 output's rounding;
  - what the engine's own code emits from the rows equals the decision (for bonus_row, the
    bonus is the engine's draw from the real row: ora_sample_f64 with the engine's uniform)."""
import math

import numpy as np
import pytest
import torch

from gollmgo_amd._lib import DType
from gollmgo_amd.batch import Batch
from gollmgo_amd.blocks import BlockPool, BlockTable
from gollmgo_amd.runner import (ACCEPT_BONUS_ROW, ACCEPT_GREEDY, ACCEPT_REJECTION, RunnerConfig, SamplingParams,
                                VerifyRunner)
from helpers import TOL, rel_err_per_vector, say
from oracle import oracle as ora

pytestmark = pytest.mark.gpu


class SynthModel:
    """Embeddings, per-layer Q/K/V/O projections and an LM head (bf16 weights, fp32 residual),
    plus a bigram bias gain[token] * onehot(succ[token]) on the logits."""

    def __init__(self, V=4096, Hd=256, L=2, Hq=8, Hkv=2, D=128, gain=12.0, seed=0):
        g = torch.Generator().manual_seed(seed)
        r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16).cuda()
        self.vocab, self.num_layers, self.num_q_heads, self.num_kv_heads, self.head_dim = V, L, Hq, Hkv, D
        self.E = r(V, Hd)
        self.Wq = [r(Hd, Hq * D, sc=1 / math.sqrt(Hd)) for _ in range(L)]
        self.Wk = [r(Hd, Hkv * D, sc=1 / math.sqrt(Hd)) for _ in range(L)]
        self.Wv = [r(Hd, Hkv * D, sc=1 / math.sqrt(Hd)) for _ in range(L)]
        self.Wo = [r(Hq * D, Hd, sc=1 / math.sqrt(Hq * D)) for _ in range(L)]
        self.Wlm = r(Hd, V, sc=1 / math.sqrt(Hd))
        perm = torch.randperm(V, generator=g)
        succ = torch.empty(V, dtype=torch.long)
        for c in range(0, V, 5):  # cycles of five tokens
            cyc = perm[c:c + 5]
            succ[cyc] = torch.roll(cyc, -1)
        # a fifth of the tokens carry no bias: after them the argmax is the noise's, so drafts
        # that follow the cycle get rejected
        biased = torch.rand(V, generator=g) < 0.8
        self.succ, self.gain = succ.cuda(), (biased.float() * gain).cuda()

    def embed(self, tokens):
        self.B, self.R = tokens.shape
        self.tok = tokens.long()
        self.x = self.E[self.tok].float().reshape(self.B * self.R, -1)

    def qkv(self, layer, positions):
        xb = self.x.to(torch.bfloat16)
        q = (xb @ self.Wq[layer]).reshape(self.B, self.R, self.num_q_heads, self.head_dim).contiguous()
        k = (xb @ self.Wk[layer]).reshape(self.B * self.R, self.num_kv_heads, self.head_dim).contiguous()
        v = (xb @ self.Wv[layer]).reshape(self.B * self.R, self.num_kv_heads, self.head_dim).contiguous()
        if layer == 0:
            self.q0 = q
        return q, k, v

    def post(self, layer, out):
        if layer == 0:
            self.out0 = out.clone()
        self.x = self.x + (out.reshape(self.B * self.R, -1) @ self.Wo[layer]).float()

    def logits(self):
        l = self.x.to(torch.bfloat16).float() @ self.Wlm.float()
        t = self.tok.reshape(-1)
        l[torch.arange(l.shape[0], device="cuda"), self.succ[t]] += self.gain[t]
        return l.reshape(self.B, self.R, self.vocab).to(torch.bfloat16).contiguous()


class Seq:
    def __init__(self, sid, tokens, table):
        self.id, self.tokens, self.table = sid, tokens, table


def prefill(runner, model, seqs, P):
    """The model's prefill of P prompt tokens per sequence (the verify path with P causal rows
    and no drafts); returns the last rows' logits."""
    kv, bs = runner.kv, runner.cfg.block_size
    B = len(seqs)
    for s in seqs:
        s.table.append_n(P)
    tables = np.full((B, runner.max_blocks), -1, np.int32)
    for i, s in enumerate(seqs):
        tables[i, :len(s.table.blocks)] = s.table.blocks
    tokens = torch.tensor([s.tokens[:P] for s in seqs], dtype=torch.int32).cuda()
    ctx = torch.full((B,), P, dtype=torch.int32).cuda()
    tb = torch.from_numpy(tables).cuda()
    ws = kv.attention_workspace(B, P, model.num_q_heads, runner.max_blocks)
    model.embed(tokens)
    kv.attention_plan(ctx, P, model.num_q_heads, runner.max_blocks, ws)
    for layer in range(model.num_layers):
        q, k, v = model.qkv(layer, None)
        out = torch.empty_like(q)
        kv.append_attention(layer, k, v, q, out, ctx, tb, 1 / math.sqrt(model.head_dim), ws)
        model.post(layer, out)
    return model.logits()[:, P - 1].float().cpu().numpy()


def engine_batch(seqs, K, n):
    """serving.go:376-417: the current token (no KV yet) and up to K n-gram drafts."""
    tok, pos, slots, counts, ctx, st, drafts = [], [], [], [], [], [], []
    for s in seqs:
        d = ora.ngram_draft(np.array(s.tokens, np.int32), n, K)[:K]
        c = 1 + len(d)
        p0 = len(s.tokens) - 1
        sl = s.table.append_n(c)
        tok += [s.tokens[-1]] + list(d)
        pos += list(range(p0, p0 + c))
        slots += sl
        counts.append(c)
        ctx.append(s.table.num_tokens)
        st.append(s.table.slot_mapping())
        drafts.append(list(d))
    return Batch([s.id for s in seqs], tok, pos, slots, [False] * len(seqs), counts, ctx, st, drafts)


@pytest.mark.parametrize("acceptance,T,top_k,top_p", [
    (ACCEPT_GREEDY, 0.0, 0, 0.0), (ACCEPT_GREEDY, 0.8, 50, 0.95), (ACCEPT_BONUS_ROW, 0.8, 0, 0.9),
    (ACCEPT_REJECTION, 0.8, 0, 0.95)])
def test_runner_step_sequence(gpu, acceptance, T, top_k, top_p):
    B, K, P, steps, bs = 16, 4, 16, 10, 16
    model = SynthModel(seed=3)
    sp = SamplingParams(temperature=T, top_k=top_k, top_p=top_p, seed=11)
    cfg = RunnerConfig(num_blocks=512, block_size=bs, kv_dtype=DType.BF16, max_drafts=K, sampling=sp,
                       acceptance=acceptance)
    runner = VerifyRunner(model, cfg)
    runner.warmup(B, P + steps * (K + 1) + 8)
    pool = BlockPool(cfg.num_blocks, bs, order=np.random.default_rng(5).permutation(cfg.num_blocks).tolist())
    rng = np.random.default_rng(7)
    # prompts that already walk the bigram cycles for a while, so n-gram drafts exist
    seqs = []
    for i in range(B):
        t = [int(rng.integers(0, model.vocab))]
        succ = model.succ.cpu().numpy()
        while len(t) < P:
            t.append(int(succ[t[-1]]) if rng.random() < 0.95 else int(rng.integers(0, model.vocab)))
        seqs.append(Seq(100 + i, t, BlockTable(pool)))
    say(f"runner prefill acceptance={acceptance}")
    last = prefill(runner, model, seqs, P)
    eng = np.random.default_rng(13)  # the engine's own random stream (its Sampler)
    for i, s in enumerate(seqs):
        s.tokens.append(ora.sample_f64(last[i], T, top_p, float(eng.random()), top_k=top_k))
    scale = 1 / math.sqrt(model.head_dim)
    n_acc = n_full = n_rej = 0
    for step in range(steps):
        batch = engine_batch(seqs, K, 3)
        say(f"runner step {step} acceptance={acceptance}")
        out = runner.step(batch)
        torch.cuda.synchronize()
        inp = runner.last_inputs
        acc, tok = runner.last_decision
        L = runner.last_logits.float().cpu().numpy()
        d, nd, u = inp.drafts, inp.n_drafts, runner.last_uniforms
        # (a) the device decision on the step's own logits
        if acceptance == ACCEPT_GREEDY:
            ea, et = ora.accept_greedy_sample(L, d, nd, T, top_k, top_p, u)
        elif acceptance == ACCEPT_BONUS_ROW:
            ea, et = ora.accept_greedy(L, d, nd)
        else:
            ea, et = ora.accept_rejection(L, d, nd, u.astype(np.float32), T, top_p)
        assert np.array_equal(acc, ea) and np.array_equal(tok, et), (step, acc, ea, tok, et)
        # (b) layer 0 attention over the pool as the step left it
        kc = runner.kv.k_pool(0).cpu().numpy()
        vc = runner.kv.v_pool(0).cpu().numpy()
        ref = ora.attention(model.q0.float().cpu().numpy(), kc, vc, "bf16", model.num_kv_heads, model.head_dim, bs,
                            inp.ctx_lens, inp.block_tables, scale, row_counts=inp.row_counts, threads=8)
        got = model.out0.float().cpu().numpy()
        for b in range(B):
            c = int(inp.row_counts[b])
            # the runner's attention output is bf16 (the model's activations): its rounding adds
            # at most 2^-9 of an element, counted as 2^-8 of the vector's largest
            assert rel_err_per_vector(got[b, :c], ref[b, :c]) <= TOL["bf16"] + 2.0 ** -8, (step, b)
        # (c) the engine's emitSpeculative on the rows, then its truncation
        ue = eng.random(B)
        rows = [out.logits_per_position[b] if out.logits_per_position[b] is not None else [out.logits[b]]
                for b in range(B)]
        a2, t2 = ora.emit_positions(d, nd, rows, T, top_p, ue, top_k=top_k)
        for b in range(B):
            n = int(nd[b])
            assert a2[b] == acc[b]
            if acceptance == ACCEPT_BONUS_ROW and acc[b] == n:
                assert t2[b] == ora.sample_f64(L[b, n], T, top_p, float(ue[b]), top_k=top_k)
            else:
                assert t2[b] == tok[b]
            s = seqs[b]
            emitted = [int(x) for x in d[b, :a2[b]]] + [int(t2[b])]
            s.table.truncate(n - int(a2[b]))  # the rejected drafts' slots (serving.go:582-591)
            assert s.table.num_tokens == len(s.tokens) + int(a2[b])  # valid KV: current + accepted
            s.tokens += emitted
            n_acc += int(a2[b])
            n_full += int(n > 0 and a2[b] == n)
            n_rej += int(a2[b] < n)
    print(f"{acceptance}: accepted drafts {n_acc}, fully accepted {n_full}, rejections {n_rej}")
    assert n_acc > 0 and n_rej > 0 and n_full > 0
    runner.close()
