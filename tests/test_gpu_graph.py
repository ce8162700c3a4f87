"""GPU: a whole verify step (n-gram lookup, attention plan, per-layer KV append and planned
attention, rejection and greedy acceptance) captured as one HIP graph and replayed. Every
replay, with eager work and synchronisations in between, must reproduce the eager step
bit for bit (the entry points allocate nothing and record no memset)."""
import math

import pytest
import torch

import gollmgo_amd.verify as gv
from gollmgo_amd._lib import DType
from gollmgo_amd.workloads import CONFIGS, build_layout, make_histories, scaled
from helpers import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cid,kv_dt,fused", [(3, DType.FP8_E4M3, True), (5, DType.BF16, False),
                                             (5, DType.BF16, True)])
def test_step_graph_replays_match_eager(gpu, cid, kv_dt, fused):
    cfg = scaled(CONFIGS[cid], num_seqs=24, layers=2, ctx=("uniform", 64, 700), vocab=5000,
                 history_len=512, repeat_rate=0.4, partition=0)
    say(f"graph step config {cid}: B={cfg.num_seqs} L={cfg.layers} fused append={fused}")
    lay = build_layout(cfg)
    B, R, K, Hq, H, D, V, L = (cfg.num_seqs, cfg.rows, cfg.max_drafts, cfg.num_q_heads, cfg.num_kv_heads,
                               cfg.head_dim, cfg.vocab, cfg.layers)
    g = torch.Generator(device="cuda")
    g.manual_seed(7 + cid)
    kv = gv.KVCache(L, lay.num_blocks, cfg.block_size, H, D, kv_dt)
    try:
        if kv_dt == DType.FP8_E4M3:
            for layer in range(L):
                kv.set_head_scales(layer, [4.0 / 448] * H, [4.0 / 448] * H)
        fill = torch.from_numpy(lay.fill_slots).cuda()
        for layer in range(L):
            kv.append(layer, torch.randn(len(fill), H, D, device="cuda", dtype=torch.bfloat16, generator=g),
                      torch.randn(len(fill), H, D, device="cuda", dtype=torch.bfloat16, generator=g), fill)
        q = torch.randn(L, B, R, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
        k_new = torch.randn(L, B * R, H, D, device="cuda", dtype=torch.bfloat16, generator=g)
        v_new = torch.randn(L, B * R, H, D, device="cuda", dtype=torch.bfloat16, generator=g)
        out = torch.empty(L, B, R, Hq, D, device="cuda", dtype=torch.bfloat16)
        keys = torch.from_numpy(lay.keys).cuda()
        bt = torch.from_numpy(lay.block_tables).cuda()
        slots = torch.from_numpy(lay.append_slots).cuda()
        ws_attn = kv.attention_workspace(B, R, Hq, bt.shape[1], 0)
        logits = torch.randn(B, R, V, device="cuda", generator=g) * 2.0
        probs = torch.softmax(logits[:, :K] * 1.5, dim=-1).contiguous()
        drafts = probs.argmax(dim=-1).to(torch.int32)
        n_drafts = torch.randint(0, K + 1, (B,), device="cuda", dtype=torch.int32, generator=g)
        uniforms = torch.rand(B, R, device="cuda", generator=g)
        hist = torch.from_numpy(make_histories(cfg, cfg.history_len)).cuda()
        hist_len = torch.full((B,), cfg.history_len, device="cuda", dtype=torch.int32)
        ws_rej = gv.rejection_workspace(B, K, V)
        ws_gr = gv.greedy_workspace(B, K, V)
        rej = (torch.empty(B, dtype=torch.int32, device="cuda"), torch.empty(B, dtype=torch.int32, device="cuda"))
        gre = (torch.empty(B, dtype=torch.int32, device="cuda"), torch.empty(B, dtype=torch.int32, device="cuda"))
        dr = (torch.zeros(B, K, dtype=torch.int32, device="cuda"), torch.empty(B, dtype=torch.int32, device="cuda"))

        def step():
            gv.ngram_draft(hist, hist_len, cfg.ngram_n, K, out=dr)
            kv.attention_plan(keys, R, Hq, bt.shape[1], ws_attn)
            for layer in range(L):
                if fused:
                    kv.append_attention(layer, k_new[layer], v_new[layer], q[layer], out[layer], keys, bt,
                                        1.0 / math.sqrt(D), ws_attn)
                    continue
                kv.append(layer, k_new[layer], v_new[layer], slots)
                kv.attention(layer, q[layer], out[layer], keys, bt, 1.0 / math.sqrt(D), workspace=ws_attn,
                             planned=True)
            gv.accept_rejection(logits, drafts, n_drafts, uniforms, cfg.temperature or 0.8, cfg.top_p,
                                draft_probs=probs, workspace=ws_rej, out=rej)
            gv.accept_greedy(logits, drafts, n_drafts, workspace=ws_gr, out=gre)

        def results():
            # Draft slots past each sequence's count are not written by the lookup.
            n = dr[1].clamp(0, K)
            valid = torch.arange(K, device="cuda")[None, :] < n[:, None]
            return [t.clone() for t in (out, rej[0], rej[1], gre[0], gre[1])] + [torch.where(valid, dr[0], -1),
                                                                                  dr[1].clone()]
        step()
        torch.cuda.synchronize()
        eager = results()
        assert int(dr[1].sum()) > 0, "the histories should give some drafts"
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        for rep in range(3):
            # Clobber the outputs and run unrelated eager work between replays.
            for t in (out, rej[0], rej[1], gre[0], gre[1], dr[0], dr[1]):
                t.fill_(-7 if t.dtype == torch.int32 else 3.0)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = results()
            for name, a, b in zip(("attention", "rej_acc", "rej_tok", "greedy_acc", "greedy_tok", "drafts", "n_drafts"),
                                  got, eager):
                assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager step"
        del graph
    finally:
        kv.close()
