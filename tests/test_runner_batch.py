"""The Batch -> ABI mapping of the runner (gollmgo_amd/batch.py; the Go runner's
PackBatch in internal/backend/rocm/batch.go is the same function). Batches are built the
way the engine builds them: per-sequence block tables over a shared block pool
(internal/kvcache/block_table.go:22-42), the step's tokens = current token + drafts, and
SeqContextLens including them (internal/backend/runner.go:43-44). CPU tests check the
packed arrays; the GPU test runs a packed step through the ABI against the oracle."""
import math

import numpy as np
import pytest

from gollmgo_amd.batch import Batch, BatchError, pack_batch


class BlockTable:
    """BlockTable.Append (block_table.go:22-42): a new block from the pool at offset 0,
    slot = block * bs + offset."""

    def __init__(self, pool: list, bs: int):
        self.pool, self.bs, self.blocks, self.n = pool, bs, [], 0

    def append_n(self, n: int) -> list:
        out = []
        for _ in range(n):
            off = self.n % self.bs
            if off == 0:
                self.blocks.append(self.pool.pop())
            out.append(self.blocks[self.n // self.bs] * self.bs + off)
            self.n += 1
        return out

    def slot_mapping(self) -> list:
        return [self.blocks[i // self.bs] * self.bs + i % self.bs for i in range(self.n)]


def engine_step(rng, B, bs, K, ctx_range, vocab=1000, num_blocks=None):
    """A decode step of B sequences with 0..K drafts each: returns the Batch and the
    number of tokens cached before the step per sequence."""
    prior = rng.integers(ctx_range[0], ctx_range[1], B)
    ndr = rng.integers(0, K + 1, B)
    need = int(sum((p + n + 1 + bs - 1) // bs for p, n in zip(prior, ndr)))
    nb = num_blocks or need + 8
    pool = [int(x) for x in rng.permutation(nb)]
    tables = [BlockTable(pool, bs) for _ in range(B)]
    for t, p in zip(tables, prior):
        t.append_n(int(p))
    tok, pos, slots, counts, ctx, st, drafts = [], [], [], [], [], [], []
    for i in range(B):
        d = [int(x) for x in rng.integers(0, vocab, ndr[i])]
        c = 1 + len(d)
        s = tables[i].append_n(c)
        tok += [int(rng.integers(0, vocab))] + d
        pos += list(range(int(prior[i]), int(prior[i]) + c))
        slots += s
        counts.append(c)
        ctx.append(int(prior[i]) + c)
        st.append(tables[i].slot_mapping())
        drafts.append(d)
    batch = Batch(list(range(100, 100 + B)), tok, pos, slots, [False] * B, counts, ctx, st, drafts)
    return batch, prior, nb


def test_pack_matches_the_engine_batch():
    rng = np.random.default_rng(1)
    bs, K = 16, 4
    batch, prior, _ = engine_step(rng, 12, bs, K, (1, 300))
    p = pack_batch(batch, bs)
    R = max(batch.seq_token_counts)
    assert p.rows_per_seq == R and p.num_seqs == 12
    t0 = 0
    for i in range(12):
        c = batch.seq_token_counts[i]
        np.testing.assert_array_equal(p.tokens[i, :c], batch.token_ids[t0:t0 + c])
        assert np.all(p.tokens[i, c:] == 0)
        assert np.all(p.slots[i * R + c:(i + 1) * R] == -1)
        assert p.ctx_lens[i] == prior[i] + c and p.row_counts[i] == c and p.n_drafts[i] == c - 1
        np.testing.assert_array_equal(p.drafts[i, :c - 1], batch.draft_tokens[i])
        # every slot of the sequence through its block table: block * bs + offset
        st = batch.seq_slot_tables[i]
        for k in range(len(st)):
            assert p.block_tables[i, k // bs] * bs + k % bs == st[k]
        # the step's rows sit at the last row_count key positions, the attention's rule
        for j in range(c):
            pos = p.ctx_lens[i] - p.row_counts[i] + j
            assert p.block_tables[i, pos // bs] * bs + pos % bs == p.slots[i * R + j]
            assert p.positions[i, j] == pos
        t0 += c
    assert np.all(p.block_tables[p.block_tables >= 0] < 10 ** 6)


def test_pack_warmed_up_shapes_and_padding():
    rng = np.random.default_rng(2)
    batch, _, _ = engine_step(rng, 3, 16, 2, (10, 40))
    p = pack_batch(batch, 16, max_blocks=9, rows_per_seq=6)
    assert p.tokens.shape == (3, 6) and p.drafts.shape == (3, 5) and p.block_tables.shape == (3, 9)
    assert np.all(p.block_tables[:, 4:] == -1)
    with pytest.raises(BatchError, match="warmed-up"):
        pack_batch(batch, 16, rows_per_seq=2)
    with pytest.raises(BatchError, match="warmed-up"):
        pack_batch(batch, 16, max_blocks=1)


def test_pack_refuses_inconsistent_batches():
    rng = np.random.default_rng(3)
    bs = 16
    good, _, _ = engine_step(rng, 2, bs, 3, (20, 60))

    def mutated(**kw):
        b = Batch(**{**good.__dict__, **kw})
        with pytest.raises(BatchError):
            pack_batch(b, bs)

    mutated(is_prefill=[True, False])
    mutated(seq_token_counts=[good.seq_token_counts[0] + 1, good.seq_token_counts[1]])
    mutated(draft_tokens=[[], []] if any(good.draft_tokens) else [[1], []])
    mutated(slot_mapping=[s + 1 for s in good.slot_mapping])
    st = [list(t) for t in good.seq_slot_tables]
    st[0][0] += 1  # a block that does not start on a block boundary
    mutated(seq_slot_tables=st)
    mutated(seq_context_lens=[good.seq_context_lens[0] + 1, good.seq_context_lens[1]])
    with pytest.raises(BatchError):
        pack_batch(Batch([], [], [], [], [], [], [], []), bs)


def test_block_runs_rule():
    from gollmgo_amd.batch import check_block_runs
    check_block_runs(np.array([32, 33, -1, 34, 16, 17, 48]), 16)  # runs of blocks 2, 1, 3
    with pytest.raises(BatchError, match="two separate runs"):
        check_block_runs(np.array([32, 33, 16, 34]), 16)
    with pytest.raises(BatchError, match="not increasing"):
        check_block_runs(np.array([33, 32]), 16)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", ["bf16", "fp8", "int8"])
def test_packed_step_through_the_abi(gpu, dt):
    """An engine-built batch packed and run through the ABI: the prior context appended,
    then the step's K/V rows (fused append for bf16 / fp8 from the block tables, gg_kv_append
    with the packed slots for PER_BLOCK int8), the planned attention against the oracle,
    then greedy acceptance handed back as one-hot rows."""
    import torch

    import gollmgo_amd.verify as gv
    from gollmgo_amd._lib import DType
    from helpers import PoolMirror, TOL, check_positions, rel_err_per_vector, say
    from oracle import oracle as ora

    rng = np.random.default_rng({"bf16": 5, "fp8": 6, "int8": 7}[dt])
    B, bs, K, H, Hq, D, V = 10, 16, 4, 2, 8, 128, 3000
    batch, prior, nb = engine_step(rng, B, bs, K, (1, 700), vocab=V)
    p = pack_batch(batch, bs)
    R = p.rows_per_seq
    say(f"packed step dt={dt} B={B} R={R} blocks={nb}")
    kv = gv.KVCache(1, nb, bs, H, D, {"bf16": DType.BF16, "fp8": DType.FP8_E4M3, "int8": DType.INT8}[dt])
    mirror = PoolMirror(kv)
    if dt == "fp8":
        kv.set_head_scales(0, [3.0 / 448] * H, [3.0 / 448] * H)
        mirror.set_head_scales([3.0 / 448] * H, [3.0 / 448] * H)
    # prior context: every cached slot of every sequence, in table order
    pslots = np.array([s for i in range(B) for s in batch.seq_slot_tables[i][:prior[i]]], np.int32)
    kx = ora.round_bf16(rng.normal(0, 1, (len(pslots), H, D)).astype(np.float32))
    vx = ora.round_bf16(rng.normal(0, 1, (len(pslots), H, D)).astype(np.float32))
    kv.append(0, torch.from_numpy(kx).to(torch.bfloat16).cuda(), torch.from_numpy(vx).to(torch.bfloat16).cuda(),
              torch.from_numpy(pslots).cuda())
    mirror.append(kx, vx, pslots)
    kn = ora.round_bf16(rng.normal(0, 1, (B * R, H, D)).astype(np.float32))
    vn = ora.round_bf16(rng.normal(0, 1, (B * R, H, D)).astype(np.float32))
    q = ora.round_bf16(rng.normal(0, 1, (B, R, Hq, D)).astype(np.float32))
    ctx_t = torch.from_numpy(p.ctx_lens).cuda()
    rc_t = torch.from_numpy(p.row_counts).cuda()
    bt_t = torch.from_numpy(p.block_tables).cuda()
    kn_t, vn_t = torch.from_numpy(kn).to(torch.bfloat16).cuda(), torch.from_numpy(vn).to(torch.bfloat16).cuda()
    q_t = torch.from_numpy(q).to(torch.bfloat16).cuda()
    out = torch.zeros(B, R, Hq, D, dtype=torch.float32, device="cuda")
    ws = kv.attention_workspace(B, R, Hq, p.max_blocks, 0)
    kv.attention_plan(ctx_t, R, Hq, p.max_blocks, ws, row_counts=rc_t)
    scale = 1 / math.sqrt(D)
    if dt == "int8":
        kv.append(0, kn_t, vn_t, torch.from_numpy(p.slots).cuda())
        kv.attention(0, q_t, out, ctx_t, bt_t, scale, row_counts=rc_t, workspace=ws, planned=True)
    else:
        kv.append_attention(0, kn_t, vn_t, q_t, out, ctx_t, bt_t, scale, ws, row_counts=rc_t)
    torch.cuda.synchronize()
    mirror.append(kn, vn, p.slots)
    mirror.compare_with_device()
    ks, vs = mirror.scales_for_oracle()
    ref = ora.attention(q, mirror.kc, mirror.vc, dt, H, D, bs, p.ctx_lens, p.block_tables, scale, ks, vs,
                        row_counts=p.row_counts)
    got = out.cpu().numpy()
    for i in range(B):
        c = p.row_counts[i]
        assert rel_err_per_vector(got[i, :c], ref[i, :c]) < TOL[dt]
        assert np.all(got[i, c:] == 0)  # padding rows are not written
    # acceptance of the packed drafts, handed back as the engine's rows
    logits = torch.randn(B, R, V, device="cuda") * 2
    acc, tok = gv.accept_greedy(logits, torch.from_numpy(p.drafts).cuda(), torch.from_numpy(p.n_drafts).cuda())
    torch.cuda.synchronize()
    ea, et = ora.accept_greedy(logits.cpu().numpy(), p.drafts, p.n_drafts)
    assert np.array_equal(acc.cpu().numpy(), ea) and np.array_equal(tok.cpu().numpy(), et)
    check_positions(p.drafts, p.n_drafts, ea, et, V, 0.0, 1.0, 0)
    kv.close()
