"""GPU parity: draft-KV append (bit-exact) and verify attention
against the CPU oracle, through the C ABI."""
import math
import os

import numpy as np
import pytest
import torch

from gollmgo_amd._lib import DType
from gollmgo_amd.verify import KVCache
from gollmgo_amd.workloads import CONFIGS, build_layout, scaled
from helpers import PoolMirror, TOL, append_rows, glibc_rand_uniform, per_head_amax_scales, rel_err_per_vector, say
from oracle import oracle as ora

pytestmark = pytest.mark.gpu

DTYPES = {"f32": DType.F32, "f16": DType.F16, "bf16": DType.BF16, "fp8": DType.FP8_E4M3, "int8": DType.INT8}


def make_cache(dt, H, D, bs, nb, layers=1):
    return KVCache(layers, nb, bs, H, D, DTYPES[dt])


# ------------------------------------------------------------------ append

@pytest.mark.parametrize("dt", ["f32", "f16", "bf16", "fp8", "int8"])
@pytest.mark.parametrize("src", ["f32", "bf16", "f16"])
def test_append_bit_exact(gpu, dt, src):
    say(f"append dt={dt} src={src}")
    H, D, bs, nb = 4, 128, 16, 40
    kv = make_cache(dt, H, D, bs, nb)
    mirror = PoolMirror(kv)
    rng = np.random.default_rng(1)
    if dt == "fp8":
        ks = np.array([0.01, 0.02, 0.005, 0.03], np.float32)
        vs = np.array([0.02, 0.01, 0.04, 0.015], np.float32)
        kv.set_head_scales(0, ks, vs)
        mirror.set_head_scales(ks, vs)
    perm = rng.permutation(nb)
    # Three calls: whole blocks, then partial runs, then single rows into partly filled blocks
    # (int8: later rows grow the block scale and re-quantise earlier rows).
    slots1 = np.concatenate([perm[b] * bs + np.arange(bs) for b in range(6)]).astype(np.int32)
    slots2 = np.concatenate([perm[6] * bs + np.arange(5), perm[7] * bs + np.arange(9), [-1]]).astype(np.int32)
    slots3 = np.array([perm[6] * bs + 5, perm[6] * bs + 6, perm[7] * bs + 9, perm[8] * bs], np.int32)
    for i, (slots, sd) in enumerate([(slots1, 1.0), (slots2, 2.0), (slots3, 8.0)]):
        k = rng.normal(0, sd, (len(slots), H, D)).astype(np.float32)
        v = rng.normal(0, sd, (len(slots), H, D)).astype(np.float32)
        append_rows(kv, mirror, k, v, slots, src)
        mirror.compare_with_device()
    kv.close()


@pytest.mark.parametrize("D", [128, 36])  # 128: vectorised kernel; 36: one element per thread
@pytest.mark.parametrize("scale", [1.0, 0.25])
def test_append_fp8_edge_values(gpu, D, scale):
    """FP8 quantise-on-write at the format's edges, bit for bit against the oracle's
    encoder (itself pinned to torch's float8_e4m3fn cast): every code and the midpoint
    between neighbouring codes (ties to even, subnormals included), both signs and zeros,
    values past 448 up to infinity (saturate), NaN (0x7F | sign)."""
    say(f"append fp8 edge values D={D} scale={scale}")
    codes = np.arange(0, 0x7F, dtype=np.uint8)
    vals = ora.fp8_decode(codes).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    near = np.concatenate([np.nextafter(mids.astype(np.float32), np.float32(0)),
                           np.nextafter(mids.astype(np.float32), np.float32(1e9))])
    big = np.array([448.0, 448.5, 460.0, 463.99, 464.0, 470.0, 480.0, 1e6, 3.4e38, np.inf, np.nan, 0.0], np.float32)
    x = np.concatenate([vals, mids, near, big, [2.0 ** -10, 2.0 ** -9 * 0.5, 2.0 ** -12, 1e-30]]).astype(np.float32)
    x = np.concatenate([x, -x]) * np.float32(scale)  # x * (1/scale) recovers the value exactly
    H, bs = 2, 16
    per_row = H * D
    n = (len(x) + per_row - 1) // per_row
    flat = np.zeros(n * per_row, np.float32)
    flat[:len(x)] = x
    k = flat.reshape(n, H, D)
    v = np.roll(flat, 7).reshape(n, H, D)
    nb = (n + bs - 1) // bs + 2
    kv = make_cache("fp8", H, D, bs, nb)
    mirror = PoolMirror(kv)
    kv.set_head_scales(0, [scale] * H, [scale] * H)
    mirror.set_head_scales(np.full(H, scale, np.float32), np.full(H, scale, np.float32))
    slots = np.arange(bs, bs + n, dtype=np.int32)
    append_rows(kv, mirror, k, v, slots, "f32")
    mirror.compare_with_device()
    kv.close()


@pytest.mark.parametrize("seed", range(15))
def test_append_random_cases(gpu, seed):
    """Seeded random append sequences: pool type, block size, head count and dim, source
    type, several calls that extend a few sequences' block runs (as BlockTable.Append
    does, so a block's rows in one call are adjacent), skipped rows; bit for bit against
    the mirror after every call."""
    r = np.random.default_rng(300 + seed)
    dt = ["f32", "f16", "bf16", "fp8", "int8"][seed % 5]
    src = str(r.choice(["f32", "bf16", "f16"]))
    bs = int(r.choice([8, 16, 32]))
    H = int(r.choice([1, 2, 8]))
    D = int(r.choice([64, 96, 128, 40]))
    nb = 64
    say(f"append random case {seed}: dt={dt} src={src} bs={bs} H={H} D={D}")
    kv = make_cache(dt, H, D, bs, nb)
    mirror = PoolMirror(kv)
    if dt == "fp8":
        ks = r.uniform(0.005, 0.05, H).astype(np.float32)
        vs = r.uniform(0.005, 0.05, H).astype(np.float32)
        kv.set_head_scales(0, ks, vs)
        mirror.set_head_scales(ks, vs)
    free = list(r.permutation(nb))
    seqs = [[] for _ in range(int(r.integers(1, 5)))]  # per sequence: its blocks
    lens = [0] * len(seqs)
    for call in range(4):
        slots = []
        for i in range(len(seqs)):
            for _ in range(int(r.integers(0, 2 * bs))):
                if lens[i] % bs == 0:
                    if not free:
                        break
                    seqs[i].append(int(free.pop()))
                slots.append(seqs[i][-1] * bs + lens[i] % bs)
                lens[i] += 1
        if r.random() < 0.3 and slots:
            slots.insert(int(r.integers(0, len(slots) + 1)), -1)  # a skipped row
        if not slots:
            continue
        slots = np.array(slots, np.int32)
        sd = float(r.choice([0.1, 1.0, 4.0])) * (call + 1)
        k = r.normal(0, sd, (len(slots), H, D)).astype(np.float32)
        v = r.normal(0, sd, (len(slots), H, D)).astype(np.float32)
        append_rows(kv, mirror, k, v, slots, src)
        mirror.compare_with_device()
    kv.close()


# ------------------------------------------------------------------ attention

def run_attention_case(dt, B, R, Hq, H, D, bs, ctx, partition=0, src="f32", seed=0, q_dt="f32",
                       row_counts=None, kv_sd=1.0, q_sd=1.0, v_sd=None):
    rng = np.random.default_rng(seed)
    keys = np.asarray(ctx, np.int32) + R
    nbs = [(int(k) + bs - 1) // bs for k in keys]
    max_blocks = max(nbs)
    nb = sum(nbs) + 4
    perm = rng.permutation(nb)
    bt = np.zeros((B, max_blocks), np.int32)
    p = 0
    for b in range(B):
        bt[b, :nbs[b]] = perm[p:p + nbs[b]]
        p += nbs[b]
    kv = make_cache(dt, H, D, bs, nb)
    mirror = PoolMirror(kv)
    slots = np.concatenate([bt[b, np.arange(keys[b]) // bs] * bs + np.arange(keys[b]) % bs for b in range(B)]).astype(np.int32)
    kk = rng.normal(0, kv_sd, (len(slots), H, D)).astype(np.float32)
    vv = rng.normal(0, kv_sd if v_sd is None else v_sd, (len(slots), H, D)).astype(np.float32)
    if dt == "fp8":
        ks, vs = per_head_amax_scales(kk), per_head_amax_scales(vv)
        kv.set_head_scales(0, ks, vs)
        mirror.set_head_scales(ks, vs)
    append_rows(kv, mirror, kk, vv, slots, src)
    mirror.sync_from_device()
    q = rng.normal(0, q_sd, (B, R, Hq, D)).astype(np.float32)
    qt = torch.from_numpy(q).to({"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[q_dt]).cuda()
    qh = qt.float().cpu().numpy()
    out = torch.zeros(B, R, Hq, D, dtype=torch.float32, device="cuda")
    rc_t = torch.from_numpy(np.asarray(row_counts, np.int32)).cuda() if row_counts is not None else None
    if row_counts is not None:
        keys = np.asarray(ctx, np.int32) + np.asarray(row_counts, np.int32)
    scale = 1.0 / math.sqrt(D)
    kv.attention(0, qt, out, torch.from_numpy(keys).cuda(), torch.from_numpy(bt).cuda(), scale,
                 row_counts=rc_t, partition_tokens=partition)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ksc, vsc = mirror.scales_for_oracle()
    ref = ora.attention(qh, mirror.kc, mirror.vc, dt, H, D, bs, keys, bt, scale, ksc, vsc,
                        row_counts=row_counts)
    if row_counts is not None:
        mask = np.arange(R)[None, :] < np.asarray(row_counts)[:, None]
        got, ref = got[mask], ref[mask]
    kv.close()
    return rel_err_per_vector(got, ref)


MFMA_SHAPES = [
    # (B, R, Hq, H, ctx) with D=128, bs=16 -> MFMA path (G*R <= 64)
    (3, 5, 24, 8, [40, 700, 1500]),          # 3B geometry, 1 row tile
    (4, 6, 32, 8, [100, 1030, 2047, 64]),    # 8B geometry, 2 row tiles
    (2, 9, 32, 8, [5000, 777]),              # config-4 geometry, 3 row tiles (stream-K: few items)
    (32, 9, 32, 8, [37 * i % 700 + 20 for i in range(32)]),  # 3 row tiles, LPT pieces
    (2, 16, 16, 4, [300, 129]),              # 4 row tiles
    (2, 1, 8, 8, [31, 65]),                  # decode-only (R=1)
]


@pytest.mark.parametrize("dt", ["bf16", "f16", "fp8", "int8"])
@pytest.mark.parametrize("shape", range(len(MFMA_SHAPES)))
def test_attention_mfma_path(gpu, dt, shape):
    B, R, Hq, H, ctx = MFMA_SHAPES[shape]
    for part in (0, 256):
        say(f"attention mfma dt={dt} shape={MFMA_SHAPES[shape]} partition={part}")
        err = run_attention_case(dt, B, R, Hq, H, 128, 16, ctx, partition=part, src="bf16", q_dt="bf16", seed=shape)
        print(f"  rel err {err:.2e}")
        assert err <= TOL[dt]


@pytest.mark.parametrize("dt", ["f16", "fp8", "int8"])
@pytest.mark.parametrize("q_sd", [3e4, 1e6])
def test_attention_large_bf16_queries_on_f16_operand_pools(gpu, dt, q_sd):
    """FP8 / INT8 / F16 pools take Q as f16 MFMA operands (|q| < 65504). bf16 queries far
    beyond that (|q| up to ~1.4e5, and ~5e6) are scaled by a power of two for the piece,
    with the score multiplier scaled back, so the result stays textbook attention. K is
    drawn at 3/q_sd so that the scores stay O(1): with scores in the tens of thousands
    the fp32 dot products themselves would decide the softmax, whatever the operands. V
    keeps N(0, 1)."""
    for shape in (0, 1, 3):
        B, R, Hq, H, ctx = MFMA_SHAPES[shape]
        for part in (0, 256):
            say(f"attention large q dt={dt} q_sd={q_sd} shape={shape} partition={part}")
            err = run_attention_case(dt, B, R, Hq, H, 128, 16, ctx, partition=part, src="bf16", q_dt="bf16",
                                     seed=shape + 7, q_sd=q_sd, kv_sd=3.0 / q_sd, v_sd=1.0)
            assert err <= TOL[dt], (dt, q_sd, shape, part, err)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16", "fp8", "int8"])
def test_attention_generic_path(gpu, dt):
    # head_dim 64 (config 1 geometry), head_dim 16 with block size 4, and G*R > 64 rows.
    for (B, R, Hq, H, D, bs, ctx) in [(4, 5, 8, 2, 64, 16, [64, 128, 192, 256]),
                                      (2, 3, 4, 4, 16, 4, [8, 30]),
                                      (2, 5, 32, 2, 128, 16, [600, 90])]:
        for part in (0, 64):
            say(f"attention generic dt={dt} shape={(B, R, Hq, H, D, bs, ctx)} partition={part}")
            err = run_attention_case(dt, B, R, Hq, H, D, bs, ctx, partition=part, seed=D)
            print(f"  rel err {err:.2e}")
            assert err <= TOL[dt]


@pytest.mark.parametrize("dt", ["bf16", "fp8"])
def test_attention_ragged_rows(gpu, dt):
    """Sequences with fewer drafts than max (row_counts) only write their own rows."""
    say(f"attention ragged dt={dt}")
    err = run_attention_case(dt, 3, 6, 32, 8, 128, 16, [300, 1000, 17], row_counts=[6, 1, 3], src="bf16",
                             q_dt="bf16", seed=7)
    assert err <= TOL[dt]


@pytest.mark.parametrize("dt,H,Hq,D,B,partition", [
    ("fp8", 8, 32, 128, 3, 0),      # MFMA, automatic schedule (stream-K at this size)
    ("bf16", 8, 32, 128, 600, 0),   # MFMA, LPT pieces (items fill the slots)
    ("bf16", 8, 32, 128, 3, 256),   # MFMA, explicit partition grid
    ("f32", 2, 8, 64, 3, 64),       # generic path
])
def test_attention_row_count_above_rows(gpu, dt, H, Hq, D, B, partition):
    """A row count above rows_per_seq is no sequence at all: its output rows stay as they
    were, and every other sequence is computed as usual."""
    say(f"attention row_count > rows dt={dt} B={B} partition={partition}")
    R, bs = 4, 16
    rng = np.random.default_rng(11)
    ctx = rng.integers(20, 700, B).astype(np.int32)
    rc = rng.integers(1, R + 1, B).astype(np.int32)
    bad = [1, B - 1]
    rc[bad] = [R + 3, R + 1]
    good_rc = rc.copy()
    good_rc[bad] = R  # the oracle's view of the other sequences; bad rows are not compared
    keys = ctx + np.where(rc > R, R, rc)
    nbs = (keys + bs - 1) // bs
    bt = np.zeros((B, int(nbs.max())), np.int32)
    perm = rng.permutation(int(nbs.sum()) + 4)
    p0 = 0
    for b in range(B):
        bt[b, :nbs[b]] = perm[p0:p0 + nbs[b]]
        p0 += nbs[b]
    kv = make_cache(dt, H, D, bs, int(nbs.sum()) + 4)
    mirror = PoolMirror(kv)
    slots = np.concatenate([bt[b, np.arange(keys[b]) // bs] * bs + np.arange(keys[b]) % bs
                            for b in range(B)]).astype(np.int32)
    kk = rng.normal(0, 1, (len(slots), H, D)).astype(np.float32)
    vv = rng.normal(0, 1, (len(slots), H, D)).astype(np.float32)
    if dt == "fp8":
        ks, vs = per_head_amax_scales(kk), per_head_amax_scales(vv)
        kv.set_head_scales(0, ks, vs)
        mirror.set_head_scales(ks, vs)
    append_rows(kv, mirror, kk, vv, slots, "bf16")
    mirror.sync_from_device()
    q = rng.normal(0, 1, (B, R, Hq, D)).astype(np.float32)
    qt = torch.from_numpy(q).to(torch.bfloat16).cuda()
    out = torch.full((B, R, Hq, D), 7.0, dtype=torch.float32, device="cuda")
    scale = 1.0 / math.sqrt(D)
    kv.attention(0, qt, out, torch.from_numpy(keys.astype(np.int32)).cuda(), torch.from_numpy(bt).cuda(), scale,
                 row_counts=torch.from_numpy(rc).cuda(), partition_tokens=partition)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(got[bad] == 7.0), "a sequence with row_counts > rows_per_seq was written"
    ksc, vsc = mirror.scales_for_oracle()
    ref = ora.attention(qt.float().cpu().numpy(), mirror.kc, mirror.vc, dt, H, D, bs, keys, bt, scale, ksc, vsc,
                        row_counts=good_rc)
    ok = np.ones(B, bool)
    ok[bad] = False
    mask = (np.arange(R)[None, :] < rc[:, None]) & ok[:, None]
    assert np.all(got[~mask & ok[:, None]] == 7.0), "rows past row_counts were written"
    err = rel_err_per_vector(got[mask], ref[mask])
    kv.close()
    assert err <= TOL[dt]


def test_attention_reference_paged_vs_naive_inputs(gpu):
    """The reference's test_paged_vs_naive inputs (srand(42), 9 tokens, 4 heads, D=16,
    block size 4, identity slots; kernels/gollmgo_paged_attn_test.cu:39-217), fp16 pool."""
    say("attention reference paged_vs_naive inputs")
    T, Hq, H, D, bs = 9, 4, 4, 16, 4
    u = glibc_rand_uniform(42, T * Hq * D + 2 * T * H * D)
    q_all = u[:T * Hq * D].reshape(T, Hq, D)
    k = u[T * Hq * D:T * Hq * D + T * H * D].reshape(T, H, D)
    v = u[T * Hq * D + T * H * D:].reshape(T, H, D)
    kv = make_cache("f16", H, D, bs, 3)
    mirror = PoolMirror(kv)
    append_rows(kv, mirror, k, v, np.arange(T, dtype=np.int32), "f16")
    q = ora.round_f16(q_all[T - 1:T]).reshape(1, 1, Hq, D)
    out = torch.zeros(1, 1, Hq, D, dtype=torch.float32, device="cuda")
    bt = np.array([[0, 1, 2]], np.int32)
    kv.attention(0, torch.from_numpy(q).half().cuda(), out, torch.tensor([T], dtype=torch.int32, device="cuda"),
                 torch.from_numpy(bt).cuda(), 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    ref = ora.attention(q, mirror.kc, mirror.vc, "f16", H, D, bs, np.array([T], np.int32), bt, 1 / math.sqrt(D))
    assert rel_err_per_vector(out.cpu().numpy(), ref) <= 2e-3
    # The reference's own bar: |paged - naive| <= 0.05 absolute.
    assert np.abs(out.cpu().numpy() - ref).max() <= 0.05
    kv.close()


V2_SWEEP = [(256, 4, 4, 64), (2048, 8, 8, 64), (4096, 8, 2, 64), (4096, 16, 8, 128), (8192, 8, 8, 64)]


@pytest.mark.parametrize("case", V2_SWEEP)
@pytest.mark.parametrize("R", [1, 5])
def test_attention_reference_v2_sweep_inputs(gpu, case, R):
    """The reference's v2 parity sweep shapes and inputs (srand(4242+seq+7H+KV),
    256-token partitions; kernels/gollmgo_paged_attn_test.cu:361-510), fp16 pool,
    extended to R verify rows."""
    S, Hq, H, D = case
    say(f"attention reference v2 sweep {case} R={R}")
    seed = 4242 + S + Hq * 7 + H
    n = R * Hq * D + 2 * S * H * D
    u = glibc_rand_uniform(seed, n)
    q = ora.round_f16(u[:R * Hq * D]).reshape(1, R, Hq, D)
    k = u[R * Hq * D:R * Hq * D + S * H * D].reshape(S, H, D)
    v = u[R * Hq * D + S * H * D:].reshape(S, H, D)
    bs = 16
    nb = (S + bs - 1) // bs
    kv = make_cache("f16", H, D, bs, nb)
    mirror = PoolMirror(kv)
    append_rows(kv, mirror, k, v, np.arange(S, dtype=np.int32), "f16")
    bt = np.arange(nb, dtype=np.int32)[None]
    out = torch.zeros(1, R, Hq, D, dtype=torch.float32, device="cuda")
    keys = np.array([S], np.int32)
    kv.attention(0, torch.from_numpy(q).half().cuda(), out, torch.from_numpy(keys).cuda(), torch.from_numpy(bt).cuda(),
                 1 / math.sqrt(D), partition_tokens=256)
    torch.cuda.synchronize()
    ref = ora.attention(q, mirror.kc, mirror.vc, "f16", H, D, bs, keys, bt, 1 / math.sqrt(D))
    assert rel_err_per_vector(out.cpu().numpy(), ref) <= 2e-3
    assert np.abs(out.cpu().numpy() - ref).max() <= 0.1  # the reference's v2-vs-v1 bar
    kv.close()


@pytest.mark.parametrize("out_dt", ["bf16", "f16"])
def test_attention_low_precision_output(gpu, out_dt):
    """bf16/f16 outputs equal the fp32 output rounded once."""
    say(f"attention output dtype {out_dt}")
    rng = np.random.default_rng(3)
    B, R, Hq, H, D, bs = 2, 5, 24, 8, 128, 16
    ctx = [900, 40]
    keys = np.asarray(ctx, np.int32) + R
    nbs = [(int(k) + bs - 1) // bs for k in keys]
    bt = np.zeros((B, max(nbs)), np.int32)
    bt[0, :nbs[0]] = np.arange(nbs[0])
    bt[1, :nbs[1]] = nbs[0] + np.arange(nbs[1])
    kv = make_cache("bf16", H, D, bs, sum(nbs))
    slots = np.concatenate([bt[b, np.arange(keys[b]) // bs] * bs + np.arange(keys[b]) % bs for b in range(B)])
    kv.append(0, torch.randn(len(slots), H, D, dtype=torch.bfloat16, device="cuda"),
              torch.randn(len(slots), H, D, dtype=torch.bfloat16, device="cuda"),
              torch.from_numpy(slots.astype(np.int32)).cuda())
    q = torch.randn(B, R, Hq, D, dtype=torch.bfloat16, device="cuda")
    o32 = torch.zeros(B, R, Hq, D, dtype=torch.float32, device="cuda")
    olo = torch.zeros(B, R, Hq, D, dtype={"bf16": torch.bfloat16, "f16": torch.float16}[out_dt], device="cuda")
    args = (torch.from_numpy(keys).cuda(), torch.from_numpy(bt).cuda(), 1 / math.sqrt(D))
    kv.attention(0, q, o32, *args)
    kv.attention(0, q, olo, *args)
    torch.cuda.synchronize()
    assert torch.equal(o32.to(olo.dtype), olo)
    kv.close()


def test_attention_config_layouts(gpu):
    """Configs 2-5 geometry and layouts (shared prefixes, shuffled pools), scaled down
    to oracle-friendly sizes."""
    for cid, kw in [(2, dict(num_seqs=4, ctx=("uniform", 512, 1200), pool_blocks=4096)),
                    (3, dict(num_seqs=4, ctx=("uniform", 1024, 1600))),
                    (4, dict(num_seqs=2, ctx=("uniform", 2000, 3000))),
                    (5, dict(num_seqs=4, ctx=("uniform", 256, 700)))]:
        cfg = scaled(CONFIGS[cid], **kw)
        say(f"attention config {cid} scaled {kw}")
        lay = build_layout(cfg)
        kv = make_cache(cfg.kv_dtype, cfg.num_kv_heads, cfg.head_dim, cfg.block_size, lay.num_blocks)
        mirror = PoolMirror(kv)
        rng = np.random.default_rng(cid)
        H, D = cfg.num_kv_heads, cfg.head_dim
        kk = rng.normal(0, 1, (len(lay.fill_slots), H, D)).astype(np.float32)
        vv = rng.normal(0, 1, (len(lay.fill_slots), H, D)).astype(np.float32)
        if cfg.kv_dtype == "fp8":
            ks, vs = per_head_amax_scales(kk), per_head_amax_scales(vv)
            kv.set_head_scales(0, ks, vs)
            mirror.set_head_scales(ks, vs)
        append_rows(kv, mirror, kk, vv, lay.fill_slots, "bf16")
        # The verify step's own append, then attention.
        R = cfg.rows
        ka = rng.normal(0, 1, (len(lay.append_slots), H, D)).astype(np.float32)
        va = rng.normal(0, 1, (len(lay.append_slots), H, D)).astype(np.float32)
        append_rows(kv, mirror, ka, va, lay.append_slots, "bf16")
        mirror.compare_with_device()
        mirror.sync_from_device()
        q = torch.randn(cfg.num_seqs, R, cfg.num_q_heads, D, dtype=torch.bfloat16, device="cuda")
        out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
        kv.attention(0, q, out, torch.from_numpy(lay.keys).cuda(), torch.from_numpy(lay.block_tables).cuda(),
                     1 / math.sqrt(D), partition_tokens=cfg.partition)
        torch.cuda.synchronize()
        ksc, vsc = mirror.scales_for_oracle()
        ref = ora.attention(q.float().cpu().numpy(), mirror.kc, mirror.vc, cfg.kv_dtype, H, D, cfg.block_size,
                            lay.keys, lay.block_tables, 1 / math.sqrt(D), ksc, vsc)
        err = rel_err_per_vector(out.cpu().numpy(), ref)
        print(f"  config {cid}: rel err {err:.2e}")
        assert err <= TOL[cfg.kv_dtype]
        kv.close()


def _random_case(seed):
    """A seeded random attention case: pool type, geometry (MFMA tiling or not), contexts
    (some empty or single-key), row counts, partition, query type and value spread."""
    r = np.random.default_rng(1000 + seed)
    dt = ["bf16", "f16", "fp8", "int8", "f32"][seed % 5]
    H = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 4, 8]))
    R = int(r.integers(1, 10))
    D = 128 if dt != "f32" and r.random() < 0.8 else int(r.choice([64, 96, 128]))
    B = int(r.integers(1, 7))
    ctx = [int(x) for x in r.integers(0, 1500, B)]
    if B > 1:
        ctx[int(r.integers(0, B))] = int(r.choice([0, 1, 15, 16, 17, 63, 64, 65]))
    rows = [int(x) for x in r.integers(0, R + 1, B)] if r.random() < 0.4 else None
    return dict(dt=dt, B=B, R=R, Hq=H * G, H=H, D=D, bs=16, ctx=ctx, partition=int(r.choice([0, 0, 64, 256])),
                src=str(r.choice(["f32", "bf16"])), seed=seed, q_dt=str(r.choice(["f32", "bf16", "f16"])),
                row_counts=rows, kv_sd=float(r.choice([0.5, 1.0, 3.0])))


@pytest.mark.parametrize("seed", range(48))
def test_attention_random_cases(gpu, seed):
    """Seeded random cases across pool types, geometries (both kernels), contexts, row
    counts, partitions and query types, against the oracle at the north-star tolerances."""
    c = _random_case(seed)
    say(f"attention random case {seed}: {c}")
    err = run_attention_case(**c)
    print(f"  rel err {err:.2e}")
    assert err <= TOL[c["dt"]]


@pytest.mark.parametrize("seed", range(4))
def test_attention_random_long_contexts(gpu, seed):
    """Seeded long contexts (8k-32k keys) with R = 9 verify rows on the 8B geometry (three
    row tiles; the automatic schedule, which is stream-K at this batch, and the 512-token
    partition grid), against the fp64 oracle at the north-star tolerance."""
    r = np.random.default_rng(3000 + seed)
    dt = ["int8", "fp8", "bf16", "int8"][seed]
    B = 2
    ctx = [int(x) for x in r.integers(8192, 32768, B)]
    partition = [0, 512][seed % 2]
    c = dict(dt=dt, B=B, R=9, Hq=32, H=8, D=128, bs=16, ctx=ctx, partition=partition, src="bf16", seed=seed,
             q_dt="bf16")
    say(f"attention random long-context case {seed}: dt={dt} ctx={ctx} partition={partition}")
    err = run_attention_case(**c)
    print(f"  rel err {err:.2e}")
    assert err <= TOL[dt]


@pytest.mark.parametrize("seed", range(10))
def test_attention_random_lpt_cases(gpu, seed):
    """Seeded random batches large enough for the LPT schedule (items fill half the
    resident workgroup slots or more): ragged short contexts, empty sequences, random row
    counts, one to three row tiles, every MFMA pool type; against the oracle."""
    r = np.random.default_rng(2000 + seed)
    dt = ["bf16", "f16", "fp8", "int8"][seed % 4]
    H = 8
    G = int(r.choice([1, 2, 4]))
    R = int(r.integers(1, 10))
    B = int(r.integers(40, 120))
    ctx = [int(x) for x in r.integers(0, 400, B)]
    for i in r.integers(0, B, 4):
        ctx[int(i)] = int(r.choice([0, 1, 16, 63, 64, 65, 1500]))
    rows = [int(x) for x in r.integers(0, R + 1, B)] if r.random() < 0.5 else None
    c = dict(dt=dt, B=B, R=R, Hq=H * G, H=H, D=128, bs=16, ctx=ctx, src="bf16", seed=seed, q_dt="bf16",
             row_counts=rows)
    say(f"attention random LPT case {seed}: dt={dt} B={B} R={R} G={G} rows={'ragged' if rows else 'all'}")
    err = run_attention_case(**c)
    print(f"  rel err {err:.2e}")
    assert err <= TOL[dt]


@pytest.mark.parametrize("dt,long_ctx", [("fp8", 3000), ("bf16", 9000), ("int8", 5000)])
def test_attention_lpt_remainder_pieces(gpu, dt, long_ctx):
    """LPT with more items than slots (72 sequences x 8 kv heads): an item longer than T
    is cut into pieces of T chunks and a shorter last piece, which runs at the end; the
    records are numbered by (sequence, piece, kv head) and the piece that finishes last
    merges them. Every sequence against the oracle."""
    r = np.random.default_rng(3300 + long_ctx)
    B = 72
    ctx = [int(x) for x in r.integers(32, 300, B)]
    ctx[int(r.integers(0, B))] = long_ctx
    c = dict(dt=dt, B=B, R=6, Hq=32, H=8, D=128, bs=16, ctx=ctx, src="bf16", seed=long_ctx, q_dt="bf16")
    say(f"attention LPT remainder pieces: dt={dt} long context {long_ctx}")
    err = run_attention_case(**c)
    print(f"  rel err {err:.2e}")
    assert err <= TOL[dt]

@pytest.mark.parametrize("dt,long_ctx", [("fp8", 24000), ("bf16", 9000), ("int8", 16000)])
def test_attention_lpt_item_split_many_ways(gpu, dt, long_ctx):
    """LPT with one long sequence among short ones: its items are cut into many pieces
    (tens), and the piece of each item that finishes last merges all of their records
    inside the launch. Every sequence against the oracle."""
    r = np.random.default_rng(3100 + long_ctx)
    B = 40
    ctx = [int(x) for x in r.integers(32, 300, B)]
    ctx[int(r.integers(0, B))] = long_ctx
    c = dict(dt=dt, B=B, R=6, Hq=32, H=8, D=128, bs=16, ctx=ctx, src="bf16", seed=long_ctx, q_dt="bf16")
    say(f"attention LPT many-piece split: dt={dt} long context {long_ctx}")
    err = run_attention_case(**c)
    print(f"  rel err {err:.2e}")
    assert err <= TOL[dt]


@pytest.mark.parametrize("R", [1, 6, 9])  # one, two and three row tiles (G = 4, D = 128)
def test_attention_int8_zero_scale_blocks(gpu, R):
    """PER_BLOCK INT8 blocks whose scale is 0: a block never written (block 0, which missing
    table entries and keys past the context read) and blocks whose rows are all zero
    (amax 0). Masked keys in them must get weight 0, not NaN; against the oracle."""
    say(f"attention int8 zero-scale blocks R={R}")
    B, Hq, H, D, bs = 3, 32, 8, 128, 16
    keys = np.array([40, 70, 10], np.int32) + R
    nbs = [(int(k) + bs - 1) // bs for k in keys]
    nb = sum(nbs) + 3
    rng = np.random.default_rng(77 + R)
    perm = 1 + rng.permutation(nb - 1)  # block 0 stays unwritten
    bt = np.zeros((B, max(nbs) + 1), np.int32)
    p = 0
    for b in range(B):
        bt[b, :nbs[b]] = perm[p:p + nbs[b]]
        p += nbs[b]
    kv = make_cache("int8", H, D, bs, nb)
    mirror = PoolMirror(kv)
    slots, kk, vv = [], [], []
    for b in range(B):
        for t in range(int(keys[b])):
            slots.append(bt[b, t // bs] * bs + t % bs)
            zero = (b == 0 and t >= 32) or b == 2  # sequence 0's third block, all of sequence 2
            kk.append(np.zeros((H, D), np.float32) if zero else rng.normal(0, 1, (H, D)).astype(np.float32))
            vv.append(np.zeros((H, D), np.float32) if zero else rng.normal(0, 1, (H, D)).astype(np.float32))
    append_rows(kv, mirror, np.stack(kk), np.stack(vv), np.array(slots, np.int32), "f32")
    mirror.sync_from_device()
    ks, _ = mirror.scales_for_oracle()
    assert ks.reshape(nb, H)[bt[0, 2]].max() == 0 and ks.reshape(nb, H)[0].max() == 0
    q = rng.normal(0, 1, (B, R, Hq, D)).astype(np.float32)
    qt = torch.from_numpy(q).to(torch.bfloat16).cuda()
    qh = qt.float().cpu().numpy()
    for part in (0, 64):
        out = torch.zeros(B, R, Hq, D, dtype=torch.float32, device="cuda")
        kv.attention(0, qt, out, torch.from_numpy(keys).cuda(), torch.from_numpy(bt).cuda(), 1 / math.sqrt(D),
                     partition_tokens=part)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ksc, vsc = mirror.scales_for_oracle()
        ref = ora.attention(qh, mirror.kc, mirror.vc, "int8", H, D, bs, keys, bt, 1 / math.sqrt(D), ksc, vsc)
        assert np.isfinite(got).all()
        # Sequence 2 attends to zero values only: its output is exactly 0.
        assert not got[2].any()
        err = rel_err_per_vector(got[:2], ref[:2])
        print(f"  partition {part}: rel err {err:.2e}")
        assert err <= TOL["int8"]
    kv.close()


@pytest.mark.parametrize("dt", ["bf16", "fp8", "int8", "f32"])
def test_attention_boundary_cases(gpu, dt):
    """Context of one key, a sequence with no rows, one with more rows than keys, key
    blocks with out-of-range ids (skipped), and a context beyond the table width
    (clamped): the ABI's boundary rules, checked against the oracle's. bf16/fp8/int8
    take the MFMA path (Hq=32, Hkv=8, D=128, R=6), f32 the generic path."""
    say(f"attention boundary cases dt={dt}")
    B, R, Hq, H, D, bs = 6, 6, 32, 8, 128, 16
    nb = 24
    rng = np.random.default_rng(31)
    perm = rng.permutation(nb)
    max_blocks = 4
    bt = np.zeros((B, max_blocks), np.int32)
    ctx = np.array([1, 40, 3, 50, 64, 30], np.int32)   # keys incl. the verify rows
    rows = np.array([1, 0, 6, 6, 6, 6], np.int32)       # seq 1: no rows; seq 2: 6 rows > 3 keys
    fill = []
    p = 0
    for b in range(B):
        nblk = (int(min(ctx[b], max_blocks * bs)) + bs - 1) // bs
        bt[b, :nblk] = perm[p:p + nblk]
        p += nblk
        fill += [bt[b, t // bs] * bs + t % bs for t in range(min(int(ctx[b]), max_blocks * bs))]
    bt[3, 1] = -1          # a skipped block in the middle of sequence 3
    bt[4, 2] = nb + 100    # an id past the pool in sequence 4
    ctx[5] = 10 ** 6       # beyond the table: clamped to max_blocks * bs
    bt[5, :] = perm[p:p + max_blocks]
    fill += [bt[5, t // bs] * bs + t % bs for t in range(max_blocks * bs)]
    slots = np.unique(np.array(fill, np.int32))
    kv = make_cache(dt, H, D, bs, nb)
    mirror = PoolMirror(kv)
    kk = rng.normal(0, 1, (len(slots), H, D)).astype(np.float32)
    vv = rng.normal(0, 1, (len(slots), H, D)).astype(np.float32)
    if dt == "fp8":
        ks, vs = per_head_amax_scales(kk), per_head_amax_scales(vv)
        kv.set_head_scales(0, ks, vs)
        mirror.set_head_scales(ks, vs)
    append_rows(kv, mirror, kk, vv, slots, "f32")
    mirror.sync_from_device()
    q = torch.randn(B, R, Hq, D, dtype=torch.float32, generator=torch.Generator().manual_seed(3)).cuda()
    sentinel = 7.0
    out = torch.full((B, R, Hq, D), sentinel, dtype=torch.float32, device="cuda")
    kv.attention(0, q, out, torch.from_numpy(ctx).cuda(), torch.from_numpy(bt).cuda(), 1 / math.sqrt(D),
                 row_counts=torch.from_numpy(rows).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ksc, vsc = mirror.scales_for_oracle()
    ref = ora.attention(q.cpu().numpy(), mirror.kc, mirror.vc, dt, H, D, bs, ctx, bt, 1 / math.sqrt(D), ksc, vsc,
                        row_counts=rows)
    # Untouched: rows past each sequence's row count, the row-less sequence, the sequence
    # with more rows than keys.
    for b in range(B):
        n = 0 if b in (1, 2) else rows[b]
        assert (got[b, n:] == sentinel).all(), f"seq {b}: rows >= {n} written"
    written = [(b, j) for b in range(B) for j in range(R) if b not in (1, 2) and j < rows[b]]
    g = np.stack([got[b, j] for b, j in written])
    r = np.stack([ref[b, j] for b, j in written])
    err = rel_err_per_vector(g, r)
    print(f"  boundary {dt}: rel err {err:.2e}")
    assert err <= TOL[dt]
    kv.close()


def _full_config_case(cid):
    """A config at its real shape, one layer, pools filled on the GPU; returns the
    pieces the full-size checks need."""
    cfg = scaled(CONFIGS[cid], layers=1)
    lay = build_layout(cfg)
    H, D, bs = cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    kv = make_cache(cfg.kv_dtype, H, D, bs, lay.num_blocks)
    gen = torch.Generator(device="cuda").manual_seed(cfg.seed)
    if cfg.kv_dtype == "fp8":
        # Values ~N(0,1): scales from a fixed amax of 4.5 (saturating the rare tail).
        kv.set_head_scales(0, [4.5 / 448] * H, [4.5 / 448] * H)
    # The context, then the step's own rows, in separate calls (INT8 pools need a block's
    # rows adjacent within one call).
    for part in (lay.fill_slots, lay.append_slots):
        slots = torch.from_numpy(part).cuda()
        for s in range(0, len(slots), 1 << 16):
            m = min(1 << 16, len(slots) - s)
            kx = torch.randn(m, H, D, device="cuda", dtype=torch.bfloat16, generator=gen)
            vx = torch.randn(m, H, D, device="cuda", dtype=torch.bfloat16, generator=gen)
            kv.append(0, kx, vx, slots[s:s + m])
    q = torch.randn(cfg.num_seqs, cfg.rows, cfg.num_q_heads, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    keys = torch.from_numpy(lay.keys).cuda()
    bt = torch.from_numpy(lay.block_tables).cuda()
    torch.cuda.synchronize()
    return cfg, lay, kv, q, keys, bt


@pytest.mark.parametrize("cid,explicit", [(2, 1024), (3, 1024), (4, 512), (5, 2048)])
def test_attention_full_size_configs(gpu, cid, explicit):
    """Configs 2-5 at their real sizes. Size-independent property over every sequence:
    the automatic schedule (LPT pieces, split items merged inside the launch) equals an
    explicit partition grid to 1e-3 (the schedules round P to the MFMA
    type against different running maxima). Then the two shortest sequences against the
    fp64 oracle at the north-star tolerance: the two shortest sequences and the longest
    (config 3's ~8k-key FP8 contexts, config 4's 16k-32k-key INT8 ones), so that deep
    block-table indices, per-block scales far into the table and merges of many pieces
    are checked against textbook attention too."""
    say(f"attention full-size config {cid}")
    cfg, lay, kv, q, keys, bt = _full_config_case(cid)
    D = cfg.head_dim
    scale = 1 / math.sqrt(D)
    outs = {}
    for p in (0, explicit):
        ws = kv.attention_workspace(cfg.num_seqs, cfg.rows, cfg.num_q_heads, bt.shape[1], p)
        o = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
        kv.attention(0, q, o, keys, bt, scale, partition_tokens=p, workspace=ws)
        torch.cuda.synchronize()
        outs[p] = o.cpu().numpy()
    agree = rel_err_per_vector(outs[0], outs[explicit])
    print(f"  config {cid}: auto vs partition {explicit}: rel diff {agree:.2e}")
    assert agree <= 1e-3
    # The step's schedule computed once (gg_verify_attention_plan), then a planned call:
    # identical to the call that plans for itself.
    ws = kv.attention_workspace(cfg.num_seqs, cfg.rows, cfg.num_q_heads, bt.shape[1], 0)
    kv.attention_plan(keys, cfg.rows, cfg.num_q_heads, bt.shape[1], ws)
    o = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    for _ in range(3):  # the plan serves any number of calls (each clears its merge counters)
        o.zero_()
        kv.attention(0, q, o, keys, bt, scale, workspace=ws, planned=True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(o.cpu().numpy(), outs[0])
    order = np.argsort(lay.keys, kind="stable")
    idx = np.array(sorted({int(order[0]), int(order[1]), int(order[-1])}))
    k_s = v_s = None
    if cfg.kv_dtype == "fp8":
        a, b = kv.scales(0)
        k_s, v_s = a.cpu().numpy()[:cfg.num_kv_heads], b.cpu().numpy()[:cfg.num_kv_heads]
    elif cfg.kv_dtype == "int8":
        a, b = kv.scales(0)
        k_s, v_s = a.float().cpu().numpy().reshape(-1), b.float().cpu().numpy().reshape(-1)
    say(f"  oracle on sequences {idx.tolist()} (keys {lay.keys[idx].tolist()})")
    ref = ora.attention(q[idx].float().cpu().numpy(), kv.k_pool(0).cpu().numpy(), kv.v_pool(0).cpu().numpy(),
                        cfg.kv_dtype, cfg.num_kv_heads, D, cfg.block_size, lay.keys[idx], lay.block_tables[idx],
                        scale, k_s, v_s, threads=min(os.cpu_count() or 1, 16))
    err = rel_err_per_vector(outs[0][idx], ref)
    print(f"  config {cid}: oracle rel err {err:.2e}")
    assert err <= TOL[cfg.kv_dtype]
    kv.close()


# ------------------------------------------------------------------ fused append + attention

def _derived_slots(lay, rows, bs, row_counts=None):
    """Slots of the verify rows from the block tables (row b*R + j -> key position
    keys[b] - row_count + j); -1 for rows past the row count."""
    B = len(lay.keys)
    slots = np.full(B * rows, -1, np.int32)
    for b in range(B):
        n = rows if row_counts is None else int(row_counts[b])
        for j in range(n):
            pos = int(lay.keys[b]) - n + j
            slots[b * rows + j] = int(lay.block_tables[b, pos // bs]) * bs + pos % bs
    return slots


@pytest.mark.parametrize("cid,dt,B,ctx,rc", [
    (3, "fp8", 64, ("uniform", 1024, 4096), False),   # LPT: append launch, then attention
    (5, "bf16", 64, ("uniform", 300, 2100), True),    # LPT, ragged row counts
    (2, "f16", 6, ("uniform", 512, 3000), False),     # stream-K: append launch, then attention
    (1, "f32", 4, ("list", 64, 128, 192, 256), True),  # generic path
    # Draft rows straddling chunk boundaries (64-token chunks for FP8, 32 for bf16), rows in
    # a piece's first chunks (short contexts), and long items that LPT splits.
    (3, "fp8", 64, ("list", *[64 * (1 + (i * 37) % 128) + (59, 60, 61, 62, 63, 0, 1, 30)[i % 8] for i in range(64)]),
     False),
    (5, "bf16", 64, ("list", *[32 * (1 + (i * 13) % 64) + (27, 28, 29, 30, 31, 0, 1, 16)[i % 8] for i in range(64)]),
     True),
    # More sequences than the LPT plan ranks: one workgroup per (sequence, kv head).
    (3, "fp8", 1100, ("uniform", 20, 400), True),
    # FP8 at three row tiles (32-token chunks, rows appended by the whole workgroup before
    # the piece starts): stream-K with few items, and LPT with rows straddling chunks.
    (4, "fp8", 8, ("uniform", 1000, 6000), True),
    (4, "fp8", 64, ("list", *[32 * (1 + (i * 13) % 64) + (27, 28, 29, 30, 31, 0, 1, 16)[i % 8] for i in range(64)]),
     False),
])
def test_append_attention_fused_equals_separate(gpu, cid, dt, B, ctx, rc):
    """gg_verify_append_attention_planned == gg_kv_append (slots from the block tables)
    followed by gg_verify_attention_planned: pool bytes and outputs bit for bit."""
    say(f"fused append+attention config {cid} dt={dt} B={B} row_counts={rc}")
    _fused_vs_separate(cid, dt, B, ctx, rc)


@pytest.mark.parametrize("dt", ["fp8", "bf16"])
def test_append_attention_fused_with_missing_blocks(gpu, dt):
    """Block-table entries outside the pool (or negative) where draft rows land: both paths
    skip those rows and mask those keys, so pools and outputs still agree bit for bit."""
    say(f"fused append+attention with missing blocks dt={dt}")
    _fused_vs_separate(3 if dt == "fp8" else 5, dt, 64, ("uniform", 300, 3000), False, corrupt=True)


def _fused_vs_separate(cid, dt, B, ctx, rc, corrupt=False):
    cfg = scaled(CONFIGS[cid], num_seqs=B, ctx=ctx, layers=1, kv_dtype=dt)
    lay = build_layout(cfg)
    H, D, bs, R, Hq = cfg.num_kv_heads, cfg.head_dim, cfg.block_size, cfg.rows, cfg.num_q_heads
    if corrupt:
        # Every fifth sequence: the block holding its last draft row leaves the pool (odd
        # sequences: past its end, even ones: negative). The context fill below still uses
        # the layout's own slots.
        tables = lay.block_tables.copy()
        for b_ in range(0, B, 5):
            pos = int(lay.keys[b_]) - 1
            tables[b_, pos // bs] = lay.num_blocks + 3 if b_ % 2 else -2
        lay = type(lay)(**{**lay.__dict__, "block_tables": tables})
    gen = torch.Generator(device="cuda").manual_seed(cfg.seed + 11)
    fill = torch.from_numpy(lay.fill_slots).cuda()
    kx = torch.randn(len(fill), H, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    vx = torch.randn(len(fill), H, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    k_new = torch.randn(B * R, H, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    v_new = torch.randn(B * R, H, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    q = torch.randn(B, R, Hq, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    row_counts = None
    if rc:
        row_counts = np.random.default_rng(cid).integers(1, R + 1, B).astype(np.int32)
    slots = _derived_slots(lay, R, bs, row_counts)
    if row_counts is None and not corrupt:
        np.testing.assert_array_equal(slots, lay.append_slots)  # the layout's own slots
    keys = torch.from_numpy(lay.keys).cuda()
    bt = torch.from_numpy(lay.block_tables).cuda()
    rc_t = torch.from_numpy(row_counts).cuda() if row_counts is not None else None
    results = []
    for fused in (True, False):
        kv = make_cache(dt, H, D, bs, lay.num_blocks)
        if dt == "fp8":
            kv.set_head_scales(0, [4.5 / 448] * H, [4.5 / 448] * H)
        kv.append(0, kx, vx, fill)
        ws = kv.attention_workspace(B, R, Hq, bt.shape[1], 0)
        kv.attention_plan(keys, R, Hq, bt.shape[1], ws, row_counts=rc_t)
        out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
        if fused:
            kv.append_attention(0, k_new, v_new, q, out, keys, bt, 1 / math.sqrt(D), ws, row_counts=rc_t)
        else:
            kv.append(0, k_new, v_new, torch.from_numpy(slots).cuda())
            kv.attention(0, q, out, keys, bt, 1 / math.sqrt(D), row_counts=rc_t, workspace=ws, planned=True)
        torch.cuda.synchronize()
        sc = kv.scales(0) if dt in ("fp8", "int8") else (torch.zeros(1), torch.zeros(1))
        results.append((kv.k_pool(0).cpu().numpy(), kv.v_pool(0).cpu().numpy(), out.cpu().numpy(),
                        tuple(t.float().cpu().numpy() for t in sc)))
        kv.close()
    (fk, fv, fo, fsc), (sk, sv, so, ssc) = results
    np.testing.assert_array_equal(fk, sk)
    np.testing.assert_array_equal(fv, sv)
    for a_, b_ in zip(fsc, ssc):  # PER_HEAD scales as set; PER_BLOCK scales as the appends left them
        np.testing.assert_array_equal(a_, b_)
    if rc:  # rows past a sequence's row count are not computed
        for b in range(B):
            fo[b, row_counts[b]:] = so[b, row_counts[b]:] = 0
    np.testing.assert_array_equal(fo, so)


@pytest.mark.parametrize("cid,B,ctx,rc", [
    (4, 8, ("uniform", 16384, 32768), False),     # config 4 shape: LPT, one CU slot per workgroup
    (4, 16, ("uniform", 100, 2000), True),        # ragged row counts, runs starting mid-block
    (4, 3, ("list", 15, 16, 33), False),          # stream-K, rows filling and opening blocks
    (4, 24, ("list", *[16 * i + (i % 5) for i in range(1, 25)]), False),  # runs straddling blocks
])
def test_append_attention_fused_per_block_int8(gpu, cid, B, ctx, rc):
    """PER_BLOCK INT8: gg_verify_append_attention_planned equals gg_kv_append with the
    derived slots followed by the planned attention: pool bytes, block scales and outputs
    bit for bit (a block's new rows re-scale it, and the rows already in it are
    re-quantised when its scale grows)."""
    say(f"fused append int8 cid={cid} B={B} ctx={ctx} rc={rc}")
    _fused_vs_separate(cid, "int8", B, ctx, rc)
