"""GPU parity: greedy Verify with the bonus token drawn by Sampler.Sample
(gg_accept_greedy_sample), bit-exact against the oracle's float64 restatement of
internal/engine/sampling.go:40-192 (ora_accept_greedy_sample / ora_emit_positions).

Every case runs twice: the normal path (parallel float64 sums, sequential replay only for
rows too close to a boundary) and GG_SAMPLE_EXACT (every draw replayed sequentially), so both
device paths are pinned to the same oracle."""
import numpy as np
import pytest
import torch

import gollmgo_amd.verify as gv
from helpers import say
from oracle import oracle as ora

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def case(B, K, V, dt, seed, sd=2.0, accept_all=0.8):
    """Logits ~ N(0, sd) in dt; with probability accept_all a sequence's drafts are its rows'
    argmaxes, so it reaches the bonus draw."""
    rng = np.random.default_rng(seed)
    lg = torch.from_numpy(rng.normal(0, sd, (B, K + 1, V)).astype(np.float32)).to(TD[dt])
    host = lg.float().numpy()
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    for b in range(B):
        if rng.random() < accept_all:
            for j in range(K):
                drafts[b, j] = ora.argmax(host[b, j])
    n = rng.integers(0, K + 1, B).astype(np.int32)
    u = rng.random(B)
    return lg, host, drafts, n, u


def run(lg, drafts, n, u, T, top_k, top_p, flags=0):
    acc, tok = gv.accept_greedy_sample(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(),
                                       torch.from_numpy(np.ascontiguousarray(u, np.float64)).cuda(), T, top_k,
                                       top_p, flags)
    torch.cuda.synchronize()
    return acc.cpu().numpy(), tok.cpu().numpy()


def check(lg, host, drafts, n, u, T, top_k, top_p, label):
    ea, et = ora.accept_greedy_sample(host, drafts, n, T, top_k, top_p, u, threads=16)
    for flags in (0, gv.SAMPLE_EXACT):
        say(f"{label} flags={flags}")
        acc, tok = run(lg, drafts, n, u, T, top_k, top_p, flags)
        bad = np.nonzero((acc != ea) | (tok != et))[0]
        assert bad.size == 0, (label, flags, bad[:5], acc[bad[:5]], ea[bad[:5]], tok[bad[:5]], et[bad[:5]])
    return ea, et


@pytest.mark.parametrize("T,top_k,top_p", [(0.8, 0, 0.0), (0.8, 50, 0.0), (0.8, 0, 0.95), (1.3, 50, 0.9),
                                           (0.6, 1, 0.5), (1.0, 4095, 0.99), (0.0, 50, 0.95)])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_sample_small_vocab(gpu, dt, T, top_k, top_p):
    lg, host, drafts, n, u = case(24, 3, 5003, dt, seed=int(T * 100) + top_k + int(top_p * 1000))
    check(lg, host, drafts, n, u, T, top_k, top_p, f"small dt={dt} T={T} k={top_k} p={top_p}")


@pytest.mark.parametrize("shape,dt", [((32, 4, 128256), "bf16"), ((8, 8, 128256), "bf16")])
@pytest.mark.parametrize("top_k,top_p", [(0, 0.0), (50, 0.0), (0, 0.95), (50, 0.95)])
def test_sample_config_shapes_via_emit_positions(gpu, shape, dt, top_k, top_p):
    """Configs 2 and 4 at T = 0.8: the device decision equals what emitSpeculative would
    compute from the full rows (ora_emit_positions reads them as Go slices)."""
    B, K, V = shape
    lg, host, drafts, n, u = case(B, K, V, dt, seed=B * 100 + K + top_k)
    say(f"config shape={shape} k={top_k} p={top_p}")
    ea, et = ora.emit_positions(drafts, n, [[host[b, j] for j in range(K + 1)] for b in range(B)], 0.8, top_p, u,
                                top_k=top_k)
    for flags in (0, gv.SAMPLE_EXACT):
        acc, tok = run(lg, drafts, n, u, 0.8, top_k, top_p, flags)
        assert np.array_equal(acc, ea) and np.array_equal(tok, et), (flags, acc, ea, tok, et)
    assert (ea == np.clip(n, 0, K)).sum() >= B // 4  # enough bonus draws


def test_sample_uniforms_on_cdf_boundaries(gpu):
    """u placed exactly on, and one ulp below, float64 CDF boundaries of the rule: the
    parallel sums cannot decide these, so the sequential replay must."""
    B, K, V = 40, 0, 20011
    rng = np.random.default_rng(5)
    host = rng.normal(0, 2, (B, 1, V)).astype(np.float32)
    lg = torch.from_numpy(host)
    drafts = np.zeros((B, 0), np.int32)
    n = np.zeros(B, np.int32)
    for top_k, top_p in [(0, 0.0), (0, 0.9), (100, 0.0), (100, 0.8)]:
        u = np.empty(B)
        for b in range(B):
            c = np.cumsum(ora.sampler_probs_f64(host[b, 0], 0.8, top_k, top_p))
            nz = np.nonzero(np.diff(c) > 0)[0]
            i = int(nz[rng.integers(0, len(nz))])
            u[b] = c[i] if b % 2 == 0 else np.nextafter(c[i], 0.0)
        check(lg, host, drafts, n, u, 0.8, top_k, top_p, f"boundaries k={top_k} p={top_p}")


def test_sample_special_rows(gpu):
    """Rows the fast path hands to the replay (NaN, +inf, all -inf, one bin holding every
    element) and edges of the uniform and the filters."""
    V = 9001
    rng = np.random.default_rng(9)
    rows = []
    r = rng.normal(0, 2, V).astype(np.float32); r[17] = np.nan; rows.append(r)
    r = rng.normal(0, 2, V).astype(np.float32); r[0] = np.nan; rows.append(r)
    r = rng.normal(0, 2, V).astype(np.float32); r[4000] = np.inf; rows.append(r)
    r = np.full(V, -np.inf, np.float32); rows.append(r)
    r = np.full(V, -np.inf, np.float32); r[123] = 1.0; rows.append(r)
    r = np.full(V, 0.5, np.float32); rows.append(r)                      # every element ties
    r = np.where(rng.random(V) < 0.5, 0.0, -0.0).astype(np.float32); rows.append(r)  # +-0 ties
    r = np.round(rng.normal(0, 2, V) * 4).astype(np.float32) / 4; rows.append(r)     # heavy ties
    r = rng.normal(0, 2, V).astype(np.float32); r[:100] = -np.inf; rows.append(r)
    r = (rng.normal(0, 1, V) * 1e-9).astype(np.float32); rows.append(r)  # tiny logits
    host = np.stack(rows)[:, None, :]
    B = host.shape[0]
    lg = torch.from_numpy(host)
    drafts = np.zeros((B, 0), np.int32)
    n = np.zeros(B, np.int32)
    for T, top_k, top_p in [(0.8, 0, 0.0), (0.8, 10, 0.0), (0.8, 0, 0.5), (2.0, 3000, 0.7), (1e30, 0, 0.0),
                            (2e-9, 0, 0.0)]:
        for u in (0.0, 0.5, 0.999999999, 1.0 - 2.0 ** -53):
            check(lg, host, drafts, n, np.full(B, u), T, top_k, top_p, f"special T={T} k={top_k} p={top_p} u={u}")


def test_sample_matches_greedy_at_zero_temperature(gpu):
    lg, host, drafts, n, u = case(16, 5, 32000, "bf16", seed=77)
    say("sample T=0 vs greedy")
    acc, tok = run(lg, drafts, n, u, 0.0, 50, 0.9)
    ga, gt = gv.accept_greedy(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(acc, ga.cpu().numpy()) and np.array_equal(tok, gt.cpu().numpy())


def _residual_boundary_uniforms(host, drafts, acc, n, q, T, top_p, rng):
    """For sequences that stop at a rejection, u on (and one ulp below) a float64 CDF
    boundary of the residual draw; others keep a random u."""
    B, R, V = host.shape
    K = R - 1
    u = rng.random(B)
    for b in range(B):
        a = int(acc[b])
        if a >= n[b]:
            continue
        p = ora.sampler_probs_f64(host[b, a], T, 0, top_p)
        qq = np.zeros(V) if q is None else np.where((q[b, a] > 0) & np.isfinite(q[b, a]), np.minimum(q[b, a], 1), 0)
        r = np.where(p > qq, p - qq, 0.0)
        r[int(drafts[b, a])] = 0.0
        s = np.cumsum(r)[-1]
        if not s > 0:
            continue
        c = np.cumsum(r / s)
        nz = np.nonzero(np.diff(c) > 0)[0]
        if len(nz):
            i = int(nz[rng.integers(0, len(nz))])
            u[b] = c[i] if b % 2 == 0 else np.nextafter(c[i], 0.0)
    return u


@pytest.mark.parametrize("dense,top_p", [(False, 1.0), (False, 0.9), (True, 1.0), (True, 0.8)])
def test_rejection_draw_on_boundaries(gpu, dense, top_p):
    """The rejection acceptance's final draw (float64, the sample module's residual mode)
    with the draw's uniform on residual CDF boundaries: the parallel sums cannot decide
    these, so the sequential replay does; the decisions stay equal to the oracle's."""
    B, K, V, T = 48, 3, 6007, 0.8
    rng = np.random.default_rng(31 + int(dense) + int(top_p * 10))
    host = rng.normal(0, 2, (B, K + 1, V)).astype(np.float32)
    q = rng.dirichlet(np.ones(V) * 0.3, (B, K)).astype(np.float32) if dense else None
    drafts = host[:, :K].argmax(-1).astype(np.int32)
    mask = rng.random((B, K)) < 0.5
    drafts[mask] = rng.integers(0, V, int(mask.sum()))
    n = np.full(B, K, np.int32)
    u = rng.random((B, K + 1)).astype(np.float32)
    acc, _ = ora.accept_rejection(host, drafts, n, u, T, top_p, q)
    ufin = _residual_boundary_uniforms(host, drafts, acc, n, q, float(np.float32(T)), float(np.float32(top_p)), rng)
    u[:, K] = ufin.astype(np.float32)  # rounded to float32: still on or next to a boundary
    ea, et = ora.accept_rejection(host, drafts, n, u, T, top_p, q)
    say(f"rejection boundaries dense={dense} top_p={top_p}")
    ga, gt = gv.accept_rejection(torch.from_numpy(host).cuda(), torch.from_numpy(drafts).cuda(),
                                 torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda(), T, top_p,
                                 torch.from_numpy(q).cuda() if dense else None)
    torch.cuda.synchronize()
    assert np.array_equal(ga.cpu().numpy(), ea) and np.array_equal(gt.cpu().numpy(), et)
    assert (ea < n).sum() > B // 4


def test_rejection_special_final_rows(gpu):
    """NaN / +inf in the final row and a draft distribution that is all ones (every residual
    0: the fallback to the row without the draft)."""
    B, K, V = 8, 1, 3001
    rng = np.random.default_rng(41)
    host = rng.normal(0, 2, (B, K + 1, V)).astype(np.float32)
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    host[0, 0, 5] = np.nan
    host[1, 1, 7] = np.inf
    host[2, 0, :] = -np.inf
    host[2, 0, 3] = 0.0
    q = np.ones((B, K, V), np.float32)
    n = np.full(B, K, np.int32)
    u = rng.random((B, K + 1)).astype(np.float32)
    for dq in (None, q):
        ea, et = ora.accept_rejection(host, drafts, n, u, 0.8, 0.9, dq)
        say(f"rejection special rows dense={dq is not None}")
        ga, gt = gv.accept_rejection(torch.from_numpy(host).cuda(), torch.from_numpy(drafts).cuda(),
                                     torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda(), 0.8, 0.9,
                                     torch.from_numpy(dq).cuda() if dq is not None else None)
        torch.cuda.synchronize()
        assert np.array_equal(ga.cpu().numpy(), ea) and np.array_equal(gt.cpu().numpy(), et)


@pytest.mark.parametrize("ties,dense", [(False, False), (True, False), (False, True)])
def test_rejection_nucleus_cut_on_float64_boundaries(gpu, ties, dense):
    """top-p (a float32) placed on or next to the float64 rule's cumulative sums of the final
    row: the acceptance's fixed-point nucleus, which the draw takes as its hint of the cut,
    can then name a neighbour of the float64 cut, and the draw has to find the rule's own
    cut. Rows with many equal logits put the cut inside a run of ties."""
    B, K, V, T = 8, 2, 5003, 0.8
    rng = np.random.default_rng(53 + 2 * int(ties) + int(dense))
    row = rng.normal(0, 2, V).astype(np.float32)
    if ties:
        row = (np.round(row * 4) / 4).astype(np.float32)
    host = np.broadcast_to(row, (B, K + 1, V)).copy()
    drafts = np.full((B, K), int(np.argmin(row)), np.int32)  # outside any nucleus: rejected
    n = np.full(B, K, np.int32)
    q = rng.dirichlet(np.ones(V) * 0.3, (B, K)).astype(np.float32) if dense else None
    p = ora.sampler_probs_f64(row, float(np.float32(T)), 0, 0.0)
    order = sorted(range(V), key=lambda i: (-p[i], i))
    c = np.cumsum(p[order])
    ks = [int(k) for k in np.searchsorted(c, np.linspace(0.3, 0.97, 8))]
    misses = 0
    for k in ks:
        for top_p in (np.float32(c[k]), np.nextafter(np.float32(c[k]), np.float32(0)),
                      np.nextafter(np.float32(c[k]), np.float32(1))):
            u = rng.random((B, K + 1)).astype(np.float32)
            ea, et = ora.accept_rejection(host, drafts, n, u, T, float(top_p), q)
            say(f"nucleus boundary ties={ties} dense={dense} k={k} top_p={float(top_p)!r}")
            ga, gt = gv.accept_rejection(torch.from_numpy(host).cuda(), torch.from_numpy(drafts).cuda(),
                                         torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda(), T, float(top_p),
                                         torch.from_numpy(q).cuda() if dense else None)
            torch.cuda.synchronize()
            assert np.array_equal(ga.cpu().numpy(), ea) and np.array_equal(gt.cpu().numpy(), et), (k, top_p)
            misses += int((ea == 0).all())
    assert misses == len(ks) * 3  # every draft rejected, so every call drew from the nucleus


@pytest.mark.parametrize("sd,top_k,top_p", [(4.0, 0, 0.95), (3.0, 2000, 0.9)])
def test_sample_wide_logits_large_vocab(gpu, sd, top_k, top_p):
    """Wide logits over a 2^18 vocab: where a top-p cut falls, a slice of the value's order
    key (1/8 octave) would hold more elements than a gather can take; the draw's coarse bins
    are 1/64-nat slices below the row max, so the parallel path resolves these rows."""
    lg, host, drafts, n, u = case(8, 2, 1 << 18, "f32", seed=71 + int(sd), sd=sd, accept_all=1.0)
    n[:] = 2
    check(lg, host, drafts, n, u, 0.9, top_k, top_p, f"wide sd={sd} k={top_k} p={top_p}")


def test_rejection_dense_draft_close_to_target(gpu):
    """A dense draft distribution within 1e-6 of the target's own probabilities, with the
    drafted token's q doubled so that u >= 0.6 rejects it. Every other element's p and q
    then nearly tie: they are more than the residual draw's list of near-ties holds, so the
    draw falls back to summing the residual from the row's total; the token is the oracle's."""
    B, K, V, T = 16, 2, 20011, 0.8
    rng = np.random.default_rng(61)
    host = rng.normal(0, 2, (B, K + 1, V)).astype(np.float32)
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    q = np.empty((B, K, V), np.float32)
    for b in range(B):
        for j in range(K):
            p = ora.sampler_probs_f64(host[b, j], float(np.float32(T)), 0, 1.0)
            q[b, j] = (p * (1.0 + 1e-6 * rng.standard_normal(V))).astype(np.float32)
            q[b, j, drafts[b, j]] = np.float32(2.0 * p[drafts[b, j]])
    n = np.full(B, K, np.int32)
    u = rng.uniform(0.6, 1.0, (B, K + 1)).astype(np.float32)
    ea, et = ora.accept_rejection(host, drafts, n, u, T, 1.0, q)
    say("rejection dense draft close to target")
    ga, gt = gv.accept_rejection(torch.from_numpy(host).cuda(), torch.from_numpy(drafts).cuda(),
                                 torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda(), T, 1.0,
                                 torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(ga.cpu().numpy(), ea) and np.array_equal(gt.cpu().numpy(), et)
    assert (ea == 0).all()  # every sequence drew from the residual of its first row


@pytest.mark.parametrize("top_k,top_p", [(0, 0.0), (40, 0.0), (0, 0.9)])
def test_sample_without_drafts_and_many_sequences(gpu, top_k, top_p):
    """No drafts (max_drafts 0: every sequence draws its token from row 0, as a plain decode
    step's Sampler.Sample) over 1000 sequences, and a batch of 600 with 2 drafts."""
    for B, K, seed in ((1000, 0, 81), (600, 2, 82)):
        lg, host, drafts, n, u = case(B, K, 3001, "bf16", seed=seed + top_k, accept_all=1.0)
        if K == 0:
            drafts = np.zeros((B, 0), np.int32)
            n = np.zeros(B, np.int32)
        check(lg, host, drafts, n, u, 0.8, top_k, top_p, f"B={B} K={K} k={top_k} p={top_p}")
