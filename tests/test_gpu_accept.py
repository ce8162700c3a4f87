"""GPU parity: greedy and rejection acceptance, bit-exact against the CPU oracle."""
import numpy as np
import pytest
import torch

import gollmgo_amd.verify as gv
from helpers import check_positions, say
from oracle import oracle as ora

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def logits_case(B, K, V, dt, seed, sd=2.0, match_rate=0.6):
    """Logits ~ N(0, sd) in dtype dt; drafts copy the row argmax with probability match_rate
    so accepted lengths spread over [0, K]."""
    rng = np.random.default_rng(seed)
    lg = torch.from_numpy(rng.normal(0, sd, (B, K + 1, V)).astype(np.float32)).to(TD[dt])
    host = lg.float().numpy()
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    for b in range(B):
        for j in range(K):
            if rng.random() < match_rate:
                drafts[b, j] = ora.argmax(host[b, j])
    n = rng.integers(0, K + 1, B).astype(np.int32)
    return lg, host, drafts, n


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", [(4, 4, 32000), (32, 4, 128256), (8, 8, 128256), (3, 0, 1000), (5, 2, 4099)])
def test_greedy_matches_oracle(gpu, dt, shape):
    B, K, V = shape
    say(f"greedy dt={dt} shape={shape}")
    lg, host, drafts, n = logits_case(B, K, V, dt, seed=B * 7 + K + V % 97)
    acc, tok = gv.accept_greedy(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda())
    torch.cuda.synchronize()
    ea, et = ora.accept_greedy(host, drafts, n)
    assert np.array_equal(acc.cpu().numpy(), ea)
    assert np.array_equal(tok.cpu().numpy(), et)


@pytest.mark.parametrize("shape", [(3, 40, 128256), (2, 64, 262144), (4, 17, 1000)])
def test_greedy_many_drafts(gpu, shape):
    """Rows past one pass of the decide block's lane groups (16 rows of 32 segments, 8 rows
    of 64, or many rows of one segment), drafts matching the argmax with probability 0.97
    so accepted lengths reach deep rows; every draft count from 0 to K."""
    B, K, V = shape
    say(f"greedy many drafts shape={shape}")
    lg, host, drafts, n = logits_case(B, K, V, "bf16", seed=K * 31 + B, match_rate=0.97)
    n[0] = K
    if B > 2:
        n[1] = 0
    acc, tok = gv.accept_greedy(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda())
    torch.cuda.synchronize()
    ea, et = ora.accept_greedy(host, drafts, n)
    assert np.array_equal(acc.cpu().numpy(), ea)
    assert np.array_equal(tok.cpu().numpy(), et)


def test_greedy_ties_nan_and_negative_zero(gpu):
    say("greedy ties/nan")
    V = 9000
    rows = np.zeros((6, 2, V), np.float32)
    rows[0, 0, [5, 4000, 8999]] = 3.0                 # tie across segments -> 5
    rows[1, 0, 0] = np.nan; rows[1, 0, 7] = 9          # NaN at index 0 -> 0
    rows[2, 0, :] = np.nan; rows[2, 0, 0] = -5; rows[2, 0, 8000] = 1  # NaN elsewhere never wins -> 8000
    rows[3, 0, :] = -np.inf                            # all -inf -> 0
    rows[4, 0, 10] = -0.0                              # -0 == +0 -> first index 0
    rows[5, 0, :] = -1; rows[5, 0, 4097] = 2; rows[5, 0, 4096] = 2  # segment boundary tie -> 4096
    drafts = np.array([[5], [0], [8000], [0], [0], [4096]], np.int32)
    n = np.ones(6, np.int32)
    for dt in ("f32", "bf16", "f16"):
        lg = torch.from_numpy(rows).to(TD[dt])
        acc, tok = gv.accept_greedy(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda())
        torch.cuda.synchronize()
        ea, et = ora.accept_greedy(lg.float().numpy(), drafts, n)
        assert np.array_equal(acc.cpu().numpy(), ea), dt
        assert np.array_equal(tok.cpu().numpy(), et), dt
        assert acc.cpu().tolist() == [1, 1, 1, 1, 1, 1]


def test_greedy_unaligned_rows(gpu):
    """Odd vocab (rows not 16-byte aligned) takes the scalar path."""
    say("greedy unaligned")
    lg, host, drafts, n = logits_case(7, 3, 5001, "bf16", seed=99)
    acc, tok = gv.accept_greedy(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda())
    torch.cuda.synchronize()
    ea, et = ora.accept_greedy(host, drafts, n)
    assert np.array_equal(acc.cpu().numpy(), ea) and np.array_equal(tok.cpu().numpy(), et)


def rejection_case(B, K, V, dt, seed, with_q, sd=2.0):
    rng = np.random.default_rng(seed)
    lg, host, drafts, n = logits_case(B, K, V, dt, seed, sd=sd, match_rate=0.8)
    q = None
    if with_q:
        # Draft distributions: a sharpened copy of the target row, so acceptances are frequent.
        qn = torch.softmax(torch.from_numpy(host[:, :K] * 1.5), dim=-1).numpy().astype(np.float32)
        q = np.ascontiguousarray(qn)
        for b in range(B):
            for j in range(K):
                if rng.random() < 0.7:
                    drafts[b, j] = int(np.argmax(q[b, j]))
    u = rng.random((B, K + 1)).astype(np.float32)
    return lg, host, drafts, n, q, u


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("with_q", [False, True])
@pytest.mark.parametrize("top_p", [1.0, 0.95, 0.5])
def test_rejection_matches_oracle(gpu, dt, with_q, top_p):
    B, K, V = 6, 5, 128256
    say(f"rejection dt={dt} q={with_q} top_p={top_p}")
    lg, host, drafts, n, q, u = rejection_case(B, K, V, dt, seed=int(top_p * 100) + with_q, with_q=with_q)
    acc, tok = gv.accept_rejection(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(),
                                   torch.from_numpy(u).cuda(), 0.8, top_p,
                                   draft_probs=torch.from_numpy(q).cuda() if q is not None else None)
    torch.cuda.synchronize()
    ea, et = ora.accept_rejection(host, drafts, n, u, 0.8, top_p, q)
    print("  accepted", acc.cpu().tolist(), "of", n.tolist())
    assert np.array_equal(acc.cpu().numpy(), ea)
    assert np.array_equal(tok.cpu().numpy(), et)


def test_rejection_ties_in_nucleus(gpu):
    """Heavily tied bf16 logits: the nucleus boundary cuts through a tie group."""
    say("rejection tied nucleus")
    rng = np.random.default_rng(21)
    B, K, V = 8, 2, 20000
    vals = rng.integers(-3, 3, (B, K + 1, V)).astype(np.float32)
    lg = torch.from_numpy(vals).to(torch.bfloat16)
    host = lg.float().numpy()
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    n = np.full(B, K, np.int32)
    u = rng.random((B, K + 1)).astype(np.float32)
    for top_p in (0.3, 0.77, 0.999):
        acc, tok = gv.accept_rejection(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(),
                                       torch.from_numpy(u).cuda(), 1.0, top_p)
        torch.cuda.synchronize()
        ea, et = ora.accept_rejection(host, drafts, n, u, 1.0, top_p)
        assert np.array_equal(acc.cpu().numpy(), ea), top_p
        assert np.array_equal(tok.cpu().numpy(), et), top_p


def test_rejection_crowded_boundary_bin(gpu):
    """Rows whose boundary coarse bin holds tens of thousands of tied logits (the exact
    row kernel resolves those) next to rows the bin sort resolves, in one call."""
    say("rejection crowded boundary bin")
    rng = np.random.default_rng(33)
    B, K, V = 4, 2, 128256
    host = rng.normal(0, 1.5, (B, K + 1, V)).astype(np.float32)
    host[:2] = rng.integers(-1, 2, (2, K + 1, V)).astype(np.float32)
    lg = torch.from_numpy(host).to(torch.bfloat16)
    host = lg.float().numpy()
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    n = np.full(B, K, np.int32)
    u = rng.random((B, K + 1)).astype(np.float32)
    for top_p in (0.2, 0.6, 0.9):
        acc, tok = gv.accept_rejection(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(),
                                       torch.from_numpy(u).cuda(), 1.0, top_p)
        torch.cuda.synchronize()
        ea, et = ora.accept_rejection(host, drafts, n, u, 1.0, top_p)
        assert np.array_equal(acc.cpu().numpy(), ea), top_p
        assert np.array_equal(tok.cpu().numpy(), et), top_p


def test_rejection_more_listed_rows_than_workgroups(gpu):
    """Rows that need the exact nucleus are listed and the later kernels loop over the
    list with grids sized by sequence (and 8 workgroups for crowded rows). Two-level tied
    logits make every row's boundary bin crowded and its bounds open, so up to B*(K+1) =
    18 rows are listed for 2 sequences, and more crowded rows than row-pass workgroups."""
    say("rejection listed rows > workgroups")
    rng = np.random.default_rng(41)
    B, K, V = 2, 8, 20000
    host = rng.integers(0, 2, (B, K + 1, V)).astype(np.float32)
    lg = torch.from_numpy(host).to(torch.bfloat16)
    host = lg.float().numpy()
    drafts = np.argmax(host[:, :K], axis=-1).astype(np.int32)  # in the top level: often accepted
    drafts[1, 3] = int(np.argmin(host[1, 3]))                  # one draft outside the nucleus
    n = np.array([K, K - 2], np.int32)
    for seed in range(4):
        u = np.random.default_rng(seed).random((B, K + 1)).astype(np.float32) * 3e-4  # p(x) ~ 1/4000 inside
        for top_p in (0.4, 0.95):
            acc, tok = gv.accept_rejection(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(),
                                           torch.from_numpy(u).cuda(), 1.0, top_p)
            torch.cuda.synchronize()
            ea, et = ora.accept_rejection(host, drafts, n, u, 1.0, top_p)
            assert np.array_equal(acc.cpu().numpy(), ea), (seed, top_p)
            assert np.array_equal(tok.cpu().numpy(), et), (seed, top_p)


@pytest.mark.parametrize("top_p", [0.95, 0.6])
def test_rejection_sixty_four_drafts_with_top_p(gpu, top_p):
    """The most drafts a call takes (64), with top-p: a sequence accepting all of them draws
    its bonus from row 64 (the row the bounds walk marks through its own branch), one is
    rejected at draft 30 (certainly, outside the nucleus), one has 10 drafts; the rows only
    drawn from get the range hint."""
    say(f"rejection 64 drafts top_p={top_p}")
    rng = np.random.default_rng(64 + int(top_p * 100))
    B, K, V = 3, 64, 32000
    host = rng.normal(0, 2.0, (B, K + 1, V)).astype(np.float32)
    for b in range(B):  # a clear mode per row, so its draft is surely accepted at a small u
        host[b, np.arange(K + 1), rng.integers(0, V, K + 1)] += 8.0
    drafts = np.argmax(host[:, :K], axis=-1).astype(np.int32)
    drafts[1, 30] = int(np.argmin(host[1, 30]))
    n = np.array([K, K, 10], np.int32)
    u = (rng.random((B, K + 1)) * 1e-3).astype(np.float32)
    acc, tok = gv.accept_rejection(torch.from_numpy(host).cuda(), torch.from_numpy(drafts).cuda(),
                                   torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda(), 0.8, top_p)
    torch.cuda.synchronize()
    ea, et = ora.accept_rejection(host, drafts, n, u, 0.8, top_p)
    assert ea.tolist() == [K, 30, 10]
    assert np.array_equal(acc.cpu().numpy(), ea)
    assert np.array_equal(tok.cpu().numpy(), et)


def test_rejection_small_temperature_is_greedy(gpu):
    say("rejection T->0")
    lg, host, drafts, n = logits_case(5, 3, 3000, "f32", seed=5)
    u = np.full((5, 4), 0.5, np.float32)
    acc, tok = gv.accept_rejection(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(),
                                   torch.from_numpy(u).cuda(), 1e-12)
    torch.cuda.synchronize()
    ea, et = ora.accept_greedy(host, drafts, n)
    assert np.array_equal(acc.cpu().numpy(), ea) and np.array_equal(tok.cpu().numpy(), et)


def test_rejection_invalid_and_nonfinite(gpu):
    say("rejection invalid drafts / non-finite logits")
    rng = np.random.default_rng(8)
    B, K, V = 4, 2, 5000
    host = rng.normal(0, 1, (B, K + 1, V)).astype(np.float32)
    host[0, 0, :] = -np.inf                    # no finite logit in a row
    host[1, :, 17] = np.nan
    host[2, :, 3] = np.inf
    drafts = np.array([[1, 2], [17, 3], [V + 5, 1], [-1, 0]], np.int32)
    n = np.array([2, 2, 2, 1], np.int32)
    u = rng.random((B, K + 1)).astype(np.float32)
    acc, tok = gv.accept_rejection(torch.from_numpy(host).cuda(), torch.from_numpy(drafts).cuda(),
                                   torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda(), 0.7, 0.9)
    torch.cuda.synchronize()
    ea, et = ora.accept_rejection(host, drafts, n, u, 0.7, 0.9)
    assert np.array_equal(acc.cpu().numpy(), ea) and np.array_equal(tok.cpu().numpy(), et)


@pytest.mark.parametrize("top_p", [1.0, 0.8])
def test_rejection_emitted_token_follows_target(gpu, top_p):
    """Speculative sampling (Leviathan et al. 2023): the first emitted token is distributed
    as the target p whatever the draft distribution q is. With top-p, p is the target
    restricted to its nucleus and renormalised (sampling.go:139-173: keep while the mass
    before an item is < p), so drafts outside the nucleus are always rejected. Checked on
    the GPU over 40000 sequences with one draft each, against float64 softmax."""
    rng = np.random.default_rng(11)
    V, N = 5, 40000
    base = np.array([1.0, 0.2, -0.5, 0.7, -1.0], np.float32)
    q = np.array([0.05, 0.3, 0.4, 0.1, 0.15], np.float32)
    drafts = rng.choice(V, size=(N, 1), p=q / q.sum()).astype(np.int32)
    u = rng.random((N, 2)).astype(np.float32)
    say(f"rejection emitted-token distribution top_p={top_p}")
    acc, tok = gv.accept_rejection(torch.from_numpy(np.broadcast_to(base, (N, 2, V)).copy()).cuda(),
                                   torch.from_numpy(drafts).cuda(), torch.ones(N, dtype=torch.int32).cuda(),
                                   torch.from_numpy(u).cuda(), 1.0, top_p,
                                   draft_probs=torch.from_numpy(np.broadcast_to(q, (N, 1, V)).copy()).cuda())
    torch.cuda.synchronize()
    acc, tok = acc.cpu().numpy(), tok.cpu().numpy()
    p = np.exp(base.astype(np.float64) - base.max())
    p /= p.sum()
    if top_p < 1.0:
        keep, cum = np.zeros(V, bool), 0.0
        for i in np.argsort(-p, kind="stable"):
            if cum >= top_p:
                break
            keep[i], cum = True, cum + p[i]
        assert keep.tolist() == [True, True, False, True, False]  # the nucleus {0, 3, 1}
        p = np.where(keep, p, 0.0)
        p /= p.sum()
        assert not acc[~keep[drafts[:, 0]]].any()  # drafts outside the nucleus never pass
    first = np.where(acc == 1, drafts[:, 0], tok)
    freq = np.bincount(first, minlength=V) / N
    assert np.abs(freq - p).max() < 0.01, (freq, p)


@pytest.mark.parametrize("seed", range(40))
def test_acceptance_random_cases(gpu, seed):
    """Seeded random acceptance calls (logit type, batch, drafts, vocabulary sizes around
    the segment and vector widths, temperature, top-p, draft distributions, value spread
    and ties), greedy and rejection, bit for bit against the oracle."""
    r = np.random.default_rng(500 + seed)
    dt = ["f32", "bf16", "f16"][seed % 3]
    B = int(r.integers(1, 9))
    K = int(r.integers(0, 9))
    V = int(r.choice([7, 100, 2048, 4099, 8191, 8192, 8193, 20000, 65537]))
    sd = float(r.choice([0.5, 2.0, 6.0]))
    T = float(r.choice([0.3, 0.8, 1.0, 1.7]))
    top_p = float(r.choice([1.0, 0.999, 0.95, 0.5, 0.1]))
    with_q = K > 0 and bool(r.random() < 0.5)
    say(f"acceptance random case {seed}: dt={dt} B={B} K={K} V={V} sd={sd} T={T} top_p={top_p} q={with_q}")
    lg, host, drafts, n, q, u = rejection_case(B, K, V, dt, seed=700 + seed, with_q=with_q, sd=sd)
    if r.random() < 0.3:  # coarse values: many ties
        host = np.round(host)
        lg = torch.from_numpy(host).to(TD[dt])
        host = lg.float().numpy()
    d_t, n_t, u_t = torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda()
    acc, tok = gv.accept_greedy(lg.cuda(), d_t, n_t)
    torch.cuda.synchronize()
    ea, et = ora.accept_greedy(host, drafts, n)
    assert np.array_equal(acc.cpu().numpy(), ea) and np.array_equal(tok.cpu().numpy(), et)
    check_positions(drafts, n, acc.cpu().numpy(), tok.cpu().numpy(), V, 0.0, 1.0, seed)
    acc, tok = gv.accept_rejection(lg.cuda(), d_t, n_t, u_t, T, top_p,
                                   draft_probs=torch.from_numpy(q).cuda() if q is not None else None)
    torch.cuda.synchronize()
    ea, et = ora.accept_rejection(host, drafts, n, u, T, top_p, q)
    assert np.array_equal(acc.cpu().numpy(), ea)
    assert np.array_equal(tok.cpu().numpy(), et)
    check_positions(drafts, n, acc.cpu().numpy(), tok.cpu().numpy(), V, T, top_p, seed)


@pytest.mark.parametrize("cid", [2, 3, 4, 5])
def test_acceptance_full_size_configs(gpu, cid):
    """Each config's acceptance at its real shape ([B, K+1, 128256] logits in the config's
    dtype; config 3 with draft distributions, config 5 with top-p 0.95), inputs generated
    as bench.py does, against the CPU oracle bit for bit."""
    from gollmgo_amd.workloads import CONFIGS
    cfg = CONFIGS[cid]
    B, K, V = cfg.num_seqs, cfg.max_drafts, cfg.vocab
    say(f"acceptance full size config {cid}: B={B} K={K} V={V} {cfg.accept}")
    g = torch.Generator(device="cuda")
    g.manual_seed(cfg.seed + 99)
    logits = (torch.randn(B, K + 1, V, device="cuda", generator=g) * 2.0).to(TD[cfg.logits_dtype])
    probs = torch.softmax(logits[:, :K].float() * 1.5, dim=-1).contiguous() if cfg.draft_probs else None
    base = probs if probs is not None else logits[:, :K].float()
    mode = base.argmax(dim=-1).to(torch.int32)
    rand = torch.randint(0, V, (B, K), device="cuda", dtype=torch.int32, generator=g)
    drafts = torch.where(torch.rand(B, K, device="cuda", generator=g) < 0.8, mode, rand).contiguous()
    n = torch.randint(0, K + 1, (B,), device="cuda", dtype=torch.int32, generator=g)
    host = logits.float().cpu().numpy()
    if cfg.accept == "greedy":
        acc, tok = gv.accept_greedy(logits, drafts, n)
        torch.cuda.synchronize()
        ea, et = ora.accept_greedy(host, drafts.cpu().numpy(), n.cpu().numpy())
    else:
        u = torch.rand(B, K + 1, device="cuda", generator=g)
        acc, tok = gv.accept_rejection(logits, drafts, n, u, cfg.temperature, cfg.top_p, draft_probs=probs)
        torch.cuda.synchronize()
        ea, et = ora.accept_rejection(host, drafts.cpu().numpy(), n.cpu().numpy(), u.cpu().numpy(),
                                      cfg.temperature, cfg.top_p,
                                      probs.cpu().numpy() if probs is not None else None)
    a, t = acc.cpu().numpy(), tok.cpu().numpy()
    print(f"  accepted {int(a.sum())} of {int(n.sum())} drafts")
    assert np.array_equal(a, ea)
    assert np.array_equal(t, et)
    # The decision handed back as the engine's LogitsPerPosition (one-hot rows).
    T = cfg.temperature if cfg.accept != "greedy" else 0.0
    check_positions(drafts.cpu().numpy(), n.cpu().numpy(), a, t, V, T, cfg.top_p, cid)


def test_greedy_ties_across_segment_boundaries(gpu):
    """Ties and a NaN around the segment boundaries of a 2^17-entry row (every segment
    length up to 2^16 that divides it has a boundary at 2^14): the first index wins."""
    say("greedy ties across segments")
    V = 1 << 17
    rows = np.full((4, 2, V), -1.0, np.float32)
    rows[0, 0, [16384, 16383]] = 5.0                          # tie straddling 2^14 -> 16383
    rows[1, 0, [32768, 100000, 16384]] = 7.0                  # ties in later segments -> 16384
    rows[2, 0, 16383] = np.nan; rows[2, 0, [16384, 65536]] = 2.0  # NaN skipped -> 16384
    rows[3, 0, V - 1] = 3.0; rows[3, 0, 65535] = 3.0          # last element ties earlier -> 65535
    drafts = np.array([[16383], [16384], [16384], [65535]], np.int32)
    n = np.ones(4, np.int32)
    for dt in ("f32", "bf16"):
        lg = torch.from_numpy(rows).to(TD[dt])
        acc, tok = gv.accept_greedy(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda())
        torch.cuda.synchronize()
        ea, et = ora.accept_greedy(lg.float().numpy(), drafts, n)
        assert np.array_equal(acc.cpu().numpy(), ea) and np.array_equal(tok.cpu().numpy(), et), dt
        assert acc.cpu().tolist() == [1, 1, 1, 1], dt
