"""Pins of the CPU oracle: the reference's own known-answer tests, library
routines (torch SDPA in float64, torch float8 casts, numpy float16 casts, libm exp),
closed forms and invariants. CPU only."""
import math

import numpy as np
import pytest
import torch


# ---------------------------------------------------------------- reference KATs

def test_ngram_reference_cases(ora, golden):
    for c in golden["ngram_draft"]:
        assert ora.ngram_draft(c["history"], c["n"], c["k"]) == c["expect"]


def test_verify_reference_cases(ora, golden):
    for c in golden["verify"]:
        # Rows may differ in length (Go slices); -inf padding leaves every argmax unchanged.
        width = max((len(r) for r in c["rows"]), default=0)
        rows = [list(r) + [-math.inf] * (width - len(r)) for r in c["rows"]]
        acc, cor = ora.verify(c["drafts"], rows)
        assert acc == c["expect_accepted"]
        if c["expect_corrected"] is not None:
            assert cor == c["expect_corrected"]


def test_verify_rows_of_different_length(ora):
    # The reference's all-accepted case uses rows of lengths 11/21/31; pad with -inf so
    # the argmax of each row is unchanged and check the same answer.
    rows = [[0.0] * 10 + [5.0], [0.0] * 20 + [5.0], [0.0] * 30 + [5.0]]
    padded = [r + [-math.inf] * (31 - len(r)) for r in rows]
    assert ora.verify([10, 20, 30], padded)[0] == 3


def test_argmax_reference_cases(ora, golden):
    for c in golden["argmax"]:
        assert ora.argmax(c["logits"]) == c["expect"]
    for c in golden["greedy_sample"]:
        assert ora.argmax(c["logits"]) == c["expect"]


def test_argmax_ties_and_nan(ora):
    assert ora.argmax([1, 3, 3, 2]) == 1
    assert ora.argmax([float("nan"), 5, 6]) == 0          # NaN at 0 never loses
    assert ora.argmax([1, float("nan"), 0.5, 2]) == 3      # NaN elsewhere never wins
    assert ora.argmax([-0.0, 0.0]) == 0                     # equal values: first index


def test_top_p_reference_case(ora, golden):
    for c in golden["top_p"]:
        out = ora.top_p_filter_f64(c["probs"], c["p"])
        for i in c["kept"]:
            assert out[i] > 0
        assert abs(out.sum() - c["sum"]) < c["tol"]


def test_softmax_reference_cases(ora, golden):
    for c in golden["softmax"]:
        x = [float(v) for v in c["logits"]]
        p = ora.softmax_f64(x)
        assert abs(p.sum() - c["sum"]) < c["tol"]
        if c.get("increasing"):
            assert p[0] < p[1] < p[2]
        if "zero_at" in c:
            assert p[c["zero_at"]] == 0


def test_categorical_closed_form(ora):
    p = [0.1, 0.2, 0.3, 0.4]
    assert ora.categorical_f64(p, 0.0) == 0
    assert ora.categorical_f64(p, 0.0999) == 0
    assert ora.categorical_f64(p, 0.1001) == 1
    assert ora.categorical_f64(p, 0.61) == 3
    assert ora.categorical_f64(p, 1.5) == 3               # fallback: last non-zero
    assert ora.categorical_f64([0.5, 0.5, 0.0], 2.0) == 1


# ---------------------------------------------------------------- n-gram brute force

def _draft_literal(hist, n, k):
    """A line-by-line Python restatement of speculative.go:24-62 (dict = Go map)."""
    if n < 2:
        n = 2
    if k < 1:
        k = 4
    if len(hist) < n:
        return []
    kl = n - 1
    table = {}
    for i in range(0, len(hist) - n + 1):
        table[tuple(hist[i:i + kl])] = hist[i + kl]
    out = []
    suffix = list(hist[len(hist) - kl:])
    while len(out) < k:
        nxt = table.get(tuple(suffix))
        if nxt is None:
            break
        out.append(nxt)
        suffix = suffix[1:] + [nxt]
    return out


@pytest.mark.parametrize("n", [2, 3, 4, 9])
def test_ngram_brute_force(ora, n):
    rng = np.random.default_rng(n)
    for trial in range(200):
        L = int(rng.integers(0, 60))
        hist = rng.integers(0, 5, size=L).tolist()
        k = int(rng.integers(0, 7))
        assert ora.ngram_draft(hist, n, k) == _draft_literal(hist, n, k), (hist, n, k)


def test_ngram_rejects_large_n(ora):
    with pytest.raises(ValueError):
        ora.ngram_draft([1, 2, 3] * 5, 10, 4)


# ---------------------------------------------------------------- number formats

def test_fp8_encode_matches_torch():
    from oracle import oracle as ora
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 100, 20000), rng.uniform(-448, 448, 20000),
                        rng.uniform(-0.02, 0.02, 20000)]).astype(np.float32)
    # Exact ties between representable values, both signs.
    codes = np.arange(0, 0x7E, dtype=np.uint8)
    vals = ora.fp8_decode(codes)
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, vals, -vals])
    # torch's cast turns |x| >= 464 into NaN; the reference convention saturates (checked below).
    x = x[np.abs(x) <= 448]
    ours = ora.fp8_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_fp8_saturates_and_decodes():
    from oracle import oracle as ora
    assert ora.fp8_encode(np.array([1e6, -1e6, 448.0, 460.0, np.inf], np.float32)).tolist() == [0x7E, 0xFE, 0x7E, 0x7E, 0x7E]
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    ours = ora.fp8_decode(codes)
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])


def test_int8_rne_and_clamp(ora):
    x = np.array([2.5, 3.5, -2.5, -3.5, 0.49, 126.6, 200, -200, np.nan], np.float32)
    assert ora.int8_encode(x).tolist() == [2, 4, -2, -4, 0, 127, 127, -127, 0]


def test_f16_round_matches_numpy(ora):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 1, 5000), rng.normal(0, 1e-5, 5000), rng.normal(0, 1e4, 5000)]).astype(np.float32)
    assert np.array_equal(ora.f16_round_c(x), x.astype(np.float16).astype(np.float32))


def test_bf16_helpers_match_torch(ora):
    rng = np.random.default_rng(2)
    x = rng.normal(0, 3, 10000).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ora.round_bf16(x), ref)


# ---------------------------------------------------------------- fixed-point exp

def test_expf_fixed_accuracy(ora):
    x = np.linspace(-80, 0, 400001).astype(np.float32)
    ours = ora.expf_fixed(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    rel = np.abs(ours - ref) / ref
    assert rel.max() < 4e-7  # ~3 ulp of fp32
    assert ora.expf_fixed(np.array([0.0, -100.0, np.nan], np.float32)).tolist()[:2] == [1.0, 0.0]


def test_weight_closed_forms(ora):
    assert ora.weight(1.0, 1.0, 1.25) == 2 ** 35
    assert ora.weight(-200.0, 0.0, 1.0) == 0
    ws = [ora.weight(float(l), 0.0, 1.25) for l in np.linspace(-10, 0, 200)]
    assert all(a <= b for a, b in zip(ws, ws[1:]))


# ---------------------------------------------------------------- rejection acceptance

def _softmax_fixed_rows(ora, logits, T):
    inv_t = np.float32(1.0) / np.float32(T)
    out = []
    for row in logits:
        m = float(np.max(row))
        out.append(np.array([ora.weight(float(l), m, float(inv_t)) for l in row], dtype=np.float64))
    return out


def test_rejection_one_hot_q_accepts_iff_u_below_p(ora):
    rng = np.random.default_rng(3)
    V, K, B = 7, 1, 400
    logits = rng.normal(0, 1, (B, K + 1, V)).astype(np.float32)
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    u = rng.random((B, K + 1)).astype(np.float32)
    acc, tok = ora.accept_rejection(logits, drafts, np.full(B, K, np.int32), u, 0.8)
    for b in range(B):
        w = _softmax_fixed_rows(ora, logits[b, :1], 0.8)[0]
        p = w[drafts[b, 0]] / w.sum()
        assert acc[b] == (1 if u[b, 0] < p else 0)
        if acc[b] == 0:
            assert tok[b] != drafts[b, 0]  # the residual excludes the rejected draft


def test_rejection_q_equal_p_always_accepts(ora):
    rng = np.random.default_rng(4)
    V, K, B = 50, 3, 64
    logits = rng.normal(0, 2, (B, K + 1, V)).astype(np.float32)
    # q = p - tiny: then p/q >= 1 and every draft is accepted.
    q = np.zeros((B, K, V), np.float32)
    for b in range(B):
        for j, w in enumerate(_softmax_fixed_rows(ora, logits[b, :K], 1.0)):
            q[b, j] = (w / w.sum() * (1 - 1e-6)).astype(np.float32)
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    u = (rng.random((B, K + 1)) * 0.999).astype(np.float32)
    acc, _ = ora.accept_rejection(logits, drafts, np.full(B, K, np.int32), u, 1.0, draft_probs=q)
    assert (acc == K).all()


def test_rejection_output_distribution_is_target(ora):
    """Leviathan et al.: the first emitted token is distributed as p whatever q is."""
    rng = np.random.default_rng(5)
    V, N = 5, 40000
    base = np.array([1.0, 0.2, -0.5, 0.7, -1.0], np.float32)
    logits = np.broadcast_to(base, (N, 2, V)).copy()
    q = np.array([0.05, 0.5, 0.3, 0.1, 0.05], np.float32)
    dp = np.broadcast_to(q, (N, 1, V)).copy()
    drafts = rng.choice(V, size=(N, 1), p=q / q.sum()).astype(np.int32)
    u = rng.random((N, 2)).astype(np.float32)
    acc, tok = ora.accept_rejection(logits, drafts, np.ones(N, np.int32), u, 1.0, draft_probs=dp)
    first = np.where(acc == 1, drafts[:, 0], tok)
    w = _softmax_fixed_rows(ora, base[None], 1.0)[0]
    p = w / w.sum()
    freq = np.bincount(first, minlength=V) / N
    assert np.abs(freq - p).max() < 0.01


def test_rejection_top_p_matches_go_rule(ora):
    """The integer nucleus equals topPFilter's float64 nucleus on generic rows."""
    rng = np.random.default_rng(6)
    V = 300
    for trial in range(20):
        row = rng.normal(0, 2, V).astype(np.float32)
        T, top_p = 0.8, 0.9
        # Float64 Go rule.
        scaled = row.astype(np.float64) * (1.0 / T)
        go_keep = ora.top_p_filter_f64(ora.softmax_f64(scaled), top_p) > 0
        # Integer rule, observed through the bonus draw: a token outside the nucleus is never drawn.
        w = _softmax_fixed_rows(ora, row[None], T)[0]
        order = sorted(range(V), key=lambda i: (-row[i], i))
        tp = math.ceil(top_p * w.sum())
        cum, keep = 0, np.zeros(V, bool)
        for i in order:
            if cum >= tp and cum > 0:
                break
            keep[i] = True
            cum += w[i]
        assert np.array_equal(keep, go_keep)
        # And the oracle's draws only land in the nucleus.
        N = 200
        logits = np.broadcast_to(row, (N, 1, V)).copy()
        u = rng.random((N, 1)).astype(np.float32)
        _, tok = ora.accept_rejection(logits, np.zeros((N, 0), np.int32), np.zeros(N, np.int32), u, T, top_p)
        assert keep[tok].all()


def _go_cdf(row, T, top_p, ora):
    """Sampler.Sample's float64 distribution (sampling.go:57-68) and its running sum in
    index order, which categoricalSample compares u against (:176-192)."""
    scaled = row.astype(np.float64) * (1.0 / T)
    probs = ora.softmax_f64(scaled)
    if 0 < top_p < 1:
        probs = ora.top_p_filter_f64(probs, top_p)
    return probs, np.cumsum(probs)


def test_rejection_bonus_draw_hits_every_nucleus_token(ora):
    """The fixed-point final draw (no drafts, so the bonus draw over row 0), driven at the
    middle of each float64 CDF bin of topPFilter(softmax(l/T)), returns that bin's token:
    every token of the Go nucleus is drawn for some u, and the boundary machinery (integer
    nucleus cut, prefix search) places each bin where the float64 rule does."""
    rng = np.random.default_rng(16)
    V = 300
    for trial in range(12):
        row = rng.normal(0, 2, V).astype(np.float32)
        T, top_p = (0.8, 0.9) if trial % 2 == 0 else (1.0, 0.95)
        probs, cdf = _go_cdf(row, T, top_p, ora)
        keep = np.nonzero(probs > 0)[0]
        lo = np.concatenate([[0.0], cdf[:-1]])
        # Bins wide enough that the midpoint is far from both boundaries in float32.
        toks = [int(k) for k in keep if probs[k] > 1e-5]
        assert len(toks) >= 0.5 * len(keep)
        u = np.array([(lo[k] + cdf[k]) / 2 for k in toks], np.float32)
        N = len(toks)
        logits = np.broadcast_to(row, (N, 1, V)).copy()
        _, tok = ora.accept_rejection(logits, np.zeros((N, 0), np.int32), np.zeros(N, np.int32), u[:, None], T,
                                      top_p)
        assert tok.tolist() == toks


def test_rejection_never_returns_the_rejected_draft(ora):
    """After a rejection at draft x the draw excludes x: max(0, p - q) is 0 at x, since
    u < 1 rejects only when p(x) < q(x). Also when the residual vanishes (q not a
    distribution: all ones), where the draw falls back to the row without x."""
    rng = np.random.default_rng(21)
    B, K, V = 300, 4, 400
    for T, top_p, dense in [(0.8, 1.0, False), (1.0, 0.9, False), (0.8, 1.0, True), (1.2, 0.95, True)]:
        lg = rng.normal(0, 1.5, (B, K + 1, V)).astype(np.float32)
        q = None
        if dense:
            q = rng.dirichlet(np.ones(V) * 0.3, (B, K)).astype(np.float32)
        drafts = lg[:, :K].argmax(-1).astype(np.int32)
        mask = rng.random((B, K)) < 0.4
        drafts[mask] = rng.integers(0, V, int(mask.sum()))
        n = rng.integers(1, K + 1, B).astype(np.int32)
        u = rng.random((B, K + 1)).astype(np.float32)
        acc, tok = ora.accept_rejection(lg, drafts, n, u, T, top_p, q)
        rej = acc < n
        assert rej.sum() > 20
        assert np.all(tok[rej] != drafts[rej, acc[rej]])
    # q = 1 everywhere: every residual is 0, and the draw takes the row without the draft.
    lg = rng.normal(0, 1.0, (50, 2, 30)).astype(np.float32)
    drafts = lg[:, 0].argmax(-1).astype(np.int32)[:, None]
    q = np.ones((50, 1, 30), np.float32)
    u = np.full((50, 2), 0.9, np.float32)
    acc, tok = ora.accept_rejection(lg, drafts, np.ones(50, np.int32), u, 1.0, 1.0, q)
    assert np.all(acc == 0) and np.all(tok != drafts[:, 0])


def _residual_draw_numpy(ora, row, T, top_p, x, qrow, u):
    """The residual draw restated in numpy: r = p - q where p > q, x excluded, normalised
    (np.cumsum gives the sequential float64 sums); fallbacks p without x, then p."""
    p = ora.sampler_probs_f64(row, T, 0, top_p)
    q = np.zeros_like(p) if qrow is None else np.where((qrow > 0) & np.isfinite(qrow), np.minimum(qrow, 1), 0)
    r = np.where(p > q, p - q, 0.0)
    if 0 <= x < len(r):
        r[x] = 0.0
    s = np.cumsum(r)[-1]
    if not s > 0:
        r = p.copy()
        if 0 <= x < len(r):
            r[x] = 0.0
        s = np.cumsum(r)[-1]
    d = r / s if s > 0 else p
    c = np.cumsum(d)
    i = int(np.searchsorted(c, u, side="right"))
    return i if i < len(d) else int(np.nonzero(d > 0)[0][-1])


@pytest.mark.parametrize("T,top_p", [(0.8, 1.0), (1.0, 0.95), (0.7, 0.5)])
def test_rejection_final_draw_is_the_float64_rule(ora, T, top_p):
    """The rejection's token is drawn by the float64 rule, not the fixed point: the bonus
    equals Sampler.Sample (ora_sample_f64), the residual draw a numpy restatement, for
    one-hot and dense draft distributions."""
    rng = np.random.default_rng(int(T * 100 + top_p * 10))
    B, K, V = 120, 3, 3000
    for dense in (False, True):
        lg = rng.normal(0, 2, (B, K + 1, V)).astype(np.float32)
        q = rng.dirichlet(np.ones(V) * 0.2, (B, K)).astype(np.float32) if dense else None
        drafts = lg[:, :K].argmax(-1).astype(np.int32)
        mask = rng.random((B, K)) < 0.5
        drafts[mask] = rng.integers(0, V, int(mask.sum()))
        n = rng.integers(0, K + 1, B).astype(np.int32)
        u = rng.random((B, K + 1)).astype(np.float32)
        acc, tok = ora.accept_rejection(lg, drafts, n, u, T, top_p, q)
        for b in range(B):
            a = int(acc[b])
            uu = float(u[b, K])
            if a == n[b]:
                assert tok[b] == ora.sample_f64(lg[b, a], float(np.float32(T)), float(np.float32(top_p)), uu)
            else:
                want = _residual_draw_numpy(ora, lg[b, a], float(np.float32(T)), float(np.float32(top_p)),
                                            int(drafts[b, a]), q[b, a] if dense else None, uu)
                assert tok[b] == want


# ---------------------------------------------------------------- attention

def _bf16_pool_case(ora, B=3, R=4, Hq=8, H=2, D=32, bs=4, ctx=(5, 17, 30), seed=0):
    rng = np.random.default_rng(seed)
    maxb = max((c + R + bs - 1) // bs for c in ctx)
    nblk = B * maxb + 3
    perm = rng.permutation(nblk)
    bt = perm[:B * maxb].reshape(B, maxb).astype(np.int32)
    keys = np.array([c + R for c in ctx], np.int32)
    kvals = ora.round_bf16(rng.normal(0, 1, (nblk, H, bs, D)).astype(np.float32))
    vvals = ora.round_bf16(rng.normal(0, 1, (nblk, H, D, bs)).astype(np.float32))
    kc = ora.bf16_bits(kvals).view(np.uint8).copy()
    vc = ora.bf16_bits(vvals).view(np.uint8).copy()
    q = rng.normal(0, 1, (B, R, Hq, D)).astype(np.float32)
    return q, kc, vc, kvals, vvals, keys, bt


def test_attention_matches_torch_sdpa(ora):
    B, R, Hq, H, D, bs = 3, 4, 8, 2, 32, 4
    q, kc, vc, kvals, vvals, keys, bt = _bf16_pool_case(ora, B, R, Hq, H, D, bs)
    scale = 1 / math.sqrt(D)
    out = ora.attention(q, kc, vc, "bf16", H, D, bs, keys, bt, scale)
    G = Hq // H
    for b in range(B):
        n = int(keys[b])
        t = np.arange(n)
        blk = bt[b, t // bs]
        k = kvals[blk, :, t % bs, :].transpose(1, 0, 2)               # [H, n, D]
        v = vvals[blk, :, :, t % bs].transpose(1, 0, 2)               # [H, n, D]
        k = np.repeat(k, G, axis=0)
        v = np.repeat(v, G, axis=0)
        qq = q[b].transpose(1, 0, 2)                                  # [Hq, R, D]
        pos = n - R + np.arange(R)
        mask = t[None, :] <= pos[:, None]                             # [R, n]
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(qq).double(), torch.from_numpy(k).double(), torch.from_numpy(v).double(),
            attn_mask=torch.from_numpy(mask), scale=scale).numpy()    # [Hq, R, D]
        np.testing.assert_allclose(out[b].transpose(1, 0, 2), ref, rtol=1e-5, atol=1e-6)


def test_attention_closed_forms(ora):
    # One visible key -> output equals that key's V; identical keys -> mean of visible V.
    B, R, Hq, H, D, bs = 1, 2, 2, 1, 16, 4
    rng = np.random.default_rng(9)
    bt = np.array([[0, 1]], np.int32)
    kvals = np.ones((2, H, bs, D), np.float32)
    vvals = ora.round_bf16(rng.normal(0, 1, (2, H, D, bs)).astype(np.float32))
    kc, vc = ora.bf16_bits(kvals).view(np.uint8).copy(), ora.bf16_bits(vvals).view(np.uint8).copy()
    q = rng.normal(0, 1, (B, R, Hq, D)).astype(np.float32)
    keys = np.array([R], np.int32)  # row 0 sees key 0 only; row 1 sees keys 0,1
    out = ora.attention(q, kc, vc, "bf16", H, D, bs, keys, bt, 0.25)
    np.testing.assert_allclose(out[0, 0, 0], vvals[0, 0, :, 0], rtol=1e-6)
    np.testing.assert_allclose(out[0, 1, 1], (vvals[0, 0, :, 0] + vvals[0, 0, :, 1]) / 2, rtol=1e-6)


def test_attention_block_permutation_invariance(ora):
    q, kc, vc, kvals, vvals, keys, bt = _bf16_pool_case(ora, seed=11)
    H, D, bs = 2, 32, 4
    out = ora.attention(q, kc, vc, "bf16", H, D, bs, keys, bt, 0.2)
    # Move every block to a new physical index, rewrite the tables accordingly.
    nblk = kvals.shape[0]
    perm = np.random.default_rng(12).permutation(nblk)
    k2, v2 = np.empty_like(kvals), np.empty_like(vvals)
    k2[perm], v2[perm] = kvals, vvals
    out2 = ora.attention(q, ora.bf16_bits(k2).view(np.uint8).copy(), ora.bf16_bits(v2).view(np.uint8).copy(),
                         "bf16", H, D, bs, keys, perm[bt].astype(np.int32), 0.2)
    np.testing.assert_array_equal(out, out2)


def test_attention_boundary_semantics(ora):
    """gg_verify_attention's boundary rules, pinned by equivalences: a key block whose
    id is out of range (negative or >= the pool's blocks) counts exactly as if it were
    removed from the table; context lengths beyond the table clamp to its width; a
    sequence with no rows or more rows than keys is left untouched."""
    H, D, bs, nblk, R = 2, 8, 4, 6, 3
    rng = np.random.default_rng(21)
    kc = rng.normal(0, 1, (nblk, H, bs, D)).astype(np.float32)
    vc = rng.normal(0, 1, (nblk, H, D, bs)).astype(np.float32)
    q = rng.normal(0, 1, (1, R, 4, D)).astype(np.float32)
    args = (kc.view(np.uint8).reshape(-1), vc.view(np.uint8).reshape(-1), "f32", H, D, bs)
    ref = ora.attention(q, *args, np.array([10], np.int32), np.array([[0, 2, 3]], np.int32), 0.3)
    assert np.abs(ref).sum() > 0
    for bad in (-1, nblk, 10 ** 6):
        got = ora.attention(q, *args, np.array([14], np.int32), np.array([[0, bad, 2, 3]], np.int32), 0.3)
        np.testing.assert_array_equal(got, ref)
    # ctx beyond the table width: clamped (3 blocks -> 12 keys).
    a = ora.attention(q, *args, np.array([99], np.int32), np.array([[4, 5, 1]], np.int32), 0.3)
    b = ora.attention(q, *args, np.array([12], np.int32), np.array([[4, 5, 1]], np.int32), 0.3)
    np.testing.assert_array_equal(a, b)
    # More rows than keys, or no rows: untouched (zeros).
    z = ora.attention(q, *args, np.array([2], np.int32), np.array([[0, 1]], np.int32), 0.3)
    assert not z.any()
    z = ora.attention(q, *args, np.array([9], np.int32), np.array([[0, 1, 2]], np.int32), 0.3,
                      row_counts=np.array([0], np.int32))
    assert not z.any()


def test_kv_append_fp8_matches_encoder(ora):
    H, D, bs, nblk = 2, 8, 4, 3
    rng = np.random.default_rng(13)
    k = rng.normal(0, 3, (5, H, D)).astype(np.float32)
    v = rng.normal(0, 3, (5, H, D)).astype(np.float32)
    slots = np.array([0, 1, 5, 11, -1], np.int32)
    kc = np.zeros(nblk * H * bs * D, np.uint8)
    vc = np.zeros(nblk * H * bs * D, np.uint8)
    kinv = np.array([1 / 0.5, 1 / 0.25], np.float32)
    ora.kv_append_q(kc, vc, "fp8", H, D, bs, k, v, slots, k_inv=kinv, v_inv=kinv)
    K = kc.reshape(nblk, H, bs, D)
    V = vc.reshape(nblk, H, D, bs)
    for r, s in enumerate(slots[:4]):
        blk, o = divmod(int(s), bs)
        for h in range(H):
            assert np.array_equal(K[blk, h, o], ora.fp8_encode(k[r, h] * kinv[h]))
            assert np.array_equal(V[blk, h, :, o], ora.fp8_encode(v[r, h] * kinv[h]))


def test_kv_append_int8_block_scales(ora):
    H, D, bs, nblk = 1, 4, 4, 2
    k = np.array([[[1, -2, 3, 4]], [[0.5, 0.5, 0.5, 0.5]], [[10, 0, 0, 0]]], np.float32)
    kc = np.zeros(nblk * H * bs * D, np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros(nblk * H, np.float32)
    vs = np.zeros(nblk * H, np.float32)
    ora.kv_append_q(kc, vc, "int8", H, D, bs, k[:2], k[:2], np.array([0, 1], np.int32), k_bscale=ks, v_bscale=vs)
    s0 = ora.f16_round_c(np.array([4 / 127], np.float32))[0]
    assert ks[0] == s0
    K = kc.view(np.int8).reshape(nblk, H, bs, D)
    assert K[0, 0, 0].tolist() == ora.int8_encode(k[0, 0] * np.float32(1 / s0)).tolist()
    # A larger row grows the scale and re-quantises the rows already in the block.
    old = K[0, 0, :2].copy()
    ora.kv_append_q(kc, vc, "int8", H, D, bs, k[2:], k[2:], np.array([2], np.int32), k_bscale=ks, v_bscale=vs)
    s1 = ora.f16_round_c(np.array([10 / 127], np.float32))[0]
    assert ks[0] == s1
    want = ora.int8_encode((old.astype(np.float32) * s0) * np.float32(1 / s1))
    assert np.array_equal(K[0, 0, :2], want)


def test_kv_append_int8_skipped_rows_inside_a_run(ora):
    """A skipped row (slot < 0) between two rows of one block does not split the block's
    run: the call equals the same call without the skipped row (one scale from the amax
    of both rows, one re-quantisation)."""
    H, D, bs, nblk = 2, 8, 8, 3
    rng = np.random.default_rng(5)
    first = rng.normal(0, 1, (3, H, D)).astype(np.float32)
    rows = rng.normal(0, 1, (3, H, D)).astype(np.float32)
    rows[2] *= 9.0  # the last row grows the scale
    pools = []
    for slots, kk in ((np.array([11, -1, 12, 13], np.int32), np.concatenate([rows[:1], rows[:1] * 0 + 99, rows[1:]])),
                      (np.array([11, 12, 13], np.int32), rows)):
        kc = np.zeros(nblk * H * bs * D, np.uint8)
        vc = np.zeros_like(kc)
        ks = np.zeros(nblk * H, np.float32)
        vs = np.zeros(nblk * H, np.float32)
        ora.kv_append_q(kc, vc, "int8", H, D, bs, first, first, np.array([8, 9, 10], np.int32), k_bscale=ks, v_bscale=vs)
        ora.kv_append_q(kc, vc, "int8", H, D, bs, kk, kk, slots, k_bscale=ks, v_bscale=vs)
        pools.append((kc, vc, ks, vs))
    for x, y in zip(*pools):
        assert np.array_equal(x, y)
    # The block's scale is the amax of every row it holds over 127 (rounded to fp16).
    amax = np.abs(np.concatenate([first, rows])).max(axis=(0, 2))
    assert np.array_equal(pools[1][2][H:2 * H], ora.f16_round_c((amax / np.float32(127)).astype(np.float32)))


def test_attention_ref_f32_is_the_same_rule(ora):
    """The fp32 restatement of the reference's v1 loop (the timed CPU baseline) computes the
    same attention as the fp64 checker, to fp32 rounding, on every pool type."""
    rng = np.random.default_rng(41)
    for dt in ("bf16", "fp8", "int8", "f32"):
        q, kc, vc, kvals, vvals, keys, bt = _bf16_pool_case(ora, seed=3)
        H, D, bs = 2, 32, 4
        ks = vs = None
        if dt != "bf16":
            kf = ora.bf16_to_f32(kc.view(np.uint16)).reshape(-1, H, bs, D)
            vf = ora.bf16_to_f32(vc.view(np.uint16)).reshape(-1, H, D, bs)
            if dt == "f32":
                kc, vc = kf.astype(np.float32).view(np.uint8).copy(), vf.astype(np.float32).view(np.uint8).copy()
            elif dt == "fp8":
                ks = vs = np.full(H, 1 / 64, np.float32)
                kc, vc = ora.fp8_encode(kf * 64), ora.fp8_encode(vf * 64)
            else:
                nb = kf.shape[0]
                ks = vs = np.full(nb * H, 1 / 32, np.float32)
                kc = ora.int8_encode(kf * 32).view(np.uint8).copy()
                vc = ora.int8_encode(vf * 32).view(np.uint8).copy()
        a = ora.attention(q, kc, vc, dt, H, D, bs, keys, bt, 0.2, ks, vs)
        b = ora.attention_ref_f32(q, kc, vc, dt, H, D, bs, keys, bt, 0.2, ks, vs)
        assert np.abs(a - b).max() <= 1e-5 * max(1.0, np.abs(a).max()), dt
