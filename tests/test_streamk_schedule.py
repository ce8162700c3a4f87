"""CPU check of the stream-K schedule used by the MFMA attention path.

Restates the integer arithmetic of attn_mfma_streamk_kernel (producer) and
attn_streamk_combine_kernel (merge) and checks, for ragged batches: every chunk of
every (sequence, kv head) item is computed exactly once; record indices stay below
grid + items (the workspace bound the host allocates); an item is written directly
iff one workgroup covers it whole; and the merge finds exactly the producing pieces.
"""
import numpy as np
import pytest

MIN_CHUNKS = 16  # kStreamKMinChunks


def seq_chunks(ctx, nrows, tok):
    if nrows <= 0 or nrows > ctx:
        return 0
    return (ctx + tok - 1) // tok


def producer(ctx, nrows, hkv, tok, grid):
    work = [hkv * seq_chunks(c, n, tok) for c, n in zip(ctx, nrows)]
    C = sum(work)
    per = max((C + grid - 1) // grid, MIN_CHUNKS)
    pieces = []  # (w, b, kvh, c0, c1, rec or None)
    for w in range(grid):
        g0 = w * per
        if g0 >= C:
            continue
        g1 = min(g0 + per, C)
        # locate the sequence holding g0
        gb, b = 0, 0
        while gb + work[b] <= g0:
            gb += work[b]
            b += 1
        g = g0
        while g < g1 and b < len(ctx):
            nch = seq_chunks(ctx[b], nrows[b], tok)
            wk = hkv * nch
            if nch == 0 or g >= gb + wk:
                gb += wk
                b += 1
                continue
            off = g - gb
            kvh, c0 = off // nch, off % nch
            c1 = min(nch, c0 + (g1 - g))
            item = b * hkv + kvh
            whole = c0 == 0 and c1 == nch
            pieces.append((w, b, kvh, c0, c1, None if whole else w + item))
            g += c1 - c0
    return pieces, C, per


def combine_lookup(ctx, nrows, hkv, tok, grid, b, kvh):
    work = [hkv * seq_chunks(c, n, tok) for c, n in zip(ctx, nrows)]
    before, total = sum(work[:b]), sum(work)
    per = max((total + grid - 1) // grid, MIN_CHUNKS)
    nch = seq_chunks(ctx[b], nrows[b], tok)
    gi0 = before + kvh * nch
    gi1 = gi0 + nch
    w0, w1 = gi0 // per, (gi1 - 1) // per
    return w0, w1


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("tok", [32, 64])
def test_streamk_covers_every_chunk_once(seed, tok):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 90))
    hkv = int(rng.choice([1, 2, 8]))
    R = int(rng.integers(1, 10))
    ctx = rng.integers(1, 9000, B).tolist()
    nrows = [int(min(R, c)) if rng.random() > 0.1 else R + 20000 for c in ctx]  # a few invalid sequences
    grid = int(rng.choice([1, 7, 256, 512]))
    pieces, C, per = producer(ctx, nrows, hkv, tok, grid)
    records = grid + B * hkv
    seen = {}
    for (w, b, kvh, c0, c1, rec) in pieces:
        assert 0 <= c0 < c1 <= seq_chunks(ctx[b], nrows[b], tok)
        for c in range(c0, c1):
            key = (b, kvh, c)
            assert key not in seen
            seen[key] = w
        if rec is not None:
            assert 0 <= rec < records
    expected = sum(hkv * seq_chunks(c, n, tok) for c, n in zip(ctx, nrows))
    assert len(seen) == expected == C
    # Direct writes happen exactly for items covered by one workgroup, and the merge
    # finds the producing workgroups.
    for b in range(B):
        for kvh in range(hkv):
            nch = seq_chunks(ctx[b], nrows[b], tok)
            if nch == 0:
                continue
            ws = sorted({seen[(b, kvh, c)] for c in range(nch)})
            w0, w1 = combine_lookup(ctx, nrows, hkv, tok, grid, b, kvh)
            assert ws == list(range(w0, w1 + 1))
            mine = [p for p in pieces if p[1] == b and p[2] == kvh]
            assert (len(mine) == 1) == (mine[0][5] is None)
            if len(mine) > 1:
                assert all(p[5] == p[0] + b * hkv + kvh for p in mine)
