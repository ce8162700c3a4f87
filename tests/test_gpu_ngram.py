"""GPU parity: n-gram draft lookup against the oracle (hash-map restatement of
NGramDrafter.Draft) and the reference's known answers."""
import numpy as np
import pytest
import torch

import gollmgo_amd.verify as gv
from gollmgo_amd.workloads import CONFIGS, make_histories, scaled
from helpers import say
from oracle import oracle as ora

pytestmark = pytest.mark.gpu


def run(hist_list, n, k):
    B = len(hist_list)
    stride = max(1, max(len(h) for h in hist_list))
    h = np.zeros((B, stride), np.int32)
    lens = np.zeros(B, np.int32)
    for b, x in enumerate(hist_list):
        h[b, :len(x)] = x
        lens[b] = len(x)
    d, nn = gv.ngram_draft(torch.from_numpy(h).cuda(), torch.from_numpy(lens).cuda(), n, k)
    torch.cuda.synchronize()
    d, nn = d.cpu().numpy(), nn.cpu().numpy()
    return [d[b, :nn[b]].tolist() for b in range(B)]


def test_ngram_reference_cases(gpu, golden):
    say("ngram reference cases")
    cases = golden["ngram_draft"]
    got = run([c["history"] for c in cases], 3, 4)
    assert got == [c["expect"] for c in cases]


@pytest.mark.parametrize("n", [2, 3, 5, 9])
@pytest.mark.parametrize("k", [0, 1, 5, 8])
def test_ngram_random_small_alphabet(gpu, n, k):
    say(f"ngram random n={n} k={k}")
    rng = np.random.default_rng(n * 10 + k)
    hists = [rng.integers(0, 4, int(rng.integers(0, 200))).tolist() for _ in range(40)]
    got = run(hists, n, k)
    want = [ora.ngram_draft(h, n, k) for h in hists]
    assert got == want


def test_ngram_config5_histories(gpu):
    """Config-5 shape: 8192-token histories with 40% injected repeats (scaled batch)."""
    say("ngram config5 histories")
    cfg = scaled(CONFIGS[5], num_seqs=16)
    h = make_histories(cfg, cfg.history_len)
    got = run([row.tolist() for row in h], cfg.ngram_n, cfg.max_drafts)
    want = [ora.ngram_draft(row, cfg.ngram_n, cfg.max_drafts) for row in h]
    assert got == want


def test_ngram_long_history_crosses_tiles(gpu):
    say("ngram long history")
    rng = np.random.default_rng(77)
    h = rng.integers(0, 50000, 20000).tolist()
    h[100:103] = [1, 2, 3]
    h[-2:] = [1, 2]     # the only match is far from the end (several LDS tiles back)
    assert run([h], 3, 3) == [ora.ngram_draft(h, 3, 3)]


@pytest.mark.parametrize("seed", range(12))
def test_ngram_random_mixed(gpu, seed):
    """Seeded batches mixing history lengths on both sides of the LDS-resident limit
    (12288 tokens) and past the tile width, small alphabets (many matches, so chained
    lookups run long) and large ones, odd row strides (unaligned rows), n = 2..9."""
    r = np.random.default_rng(900 + seed)
    n = int(r.integers(2, 10))
    k = int(r.integers(0, 9))
    B = int(r.integers(1, 12))
    alphabet = int(r.choice([2, 5, 50, 32000]))
    lens = [int(r.choice([0, 1, n - 1, n, int(r.integers(0, 4000)), 12287, 12288, 12289, int(r.integers(12289, 30000))]))
            for _ in range(B)]
    hists = []
    for L in lens:
        h = r.integers(0, alphabet, L)
        if L > 2 * n and r.random() < 0.5:  # plant the final key far back in the history
            pos = int(r.integers(0, L - 2 * n))
            h[pos:pos + n - 1] = h[L - (n - 1):]
        hists.append(h.tolist())
    stride = max(1, max(lens)) + int(r.integers(0, 3))  # 1 or 2 extra: rows not 16-byte aligned
    say(f"ngram random case {seed}: n={n} k={k} lens={lens} alphabet={alphabet} stride={stride}")
    h = np.zeros((B, stride), np.int32)
    ln = np.zeros(B, np.int32)
    for b, x in enumerate(hists):
        h[b, :len(x)] = x
        ln[b] = len(x)
    d, nn = gv.ngram_draft(torch.from_numpy(h).cuda(), torch.from_numpy(ln).cuda(), n, k)
    torch.cuda.synchronize()
    d, nn = d.cpu().numpy(), nn.cpu().numpy()
    got = [d[b, :nn[b]].tolist() for b in range(B)]
    want = [ora.ngram_draft(x, n, k) for x in hists]
    assert got == want
