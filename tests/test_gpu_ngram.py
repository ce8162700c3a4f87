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
