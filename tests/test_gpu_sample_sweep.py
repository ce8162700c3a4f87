"""GPU: the float64 draw against the oracle's float64 rule over many rows per setting, as a
count of disagreements that must be zero. Sampled bonuses (gg_accept_greedy_sample with no
drafts: every sequence draws its token from its row by Sampler.Sample) and rejection
residuals (gg_accept_rejection, every draft rejected, dense and one-hot q) on random rows of
a 32000-entry vocab. The suite runs GG_SAMPLE_SWEEP_ROWS rows per setting (default 2000);
the count recorded in the design notes was run with 100000."""
import os

import numpy as np
import pytest
import torch

import gollmgo_amd.verify as gv
from helpers import say
from oracle import oracle as ora

pytestmark = pytest.mark.gpu

ROWS = int(os.environ.get("GG_SAMPLE_SWEEP_ROWS", "2000"))
V = 32000
CHUNK = 2000


@pytest.mark.parametrize("T,top_k,top_p", [(0.8, 0, 0.0), (0.8, 50, 0.0), (0.8, 0, 0.95), (1.0, 50, 0.9)])
def test_sampled_bonus_sweep(gpu, T, top_k, top_p):
    rng = np.random.default_rng(1000 + top_k + int(top_p * 100))
    bad = done = 0
    while done < ROWS:
        B = min(CHUNK, ROWS - done)
        sd = rng.uniform(1.0, 4.0)
        lg = torch.from_numpy(rng.normal(0, sd, (B, 1, V)).astype(np.float32)).to(torch.bfloat16)
        host = lg.float().numpy()
        u = rng.random(B)
        drafts, n = np.zeros((B, 0), np.int32), np.zeros(B, np.int32)
        ea, et = ora.accept_greedy_sample(host, drafts, n, T, top_k, top_p, u, threads=16)
        acc, tok = gv.accept_greedy_sample(lg.cuda(), torch.from_numpy(drafts).cuda(), torch.from_numpy(n).cuda(),
                                           torch.from_numpy(u).cuda(), T, top_k, top_p)
        torch.cuda.synchronize()
        bad += int(((acc.cpu().numpy() != ea) | (tok.cpu().numpy() != et)).sum())
        done += B
        if done % 20000 == 0:
            say(f"  {done} rows, {bad} disagreements")
    say(f"sampled bonus T={T} k={top_k} p={top_p}: {done} rows, {bad} disagreements")
    assert bad == 0


@pytest.mark.parametrize("dense,top_p", [(False, 1.0), (False, 0.95), (True, 1.0)])
def test_rejection_residual_sweep(gpu, dense, top_p):
    rng = np.random.default_rng(2000 + int(dense) + int(top_p * 100))
    T = 0.8
    bad = done = 0
    while done < ROWS:
        B = min(CHUNK // 2, ROWS - done)
        host = rng.normal(0, rng.uniform(1.0, 3.0), (B, 2, V)).astype(np.float32)
        drafts = np.argmin(host[:, :1], axis=-1).astype(np.int32)  # outside any nucleus
        q = rng.dirichlet(np.ones(V) * 0.3, (B, 1)).astype(np.float32) if dense else None
        if dense:
            q[np.arange(B), 0, drafts[:, 0]] = 0.5  # q(x) > p(x): rejected for any u
        n = np.ones(B, np.int32)
        u = rng.random((B, 2)).astype(np.float32)
        ea, et = ora.accept_rejection(host, drafts, n, u, T, top_p, q)
        ga, gt = gv.accept_rejection(torch.from_numpy(host).cuda(), torch.from_numpy(drafts).cuda(),
                                     torch.from_numpy(n).cuda(), torch.from_numpy(u).cuda(), T, top_p,
                                     torch.from_numpy(q).cuda() if dense else None)
        torch.cuda.synchronize()
        bad += int(((ga.cpu().numpy() != ea) | (gt.cpu().numpy() != et)).sum())
        assert (ea == 0).all()
        done += B
        if done % 10000 == 0:
            say(f"  {done} rows, {bad} disagreements")
    say(f"rejection residual dense={dense} top_p={top_p}: {done} rows, {bad} disagreements")
    assert bad == 0
