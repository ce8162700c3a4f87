"""Shared helpers of the GPU parity tests: building pools through the HIP append,
mirroring them on the host, and comparing attention outputs."""
from __future__ import annotations

import ctypes as C
import math
import sys

import numpy as np
import torch

from gollmgo_amd._lib import DType
from gollmgo_amd.verify import KVCache
from oracle import oracle as ora

DT_NAME = {DType.F32: "f32", DType.F16: "f16", DType.BF16: "bf16", DType.FP8_E4M3: "fp8", DType.INT8: "int8"}
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
TOL = {"f32": 2e-3, "f16": 2e-3, "bf16": 2e-3, "fp8": 2e-2, "int8": 2e-2}


def say(msg: str) -> None:
    """Name the case before each GPU step (flushed, so it survives a crash)."""
    print(msg, flush=True)
    sys.stdout.flush()


def host_round(x: np.ndarray, dt: str) -> np.ndarray:
    if dt == "bf16":
        return ora.round_bf16(x)
    if dt == "f16":
        return ora.round_f16(x)
    return x.astype(np.float32)


class PoolMirror:
    """Host copy of one layer's pools, updated with the oracle's append rules."""

    def __init__(self, kv: KVCache):
        self.kv = kv
        self.H, self.D, self.bs, self.nb = kv.num_kv_heads, kv.head_dim, kv.block_size, kv.num_blocks
        self.dt = DT_NAME[kv.dtype]
        eb = {"f32": 4, "f16": 2, "bf16": 2, "fp8": 1, "int8": 1}[self.dt]
        n = self.nb * self.H * self.bs * self.D
        self.kc = np.zeros(n * eb, np.uint8)
        self.vc = np.zeros(n * eb, np.uint8)
        self.written = np.zeros((self.nb, self.bs), bool)
        self.k_inv = np.ones(self.H, np.float32)
        self.v_inv = np.ones(self.H, np.float32)
        self.k_scale = np.ones(self.H, np.float32)
        self.v_scale = np.ones(self.H, np.float32)
        self.k_bscale = np.zeros(self.nb * self.H, np.float32)
        self.v_bscale = np.zeros(self.nb * self.H, np.float32)

    def set_head_scales(self, ks, vs):
        self.k_scale = np.asarray(ks, np.float32)
        self.v_scale = np.asarray(vs, np.float32)
        self.k_inv = (np.float32(1.0) / self.k_scale).astype(np.float32)
        self.v_inv = (np.float32(1.0) / self.v_scale).astype(np.float32)

    def append(self, k: np.ndarray, v: np.ndarray, slots: np.ndarray):
        """k, v: [n, H, D] fp32 values (already exact in the source dtype)."""
        H, D, bs = self.H, self.D, self.bs
        if self.dt in ("fp8", "int8"):
            ora.kv_append_q(self.kc, self.vc, self.dt, H, D, bs, k, v, slots, self.k_inv, self.v_inv,
                            self.k_bscale, self.v_bscale)
        else:
            if self.dt == "f32":
                kview, vview, kk, vv = self.kc.view(np.float32), self.vc.view(np.float32), k, v
            elif self.dt == "f16":
                kview, vview = self.kc.view(np.float16), self.vc.view(np.float16)
                kk, vv = k.astype(np.float16), v.astype(np.float16)
            else:
                kview, vview = self.kc.view(np.uint16), self.vc.view(np.uint16)
                kk, vv = ora.bf16_bits(k), ora.bf16_bits(v)
            K = kview.reshape(self.nb, H, bs, D)
            V = vview.reshape(self.nb, H, D, bs)
            for r, s in enumerate(slots):
                if s < 0:
                    continue
                blk, o = divmod(int(s), bs)
                K[blk, :, o, :] = kk[r]
                V[blk, :, :, o] = vv[r]
        for s in slots:
            if s >= 0:
                self.written[int(s) // bs, int(s) % bs] = True

    def scales_for_oracle(self):
        if self.dt == "fp8":
            return self.k_scale, self.v_scale
        if self.dt == "int8":
            return self.k_bscale, self.v_bscale
        return None, None

    def compare_with_device(self, layer: int = 0):
        """Assert the device pools equal the mirror on every written slot."""
        eb = len(self.kc) // (self.nb * self.H * self.bs * self.D)
        kd = self.kv.k_pool(layer).cpu().numpy()
        vd = self.kv.v_pool(layer).cpu().numpy()
        K1 = kd.reshape(self.nb, self.H, self.bs, self.D * eb)
        K2 = self.kc.reshape(self.nb, self.H, self.bs, self.D * eb)
        V1 = vd.reshape(self.nb, self.H, self.D, self.bs, eb)
        V2 = self.vc.reshape(self.nb, self.H, self.D, self.bs, eb)
        blk, off = np.nonzero(self.written)
        np.testing.assert_array_equal(K1[blk, :, off], K2[blk, :, off])
        np.testing.assert_array_equal(V1[blk, :, :, off], V2[blk, :, :, off])
        if self.dt == "int8":
            ks, vs = self.kv.scales(layer)
            used = np.unique(blk)
            np.testing.assert_array_equal(ks.float().cpu().numpy()[used], self.k_bscale.reshape(self.nb, self.H)[used])
            np.testing.assert_array_equal(vs.float().cpu().numpy()[used], self.v_bscale.reshape(self.nb, self.H)[used])

    def sync_from_device(self, layer: int = 0):
        """Adopt the device's bytes (used after the append itself has been checked)."""
        self.kc = self.kv.k_pool(layer).cpu().numpy().copy()
        self.vc = self.kv.v_pool(layer).cpu().numpy().copy()
        if self.dt == "int8":
            ks, vs = self.kv.scales(layer)
            self.k_bscale = ks.float().cpu().numpy().reshape(-1).copy()
            self.v_bscale = vs.float().cpu().numpy().reshape(-1).copy()


def rel_err_per_vector(got: np.ndarray, ref: np.ndarray) -> float:
    """max over (row, head) vectors of max|got-ref| / max|ref|."""
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    num = np.abs(g - r).max(axis=1)
    den = np.maximum(np.abs(r).max(axis=1), 1e-12)
    return float((num / den).max())


def append_rows(kv: KVCache, mirror: PoolMirror, k: np.ndarray, v: np.ndarray, slots: np.ndarray,
                src: str = "f32", layer: int = 0):
    """Round k/v to the source dtype, append on the device and in the mirror."""
    k = host_round(k.astype(np.float32), src)
    v = host_round(v.astype(np.float32), src)
    kt = torch.from_numpy(k).to(TORCH_DT[src]).cuda()
    vt = torch.from_numpy(v).to(TORCH_DT[src]).cuda()
    st = torch.from_numpy(slots.astype(np.int32)).cuda()
    kv.append(layer, kt, vt, st)
    torch.cuda.synchronize()
    mirror.append(k, v, slots.astype(np.int32))


def glibc_rand_uniform(seed: int, n: int) -> np.ndarray:
    """((float)rand()/RAND_MAX - 0.5f) * 0.5f with glibc's srand/rand, as the reference's
    kernel tests draw their inputs (kernels/gollmgo_paged_attn_test.cu:61-63)."""
    libc = C.CDLL("libc.so.6")
    libc.srand(C.c_uint(seed))
    vals = np.array([libc.rand() for _ in range(n)], dtype=np.float32)
    return ((vals / np.float32(2147483647.0)) - np.float32(0.5)) * np.float32(0.5)


def per_head_amax_scales(x: np.ndarray) -> np.ndarray:
    """amax/448 per kv head over rows [n, H, D] (the reference's fp8 scale rule)."""
    amax = np.abs(x).max(axis=(0, 2)).astype(np.float32)
    return np.maximum(amax / np.float32(448.0), np.float32(1e-8)).astype(np.float32)


__all__ = ["PoolMirror", "rel_err_per_vector", "append_rows", "glibc_rand_uniform", "TOL", "say", "math"]


def check_positions(drafts, n, acc, tok, vocab: int, temperature: float, top_p: float, seed: int) -> None:
    """The engine's own Verify + Sample over the one-hot LogitsPerPosition rows built from a
    device decision must give that decision back, and a rejected draft is never the token."""
    from gollmgo_amd.positions import LogitsPerPosition

    drafts, n, acc, tok = (np.asarray(x) for x in (drafts, n, acc, tok))
    K = drafts.shape[1] if drafts.ndim == 2 else 0
    for b in range(len(acc)):
        nb = min(max(int(n[b]), 0), K)
        if acc[b] < nb:
            assert tok[b] != drafts[b, acc[b]], f"sequence {b}: the token after a rejection is the draft"
    pos = LogitsPerPosition(vocab).batch(drafts, n, acc, tok)
    u = np.random.default_rng(seed).random(len(acc))
    ea, et = ora.emit_positions(drafts, n, pos, temperature, top_p, u)
    assert np.array_equal(ea, acc) and np.array_equal(et, tok)
