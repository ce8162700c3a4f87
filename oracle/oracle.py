"""Python face of the CPU oracle (oracle/gg_oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, as the checker or as the timed CPU baseline; the product never does.
Every function here calls the C restatement or does plain numpy bookkeeping
(dtype conversions, array marshalling).
"""
from __future__ import annotations

import ctypes as C
import time
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libgg_oracle.so"

_lib = None


def build(force: bool = False) -> Path:
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "gg_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE), "-B" if force else "all"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- dtype helpers

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


def round_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def fp8_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().ora_fp8_encode_n(_p(x), _p(out), C.c_long(x.size))
    return out


def fp8_decode(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.shape, dtype=np.float32)
    lib().ora_fp8_decode_n(_p(b), _p(out), C.c_long(b.size))
    return out


def int8_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.int8)
    lib().ora_int8_encode_n(_p(x), _p(out), C.c_long(x.size))
    return out


def f16_round_c(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().ora_f16_round_n(_p(x), _p(out), C.c_long(x.size))
    return out


def expf_fixed(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().ora_expf_fixed_n(_p(x), _p(out), C.c_long(x.size))
    return out


def weight(l: float, m: float, inv_t: float) -> int:
    f = lib().ora_weight
    f.restype = C.c_uint64
    f.argtypes = [C.c_float, C.c_float, C.c_float]
    return int(f(l, m, inv_t))


# ---------------------------------------------------------------- Go host logic

def argmax(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().ora_argmax(_p(x), len(x)))


def verify(drafts, rows) -> tuple[int, int]:
    """speculative.go:68-84 on rows [n][V] (list of equal-length rows)."""
    d = np.ascontiguousarray(drafts, dtype=np.int32)
    if len(rows) == 0:
        r = np.zeros((0, 1), dtype=np.float32)
    else:
        r = np.ascontiguousarray(np.stack([np.asarray(x, dtype=np.float32) for x in rows]))
    acc, cor = C.c_int(), C.c_int()
    lib().ora_verify(_p(d), len(d), _p(r), r.shape[0], r.shape[1] if r.ndim == 2 else 0,
                     C.byref(acc), C.byref(cor))
    return acc.value, cor.value


def accept_greedy(logits_f32: np.ndarray, drafts: np.ndarray, n_drafts: np.ndarray):
    lg = np.ascontiguousarray(logits_f32, dtype=np.float32)
    B, R, V = lg.shape
    d = np.ascontiguousarray(drafts, dtype=np.int32).reshape(B, R - 1) if R > 1 else np.zeros((B, 0), np.int32)
    nd = np.ascontiguousarray(n_drafts, dtype=np.int32)
    acc = np.empty(B, np.int32)
    tok = np.empty(B, np.int32)
    lib().ora_accept_greedy(_p(lg), B, R - 1, V, _p(d), _p(nd), _p(acc), _p(tok))
    return acc, tok


def accept_rejection(logits_f32, drafts, n_drafts, uniforms, temperature, top_p=1.0, draft_probs=None):
    lg = np.ascontiguousarray(logits_f32, dtype=np.float32)
    B, R, V = lg.shape
    d = np.ascontiguousarray(drafts, dtype=np.int32).reshape(B, R - 1) if R > 1 else np.zeros((B, 0), np.int32)
    nd = np.ascontiguousarray(n_drafts, dtype=np.int32)
    u = np.ascontiguousarray(uniforms, dtype=np.float32)
    dp = np.ascontiguousarray(draft_probs, dtype=np.float32) if draft_probs is not None else None
    acc = np.empty(B, np.int32)
    tok = np.empty(B, np.int32)
    f = lib().ora_accept_rejection
    f.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                  C.c_float, C.c_float, C.c_void_p, C.c_void_p]
    f(_p(lg), B, R - 1, V, _p(dp) if dp is not None else None, _p(d), _p(nd), _p(u), float(temperature),
      float(top_p), _p(acc), _p(tok))
    return acc, tok


def ngram_draft(history, n: int, max_drafts: int) -> list[int]:
    h = np.ascontiguousarray(history, dtype=np.int32)
    k = max_drafts if max_drafts >= 1 else 4
    out = np.zeros(max(k, 1), np.int32)
    c = lib().ora_ngram_draft(_p(h), len(h), n, max_drafts, _p(out))
    if c < 0:
        raise ValueError("n must be <= 9")
    return [int(x) for x in out[:c]]


def ngram_draft_batch(hist: np.ndarray, lens: np.ndarray, n: int, K: int, threads: int = 1):
    h = np.ascontiguousarray(hist, dtype=np.int32)
    B, stride = h.shape
    ln = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.zeros((B, K), np.int32)
    out_n = np.zeros(B, np.int32)
    lib().ora_ngram_draft_batch(_p(h), stride, _p(ln), B, n, K, _p(out), _p(out_n), threads)
    return out, out_n


def softmax_f64(x):
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty_like(x)
    lib().ora_softmax_f64(_p(x), len(x), _p(out))
    return out


def top_p_filter_f64(p, top_p):
    p = np.ascontiguousarray(p, dtype=np.float64)
    out = np.empty_like(p)
    f = lib().ora_top_p_filter_f64
    f.argtypes = [C.c_void_p, C.c_int, C.c_double, C.c_void_p]
    f(_p(p), len(p), float(top_p), _p(out))
    return out


def categorical_f64(p, u: float) -> int:
    p = np.ascontiguousarray(p, dtype=np.float64)
    f = lib().ora_categorical_f64
    f.argtypes = [C.c_void_p, C.c_int, C.c_double]
    return int(f(_p(p), len(p), float(u)))


def sample_f64(logits, temperature: float, top_p: float, u: float, top_k: int = 0) -> int:
    """Sampler.Sample (sampling.go:40-72) with the uniform supplied."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    f = lib().ora_sample_f64
    f.argtypes = [C.c_void_p, C.c_int, C.c_double, C.c_int, C.c_double, C.c_double]
    return int(f(_p(x), len(x), float(temperature), int(top_k), float(top_p), float(u)))


def sampler_probs_f64(logits, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
    """The distribution Sampler.Sample hands to categoricalSample (temperature > 1e-9)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty(len(x), np.float64)
    f = lib().ora_sampler_probs_f64
    f.argtypes = [C.c_void_p, C.c_int, C.c_double, C.c_int, C.c_double, C.c_void_p]
    f(_p(x), len(x), float(temperature), int(top_k), float(top_p), _p(out))
    return out


def top_k_filter_f64(x, k: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty_like(x)
    f = lib().ora_top_k_filter_f64
    f.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    f(_p(x), len(x), int(k), _p(out))
    return out


def exp64(x) -> np.ndarray:
    """The float64 exponential of the sampler (fdlibm's method, as Go's portable math.Exp)."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty_like(x)
    f = lib().ora_exp64_n
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
    f(_p(x), _p(out), x.size)
    return out


def accept_greedy_sample(logits_f32, drafts, n_drafts, temperature: float, top_k: int, top_p: float,
                         uniforms, threads: int = 0):
    """Greedy Verify with the bonus drawn by Sampler.Sample (gg_accept_greedy_sample's rule)."""
    lg = np.ascontiguousarray(logits_f32, dtype=np.float32)
    B, R, V = lg.shape
    d = np.ascontiguousarray(drafts, dtype=np.int32).reshape(B, R - 1)
    nd = np.ascontiguousarray(n_drafts, dtype=np.int32)
    u = np.ascontiguousarray(uniforms, dtype=np.float64)
    acc = np.empty(B, np.int32)
    tok = np.empty(B, np.int32)
    f = lib().ora_accept_greedy_sample
    f.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_double, C.c_int,
                  C.c_double, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
    f(_p(lg), B, R - 1, V, _p(d) if d.size else None, _p(nd), float(temperature), int(top_k), float(top_p),
      _p(u), _p(acc), _p(tok), threads)
    return acc, tok


def emit_positions(drafts, n_drafts, positions, temperature: float = 0.0, top_p: float = 1.0,
                   uniforms=None, timer=None, top_k: int = 0):
    """What emitSpeculative (serving.go:496-570) takes from LogitsPerPosition: per sequence
    (accepted, token), token -1 when every draft is accepted and no further row is given.
    positions[b] is a list of 1-D float32 rows (ragged, as Go slices). timer: a list that
    receives the seconds spent in the C routine alone."""
    d = np.ascontiguousarray(drafts, dtype=np.int32)
    B = len(positions)
    K = d.shape[1] if d.ndim == 2 else 0
    nd = np.ascontiguousarray(n_drafts, dtype=np.int32)
    flat = [np.ascontiguousarray(r, dtype=np.float32) for rows in positions for r in rows]
    ptrs = (C.c_void_p * max(1, len(flat)))(*[r.ctypes.data for r in flat])
    lens = np.array([len(r) for r in flat] or [0], np.int32)
    counts = np.array([len(rows) for rows in positions], np.int32)
    u = np.ascontiguousarray(uniforms if uniforms is not None else np.zeros(B), dtype=np.float64)
    acc = np.empty(B, np.int32)
    tok = np.empty(B, np.int32)
    f = lib().ora_emit_positions
    f.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                  C.c_double, C.c_int, C.c_double, C.c_void_p, C.c_void_p, C.c_void_p]
    t0 = time.perf_counter()
    f(B, K, _p(d) if d.size else None, _p(nd), ptrs, _p(lens), _p(counts), float(temperature),
      int(top_k), float(top_p), _p(u), _p(acc), _p(tok))
    if timer is not None:
        timer.append(time.perf_counter() - t0)
    return acc, tok


# ---------------------------------------------------------------- KV cache

DT_CODE = {"f32": 0, "f16": 1, "bf16": 2, "fp8": 3, "int8": 4}


def kv_append_q(kc: np.ndarray, vc: np.ndarray, dt: str, H: int, D: int, bs: int, k: np.ndarray,
                v: np.ndarray, slots: np.ndarray, k_inv=None, v_inv=None, k_bscale=None, v_bscale=None):
    """Quantised append for fp8 / int8 pools, in place on the numpy byte pools."""
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    s = np.ascontiguousarray(slots, dtype=np.int32)
    ki = np.ascontiguousarray(k_inv if k_inv is not None else np.ones(H), dtype=np.float32)
    vi = np.ascontiguousarray(v_inv if v_inv is not None else np.ones(H), dtype=np.float32)
    kb = k_bscale if k_bscale is not None else np.zeros(1, np.float32)
    vb = v_bscale if v_bscale is not None else np.zeros(1, np.float32)
    assert kc.flags.c_contiguous and vc.flags.c_contiguous and kb.dtype == np.float32
    lib().ora_kv_append_q(_p(kc), _p(vc), DT_CODE[dt], H, D, bs, _p(k), _p(v), _p(s), len(s), _p(ki), _p(vi),
                          _p(kb), _p(vb))


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, dt: str, H: int, D: int, bs: int,
              ctx_lens: np.ndarray, block_tables: np.ndarray, scale: float, k_scale=None, v_scale=None,
              row_counts=None, threads: int = 0, fn: str = "ora_attention") -> np.ndarray:
    """fp64 textbook attention; q [B,R,Hq,D] fp32 values; pools as raw bytes (one
    layer, all blocks: the block count is taken from their size)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, R, Hq, Dq = q.shape
    assert Dq == D
    out = np.zeros_like(q)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    rc = np.ascontiguousarray(row_counts, dtype=np.int32) if row_counts is not None else None
    ks = np.ascontiguousarray(k_scale, dtype=np.float32) if k_scale is not None else None
    vs = np.ascontiguousarray(v_scale, dtype=np.float32) if v_scale is not None else None
    kc = np.ascontiguousarray(kc)
    vc = np.ascontiguousarray(vc)
    eb = {"f32": 4, "f16": 2, "bf16": 2, "fp8": 1, "int8": 1}[dt]
    num_blocks = kc.nbytes // (H * bs * D * eb)
    f = getattr(lib(), fn)
    f.argtypes = [C.c_void_p] * 4 + [C.c_int] * 4 + [C.c_void_p] * 5 + [C.c_int] * 4 + [C.c_float, C.c_int, C.c_int]
    f(_p(q), _p(out), _p(kc), _p(vc), DT_CODE[dt], H, D, bs,
      _p(ks) if ks is not None else None, _p(vs) if vs is not None else None, _p(cl),
      _p(rc) if rc is not None else None, _p(bt), bt.shape[1], B, R, Hq, float(scale), threads, int(num_blocks))
    return out


def attention_ref_f32(q, kc, vc, dt, H, D, bs, ctx_lens, block_tables, scale, k_scale=None, v_scale=None,
                      row_counts=None, threads: int = 0) -> np.ndarray:
    """The reference's v1 attention semantics in fp32 (kernels/gollmgo_paged_attn.cu:38-119):
    the timed CPU baseline of bench.py, not the checker (that is `attention`, fp64)."""
    return attention(q, kc, vc, dt, H, D, bs, ctx_lens, block_tables, scale, k_scale, v_scale, row_counts, threads,
                     fn="ora_attention_ref_f32")
