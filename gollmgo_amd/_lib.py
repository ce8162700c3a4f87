"""ctypes binding of libgg_verify.so (the C ABI declared in include/gg_verify.h).

The library is loaded from this package directory only. There is no fallback:
if it is missing, every entry point raises, so a GPU run can never silently
take another code path. GG_VERIFY_TRACE=1 loads the timeline build instead
(libgg_verify_trace.so, compiled with -DGG_TRACE by build.build_trace; same
kernels, plus per-workgroup timestamps of the LPT attention kernel).
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from pathlib import Path

_TRACE = os.environ.get("GG_VERIFY_TRACE", "") == "1"
LIB_PATH = Path(__file__).resolve().parent / ("libgg_verify_trace.so" if _TRACE else "libgg_verify.so")


class Status(enum.IntEnum):
    OK = 0
    ERR_HIP = 1
    ERR_OOM = 2
    ERR_INVALID = 3
    ERR_INTERNAL = 4


class DType(enum.IntEnum):
    F32 = 0
    F16 = 1
    BF16 = 2
    FP8_E4M3 = 3
    INT8 = 4


class ScaleMode(enum.IntEnum):
    NONE = 0
    PER_HEAD = 1
    PER_BLOCK = 2


class GGError(RuntimeError):
    def __init__(self, status: int, where: str, msg: str):
        super().__init__(f"{where}: status {Status(status).name}: {msg}")
        self.status = Status(status)


_vp = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t
_i32p = C.POINTER(C.c_int32)

# name -> (restype, argtypes)
SIGNATURES = {
    "gg_last_error": (C.c_char_p, []),
    "gg_version": (C.c_char_p, []),
    "gg_set_device": (_i, [_i]),
    "gg_sync": (_i, [_vp]),
    "gg_kv_create": (_i, [_i, _i, _i, _i, _i, _i, _i, C.POINTER(_vp)]),
    "gg_kv_destroy": (_i, [_vp]),
    "gg_kv_k_layer_ptr": (_vp, [_vp, _i]),
    "gg_kv_v_layer_ptr": (_vp, [_vp, _i]),
    "gg_kv_k_scale_ptr": (_vp, [_vp, _i]),
    "gg_kv_v_scale_ptr": (_vp, [_vp, _i]),
    "gg_kv_layer_bytes": (_sz, [_vp]),
    "gg_kv_set_head_scales": (_i, [_vp, _i, C.POINTER(_f), C.POINTER(_f)]),
    "gg_kv_append": (_i, [_vp, _i, _vp, _vp, _i, _vp, _i, _vp]),
    "gg_kv_snapshot_bytes": (_sz, [_vp, _i]),
    "gg_kv_snapshot": (_i, [_vp, _vp, _i, _vp, _sz, _vp, _vp]),
    "gg_kv_restore": (_i, [_vp, _vp, _i, _vp, _sz, _vp, _vp]),
    "gg_verify_attention_workspace_size": (_sz, [_vp, _i, _i, _i, _i, _i]),
    "gg_verify_attention": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i,
                                 _vp, _sz, _vp]),
    "gg_verify_attention_plan": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "gg_verify_attention_planned": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _f,
                                         _vp, _sz, _vp]),
    "gg_verify_append_attention_planned": (_i, [_vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i, _vp, _vp, _vp, _i,
                                                _i, _i, _i, _f, _vp, _sz, _vp]),
    "gg_verify_attention_noalloc_max_bytes": (_sz, []),
    "gg_verify_attention_noalloc": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp]),
    "gg_accept_greedy_workspace_size": (_sz, [_i, _i, _i]),
    "gg_accept_greedy": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "gg_accept_greedy_sample_workspace_size": (_sz, [_i, _i, _i]),
    "gg_accept_greedy_sample": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, C.c_double, _i, C.c_double, _vp, C.c_uint,
                                     _vp, _vp, _vp, _sz, _vp]),
    "gg_accept_rejection_workspace_size": (_sz, [_i, _i, _i]),
    "gg_accept_rejection": (_i, [_vp, _i, _vp, _i, _i, _i, _vp, _vp, _vp, _f, _f, _vp, _vp, _vp,
                                 _sz, _vp]),
    "gg_ngram_draft": (_i, [_vp, _i, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "gg_history_append_draft": (_i, [_vp, _i, _vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i, _vp, _vp, _vp]),
}

_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load libgg_verify.so (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(the verify path has no non-HIP fallback)")
        handle = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if _TRACE:
            handle.gg_debug_trace_ptr.restype = C.c_void_p
            handle.gg_debug_trace_ptr.argtypes = []
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().gg_last_error().decode()


def check(status: int, where: str) -> None:
    if status != Status.OK:
        raise GGError(status, where, last_error())
