"""The C ABI library loads and exports every entry point include/gg_verify.h declares;
argument checks that run before any HIP call behave like the reference's C ABI
(NULL / invalid -> GG_ERR_INVALID with a message, destroy(NULL) -> OK). CPU only."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from gollmgo_amd import _lib
from gollmgo_amd._lib import DType, Status

HEADER = Path(__file__).resolve().parent.parent / "include" / "gg_verify.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_surface():
    names = declared()
    for n in ["gg_kv_create", "gg_kv_append", "gg_verify_attention", "gg_accept_greedy",
              "gg_accept_rejection", "gg_ngram_draft", "gg_last_error"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for n in declared():
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\b(gg_[a-z0-9_]+)\b", out))
    assert set(declared()) <= exported
    # The Python binding covers the whole surface.
    assert set(declared()) == set(_lib.SIGNATURES)


def test_library_is_built_for_gfx950():
    data = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data


def test_invalid_arguments_return_status():
    lib = _lib.lib()
    assert lib.gg_kv_create(1, 1, 16, 1, 128, int(DType.BF16), 0, None) == Status.ERR_INVALID
    assert "out is NULL" in _lib.last_error()
    h = C.c_void_p()
    assert lib.gg_kv_create(0, 1, 16, 1, 128, int(DType.BF16), 0, C.byref(h)) == Status.ERR_INVALID
    assert lib.gg_kv_create(1, 1, 16, 1, 128, int(DType.FP8_E4M3), 0, C.byref(h)) == Status.ERR_INVALID
    assert "PER_HEAD" in _lib.last_error()
    assert lib.gg_kv_destroy(None) == Status.OK
    assert lib.gg_kv_append(None, 0, None, None, 0, None, 1, None) == Status.ERR_INVALID
    assert lib.gg_verify_attention(None, 0, None, 0, None, 0, None, None, None, 1, 1, 1, 1, 1.0, 0, None, 0,
                                   None) == Status.ERR_INVALID
    assert lib.gg_accept_greedy(None, 0, 1, 4, 0, None, None, None, None, None, 0, None) == Status.ERR_INVALID
    assert lib.gg_accept_rejection(None, 0, None, 1, 4, 1 << 19, None, None, None, 0.8, 1.0, None, None, None, 0,
                                   None) == Status.ERR_INVALID
    assert "vocab" in _lib.last_error()
    assert lib.gg_accept_greedy_sample(None, 0, 1, 4, 100, None, None, 0.8, 0, 0.9, None, 0, None, None, None, 0,
                                       None) == Status.ERR_INVALID
    assert "NULL buffer" in _lib.last_error()
    assert lib.gg_ngram_draft(None, 0, None, 1, 10, 4, None, None, None) == Status.ERR_INVALID
    assert "n must be <= 9" in _lib.last_error()
    assert lib.gg_history_append_draft(None, 16, None, None, 1, None, 0, None, None, 3, 4, None, None,
                                       None) == Status.ERR_INVALID
    assert "NULL buffer" in _lib.last_error()
    assert lib.gg_history_append_draft(None, 16, None, None, 1, None, 65, None, None, 3, 4, None, None,
                                       None) == Status.ERR_INVALID
    assert "bad shape" in _lib.last_error()
    assert lib.gg_kv_k_layer_ptr(None, 0) is None


def test_workspace_sizes_are_host_only():
    lib = _lib.lib()
    g = lib.gg_accept_greedy_workspace_size(64, 5, 128256)
    assert g == 64 * 6 * ((128256 + 4095) // 4096) * 8
    assert lib.gg_accept_rejection_workspace_size(64, 5, 128256) >= g
    assert lib.gg_accept_greedy_workspace_size(0, 5, 100) == 0
