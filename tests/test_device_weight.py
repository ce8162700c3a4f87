"""The device's fixed-point weight (gollmgo_amd/csrc/gg_fixed_exp.h, gg_weight) compiled for
the host and compared with the oracle's floor(expf_fixed(x) * 2^35). The device writes the
weight without per-element branches (x clamped to -80 instead of a zero select, and the
floor to 64 bits as two 32-bit conversions); this pins that formulation to the oracle's
rule over every float class: a strided sweep of all 2^32 bit patterns, the whole range
where the weight is non-zero at a fine step, and the special values. CPU only."""
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = r"""
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "gg_fixed_exp.h"
int main(int argc, char** argv) {
    FILE* f = fopen(argv[1], "rb");
    FILE* g = fopen(argv[2], "wb");
    float x;
    while (fread(&x, 4, 1, f) == 1) {
        unsigned long long w = gg_weight(x, 0.0f, 1.0f);
        fwrite(&w, 8, 1, g);
    }
    fclose(f);
    fclose(g);
    return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_device_weight_equals_oracle_rule(ora, tmp_path):
    c = tmp_path / "w.c"
    c.write_text(SRC)
    exe = tmp_path / "w"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", str(ROOT / "gollmgo_amd" / "csrc"), str(c), "-o",
                    str(exe), "-lm"], check=True)
    pats = np.arange(0, 1 << 32, 4093, dtype=np.uint64).astype(np.uint32).view(np.float32)
    dense = np.arange(-85.0, 1.0, 1.0 / 4096, dtype=np.float64).astype(np.float32)
    special = np.array([0.0, -0.0, 1.0, -80.0, np.nextafter(np.float32(-80), np.float32(0)),
                        np.nextafter(np.float32(-80), np.float32(-100)), -24.26, -np.inf, np.inf, np.nan,
                        np.float32(1e-45), np.float32(-1e-45), 3.4e38, -3.4e38], np.float32)
    x = np.concatenate([pats, dense, special]).astype(np.float32)
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    subprocess.run([str(exe), str(tmp_path / "x.bin"), str(tmp_path / "w.bin")], check=True)
    got = np.frombuffer((tmp_path / "w.bin").read_bytes(), np.uint64)
    e = ora.expf_fixed(x)
    with np.errstate(invalid="ignore"):
        want = np.floor(e * np.float32(2.0 ** 35)).astype(np.float64)
    want = np.where(np.isfinite(want), want, 0).astype(np.uint64)
    assert got.shape == want.shape
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (x[bad[:5]], got[bad[:5]], want[bad[:5]])
    assert got[np.nonzero(x == 0)[0][0]] == 1 << 35
