"""The oracle's float64 sampler (ora_sampler_probs_f64 / ora_sample_f64, the rule of
gg_accept_greedy_sample) pinned without Go: the reference's known answers, an independent
numpy restatement, closed forms, and its exponential (ora_exp64) against libm. CPU only."""
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def ulp_diff(a, b):
    return np.abs(a.view(np.int64) - b.view(np.int64))


def test_exp64_against_libm(ora):
    """fdlibm's method is within 1 ulp of glibc's exp (which is within about half an ulp of
    the true value) over the domain the sampler uses (x <= 0) and beyond."""
    rng = np.random.default_rng(0)
    x = np.concatenate([-rng.random(1_000_000) * 745.2, -rng.random(500_000) * 40, -rng.random(100_000) * 1e-6,
                        rng.random(100_000) * 709, -np.logspace(-300, 2.87, 10_000)])
    a, b = ora.exp64(x), np.exp(x)
    d = ulp_diff(a, b)
    assert d.max() <= 1
    assert (d == 0).mean() > 0.85
    assert ora.exp64(np.array([0.0]))[0] == 1.0 and ora.exp64(np.array([-0.0]))[0] == 1.0
    sp = ora.exp64(np.array([-np.inf, np.inf, -746.0, 710.0, 1e-300, -1e-300]))
    assert sp[0] == 0 and np.isinf(sp[1]) and sp[2] == 0 and np.isinf(sp[3]) and sp[4] == 1 and sp[5] == 1
    assert np.isnan(ora.exp64(np.array([np.nan])))[0]
    # subnormal results round once: e^-740 = 4.2e-322
    assert abs(ora.exp64(np.array([-740.0]))[0] - np.exp(-740.0)) <= 5e-324


def test_exp64_is_monotone(ora):
    """Non-decreasing over dense sorted sweeps and at consecutive doubles (the device's
    nucleus tie check relies on it)."""
    rng = np.random.default_rng(1)
    x = np.sort(np.concatenate([-rng.random(2_000_000) * 745, np.linspace(-50, 0, 1_000_001)]))
    e = ora.exp64(x)
    assert np.all(np.diff(e) >= 0)
    base = -rng.random(200_000) * 700
    nxt = np.nextafter(base, 0.0)
    assert np.all(ora.exp64(nxt) >= ora.exp64(base))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_device_exp64_equals_oracle(ora, tmp_path):
    """The device header gg_exp64.h compiled for the host gives the oracle's bits."""
    src = tmp_path / "e.c"
    src.write_text(r"""
#include <stdio.h>
#include "gg_exp64.h"
int main(int argc, char** argv) {
    FILE* f = fopen(argv[1], "rb"); FILE* g = fopen(argv[2], "wb"); double x;
    while (fread(&x, 8, 1, f) == 1) { double y = gg_exp64(x); fwrite(&y, 8, 1, g); }
    fclose(f); fclose(g); return 0;
}
""")
    exe = tmp_path / "e"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", str(ROOT / "gollmgo_amd" / "csrc"), str(src), "-o",
                    str(exe), "-lm"], check=True)
    rng = np.random.default_rng(2)
    x = np.concatenate([-rng.random(1_000_000) * 746, -rng.random(100_000) * 1e-8, [0.0, -0.0, -np.inf, np.nan,
                                                                                     -745.13, -708.4, 3.0]])
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    subprocess.run([str(exe), str(tmp_path / "x.bin"), str(tmp_path / "y.bin")], check=True)
    got = np.frombuffer((tmp_path / "y.bin").read_bytes(), np.float64)
    want = ora.exp64(x)
    same = (got.view(np.int64) == want.view(np.int64)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), x[~same][:5]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fast_exp64_error_bound(ora, tmp_path):
    """The device's parallel-path exponential stays within 2e-14 relative of ora_exp64 on
    [-708, 0] (the draw's margins count 1e-12), and gives 0 below -745.2."""
    src = tmp_path / "f.c"
    src.write_text(r"""
#include <stdio.h>
#include "gg_exp64.h"
int main(int argc, char** argv) {
    FILE* f = fopen(argv[1], "rb"); FILE* g = fopen(argv[2], "wb"); double x;
    double tab[64]; gg_exp64_table(tab);
    int use_tab = argc > 3;
    while (fread(&x, 8, 1, f) == 1) {
        double y = use_tab ? gg_fast_exp64_tab(x, tab) : gg_fast_exp64(x);
        fwrite(&y, 8, 1, g);
    }
    fclose(f); fclose(g); return 0;
}
""")
    exe = tmp_path / "f"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", str(ROOT / "gollmgo_amd" / "csrc"), str(src), "-o",
                    str(exe), "-lm"], check=True)
    rng = np.random.default_rng(3)
    x = np.concatenate([-rng.random(2_000_000) * 708, -rng.random(500_000) * 2, np.linspace(-708, 0, 200_001)])
    want = ora.exp64(x)
    for extra in ([], ["tab"]):  # gg_fast_exp64, then the table-driven gg_fast_exp64_tab
        (tmp_path / "x.bin").write_bytes(x.tobytes())
        subprocess.run([str(exe), str(tmp_path / "x.bin"), str(tmp_path / "y.bin"), *extra], check=True)
        got = np.frombuffer((tmp_path / "y.bin").read_bytes(), np.float64)
        rel = np.abs(got - want) / want
        assert rel.max() < 2e-14, (extra, rel.max())
        (tmp_path / "x.bin").write_bytes(np.array([-745.3, -1000.0, np.nan, -np.inf]).tobytes())
        subprocess.run([str(exe), str(tmp_path / "x.bin"), str(tmp_path / "y.bin"), *extra], check=True)
        assert (np.frombuffer((tmp_path / "y.bin").read_bytes(), np.float64) == 0).all()


def test_top_k_reference_case(ora, golden):
    """sampling_test.go:56-71: top-2 of {1,5,3,2,4} keeps indices 1 and 4."""
    f = ora.top_k_filter_f64(np.array([1.0, 5.0, 3.0, 2.0, 4.0]), 2)
    assert np.isinf(f[[0, 2, 3]]).all() and (f[[0, 2, 3]] < 0).all()
    assert f[1] == 5.0 and f[4] == 4.0


def test_top_k_ties_and_nan(ora):
    f = ora.top_k_filter_f64(np.array([1.0, 3.0, 3.0, np.nan, 3.0, -0.0, 0.0]), 2)
    assert f[1] == 3.0 and f[2] == 3.0 and np.isneginf(f[4])  # equal values: lower index first
    f = ora.top_k_filter_f64(np.array([np.nan, 1.0, -np.inf]), 3)
    assert np.isnan(f[0]) and f[1] == 1.0
    f = ora.top_k_filter_f64(np.array([np.nan, 1.0, -np.inf]), 2)
    assert np.isneginf(f[0]) and f[1] == 1.0 and np.isneginf(f[2])  # NaN after every number


def numpy_sampler_probs(logits, T, top_k, top_p, exp64):
    """An independent restatement of sampling.go:57-71 in numpy (finite logits): stable sorts
    for the open tie order, np.cumsum for the sequential float64 sums."""
    v = logits.astype(np.float64) * (1.0 / T)
    n = len(v)
    if 0 < top_k < n:
        order = np.argsort(-v, kind="stable")
        kept = np.full(n, -np.inf)
        kept[order[:top_k]] = v[order[:top_k]]
        v = kept
    mx = v.max()
    e = np.where(np.isneginf(v), 0.0, exp64(np.where(np.isneginf(v), 0.0, v - mx)))
    s = np.cumsum(e)[-1]
    p = e / s if s > 0 else e
    if 0 < top_p < 1:
        order = np.argsort(-p, kind="stable")
        c = np.concatenate([[0.0], np.cumsum(p[order])])
        stop = np.nonzero((c >= top_p) & (c > 0))[0]
        m = stop[0] if len(stop) else n
        r = np.zeros(n)
        r[order[:m]] = p[order[:m]]
        s2 = np.cumsum(r)[-1]
        p = r / s2 if s2 > 0 else r
    return p


@pytest.mark.parametrize("T,top_k,top_p", [(0.8, 0, 0.0), (0.8, 50, 0.0), (1.0, 0, 0.9), (0.7, 20, 0.6),
                                           (2.5, 999, 0.99), (0.3, 1, 0.5)])
def test_sampler_probs_match_numpy_restatement(ora, T, top_k, top_p):
    rng = np.random.default_rng(int(T * 10) + top_k)
    for trial in range(6):
        V = int(rng.integers(50, 5000))
        lg = rng.normal(0, 2, V).astype(np.float32)
        if trial % 2:
            lg = np.round(lg * 2) / 2  # ties
        want = numpy_sampler_probs(lg, T, top_k, top_p, ora.exp64)
        got = ora.sampler_probs_f64(lg, T, top_k, top_p)
        assert np.array_equal(got, want)
        c = np.cumsum(want)
        for u in rng.random(20):
            i = int(np.searchsorted(c, u, side="right"))
            if i >= V:
                i = int(np.nonzero(want > 0)[0][-1])
            assert ora.sample_f64(lg, T, top_p, float(u), top_k=top_k) == i


def test_sample_closed_forms(ora):
    rng = np.random.default_rng(4)
    lg = rng.normal(0, 2, 1000).astype(np.float32)
    am = ora.argmax(lg)
    for u in (0.0, 0.3, 0.999999):
        assert ora.sample_f64(lg, 0.8, 0.0, u, top_k=1) == am      # top-1 is the argmax
        assert ora.sample_f64(lg, 0.0, 0.9, u, top_k=5) == am      # T <= 1e-9 is greedy
        assert ora.sample_f64(lg, 1e-9, 0.9, u, top_k=5) == am
    # top_k >= n is off; top_p >= 1 or <= 0 is off
    for u in (0.1, 0.7):
        a = ora.sample_f64(lg, 0.8, 0.0, u)
        assert ora.sample_f64(lg, 0.8, 0.0, u, top_k=1000) == a
        assert ora.sample_f64(lg, 0.8, 1.0, u, top_k=0) == a
    # sampling_test.go's TestTemperatureSampling logits {10,0,0,0}: at T = 0.01 index 0
    # holds all the mass; at T = 100 the four are near uniform, so u = 0.6 picks index 2.
    t = np.array([10, 0, 0, 0], np.float32)
    assert all(ora.sample_f64(t, 0.01, 0.0, u) == 0 for u in (0.0, 0.5, 0.999))
    assert ora.sample_f64(t, 100.0, 0.0, 0.6) == 2


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_exp64_table_literals(ora, tmp_path):
    """The fast exponential's table literals (GG_EXP64_TAB64) are gg_exp64(j ln2 / 64) bit
    for bit, and equal the oracle's exp64 there."""
    src = tmp_path / "t.c"
    src.write_text(r"""
#include <stdio.h>
#include <string.h>
#include "gg_exp64.h"
int main(void) {
    double t[64];
    gg_exp64_table(t);
    int bad = 0;
    for (int j = 0; j < 64; ++j) {
        const double v = gg_exp64((double)j * (6.93147180559945286227e-01 / 64.0));
        if (memcmp(&v, &t[j], 8) != 0) ++bad;
        printf("%a\n", t[j]);
    }
    return bad;
}
""")
    exe = tmp_path / "t"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", str(ROOT / "gollmgo_amd" / "csrc"), str(src), "-o",
                    str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0
    got = np.array([float.fromhex(v) for v in res.stdout.split()])
    want = ora.exp64(np.arange(64) * (0.693147180559945286227 / 64.0))
    assert np.array_equal(got.view(np.int64), want.view(np.int64))
