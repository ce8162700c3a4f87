"""Build the gfx950 verify-path library (libgg_verify.so) in-tree with hipcc.

Every .hip / .cpp file under csrc/ is compiled to an object for gfx950 and
linked into one shared library next to this file. Objects are rebuilt only when
a source or header is newer, unless ``force`` is set.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libgg_verify.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
# Packed-fp32 instructions are kept out of generated code: the feature is turned
# off for the device pass (the host pass warns that it does not know it).
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
# Per-source flags. The attention kernels are scheduled by LLVM's ILP-first machine
# scheduler: in their chunk loop it places the next chunk's loads and the independent
# decode and softmax work further from their uses than the default occupancy-first
# strategy, with the same occupancy (two workgroups per CU). Same box, HIP events, µs per
# call: config 3 119.1 -> 117.9 (eight seeded layouts 123.7 -> 121.0), configs 2 and 5
# unchanged, config 4 117.8 -> 118.1.
SOURCE_FLAGS = {
    "attention_mfma.hip": ("-mllvm", "-amdgpu-sched-strategy=max-ilp"),
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the verify-path library needs ROCm's hipcc")


def _sources() -> list[Path]:
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])


def _headers() -> list[Path]:
    return sorted([*CSRC.glob("*.h"), *INCLUDE.glob("*.h")])


def _compile(src: Path, force: bool, obj_dir: Path = OBJ, extra: tuple = ()) -> Path:
    obj = obj_dir / (src.name + ".o")
    newest_dep = max([src.stat().st_mtime] + [h.stat().st_mtime for h in _headers()])
    if not force and obj.exists() and obj.stat().st_mtime >= newest_dep:
        return obj
    flags = [*HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, ()), *extra]
    cmd = [hipcc(), *flags, "-I", str(INCLUDE), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [hipcc(), *flags, "-x", "hip", "-I", str(INCLUDE), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(force: bool = False, verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = _sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    need_link = force or not LIB.exists() or any(o.stat().st_mtime > LIB.stat().st_mtime for o in objs)
    if need_link:
        tmp = LIB.with_suffix(".so.tmp")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stderr}")
        os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_trace(force: bool = False) -> Path:
    """The timeline build: every source with -DGG_TRACE, linked to libgg_verify_trace.so
    (loaded instead of the library when GG_VERIFY_TRACE=1). Diagnostics only."""
    obj_dir = OBJ / "trace"
    obj_dir.mkdir(parents=True, exist_ok=True)
    out = PKG / "libgg_verify_trace.so"
    with ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(lambda s: _compile(s, force, obj_dir, ("-DGG_TRACE",)), _sources()))
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    return out


if __name__ == "__main__":
    build(force="--force" in sys.argv, verbose=True)
