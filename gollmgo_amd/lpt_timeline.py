"""Slot occupancy of the LPT attention kernel over time (diagnostics).

Runs bench.py's step for a config on the timeline build of the library
(libgg_verify_trace.so: every LPT workgroup records its start and end in 100 MHz wall-clock
ticks) and prints, for the last attention launch, how many workgroups were busy over the
kernel's span and over its last 20 us. Build the timeline library first:
    python -c "from gollmgo_amd.build import build_trace; build_trace()"
Run on the GPU:
    python -m gollmgo_amd.lpt_timeline --config 3
"""
from __future__ import annotations

import argparse
import os
import runpy
import sys
from pathlib import Path


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, default=3)
    args = ap.parse_args()
    os.environ["GG_VERIFY_TRACE"] = "1"
    root = Path(__file__).resolve().parent.parent
    sys.argv = ["bench.py", "--config", str(args.config), "--steps", "3", "--warmup", "1", "--no-cpu-baseline"]
    runpy.run_path(str(root / "bench.py"), run_name="__main__")
    import numpy as np
    import torch

    from gollmgo_amd import verify as gv
    from gollmgo_amd._lib import lib

    t = gv.device_bytes(lib().gg_debug_trace_ptr(), 65536 * 4 * 8).view(torch.int64).cpu().numpy().reshape(-1, 4)
    t = t[((t[:, 2] >> 32) & 1) == 1]
    st, en = t[:, 0].astype(np.float64), t[:, 1].astype(np.float64)
    t0 = st.min()
    st, en = (st - t0) / 100.0, (en - t0) / 100.0
    span = en.max()
    slots = len(set((t[:, 2] & 0xFFFFFFFF).tolist()))

    def busy(x):
        return int(((st <= x) & (en > x)).sum())

    print(f"config {args.config}: {len(st)} pieces, span {span:.1f} us, {slots} CUs seen")
    print("| time (fraction of span) | busy workgroups |\n|---|---|")
    for f in (0.5, 0.6, 0.7, 0.8, 0.85, 0.9, 0.95):
        print(f"| {f * span:.1f} us ({f:.2f}) | {busy(f * span)} |")
    print("| time before the end | busy workgroups |\n|---|---|")
    for dt in (20, 15, 10, 5, 2):
        print(f"| {dt} us | {busy(span - dt)} |")
    whole = np.mean([busy(x) for x in np.linspace(0, span, 401)])
    last = np.mean([busy(x) for x in np.linspace(span - 20, span, 201)])
    print(f"mean busy workgroups: whole span {whole:.1f}, last 20 us {last:.1f}")
    q = np.percentile(en - st, [0, 25, 50, 75, 100])
    print("piece durations (us) min/25/50/75/max: " + " / ".join(f"{v:.1f}" for v in q))


if __name__ == "__main__":
    main()
