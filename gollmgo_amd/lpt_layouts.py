"""Attention call time over seeded layouts of a configuration's context distribution
(diagnostics).

The LPT schedule's piece factors are tuned constants whose effect moves in steps as items
cross piece boundaries, so they are judged on several layouts of the same distribution,
not on the bench layout alone. For each seed this builds the config's layout (one layer,
contexts drawn from the config's distribution with that seed), fills the pool with seeded
random K/V, plans the schedule once and times 30 planned calls with the draft-KV append
inside (gg_verify_append_attention_planned), as the bench step makes them. Run on the GPU:
    python -m gollmgo_amd.lpt_layouts --config 3 --seeds 1,2,3,4,5,6,7,8
"""
from __future__ import annotations

import argparse
import math


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, default=3, choices=[2, 3, 5])  # the bf16-query LPT configs
    ap.add_argument("--seeds", default="1,2,3,4,5,6,7,8")
    ap.add_argument("--calls", type=int, default=30)
    args = ap.parse_args()
    import torch

    from gollmgo_amd import verify as gv
    from gollmgo_amd._lib import DType
    from gollmgo_amd.workloads import CONFIGS, build_layout, scaled

    dev = "cuda"
    seeds = [int(x) for x in args.seeds.split(",")]
    res = []
    for seed in seeds:
        cfg = scaled(CONFIGS[args.config], layers=1, seed=seed)
        B, R, Hq, H, D, bs = cfg.num_seqs, cfg.rows, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
        kv_dt = {"bf16": DType.BF16, "f16": DType.F16, "fp8": DType.FP8_E4M3, "int8": DType.INT8}[cfg.kv_dtype]
        lay = build_layout(cfg)
        kv = gv.KVCache(1, lay.num_blocks, bs, H, D, kv_dt)
        if cfg.kv_dtype == "fp8":
            kv.set_head_scales(0, [4.5 / 448] * H, [4.5 / 448] * H)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        fs = torch.from_numpy(lay.fill_slots).to(dev)
        for s in range(0, len(fs), 1 << 16):
            m = min(1 << 16, len(fs) - s)
            kv.append(0, torch.randn(m, H, D, device=dev, dtype=torch.bfloat16, generator=g),
                      torch.randn(m, H, D, device=dev, dtype=torch.bfloat16, generator=g), fs[s:s + m])
        q = torch.randn(B, R, Hq, D, device=dev, dtype=torch.bfloat16, generator=g)
        out = torch.empty(B, R, Hq, D, device=dev, dtype=torch.bfloat16)
        kn = torch.randn(B * R, H, D, device=dev, dtype=torch.bfloat16, generator=g)
        vn = torch.randn(B * R, H, D, device=dev, dtype=torch.bfloat16, generator=g)
        keys = torch.from_numpy(lay.keys).to(dev)
        bt = torch.from_numpy(lay.block_tables).to(dev)
        ws = kv.attention_workspace(B, R, Hq, bt.shape[1], 0)
        kv.attention_plan(keys, R, Hq, bt.shape[1], ws)
        sc = 1 / math.sqrt(D)
        for _ in range(5):
            kv.append_attention(0, kn, vn, q, out, keys, bt, sc, ws)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.calls):
            kv.append_attention(0, kn, vn, q, out, keys, bt, sc, ws)
        e1.record()
        torch.cuda.synchronize()
        res.append(e0.elapsed_time(e1) * 1000 / args.calls)
        kv.close()
        print(f"config {args.config} seed {seed}: {res[-1]:.1f} us per call", flush=True)
    print(f"config {args.config}: mean {sum(res) / len(res):.2f} us over seeds {args.seeds}", flush=True)


if __name__ == "__main__":
    main()
