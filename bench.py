#!/usr/bin/env python3
"""Spec-verify benchmark of the gfx950 verify path (one GPU).

One step = one verify pass of a batch: the n-gram draft lookup (configs with a token
history), the attention schedule of the step, then for each of L layers the draft-KV
append of the B*(k+1) verify rows followed by multi-query paged attention over the whole
context; then one acceptance over the full-vocabulary logits. Inputs are synthetic, seeded,
and resident in HBM before the timed region starts.

value = verified tokens/s = B*(k+1) / (L*(t_append + t_attn) + t_accept), taken from
the wall clock of the timed steps (the same formula the measurement plan uses).
The roofline object describes the attention call (the dominant kernel); its
duration is the HIP-event average over every attention call in the timed region, and
its traffic comes from the committed rocprofv3 PMC summary of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, help="workload config id (default 3 = 8B fp8)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seqs", type=int, default=32, help="sequences in the CPU baseline sample")
    ap.add_argument("--partition", type=int, default=-1, help="override split-K partition tokens")
    ap.add_argument("--layers", type=int, default=0, help="override layer count (0 = config)")
    ap.add_argument("--separate-append", action="store_true",
                    help="append the draft KV with gg_kv_append before gg_verify_attention_planned instead of "
                         "inside the attention call (gg_verify_append_attention_planned, the default where "
                         "the pool allows it)")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches for `value` instead of replays of the captured step graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of known size (for PMC byte calibration)")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch

    import gollmgo_amd.verify as gv
    from gollmgo_amd._lib import DType
    from gollmgo_amd.workloads import CONFIGS, build_layout, scaled

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.set_device(0)
    dev = "cuda"

    if args.copy_calibration:
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n}))
        return

    cfg = CONFIGS[args.config]
    if args.layers:
        cfg = scaled(cfg, layers=args.layers)
    # The library's automatic schedule unless --partition asks for a fixed split-K
    # partition. (Config 4 names 512-token partitions, the reference kernel's setting;
    # the schedule changes only the fp32 summation order, which the parity tests cover
    # at 512-token partitions too.)
    cfg = scaled(cfg, partition=max(args.partition, 0))
    B, R, K = cfg.num_seqs, cfg.rows, cfg.max_drafts
    Hq, H, D, bs, V, L = cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size, cfg.vocab, cfg.layers
    kv_dt = {"bf16": DType.BF16, "f16": DType.F16, "fp8": DType.FP8_E4M3, "int8": DType.INT8, "f32": DType.F32}[cfg.kv_dtype]
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}

    t_setup = time.time()
    lay = build_layout(cfg)
    kv = gv.KVCache(L, lay.num_blocks, bs, H, D, kv_dt)
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg.seed)
    fill_slots = torch.from_numpy(lay.fill_slots).to(dev)
    append_slots = torch.from_numpy(lay.append_slots).to(dev)
    n_fill = len(lay.fill_slots)
    chunk = 1 << 16
    for layer in range(L):
        if cfg.kv_dtype == "fp8":
            # Per-head amax/448 scales over this layer's context (the reference's fp8 convention).
            kmax = torch.zeros(H, device=dev)
            vmax = torch.zeros(H, device=dev)
            for s in range(0, n_fill, chunk):
                m = min(chunk, n_fill - s)
                torch.manual_seed(cfg.seed * 1000 + layer * 100 + s // chunk)
                kx = torch.randn(m, H, D, device=dev, dtype=torch.bfloat16)
                vx = torch.randn(m, H, D, device=dev, dtype=torch.bfloat16)
                kmax = torch.maximum(kmax, kx.float().abs().amax(dim=(0, 2)))
                vmax = torch.maximum(vmax, vx.float().abs().amax(dim=(0, 2)))
            kv.set_head_scales(layer, (kmax / 448).clamp_min(1e-8).tolist(), (vmax / 448).clamp_min(1e-8).tolist())
        for s in range(0, n_fill, chunk):
            m = min(chunk, n_fill - s)
            torch.manual_seed(cfg.seed * 1000 + layer * 100 + s // chunk)
            kx = torch.randn(m, H, D, device=dev, dtype=torch.bfloat16)
            vx = torch.randn(m, H, D, device=dev, dtype=torch.bfloat16)
            kv.append(layer, kx, vx, fill_slots[s:s + m])
    torch.cuda.synchronize()

    q = torch.randn(L, B, R, Hq, D, device=dev, dtype=tdt[cfg.q_dtype], generator=gen)
    out = torch.empty(B, R, Hq, D, device=dev, dtype=torch.bfloat16)
    k_new = torch.randn(L, B * R, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
    v_new = torch.randn(L, B * R, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
    keys = torch.from_numpy(lay.keys).to(dev)
    bt = torch.from_numpy(lay.block_tables).to(dev)
    ws_attn = kv.attention_workspace(B, R, Hq, bt.shape[1], cfg.partition)

    # Acceptance inputs: target logits, draft distributions (a sharpened copy of the
    # target row) and drafts that mostly follow the draft distribution's mode.
    logits = (torch.randn(B, R, V, device=dev, generator=gen) * 2.0).to(tdt[cfg.logits_dtype])
    draft_probs = torch.softmax(logits[:, :K].float() * 1.5, dim=-1).contiguous() if cfg.draft_probs else None
    drafts = torch.randint(0, V, (B, K), device=dev, dtype=torch.int32, generator=gen)
    base = draft_probs if draft_probs is not None else logits[:, :K].float()
    mode = base.argmax(dim=-1).to(torch.int32)
    pick = torch.rand(B, K, device=dev, generator=gen) < 0.8
    drafts = torch.where(pick, mode, drafts).contiguous()
    n_drafts = torch.full((B,), K, device=dev, dtype=torch.int32)
    uniforms = torch.rand(B, R, device=dev, generator=gen)
    acc_out = (torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev))
    # n-gram draft lookup over each sequence's token history (configs that define one); its
    # drafts are timed as part of the step, the acceptance below keeps its own synthetic drafts.
    hist = None
    if cfg.history_len:
        from gollmgo_amd.workloads import make_histories
        hist_np = make_histories(cfg, cfg.history_len)
        hist = torch.from_numpy(hist_np).to(dev)
        hist_len = torch.full((B,), cfg.history_len, device=dev, dtype=torch.int32)
        draft_out = (torch.zeros(B, K, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev))
    if cfg.accept == "rejection":
        ws_acc = gv.rejection_workspace(B, K, V)
    else:
        ws_acc = gv.greedy_workspace(B, K, V)
    torch.cuda.synchronize()
    setup_s = time.time() - t_setup

    scale = 1.0 / math.sqrt(D)
    ev = {name: [] for name in ("append", "attn", "accept", "plan", "draft")}

    # The attention schedule depends only on the context lengths, shared by all layers of
    # a step: computed once per step (gg_verify_attention_plan), used by every layer.
    use_plan = cfg.partition == 0
    # The draft rows' KV append goes through the attention entry point
    # (gg_verify_append_attention_planned; PER_BLOCK INT8 pools included).
    fused = use_plan and not args.separate_append

    def step(record: bool):
        if hist is not None:
            if record:
                d0, d1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                d0.record()
            gv.ngram_draft(hist, hist_len, cfg.ngram_n, K, out=draft_out)
            if record:
                d1.record()
                ev["draft"].append((d0, d1))
        if use_plan:
            if record:
                p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                p0.record()
            kv.attention_plan(keys, R, Hq, bt.shape[1], ws_attn)
            if record:
                p1.record()
                ev["plan"].append((p0, p1))
        for layer in range(L):
            if record:
                e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
                if not fused:
                    e0.record()
            if not fused:
                kv.append(layer, k_new[layer], v_new[layer], append_slots)
            if record:
                e1.record()
            if fused:
                kv.append_attention(layer, k_new[layer], v_new[layer], q[layer], out, keys, bt, scale, ws_attn)
            else:
                kv.attention(layer, q[layer], out, keys, bt, scale, partition_tokens=cfg.partition,
                             workspace=ws_attn, planned=use_plan)
            if record:
                e2.record()
                if not fused:  # (fused: the append is inside the attention call)
                    ev["append"].append((e0, e1))
                ev["attn"].append((e1, e2))
        if record:
            a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a0.record()
        if cfg.accept == "rejection":
            gv.accept_rejection(logits, drafts, n_drafts, uniforms, cfg.temperature, cfg.top_p,
                                draft_probs=draft_probs, workspace=ws_acc, out=acc_out)
        else:
            gv.accept_greedy(logits, drafts, n_drafts, workspace=ws_acc, out=acc_out)
        if record:
            a1.record()
            ev["accept"].append((a0, a1))

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    # Per-kernel durations: eager steps with HIP events (on the stream the library launches
    # on, torch's current stream) around every call.
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    wall_eager = time.perf_counter() - t0
    eager_out = (acc_out[0].clone(), acc_out[1].clone(), out.clone())
    wall = wall_eager
    graph_ok = None
    if not args.eager:
        # `value`: the same step (draft lookup, plan, every layer's append and attention,
        # acceptance) captured once as a HIP graph and replayed, so the launch gaps between
        # the ~2L+4 kernels go away. The entry points allocate nothing and record no memset,
        # so the graph holds only their kernels; every replay recomputes everything.
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cs):
            step(False)
        torch.cuda.current_stream().wait_stream(cs)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(False)
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        graph_ok = bool(torch.equal(acc_out[0], eager_out[0]) and torch.equal(acc_out[1], eager_out[1])
                        and torch.equal(out, eager_out[2]))

    def avg_us(name):
        xs = [s.elapsed_time(e) * 1000.0 for s, e in ev[name]]
        if not xs:
            return 0.0, 0.0
        xs.sort()
        return sum(xs) / len(xs), xs[len(xs) // 2]

    t_app, t_app_med = avg_us("append")
    t_attn, t_attn_med = avg_us("attn")
    t_acc, t_acc_med = avg_us("accept")
    t_plan, _ = avg_us("plan")
    t_draft, _ = avg_us("draft")
    ms_per_step = wall * 1000.0 / args.steps
    ms_per_step_eager = wall_eager * 1000.0 / args.steps
    tokens = B * R
    value = tokens / (ms_per_step / 1000.0)
    kernel_formula_tps = tokens / ((L * (t_app + t_attn) + t_acc + t_plan + t_draft) * 1e-6)
    accepted = acc_out[0].cpu()
    accepted_tps = float((accepted + 1).sum()) / (ms_per_step / 1000.0)

    # Algorithmic bytes of one attention call (one layer): K+V once per sequence, Q in, out, scales, tables.
    eb = {"bf16": 2, "f16": 2, "fp8": 1, "int8": 1, "f32": 4}[cfg.kv_dtype]
    keys_np = lay.keys.astype(np.int64)
    kv_bytes = int(keys_np.sum()) * H * D * eb * 2
    q_bytes = B * R * Hq * D * q.element_size()
    o_bytes = B * R * Hq * D * out.element_size()
    blocks_used = int(((keys_np + bs - 1) // bs).sum())
    scale_bytes = H * 4 * 2 if cfg.kv_dtype == "fp8" else (blocks_used * H * 2 * 2 if cfg.kv_dtype == "int8" else 0)
    attn_bytes = kv_bytes + q_bytes + o_bytes + scale_bytes + blocks_used * 4
    if fused:  # the draft rows' K/V read (bf16) and written to the pool by the same call
        attn_bytes += B * R * H * D * 2 * (k_new.element_size() + eb)
    achieved = attn_bytes / (t_attn * 1e-6) / 1e9
    # The same with every pool block counted once: sequences that share prefix blocks read
    # them once each in the algorithmic count, but HBM serves a shared block once when its
    # readers meet in cache. A block counts with the most tokens any reader uses of it.
    used = {}
    for i in range(B):
        n_tok = int(keys_np[i])
        for blk in range((n_tok + bs - 1) // bs):
            pid = int(lay.block_tables[i, blk])
            used[pid] = max(used.get(pid, 0), min(bs, n_tok - blk * bs))
    unique_bytes = attn_bytes - kv_bytes + sum(used.values()) * H * D * eb * 2
    achieved_unique = unique_bytes / (t_attn * 1e-6) / 1e9
    # One gg_verify_attention call: a single-piece plan (no workspace) is one launch of the
    # MFMA kernel; otherwise stream-K (or an explicit partition grid) plus its merge.
    from gollmgo_amd._lib import lib as _gglib
    ws_need = _gglib().gg_verify_attention_workspace_size(kv.handle, B, R, Hq, bt.shape[1], cfg.partition)
    if ws_need == 0:
        attn_kernels = "attn_mfma_kernel (one workgroup per sequence x kv head)"
    elif cfg.partition:
        attn_kernels = "attn_mfma_kernel + attn_combine_kernel (partition grid)"
    elif fused:
        attn_kernels = ("gg_verify_append_attention_planned: the library's automatic schedule (LPT pieces or "
                        "stream-K), each piece appending its draft rows, + merge")
    else:
        attn_kernels = "gg_verify_attention_planned: the library's automatic schedule (LPT pieces or stream-K) + merge"
    traffic, traffic_src = pmc_traffic(args.config)
    lb = logits.element_size()
    acc_bytes = B * R * V * lb + (B * K * V * 4 if draft_probs is not None else 0)

    result = {
        "metric": "spec-verify tokens/s at Llama-3.1-8B shape, FP8 KV; achieved HBM GB/s",
        "value": round(value, 1),
        "unit": "verified tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp8": "fp8-e4m3 KV, f16 MFMA, fp32 softmax", "bf16": "bf16", "int8": "int8 KV, f16 MFMA",
                  "f16": "f16", "f32": "f32"}[cfg.kv_dtype],
        "data": "synthetic (seeded N(0,1) K/V/Q, N(0,2) logits), random-permuted paged pool",
        "config": {
            "workload": f"config {args.config}: {cfg.name} verify step",
            "batch": B, "draft_k": K, "rows_per_seq": R, "q_heads": Hq, "kv_heads": H, "head_dim": D,
            "block_size": bs, "ctx": list(cfg.ctx), "mean_keys": float(keys_np.mean()), "kv_dtype": cfg.kv_dtype,
            "layers": L, "vocab": V, "accept": cfg.accept, "temperature": cfg.temperature, "top_p": cfg.top_p,
            "draft_probs": cfg.draft_probs, "partition_tokens": cfg.partition or "auto",
            "shared_prefix_frac": cfg.shared_prefix_frac,
            "draft_kv_append": "gg_verify_append_attention_planned" if fused else "gg_kv_append",
        },
        "kernels_us": {"append_avg": round(t_app, 2), "attention_avg": round(t_attn, 2),
                       "attention_median": round(t_attn_med, 2), "accept_avg": round(t_acc, 2),
                       "attention_plan_per_step": round(t_plan, 2), "ngram_draft_per_step": round(t_draft, 2)},
        "timing": "graph replay of the whole step" if graph_ok is not None else "eager launches",
        "graph_matches_eager": graph_ok,
        "ms_per_step_eager": round(ms_per_step_eager, 4),
        "tokens_per_s_from_kernel_times": round(kernel_formula_tps, 1),
        "accepted_tokens_per_s": round(accepted_tps, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": attn_kernels, "algorithmic_bytes_per_launch": attn_bytes,
                     "traffic_source": traffic_src, "unique_block_bytes_per_launch": unique_bytes,
                     "achieved_unique_block_bytes": round(achieved_unique, 1),
                     "frac_unique_block_bytes": round(achieved_unique / HBM_PEAK_GBS, 4)},
        "accept_roofline": {"achieved": round(acc_bytes / (t_acc * 1e-6) / 1e9, 1), "unit": "GB/s",
                            "algorithmic_bytes_per_launch": acc_bytes},
        "setup_s": round(setup_s, 1),
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, cfg, lay, kv, q, logits, draft_probs, drafts, n_drafts,
                                              uniforms, scale, acc_out)
    kv.close()
    print(json.dumps(result))


def pmc_traffic(config_id: int):
    """HBM bytes per attention launch from the committed rocprofv3 PMC summary of this
    workload (FETCH_SIZE and WRITE_SIZE per dispatch, scaled by the copy-kernel
    calibration recorded there), or None when no summary exists for it."""
    import re
    path = ROOT / "profiles" / f"attention_config{config_id}_pmc.md"
    if not path.exists():
        return None, None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", path.read_text(), re.M)
    if not m:
        return None, None
    return int(m.group(1)), str(path.relative_to(ROOT))


def cpu_baseline(args, cfg, lay, kv, q, logits, draft_probs, drafts, n_drafts, uniforms, scale, decision):
    """A C port of the reference's host logic and of its attention (the v1 kernel's loop,
    kernels/gollmgo_paged_attn.cu:38-119, at its fp32 precision: ora_attention_ref_f32, not
    the fp64 checker) timed on this host on bounded samples of the same workload, at every
    usable core and at one thread. A sample is the attention of layer 0 for the first S sequences,
    scaled by L layers, plus the acceptance of the same S sequences (and their n-gram
    drafts when the config has token histories). `value` is the all-cores figure; the
    one-thread figure uses a smaller sample of the same shape. The Go engine's own host
    loops (NGramDrafter.Draft and Verify, internal/engine/speculative.go:24-84) are also
    timed at one thread per sequence, and so is the return path of the device decision:
    the one-hot LogitsPerPosition rows built from the step's (accepted, token) and the
    engine's Verify + bonus Sample over them (serving.go:496-570), for the whole batch."""
    import numpy as np

    from oracle import oracle as ora

    nproc = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = nproc
    kc = kv.k_pool(0).cpu().numpy()
    vc = kv.v_pool(0).cpu().numpy()
    ks = vs = None
    if cfg.kv_dtype == "fp8":
        k_s, v_s = kv.scales(0)
        ks, vs = k_s.cpu().numpy()[:cfg.num_kv_heads], v_s.cpu().numpy()[:cfg.num_kv_heads]
    elif cfg.kv_dtype == "int8":
        k_s, v_s = kv.scales(0)
        ks, vs = k_s.float().cpu().numpy().reshape(-1), v_s.float().cpu().numpy().reshape(-1)
    hist = None
    if cfg.history_len:
        from gollmgo_amd.workloads import make_histories
        hist = make_histories(cfg, cfg.history_len)

    def sample(S, threads):
        qh = q[0, :S].float().cpu().numpy()
        t0 = time.perf_counter()
        ora.attention_ref_f32(qh, kc, vc, cfg.kv_dtype, cfg.num_kv_heads, cfg.head_dim, cfg.block_size,
                              lay.keys[:S], lay.block_tables[:S], scale, ks, vs, threads=threads)
        t_attn = time.perf_counter() - t0
        t_dr = 0.0
        if hist is not None:
            t0 = time.perf_counter()
            ora.ngram_draft_batch(hist[:S], np.full(S, hist.shape[1], np.int32), cfg.ngram_n, cfg.max_drafts,
                                  threads=threads)
            t_dr = time.perf_counter() - t0
        lg = logits[:S].float().cpu().numpy()
        dp = draft_probs[:S].cpu().numpy() if draft_probs is not None else None
        dr, nd, un = drafts[:S].cpu().numpy(), n_drafts[:S].cpu().numpy(), uniforms[:S].cpu().numpy()
        t0 = time.perf_counter()
        if cfg.accept == "rejection":
            ora.accept_rejection(lg, dr, nd, un, cfg.temperature, cfg.top_p, dp)
        else:
            ora.accept_greedy(lg, dr, nd)
        t_acc = time.perf_counter() - t0
        step_s = cfg.layers * t_attn + t_acc + t_dr
        desc = (f"{S} of {cfg.num_seqs} sequences: layer-0 attention ({t_attn:.2f} s, the reference's v1 loop in fp32, {threads} thread(s)) "
                f"x {cfg.layers} layers + {cfg.accept} acceptance ({t_acc:.2f} s, 1 thread)"
                + (f" + n-gram drafts ({t_dr:.3f} s)" if hist is not None else ""))
        return {"value": round(S * cfg.rows / step_s, 2), "threads": threads, "sample": desc,
                "attention_s_per_layer": round(t_attn, 3), "accept_s": round(t_acc, 3)}

    S = min(args.cpu_seqs, cfg.num_seqs)
    all_cores = sample(S, usable)
    one_thread = sample(max(1, S // 16), 1)

    # The Go engine's host loops, one thread: Draft over a history of the config's (or, for
    # configs without one, config 5's 8192-token) shape, Verify over one sequence's K draft
    # rows of the config's logits (greedy argmax scan, the engine's own check).
    if hist is None:
        from gollmgo_amd.workloads import CONFIGS, make_histories
        dh = make_histories(CONFIGS[5], CONFIGS[5].history_len)[:16]
    else:
        dh = hist[:16]
    t0 = time.perf_counter()
    ora.ngram_draft_batch(dh, np.full(len(dh), dh.shape[1], np.int32), 3, cfg.max_drafts, threads=1)
    draft_us = (time.perf_counter() - t0) / len(dh) * 1e6
    nv = min(16, cfg.num_seqs)
    lg = logits[:nv].float().cpu().numpy()
    t0 = time.perf_counter()
    ora.accept_greedy(lg, drafts[:nv].cpu().numpy(), n_drafts[:nv].cpu().numpy())
    verify_us = (time.perf_counter() - t0) / nv * 1e6
    # Return path: rows from the device decision of the bench step, then the engine's reads.
    from gollmgo_amd.positions import LogitsPerPosition
    dr_h, nd_h = drafts.cpu().numpy(), n_drafts.cpu().numpy()
    acc_h, tok_h = decision[0].cpu().numpy(), decision[1].cpu().numpy()
    lpp = LogitsPerPosition(int(logits.shape[-1]))
    t0 = time.perf_counter()
    pos = lpp.batch(dr_h, nd_h, acc_h, tok_h)
    build_us = (time.perf_counter() - t0) * 1e6
    T = cfg.temperature if cfg.accept == "rejection" else 0.0
    ub = np.random.default_rng(0).random(len(pos))
    tm = []
    ea, et = ora.emit_positions(dr_h, nd_h, pos, T, cfg.top_p, ub, timer=tm)
    emit_us = tm[0] * 1e6
    return_ok = bool(np.array_equal(ea, acc_h) and np.array_equal(et, tok_h))
    row_floats = int(sum(len(r) for rows in pos for r in rows))
    return {"value": all_cores["value"], "unit": "verified tokens/s", "cores": usable, "kind": "port",
            "sample": all_cores["sample"], "nproc": nproc, "usable_cpus": usable,
            "all_cores": all_cores, "one_thread": one_thread,
            "go_engine_loops_one_thread": {
                "ngram_draft_us_per_seq": round(draft_us, 1),
                "ngram_history_tokens": int(dh.shape[1]),
                "verify_greedy_us_per_seq": round(verify_us, 1),
                "verify_rows_x_vocab": [cfg.rows, int(logits.shape[-1])]},
            "return_path_one_thread": {
                "rows_build_us_per_step": round(build_us, 1),
                "engine_verify_sample_us_per_step": round(emit_us, 1),
                "row_floats_scanned": row_floats,
                "sampler": f"T={T} top_p={cfg.top_p}",
                "reproduces_device_decision": return_ok}}


if __name__ == "__main__":
    main()
