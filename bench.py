#!/usr/bin/env python3
"""Benchmark: NN positions/sec at batch 256 for the BT4-shape net on one MI355X.

A "step" is one forward pass of the BT4-shape transformer (
d_model 1024, 15 encoder layers, 32 heads, FFN 1536 Mish, smolgen 32 -> 256 ->
32 x 256, attention policy head, WDL head) over one batch of 256 seeded
random-playout positions, with packed inputs already resident in HBM and the
outputs left in HBM (mfh_net_eval_device).  Weights are random-init (seeded,
N(0, 1/fan_in)) stored as bf16; there is no network access for real nets.

Prints one JSON line.  Besides the contract fields it carries:
  roofline      -- the dominant kernel (the bf16 MFMA GEMM): algorithmic
                   FLOPs of its launches / their summed duration, from HIP
                   events recorded on the launch stream (mfh stage profiler);
  cpu_baseline  -- the CPU oracle (a restatement of the reference CPU
                   backend) timed on a bounded sample on this host's cores;
  latency_batch1_ms -- p50 / p99 of single-position forwards;
  mfma_util_pct -- executed MFMA work of the GEMMs against the dense bf16
                   peak (twice the algorithmic work in bf16x2 precision).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 (no sparsity)
PEAK_HBM_GBS = 8000.0
METRIC = "NN positions/sec at batch 256 (BT4-shape bf16, 1 GPU)"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--precision", choices=["bf16x2", "bf16"], default="bf16x2")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--latency-iters", type=int, default=100)
    ap.add_argument("--cpu-positions", type=int, default=16,
                    help="positions in the CPU-baseline sample (0 skips it)")
    ap.add_argument("--cpu-threads", type=int, default=16)
    return ap.parse_args()


def cpu_baseline(spec, weights, planes, n, threads):
    """Times the CPU oracle on n positions with `threads` worker threads."""
    import oracle

    net = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads), weights)
    sample = planes[:n]
    t0 = time.perf_counter()
    net.evaluate_batch(sample, threads=threads)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 4), "unit": "positions/s", "cores": threads,
            "kind": "port",
            "sample": f"{n} positions of the BT4-shape net (config 2), fp32 oracle "
                      f"(restated reference CPU backend, -O3 no FMA contraction), one "
                      f"position per thread, {dt:.1f} s wall"}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the "
              "transformer evaluation shards as independent positions per GPU with no "
              "collectives, so there is no multi-GPU step to time here.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from metalfish_amd import backend, synth

    spec = synth.SPECS["bt4"]
    B = args.batch
    weights = synth.make_weights(spec, seed=args.seed)
    planes, _ = synth.playout_positions(B, seed=args.seed)
    masks, values = backend.pack_planes(planes)

    net = backend.create_network(spec, weights, max_batch=B, device=0,
                                 precision=args.precision)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    s = stream.cuda_stream
    d_masks = torch.from_numpy(masks.view(np.int64)).cuda()
    d_values = torch.from_numpy(values).cuda()
    d_policy = torch.empty((B, 1858), dtype=torch.float32, device="cuda")
    d_wdl = torch.empty((B, 3), dtype=torch.float32, device="cuda")
    ptrs = (d_masks.data_ptr(), d_values.data_ptr(), d_policy.data_ptr(), d_wdl.data_ptr())

    def step(b=B):
        net.eval_device(b, *ptrs, stream=s)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly `steps` forwards, synchronised on both sides.
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value = B / (ms_per_step * 1e-3)

    # Per-kernel breakdown: the same steps again with the stage profiler's
    # HIP events on the launch stream.
    net.profile_reset()
    net.set_profiling(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    prof = net.profile()
    net.set_profiling(False)
    gemm = prof.get("gemm_bf16", {"ms": 0.0, "flops": 0.0, "launches": 0, "bytes": 0.0})
    gemm_ms = gemm["ms"]
    achieved = gemm["flops"] / (gemm_ms * 1e-3) / 1e12 if gemm_ms else 0.0
    mfma_mult = 2.0 if args.precision == "bf16x2" else 1.0
    total_prof_ms = sum(v["ms"] for v in prof.values())
    breakdown = {k: {"ms_per_step": round(v["ms"] / args.steps, 4),
                     "launches_per_step": v["launches"] // args.steps,
                     "share": round(v["ms"] / total_prof_ms, 4) if total_prof_ms else 0.0}
                 for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}

    # Batch-1 latency (MCTS single-leaf regime).
    for _ in range(5):
        step(1)
    torch.cuda.synchronize()
    lat = []
    for _ in range(args.latency_iters):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        step(1)
        b.record(stream)
        b.synchronize()
        lat.append(a.elapsed_time(b))
    lat = np.array(lat)

    cpu = None
    if args.cpu_positions > 0:
        cpu = cpu_baseline(spec, weights, planes, args.cpu_positions, args.cpu_threads)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded random-init BT4-shape weights (bf16), seeded random-playout "
                "positions encoded as 112x8x8 planes with 8-ply history",
        "config": {
            "workload": "BT4-shape transformer forward (config 2): E=1024, 15 layers, 32 heads "
                        "(depth 32), FFN 1536 Mish, smolgen 32->256->32x256 swish, attention "
                        "policy (1858), WDL value; batch 256, inputs resident in HBM",
            "batch": B,
            "precision": args.precision,
            "weights": "bf16",
            "algorithmic_gflop_per_position": 16.33,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_bf16 (GemmKernel, all dense layers)",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": None,
            "launches_per_step": gemm["launches"] // args.steps,
            "avg_launch_us": round(gemm_ms * 1e3 / max(1, gemm["launches"]), 3),
        },
        "mfma_util_pct": round(100.0 * achieved * mfma_mult / PEAK_BF16_TFLOPS, 2),
        "whole_forward_tflops": round(16.33e9 * value / 1e12, 2),
        "latency_batch1_ms": {"p50": round(float(np.percentile(lat, 50)), 4),
                              "p99": round(float(np.percentile(lat, 99)), 4)},
        "kernel_breakdown": breakdown,
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
        "device": net.capabilities()["arch"],
    }
    net.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
