"""Benchmark of the quantized matrix-product hot path on one MI355X.

Headline (BASELINE.json metric, config 1): Q8 GEMV HBM GB/s. One step is one
pass of the GEMV over a rotation of distinct 4096x4096 int8 weight sets with
fp32 block-32 scales (more than 256 MB in total, so HBM, not the Infinity
Cache, serves the weights), all resident in HBM before timing starts. Kernels
are launched on torch's current stream and timed with HIP events on that
stream; the step sequence is replayed as a HIP graph.

Prints ONE JSON line (rank 0). `python bench.py --gpus N` with N > 1 exits:
this build targets one GPU.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rotations", type=int, default=32)
    ap.add_argument("--mode", choices=["graph", "eager"], default="graph")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def gemv_config1(args, torch, gphq):
    """Config 1: Q8 GEMV, K = N = 4096, int8 U[-127,127], fp32 block-32 scales |N(0,1)|*0.01, x ~ N(0,1)."""
    K = N = 4096
    R = args.rotations
    g = torch.Generator(device="cuda").manual_seed(0x5147)
    codes = torch.randint(-127, 128, (R, N, K), dtype=torch.int8, device="cuda", generator=g)
    scales = (torch.randn((R, N, K // 32), device="cuda", generator=g).abs() * 0.01).contiguous()
    x = torch.randn((K,), device="cuda", generator=g)
    y = torch.empty((R, N), device="cuda")
    fmt = gphq.FMT_Q8B_F32
    stream = torch.cuda.current_stream()

    def step():
        for r in range(R):
            gphq.gemv(fmt, codes[r], scales[r], x, y[r], K, N, stream=stream)

    torch.cuda.synchronize()
    runner = step
    if args.mode == "graph":
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()  # warm the capture stream
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cap_stream = torch.cuda.current_stream()
            for r in range(R):
                gphq.gemv(fmt, codes[r], scales[r], x, y[r], K, N, stream=cap_stream)
        runner = graph.replay
    for _ in range(args.warmup):
        runner()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        runner()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    launches = args.steps * R
    per_launch_s = ms / 1e3 / launches
    unit_bytes = N * K + N * (K // 32) * 4 + K * 4 + N * 4  # 18,907,136
    achieved = unit_bytes / per_launch_s / 1e9
    # Spot-check the last rotation against a float64 product on the device.
    deq = codes[R - 1].double() * scales[R - 1].double().repeat_interleave(32, dim=1)
    ref = deq @ x.double()
    rel = float(((y[R - 1].double() - ref).norm() / ref.norm()).item())
    if not rel <= 1e-5:
        raise SystemExit(f"bench: GEMV result check failed (relative L2 {rel:.3g})")
    return {
        "ms_total": ms,
        "ms_per_step": ms / args.steps,
        "launches": launches,
        "unit_bytes": unit_bytes,
        "achieved_gbs": achieved,
        "per_launch_us": per_launch_s * 1e6,
        "rel_l2": rel,
        "K": K,
        "N": N,
        "R": R,
    }


def cpu_baseline(seconds):
    """The reference's amd64 q8gemv path (scalarMulInto, single thread),
    restated in C (oracle), on the config-1 shape with per-row scales."""
    from oracle import oracle as orc

    K = N = 4096
    rng = np.random.default_rng(1)
    x = rng.standard_normal(K).astype(np.float32)
    q = rng.integers(-127, 128, N * K).astype(np.int8)
    s = (np.abs(rng.standard_normal(N)) * 0.01).astype(np.float32)
    orc.q8gemv_mul_into(x, q, s, K, N)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.q8gemv_mul_into(x, q, s, K, N)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    unit = N * K + N * 4 + K * 4 + N * 4
    return {
        "value": unit * reps / el / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{reps} x q8gemv.scalarMulInto 4096x4096 (per-row fp32 scales, the reference's amd64 path), "
        f"C restatement -O2 -ffp-contract=off, 1 thread, {el:.1f} s",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    import torch

    from gophonic_amd import gphq

    gphq.load()
    torch.cuda.set_device(0)
    r = gemv_config1(args, torch, gphq)
    total_bytes = r["unit_bytes"] * r["launches"]
    value = total_bytes / (r["ms_total"] / 1e3) / 1e9
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    out = {
        "metric": "Q8 GEMV HBM GB/s (% of peak) + Qwen3-8B Q8 decode ms/token, 1 MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 codes x fp32 activations, fp32 accumulate",
        "data": "synthetic (seeded torch generator): int8 U[-127,127], fp32 block-32 scales |N(0,1)|*0.01, x ~ N(0,1)",
        "config": {
            "workload": f"config 1: Q8 GEMV 4096x4096 with fp32 block-32 scales; one step = {r['R']} distinct "
            f"(W, scales) sets ({r['R'] * r['unit_bytes'] / 1e6:.0f} MB) through gphq_gemv, {args.mode} mode",
            "K": r["K"],
            "N": r["N"],
            "rotations": r["R"],
            "mode": args.mode,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(r["achieved_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "gemv8_kernel<Q8B_F32>",
            "per_launch_us": round(r["per_launch_us"], 3),
            "bytes_per_launch": r["unit_bytes"],
        },
        "cpu_baseline": cpu,
        "decode_ms_per_token": None,
        "check": {"rel_l2_vs_float64": r["rel_l2"]},
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
