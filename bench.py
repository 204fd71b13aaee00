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
    ap.add_argument("--warmup", type=int, default=300,
                    help="untimed config-1 steps first; the GPU's clocks take about 20 ms of sustained load "
                    "(about 200 batch launches) to settle, and shorter warmups time the ramp")
    ap.add_argument("--rotations", type=int, default=32)
    ap.add_argument("--mode", choices=["batch", "graph", "eager"], default="batch")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="bound of the config-1 CPU baseline sample (each other CPU line takes half)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true", help="skip the config-2 int8 GEMM lines")
    ap.add_argument("--no-gptq", action="store_true", help="skip the config-5 GPTQ int4 lines")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-3/4b decode lines")
    ap.add_argument("--decode-fmt", choices=["q8b", "q8b_f32", "q8", "q4"], default="q8b",
                    help="layer weight format of the decode models (the reference's decode batch uses Q8B)")
    ap.add_argument("--decode-eager", action="store_true", help="launch decode steps without the HIP graph")
    ap.add_argument("--decode-configs", default="3,4a,4a8,4b1,4b16",
                    help="model lines to run: 3 (Qwen3-0.6B decode), 4a (Qwen3-8B 4096-token prefill), "
                    "4a8 (4a on the int8 route, Q8 layers), 4b1 / 4b16 (Qwen3-8B decode, 1 / 16 lanes)")
    return ap.parse_args()


def gemv_config1(args, torch, gphq, mode):
    """Config 1: Q8 GEMV, K = N = 4096, int8 U[-127,127], fp32 block-32 scales |N(0,1)|*0.01, x ~ N(0,1).

    mode "batch": one gphq_gemv_batch launch per step covering all rotations;
    "graph": one gphq_gemv launch per rotation, the step replayed as a HIP graph;
    "eager": the same launches issued from the host each step.
    """
    K = N = 4096
    R = args.rotations
    g = torch.Generator(device="cuda").manual_seed(0x5147)
    codes = torch.randint(-127, 128, (R, N, K), dtype=torch.int8, device="cuda", generator=g)
    scales = (torch.randn((R, N, K // 32), device="cuda", generator=g).abs() * 0.01).contiguous()
    x = torch.randn((K,), device="cuda", generator=g)
    y = torch.empty((R, N), device="cuda")
    fmt = gphq.FMT_Q8B_F32
    stream = torch.cuda.current_stream()
    cl, sl, xl, yl = [codes[r] for r in range(R)], [scales[r] for r in range(R)], [x] * R, [y[r] for r in range(R)]

    def launch_all(st):
        if mode == "batch":
            for i in range(0, R, gphq.GEMV_MAX_BATCH):
                j = min(R, i + gphq.GEMV_MAX_BATCH)
                gphq.gemv_batch(fmt, cl[i:j], sl[i:j], xl[i:j], yl[i:j], K, N, stream=st)
        else:
            for r in range(R):
                gphq.gemv(fmt, cl[r], sl[r], x, yl[r], K, N, stream=st)

    torch.cuda.synchronize()
    runner = lambda: launch_all(stream)  # noqa: E731
    if mode == "graph":
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            launch_all(s)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            launch_all(torch.cuda.current_stream())
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
    per_launch = (R + gphq.GEMV_MAX_BATCH - 1) // gphq.GEMV_MAX_BATCH if mode == "batch" else R
    launches = args.steps * per_launch
    gemvs_per_launch = R / per_launch
    unit_bytes = N * K + N * (K // 32) * 4 + K * 4 + N * 4  # 18,907,136 per GEMV
    launch_s = ms / 1e3 / launches
    # Every rotation's output against a float64 product on the device.
    rel = 0.0
    for r in range(R):
        deq = codes[r].double() * scales[r].double().repeat_interleave(32, dim=1)
        ref = deq @ x.double()
        rel = max(rel, float(((y[r].double() - ref).norm() / ref.norm()).item()))
        del deq, ref
    if not rel <= 1e-5:
        raise SystemExit(f"bench: GEMV result check failed (relative L2 {rel:.3g})")
    return {
        "mode": mode,
        "ms_total": ms,
        "ms_per_step": ms / args.steps,
        "launches": launches,
        "unit_bytes": unit_bytes,
        "bytes_per_launch": int(unit_bytes * gemvs_per_launch),
        "gemvs_per_launch": gemvs_per_launch,
        "per_launch_us": launch_s * 1e6,
        "per_gemv_us": launch_s / gemvs_per_launch * 1e6,
        "value_gbs": unit_bytes * R * args.steps / (ms / 1e3) / 1e9,
        "achieved_gbs": unit_bytes * gemvs_per_launch / launch_s / 1e9,
        "rel_l2": rel,
        "K": K,
        "N": N,
        "R": R,
    }


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, AMD published (POP/s)
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, AMD published


def gemm_config2(args, torch, gphq, ms=(1, 16, 128, 512), rotations=6, steps=20):
    """Config 2 (reference semantics): x fp32 [M, 4096] quantized per row (WorkspaceI8),
    int8 weights [12288, 4096] with fp32 per-row scales, exact int32 GEMM
    (MulPanelsI8). Times the GEMM launch over `rotations` distinct weight sets
    (> 256 MB) and, separately, the activation quantizer."""
    K, N = 4096, 12288
    rng = np.random.default_rng(2)
    ws_list = []
    for r in range(rotations):
        w = gphq.WeightsI8(K, N)
        w.pack(rng.integers(-127, 128, N * K, dtype=np.int8), (np.abs(rng.standard_normal(N)) * 0.01).astype(np.float32))
        ws_list.append(w)
    stream = torch.cuda.current_stream()
    out = {}
    for m in ms:
        x = torch.randn((m, K), device="cuda")
        ws = gphq.WorkspaceI8(K, m)
        ws.pack(x, m, K, stream=stream)
        dst = torch.empty((m, N), device="cuda")
        for w in ws_list:
            gphq.mul_panels_i8(dst, N, ws, w, 0, w.panels(), stream=stream)
        torch.cuda.synchronize()
        # Replay captured launches so host launch cost does not enter the timing.
        g_gemm, g_quant = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_gemm):
            cs = torch.cuda.current_stream()
            for w in ws_list:
                gphq.mul_panels_i8(dst, N, ws, w, 0, w.panels(), stream=cs)
        with torch.cuda.graph(g_quant):
            cs = torch.cuda.current_stream()
            for _ in range(rotations):
                ws.pack(x, m, K, stream=cs)
        g_gemm.replay()
        g_quant.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            g_gemm.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (steps * rotations)
        e0.record(stream)
        for _ in range(steps):
            g_quant.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        q_us = e0.elapsed_time(e1) * 1e3 / (steps * rotations)
        gemm_bytes = N * K + 4 * N + m * K + 4 * m + 4 * m * N
        ops = 2.0 * m * N * K
        out[f"M{m}"] = {
            "gemm_us": round(us, 3),
            "gemm_gbs": round(gemm_bytes / us / 1e3, 1),
            "hbm_frac": round(gemm_bytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "tops": round(ops / us / 1e6, 1),
            "int8_frac": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4),
            "quantize_us": round(q_us, 3),
        }
        del ws
    for w in ws_list:
        w.close()
    return out


def gemm_config2_block32(args, torch, gphq, ms=(1, 16, 128, 512), steps=20):
    """Config 2 with BASELINE's per-32-block weight scales: int8 codes [12288, 4096]
    U[-127,127] with one fp32 scale per 32-value block |N(0,1)|*0.01 (GPHQ_FMT_Q8B_F32),
    x fp32 [M, 4096] N(0,1). The reference has no block-scaled int8 x int8 GEMM (its
    q8gemm int8 path scales per row, gemm_config2); block-scaled weights go through
    qwen3lm's kernels as the reference runs them: one row through the GEMV
    (gphq_gemv, fp32), up to 16 rows through the multi-vector GEMV (gphq_gemv_vec, as
    decode lanes), more through mm (gphq_mm: FP16 tiles, fp32 sums). Rotates > 256 MB
    of weights."""
    K, N = 4096, 12288
    per = N * K + N * (K // 32) * 4
    rotations = (300 << 20) // per + 1
    g = torch.Generator(device="cuda")
    g.manual_seed(22)
    sets = []
    for _ in range(rotations):
        codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
        scales = torch.randn((N, K // 32), device="cuda", generator=g).abs() * 0.01
        sets.append((codes, scales))
    stream = torch.cuda.current_stream()
    out = {}
    for m in ms:
        x = torch.randn((m, K), device="cuda", generator=g)
        y = torch.empty((m, N), device="cuda")
        if m == 1:
            path = "gphq_gemv"
            run = lambda c, sc, st: gphq.gemv(gphq.FMT_Q8B_F32, c, sc, x, y, K, N, stream=st)
        elif m <= 16:
            path = "gphq_gemv_vec"
            work = torch.empty(gphq.gemv_vec_workspace_bytes(m, K), dtype=torch.uint8, device="cuda")
            run = lambda c, sc, st: gphq.gemv_vec(gphq.FMT_Q8B_F32, c, sc, x, y, m, K, N, work, stream=st)
        else:
            path = "gphq_mm"
            work = torch.empty(gphq.mm_split_workspace_bytes(m, K, N), dtype=torch.uint8, device="cuda")
            run = lambda c, sc, st: gphq.mm(gphq.FMT_Q8B_F32, c, sc, x, y, m, K, N, work, stream=st)
        for c, sc in sets:
            run(c, sc, stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cs = torch.cuda.current_stream()
            for c, sc in sets:
                run(c, sc, cs)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (steps * rotations)
        nbytes = per + 4 * m * K + 4 * m * N
        flops = 2.0 * m * N * K
        out[f"M{m}"] = {
            "us": round(us, 3),
            "gbs": round(nbytes / us / 1e3, 1),
            "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "tflops": round(flops / us / 1e6, 2),
            "fp16_frac": round(flops / us / 1e6 / FP16_PEAK_TFLOPS, 4),
            "rotations": rotations,
            "path": path,
        }
    del sets
    torch.cuda.empty_cache()
    return out


def gemm_config2_block32_int8(args, torch, gphq, ms=(1, 16, 128, 512), steps=20):
    """Config 2 as BASELINE words it, exactly: x fp32 [M, 4096] N(0,1) quantized to
    int8 per 32-value block (WorkspaceI8's rule per block) and int8 weights [12288, 4096]
    U[-127,127] with fp32 block scales |N(0,1)|*0.01; exact int32 per block, then the
    block-ordered fp32 scale-accumulate (gphq_q8b_quantize + gphq_q8b_gemm; no
    counterpart in the reference). Rotates > 256 MB of weights; times the GEMM and,
    separately, the activation quantizer."""
    K, N = 4096, 12288
    per = N * K + N * (K // 32) * 4
    rotations = (300 << 20) // per + 1
    g = torch.Generator(device="cuda")
    g.manual_seed(23)
    sets = []
    for _ in range(rotations):
        codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
        scales = torch.randn((N, K // 32), device="cuda", generator=g).abs() * 0.01
        sets.append((codes, scales))
    stream = torch.cuda.current_stream()
    out = {}
    for m in ms:
        x = torch.randn((m, K), device="cuda", generator=g)
        q = torch.empty((m, K), dtype=torch.int8, device="cuda")
        d = torch.empty((m, K // 32), device="cuda")
        y = torch.empty((m, N), device="cuda")
        gphq.q8b_quantize(x, m, K, q, d, stream=stream)
        for c, sc in sets:
            gphq.q8b_gemm(q, d, c, sc, y, m, K, N, stream=stream)
        torch.cuda.synchronize()
        g_gemm, g_quant = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_gemm):
            cs = torch.cuda.current_stream()
            for c, sc in sets:
                gphq.q8b_gemm(q, d, c, sc, y, m, K, N, stream=cs)
        with torch.cuda.graph(g_quant):
            cs = torch.cuda.current_stream()
            for _ in range(rotations):
                gphq.q8b_quantize(x, m, K, q, d, stream=cs)
        g_gemm.replay()
        g_quant.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            g_gemm.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (steps * rotations)
        e0.record(stream)
        for _ in range(steps):
            g_quant.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        q_us = e0.elapsed_time(e1) * 1e3 / (steps * rotations)
        nbytes = per + m * K + m * (K // 32) * 4 + 4 * m * N
        ops = 2.0 * m * N * K
        out[f"M{m}"] = {
            "gemm_us": round(us, 3),
            "gemm_gbs": round(nbytes / us / 1e3, 1),
            "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "tops": round(ops / us / 1e6, 1),
            "int8_frac": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4),
            "quantize_us": round(q_us, 3),
            "rotations": rotations,
        }
    del sets
    torch.cuda.empty_cache()
    return out


def gptq_config5(args, torch, gphq, ms=(1, 256), steps=20):
    """Config 5: GPTQ int4 dequant-matmul at the Qwen3-8B shapes K=4096 -> N=12288 and
    K=12288 -> N=4096 (gphq_mm, GPHQ_FMT_GPTQ4_G128: nibbles U[0,15] 8 per int32 along K,
    fp16 group-128 scales |N(0,1)|*0.01, 4-bit zero points U[0,15]); activations fp32
    N(0,1) converted to FP16 inside the call, fp32 accumulation. Each shape rotates
    through distinct weight sets totalling > 256 MB."""
    out = {}
    stream = torch.cuda.current_stream()
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    for k, n in ((4096, 12288), (12288, 4096)):
        per = n * k // 2 + n * (k // 128) * 3
        rotations = (320 << 20) // per + 1
        sets = []
        for _ in range(rotations):
            codes = torch.randint(0, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device="cuda", generator=g)
            scales = (torch.randn((n, k // 128), device="cuda", generator=g).abs() * 0.01).half()
            zeros = torch.randint(0, 16, (n, k // 128), dtype=torch.uint8, device="cuda", generator=g)
            sets.append((codes, scales, zeros))
        for m in ms:
            x = torch.randn((m, k), device="cuda", generator=g)
            y = torch.empty((m, n), device="cuda")
            work = torch.empty(gphq.mm_split_workspace_bytes(m, k, n), dtype=torch.uint8, device="cuda")
            for c, sc, z in sets:
                gphq.mm(gphq.FMT_GPTQ4_G128, c, sc, x, y, m, k, n, work, zeros=z, stream=stream)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                cs = torch.cuda.current_stream()
                for c, sc, z in sets:
                    gphq.mm(gphq.FMT_GPTQ4_G128, c, sc, x, y, m, k, n, work, zeros=z, stream=cs)
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (steps * rotations)
            nbytes = per + 4 * m * k + 4 * m * n
            flops = 2.0 * m * n * k
            out[f"K{k}_N{n}_M{m}"] = {
                "us": round(us, 3),
                "gbs": round(nbytes / us / 1e3, 1),
                "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                "tflops": round(flops / us / 1e6, 2),
                "fp16_frac": round(flops / us / 1e6 / FP16_PEAK_TFLOPS, 4),
                "rotations": rotations,
            }
        del sets
        torch.cuda.empty_cache()
    return out


QWEN3_06B = dict(hidden=1024, layers=28, heads=16, kv_heads=8, head_dim=128, intermediate=3072, vocab=151936,
                 max_positions=40960)
QWEN3_8B = dict(hidden=4096, layers=36, heads=32, kv_heads=8, head_dim=128, intermediate=12288, vocab=151936,
                max_positions=40960)


def decode_model(torch, gphq, geom, fmt, seed):
    """A random-init Qwen3-shaped model in the qwen3lm GPU layout, generated on
    the device (gphq.lm_random): int8 codes U[-127,127] (Q4: bytes U[0,255]),
    scales |N(0,1)|*0.02, norms 1 + N(0,0.02), BF16 embeddings N(0,1), a Q8B
    head padded to 16 rows. Returns (lm, algorithmic weight bytes read per step)."""
    lm, weight_bytes, _ = gphq.lm_random(geom, fmt, seed)
    return lm, weight_bytes


def decode_config(torch, gphq, lm, weight_bytes, geom, lanes, ctx, steps, warmup, graph, label, cap_factor=1):
    """Greedy decode of `steps` tokens per lane at context `ctx` (the K/V
    cache prefilled by the batched pass over random ids, lane 0's prefix
    copied to the others), timed with HIP events on the launch stream. Each
    prefix holds cap_factor times the rows the run needs (the reference's
    callers double capacity, qwen3/chat.go:760-769)."""
    stream = torch.cuda.current_stream()
    ws = gphq.DecodeBatch(lm, lanes)
    ws.set_graph(graph)
    cap = cap_factor * (ctx + max(steps, warmup) + 1)
    kvs = [gphq.Prefix(lm, cap) for _ in range(lanes)]
    rng = np.random.default_rng(ctx + lanes)
    t0 = time.perf_counter()
    pf = gphq.Prefill(lm, ctx)  # the batched pass fills lane 0's cache
    pf.extend(kvs[0], 0, rng.integers(0, geom["vocab"], ctx), torch.empty(geom["hidden"], device="cuda"))
    pf.check()
    del pf
    for kv in kvs[1:]:
        kv.copy_from(kvs[0], ctx)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    first = rng.integers(0, geom["vocab"], lanes)
    out = torch.empty((max(steps, warmup), lanes), dtype=torch.int32, device="cuda")
    ws.greedy_run(kvs, [ctx] * lanes, first, warmup, out[:warmup])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    ws.greedy_run(kvs, [ctx] * lanes, first, steps, out[:steps])
    e1.record(stream)
    torch.cuda.synchronize()
    ws.check()
    ms = e0.elapsed_time(e1)
    toks = out[:steps].cpu().numpy()
    layers, kvd = geom["layers"], geom["kv_heads"] * 128
    mean_ctx = ctx + (steps + 1) / 2.0  # keys read per layer, averaged over the timed steps
    kv_bytes = lanes * layers * 2 * kvd * 4 * mean_ctx
    step_bytes = weight_bytes + kv_bytes
    ms_tok = ms / steps
    return {
        "workload": label,
        "lanes": lanes,
        "context": ctx,
        "steps": steps,
        "ms_per_step": round(ms_tok, 4),
        "tokens_per_s": round(lanes * steps / (ms / 1e3), 1),
        "bytes_per_step": int(step_bytes),
        "achieved_gbs": round(step_bytes / (ms_tok / 1e3) / 1e9, 1),
        "hbm_frac": round(step_bytes / (ms_tok / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "graph": bool(graph),
        "capacity": int(cap),
        "prefill_s": round(prefill_s, 2),
        "distinct_tokens": int(len(np.unique(toks))),
    }


def prefill_config(torch, gphq, lm, geom, tokens, reps, label, int8=False):
    """Config 4a: one `tokens`-token prompt evaluated by the batched pass
    (gphq_prefill_extend, one pass of `tokens` rows) into a fresh prefix, timed
    with HIP events on the launch stream over `reps` prefills after one
    untimed prefill. FLOPs are algorithmic: 2 per weight per token for the
    projections, 4 * head_dim per (query head, visible key) for attention.
    int8: the int8 route (Q8 layers; per-row int8 activations, exact int32
    products on int8 MFMA)."""
    stream = torch.cuda.current_stream()
    ws = gphq.Prefill(lm, tokens)
    if int8:
        ws.set_arith(gphq.PASS_INT8)
    kv = gphq.Prefix(lm, tokens)
    rng = np.random.default_rng(tokens)
    ids = rng.integers(0, geom["vocab"], tokens)
    hidden = torch.empty(geom["hidden"], device="cuda")
    ws.extend(kv, 0, ids, hidden)
    ws.check()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        ws.extend(kv, 0, ids, hidden)
    e1.record(stream)
    ws.check()
    ms = e0.elapsed_time(e1) / reps
    H, I, L = geom["hidden"], geom["intermediate"], geom["layers"]
    qd, kvd = geom["heads"] * 128, geom["kv_heads"] * 128
    weights = L * (H * (qd + 2 * kvd) + qd * H + H * 2 * I + I * H)
    proj = 2.0 * weights * tokens
    attn = 4.0 * 128 * geom["heads"] * L * tokens * (tokens + 1) / 2
    tf = (proj + attn) / (ms / 1e3) / 1e12
    rec = {
        "workload": label,
        "tokens": tokens,
        "reps": reps,
        "ms": round(ms, 3),
        "tokens_per_s": round(tokens / (ms / 1e3), 1),
        "tflops": round(tf, 1),
        "fp16_mfma_frac": round(tf / FP16_PEAK_TFLOPS, 4),
        "projection_tflop": round(proj / 1e12, 3),
        "attention_tflop": round(attn / 1e12, 3),
        "arithmetic": "FP16 weight/activation tiles, fp32 accumulate (the reference mm); FP16 attention tiles",
        "finite": bool(torch.isfinite(hidden).all().item()),
    }
    if int8:
        # Projections on int8 MFMA, attention on FP16 MFMA: the fraction of
        # each peak the whole pass would reach if it ran at that rate alone.
        del rec["fp16_mfma_frac"]
        rec["arithmetic"] = ("int8 route: per-row int8 activations (WorkspaceI8) x Q8 per-row int8 weights, exact "
                             "int32 sums, MulPanelsI8 scaling (the reference's CPU int8 path); FP16 attention tiles")
        rec["int8_mfma_frac_of_projection_ops"] = round(proj / (ms / 1e3) / 1e12 / INT8_PEAK_TOPS, 4)
    return rec


FORMAT_DESC = {
    "q8b": "Q8B: int8 codes with one FP16 scale per 32-value block (the reference's gpu-q8 format), Q8B head",
    "q8b_f32": "Q8B_F32: int8 codes with one fp32 scale per 32-value block (BASELINE config 1's scales), Q8B head",
    "q8": "Q8: int8 codes with one fp32 scale per row (the reference's gpu format), Q8B head",
    "q4": "Q4: 4-bit codes with one FP16 scale per 32-value block (the reference's gpu-q4 format), Q8B head",
}


def decode_benchmarks(args, torch, gphq):
    fmt = {"q8b": gphq.FMT_Q8B, "q8b_f32": gphq.FMT_Q8B_F32, "q8": gphq.FMT_Q8, "q4": gphq.FMT_Q4}[args.decode_fmt]
    graph = not args.decode_eager
    want = set(args.decode_configs.split(","))
    res = {"fmt": args.decode_fmt, "weights": FORMAT_DESC[args.decode_fmt]}
    if "3" in want:
        lm, wb = decode_model(torch, gphq, QWEN3_06B, fmt, 3)
        res["config3"] = decode_config(torch, gphq, lm, wb, QWEN3_06B, 1, 1024, 256, 16, graph,
                                       "config 3: Qwen3-0.6B-shaped, batch 1, 1024-token K/V prefill, 256 greedy steps")
        del lm
        torch.cuda.empty_cache()
    if want & {"4a", "4b1", "4b16"}:
        lm, wb = decode_model(torch, gphq, QWEN3_8B, fmt, 4)
        if "4a" in want:
            res["config4a"] = prefill_config(torch, gphq, lm, QWEN3_8B, 4096, 3,
                                             "config 4a: Qwen3-8B-shaped 4096-token prefill, one batched pass")
        if "4b1" in want:
            res["config4b_1"] = decode_config(torch, gphq, lm, wb, QWEN3_8B, 1, 4096, 64, 8, graph,
                                              "config 4b: Qwen3-8B-shaped decode at context 4096, 1 lane")
            res["config4b_1_cap2x"] = decode_config(
                torch, gphq, lm, wb, QWEN3_8B, 1, 4096, 64, 8, graph,
                "config 4b: Qwen3-8B-shaped decode at context 4096, 1 lane, prefix capacity twice the need", 2)
        if "4b16" in want:
            res["config4b_16"] = decode_config(torch, gphq, lm, wb, QWEN3_8B, 16, 4096, 32, 4, graph,
                                               "config 4b: Qwen3-8B-shaped decode at context 4096, 16 lanes")
        del lm
        torch.cuda.empty_cache()
    if "4a8" in want:
        # Config 4a on the int8 route: Q8 layers (one fp32 scale per row, the
        # format the int8 route multiplies exactly).
        lm, _ = decode_model(torch, gphq, QWEN3_8B, gphq.FMT_Q8, 4)
        line = prefill_config(torch, gphq, lm, QWEN3_8B, 4096, 3,
                              "config 4a: Qwen3-8B-shaped 4096-token prefill, one batched pass, int8 route", int8=True)
        line["weights"] = FORMAT_DESC["q8"]
        res["config4a_int8"] = line
        del lm
        torch.cuda.empty_cache()
    if "4b1" in want and fmt != gphq.FMT_Q8B_F32:
        # The same line with fp32 block scales (config 1's scale format, 9.72 GB a step).
        lm, wb = decode_model(torch, gphq, QWEN3_8B, gphq.FMT_Q8B_F32, 4)
        line = decode_config(torch, gphq, lm, wb, QWEN3_8B, 1, 4096, 64, 8, graph,
                             "config 4b: Qwen3-8B-shaped decode at context 4096, 1 lane, fp32 block scales")
        line["weights"] = FORMAT_DESC["q8b_f32"]
        res["config4b_1_q8b_f32"] = line
        del lm
        torch.cuda.empty_cache()
    return res


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE / WRITE_SIZE
    profile (profiles/gemvb_config1_traffic.md), or None."""
    path = os.path.join(ROOT, "profiles", "gemvb_config1_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return rec["traffic_bytes_per_launch"] if rec.get("kernel") == kernel else None


def profiled_launch(kernel):
    """The committed rocprofv3 kernel-trace summary of `kernel`
    (profiles/gemvb_config1_kernel_stats.json, made from the run in
    profiles/gemvb_config1_kernel_stats.md), or None: its average duration per
    launch over all dispatches and over the timed ones, the host it ran on and
    when."""
    path = os.path.join(ROOT, "profiles", "gemvb_config1_kernel_stats.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return rec if rec.get("kernel") == kernel else None


def cpu_baseline(seconds):
    """The reference's amd64 q8gemv path (scalarMulInto, single thread),
    restated in C (oracle), on the config-1 shape with per-row scales; with
    the host's core count and CPU model."""
    from oracle import cpu_baseline as cb

    out = cb.config1(seconds)
    out.update(cb.host_info())
    return out


def cpu_baselines(seconds):
    """The reference's CPU paths for configs 2, 3 and 4b (C restatements of
    its amd64 code: scalar int8 panels split across T workers), at T = 1 and
    T = min(cores, 16) (the reference's default worker cap)."""
    from oracle import cpu_baseline as cb

    T = cb.max_threads()
    ts = [1, T] if T > 1 else [1]
    q06 = dict(QWEN3_06B, head_dim=128)
    q8 = dict(QWEN3_8B, head_dim=128)
    return {
        "host": cb.host_info(),
        "config2_int8_tile": [cb.config2(seconds, t) for t in ts],
        "config3_decode": cb.decode(q06, 1024, seconds, ts),
        "config4b_decode": cb.decode(q8, 4096, seconds, [T], layers_run=2),
        "path": "the reference's CPU int8 path (WorkspaceI8 per-row activation quantization, scalarMulPanelsI8 "
        "over 64-column panels per worker, fp32 attention): C restatement, -O2 -ffp-contract=off",
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
    r = gemv_config1(args, torch, gphq, args.mode)
    single = gemv_config1(args, torch, gphq, "graph") if args.mode == "batch" else None
    value = r["value_gbs"]
    gemm = None if args.no_gemm else gemm_config2(args, torch, gphq)
    gemm_b32 = None if args.no_gemm else gemm_config2_block32(args, torch, gphq)
    gemm_b32i8 = None if args.no_gemm else gemm_config2_block32_int8(args, torch, gphq)
    gptq = None if args.no_gptq else gptq_config5(args, torch, gphq)
    decode = None if args.no_decode else decode_benchmarks(args, torch, gphq)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    cpus = None if args.no_cpu else cpu_baselines(args.cpu_seconds / 2)
    # The config-1 kernels (gemv.hip): the batch kernel <format, K steps per wave, slices,
    # rows per group, waves per block>; the single-GEMV persistent kernel <format, K steps
    # per wave, rows per group, K slices, waves per block, GEMVs per launch>.
    kernel = "gemvb_kernel<Q8B_F32,4,2,2,4>" if args.mode == "batch" else "gemvp_kernel<Q8B_F32,2,4,2,8,1>"
    traffic = measured_traffic(kernel) if args.rotations == 32 else None
    prof = profiled_launch(kernel) if args.rotations == 32 else None
    prof_us = None if prof is None else prof.get("timed_avg_us", prof["avg_us"])
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
            f"(W, scales) sets ({r['R'] * r['unit_bytes'] / 1e6:.0f} MB, > 256 MB Infinity Cache), "
            + ("one gphq_gemv_batch launch per step" if args.mode == "batch" else f"{r['R']} gphq_gemv launches ({args.mode})"),
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
            "traffic": traffic,
            "traffic_source": None if traffic is None else
            "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this launch, copy-kernel calibrated "
            "(profiles/gemvb_config1_traffic.md)",
            "kernel": kernel,
            "per_launch_us": round(r["per_launch_us"], 3),
            "bytes_per_launch": r["bytes_per_launch"],
            # The same launch's average duration over the timed dispatches of
            # the committed rocprofv3 kernel trace (another run, usually another
            # box of the pool) and the fraction it gives, beside this run's
            # HIP-event figures.
            "profile_us": None if prof is None else prof_us,
            "frac_profile": None if prof is None else
            round(r["bytes_per_launch"] / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "profile_source": None if prof is None else
            f"profiles/gemvb_config1_kernel_stats.md ({prof.get('timed_calls', prof['calls'])} timed launches on "
            f"{prof['host']}, {prof['date']})",
        },
        "cpu_baseline": cpu,
        "cpu_baselines": cpus,
        "single_launch": None if single is None else {
            "gbs": round(single["achieved_gbs"], 2),
            "frac": round(single["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "per_gemv_us": round(single["per_gemv_us"], 3),
            "mode": "one gphq_gemv launch per 4096x4096 GEMV, HIP graph of 32 launches",
        },
        "gemm_config2": gemm,
        "gemm_config2_block32": gemm_b32,
        "gemm_config2_block32_int8": gemm_b32i8,
        "gptq_config5": gptq,
        "decode_ms_per_token": (decode or {}).get("config4b_1", {}).get("ms_per_step"),
        "decode_weights": (decode or {}).get("weights"),
        "prefill_4096_ms": (decode or {}).get("config4a", {}).get("ms"),
        "decode": decode,
        "check": {"rel_l2_vs_float64": r["rel_l2"]},
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
