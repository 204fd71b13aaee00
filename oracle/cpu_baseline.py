"""CPU baselines for bench.py (timed on the GPU box's host cores, beside the
GPU numbers): the reference's amd64 code paths restated in C
(oracle/gphq_oracle.c), which is what the reference runs on x86-64 (its SIMD,
SME and NEON kernels are arm64-only).

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product library never does.

* config 1: q8gemv.scalarMulInto (q8gemv/scalar.go:6-17), one thread.
* config 2: q8gemm's int8 path for one 16-row activation tile
  (WorkspaceI8 quantizer int8.go:106-168, scalarMulPanelsI8 int8.go:200-211)
  with 64-column panels split across T workers (qwen3lm/ops.go:153-214).
* configs 3 / 4b: one decode step of the CPU int8 path (orc_lm_step_i8:
  qwen3lm/ops.go:96-254 over WeightsInt8 rows, with the reference's
  hidden / context / intermediate input rotations), T workers; equal to the
  float64 CpuInt8Oracle to relative 1e-5 (tests/test_cpu_baseline.py).

T is 1 and min(cores, 16): the reference's default worker cap
(qwen3/model.go:39,99-108).
"""
import ctypes
import os
import time

import numpy as np

from . import oracle as orc


def host_info():
    """Core count and CPU model of this host."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"nproc": os.cpu_count(), "usable_cores": usable, "cpu_model": model}


def max_threads():
    return max(1, min(host_info()["usable_cores"], 16))


def _timed(fn, seconds, min_reps=1):
    fn()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds and reps >= min_reps:
            return reps, el


def config1(seconds):
    """q8gemv.scalarMulInto, 4096 x 4096 with per-row fp32 scales, 1 thread: GB/s."""
    K = N = 4096
    rng = np.random.default_rng(1)
    x = rng.standard_normal(K).astype(np.float32)
    q = rng.integers(-127, 128, N * K).astype(np.int8)
    s = (np.abs(rng.standard_normal(N)) * 0.01).astype(np.float32)
    reps, el = _timed(lambda: orc.q8gemv_mul_into(x, q, s, K, N), seconds)
    unit = N * K + N * 4 + K * 4 + N * 4
    return {
        "value": unit * reps / el / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{reps} x q8gemv.scalarMulInto 4096x4096 (per-row fp32 scales, the reference's amd64 path), "
        f"C restatement -O2 -ffp-contract=off, 1 thread, {el:.1f} s",
    }


def config2(seconds, threads):
    """q8gemm int8 path on one 16-row tile (K = 4096, N = 12288): quantizer +
    panel-parallel scalarMulPanelsI8 at T threads: int8 TOPS and ms per tile."""
    K, N, M = 4096, 12288, 16
    rng = np.random.default_rng(2)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = rng.integers(-127, 128, N * K).astype(np.int8)
    sw = (np.abs(rng.standard_normal(N)) * 0.01).astype(np.float32)
    dst = np.zeros(M * N, np.float32)

    def run():
        qa, rs, _ = orc.i8_pack_rows(x, M, K)
        orc.i8_mul_panels(qa, rs, w, sw, K, N, dst=dst, threads=threads)

    reps, el = _timed(run, seconds)
    ms = el / reps * 1e3
    return {"threads": threads, "ms_per_tile": round(ms, 2), "tops": round(2.0 * M * N * K / (ms / 1e3) / 1e12, 4),
            "sample": f"{reps} tiles of 16 x 4096 activations x 12288 int8 rows, {el:.1f} s"}


class _Geom(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("hidden", "heads", "kv_heads", "head_dim", "inter", "vocab", "layers",
                                               "cap")] + [("eps", ctypes.c_float)]


class _Layer(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p * 7), ("s", ctypes.c_void_p * 7), ("attn_norm", ctypes.c_void_p),
                ("mlp_norm", ctypes.c_void_p), ("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p)]


def decode(geom, ctx, seconds, threads_list, layers_run=None, seed=3):
    """Decode steps of the CPU int8 path at context `ctx` for each T in
    threads_list: ms per token. geom: dict(hidden, layers, heads, kv_heads,
    head_dim=128, intermediate, vocab). layers_run < layers times that many
    layers (one shared set of random weights) and scales the layer time up
    to the full depth; the head is timed once per step."""
    lib = orc.lib()
    lib.orc_lm_step_i8.restype = None
    lib.orc_lm_step_i8.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] + [ctypes.c_void_p] * 7 + [ctypes.c_int]
    H, I, hd = geom["hidden"], geom["intermediate"], geom.get("head_dim", 128)
    qd, kvd = geom["heads"] * hd, geom["kv_heads"] * hd
    L = geom["layers"] if layers_run is None else layers_run
    rng = np.random.default_rng(seed)
    shapes = [(qd, H), (kvd, H), (kvd, H), (H, qd), (I, H), (I, H), (H, I)]
    keep = []
    layers = (_Layer * L)()
    for li in range(L):
        for p, (n, k) in enumerate(shapes):
            w = rng.integers(-127, 128, n * k, dtype=np.int8)
            s = (np.abs(rng.standard_normal(n)) * 0.0002).astype(np.float32)
            keep += [w, s]
            layers[li].w[p], layers[li].s[p] = w.ctypes.data, s.ctypes.data
        for name, n in (("attn_norm", H), ("mlp_norm", H), ("q_norm", hd), ("k_norm", hd)):
            v = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
            keep.append(v)
            setattr(layers[li], name, v.ctypes.data)
    cap = ctx + 8
    g = _Geom(H, geom["heads"], geom["kv_heads"], hd, I, geom["vocab"], L, cap, 1e-6)
    kc = rng.standard_normal(L * cap * kvd).astype(np.float32)
    vc = rng.standard_normal(L * cap * kvd).astype(np.float32)
    half = hd // 2
    inv = 1.0 / np.power(1e6, (2.0 * np.arange(half)) / hd)
    cosv, sinv = np.cos(ctx * inv).astype(np.float32), np.sin(ctx * inv).astype(np.float32)
    head = rng.integers(-127, 128, geom["vocab"] * H, dtype=np.int8)
    head_s = (np.abs(rng.standard_normal(geom["vocab"])) * 0.0002).astype(np.float32)
    fnorm = np.ones(H, np.float32)
    logits = np.zeros(geom["vocab"], np.float32)
    out = []
    for T in threads_list:
        h = rng.standard_normal(H).astype(np.float32)

        def step():
            lib.orc_lm_step_i8(ctypes.byref(g), layers, kc.ctypes.data, vc.ctypes.data, ctx, cosv.ctypes.data,
                               sinv.ctypes.data, fnorm.ctypes.data, head.ctypes.data, head_s.ctypes.data,
                               h.ctypes.data, logits.ctypes.data, T)

        reps, el = _timed(step, seconds)
        ms = el / reps * 1e3
        rec = {"threads": T, "context": ctx, "steps": reps}
        if L != geom["layers"]:
            # Head once per step; layers scaled to the full depth.
            g0 = _Geom(H, geom["heads"], geom["kv_heads"], hd, I, geom["vocab"], 0, cap, 1e-6)

            def head_only():
                lib.orc_lm_step_i8(ctypes.byref(g0), layers, kc.ctypes.data, vc.ctypes.data, ctx, cosv.ctypes.data,
                                   sinv.ctypes.data, fnorm.ctypes.data, head.ctypes.data, head_s.ctypes.data,
                                   h.ctypes.data, logits.ctypes.data, T)

            hr, he = _timed(head_only, max(1.0, seconds / 4))
            head_ms = he / hr * 1e3
            ms = head_ms + (ms - head_ms) * geom["layers"] / L
            rec["sample"] = f"{L} of {geom['layers']} layers timed ({reps} steps, {el:.1f} s) and scaled, head timed"
        else:
            rec["sample"] = f"{reps} steps, {el:.1f} s"
        rec["ms_per_token"] = round(ms, 2)
        rec["tokens_per_s"] = round(1e3 / ms, 2)
        out.append(rec)
    return out
