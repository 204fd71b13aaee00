"""Writes the golden fixtures in this directory. numpy only: the expected
outputs come from exact or float64 arithmetic, never from the oracle or the
HIP library, so they pin both.

Inputs follow the deterministic generators in the reference's own tests
(gophonic tree; only those that do not depend on Go's math/rand, which cannot
be replayed without Go):
  q8gemv_extremes  q8gemv/q8gemv_test.go:45-73   (k=35, n=3)
  q8gemv_nonfinite q8gemv/q8gemv_test.go:75-89
  q8b_stream       qwen3lm/gpu_projection_stream_darwin_test.go:44-68,89-98
                   (weight/activation generator; 2 of the 28 matrices, 64 rows)
  f16_buffer       q8gemm/buffer_test.go:12-50 (BF16 values (i%29-14)/8)
  i8_tile          q8gemm/int8_test.go:123-128 activations (i%13 - 6), with a
                   documented deterministic weight pattern in place of the
                   test's math/rand weights
  q4_pattern       qwen3lm/gpu_darwin_test.go:44-56 dequantization rule over a
                   documented deterministic nibble/scale pattern

Run: python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_round(v):
    """IEEE float32 -> float16 -> float32 (numpy rounds to nearest even)."""
    return np.float32(v).astype(np.float16).astype(np.float32)


def q8gemv_extremes():
    k, n = 35, 3
    x = np.array([((i % 9) - 4) * 0.25 for i in range(k)], dtype=np.float32)
    pat = [-128, 127, -1, 1]
    q = np.array([pat[i % 4] for i in range(k * n)], dtype=np.int8)
    scales = np.array([1, -0.03125, 0.0001], dtype=np.float32)
    want = np.zeros(n, dtype=np.float32)
    for r in range(n):
        # Every partial sum is a multiple of 0.25 below 2^12 in magnitude, so
        # the sequential fp32 sum is exact; one fp32 multiply by the scale.
        s = sum(float(x[c]) * float(q[r * k + c]) for c in range(k))
        want[r] = np.float32(s) * scales[r]
    np.savez(os.path.join(HERE, "q8gemv_extremes.npz"), x=x, q=q, scales=scales, want=want, k=k, n=n)


def q8gemv_nonfinite():
    x = np.zeros(20, dtype=np.float32)
    q = np.zeros(20, dtype=np.int8)
    x[0] = np.inf
    x[4] = np.nan
    x[19] = -0.0
    q[0], q[4], q[19] = 0, 3, -4
    np.savez(os.path.join(HERE, "q8gemv_nonfinite.npz"), x=x, q=q, scales=np.array([2], np.float32), k=20, n=1)


def q8b_stream(matrices=(0, 27), rows=64, cols=2048):
    codes, scales, ys = [], [], []
    x = np.array([((i % 31) - 15) * 0.017 for i in range(cols)], dtype=np.float32)
    for m in matrices:
        r = np.arange(rows)[:, None]
        c = np.arange(cols)[None, :]
        v = (((((r + m * 13) * 3 + c * 7) % 101) - 50).astype(np.float32) * np.float32(0.001)).astype(np.float32)
        vb = v.reshape(rows, cols // 32, 32)
        maxabs = np.abs(vb).max(axis=2)
        d = f16_round(maxabs / np.float32(127))  # fp32 divide, then FP16 round
        with np.errstate(divide="ignore", invalid="ignore"):
            qv = np.rint(vb / d[:, :, None])  # fp32 divide, round half to even
        qv = np.where(d[:, :, None] == 0, 0, qv)
        q = qv.astype(np.int8).reshape(rows, cols)
        sbits = d.astype(np.float16).view(np.uint16)
        deq = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32, axis=1)
        y = deq @ x.astype(np.float64)
        codes.append(q)
        scales.append(sbits)
        ys.append(y)
    np.savez(
        os.path.join(HERE, "q8b_stream.npz"), codes=np.stack(codes), scales=np.stack(scales), x=x,
        want=np.stack(ys), rows=rows, cols=cols, matrices=np.array(matrices),
    )


def f16_buffer():
    out = {}
    for k, n in [(3, 65), (32, 129)]:
        raw = np.array([((i % 29) - 14) * 0.125 for i in range(k * n)], dtype=np.float32)
        bf = (raw.view(np.uint32) >> 16).astype(np.uint16)
        vals = (bf.astype(np.uint32) << 16).view(np.float32).reshape(n, k)
        maxabs = np.abs(vals).max(axis=1)
        h = np.zeros((n, k), dtype=np.uint16)
        sc = np.zeros(n, dtype=np.float32)
        for row in range(n):
            e = 0
            if maxabs[row] > 0:
                _, ex = np.frexp(np.float64(maxabs[row]))
                e = int(min(max(15 - ex, -100), 100))
            h[row] = (vals[row] * np.float32(2.0 ** e)).astype(np.float16).view(np.uint16)
            sc[row] = np.float32(2.0 ** -e)
        out[f"bf16_{k}_{n}"] = bf
        out[f"h_{k}_{n}"] = h
        out[f"scales_{k}_{n}"] = sc
    np.savez(os.path.join(HERE, "f16_buffer.npz"), **out)


def i8_tile(rows=16, k=256, n=96):
    x = np.array([(i % 13) - 6 for i in range(rows * k)], dtype=np.float32).reshape(rows, k)
    # Deterministic weights and scales (documented pattern, not the test's rand).
    idx = np.arange(n * k).reshape(n, k)
    w = (((idx * 37 + 11) % 255) - 127).astype(np.int8)
    scales = ((np.arange(n) % 100) + 1).astype(np.float32) / np.float32(997)
    maxabs = np.abs(x).max(axis=1)
    row_scale = (maxabs / np.float32(127)).astype(np.float32)
    row_inv = (np.float32(127) / maxabs).astype(np.float32)
    prod = (x * row_inv[:, None]).astype(np.float32)
    qa = np.clip(np.rint(prod), -128, 127).astype(np.int8)
    acc = qa.astype(np.int64) @ w.astype(np.int64).T
    want = (acc.astype(np.float32) * scales[None, :]).astype(np.float32) * row_scale[:, None]
    np.savez(
        os.path.join(HERE, "i8_tile.npz"), x=x, w=w, scales=scales, qa=qa, row_scale=row_scale, acc=acc,
        want=want.astype(np.float32),
    )


def q4_pattern(rows=32, k=1024):
    idx = np.arange(rows * k // 2).reshape(rows, k // 2)
    codes = ((idx * 29 + 7) % 256).astype(np.uint8)
    sidx = np.arange(rows * k // 32).reshape(rows, k // 32)
    svals = ((((sidx * 13) % 41) + 1) * 0.0007).astype(np.float32)
    sbits = svals.astype(np.float16).view(np.uint16)
    x = np.array([np.sin(0.37 * i) for i in range(k)], dtype=np.float32)
    deq = np.zeros((rows, k), dtype=np.float64)
    for i in range(k):
        b = codes[:, (i // 32) * 16 + i % 16]
        q = (b >> 4).astype(np.int64) - 8 if i % 32 >= 16 else (b & 15).astype(np.int64) - 8
        deq[:, i] = q * sbits.view(np.float16)[:, i // 32].astype(np.float64)
    want = deq @ x.astype(np.float64)
    np.savez(os.path.join(HERE, "q4_pattern.npz"), codes=codes, scales=sbits, x=x, want=want, rows=rows, k=k)


if __name__ == "__main__":
    q8gemv_extremes()
    q8gemv_nonfinite()
    q8b_stream()
    f16_buffer()
    i8_tile()
    q4_pattern()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
