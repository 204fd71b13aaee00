"""GPU parity of the q8gemm FP16 path (Weights / Workspace / MulPanels /
MulInto / PackBF16) through the C ABI, with the reference's own bounds:
  * packed activations are bit-identical to f32ToF16(x * rowScale)
    (q8gemm_test.go:244-288);
  * against float64, |got - want| <= 1e-6 + (1/2048 + 1e-5) * sum|x w| * scale
    (q8gemm_test.go:63-87);
  * against the scalar oracle on Qwen3-8B shapes, 2e-5 * sqrt(K) relative
    (q8gemm_test.go:41-61);
  * BF16 weights pack exactly (q8gemm_test.go:290-352, buffer_test.go).
"""
import math
import os

import numpy as np
import pytest

from gophonic_amd import gphq
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def fill(n, v=-7.0):
    import torch

    return torch.full((max(n, 1),), v, dtype=torch.float32, device="cuda")


def fixture(rows, k, n, seed):
    # q8gemm_test.go:89-113: weights [-127,127], scales (1..100)/1000, x in (-1,1).
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, k * n).astype(np.int8)
    scales = (rng.integers(1, 101, n) / np.float32(1000)).astype(np.float32)
    w = gphq.Weights(k, n)
    w.pack(q, scales)
    x = (rng.random(rows * k, dtype=np.float32) * 2 - 1).astype(np.float32)
    return w, q.reshape(n, k), scales, x


def run_mul_into(x, rows, w, k, n):
    ws = gphq.Workspace(k, max(rows, 1))
    dst = fill(rows * n)
    gphq.mul_into(dst, dev(x), rows, w, ws)
    return host(dst)[: rows * n].reshape(rows, n), ws


@pytest.mark.parametrize("k", [1, 3, 7, 16, 31, 65, 257])
@pytest.mark.parametrize("n", [1, 15, 16, 17, 63, 64, 65, 129])
@pytest.mark.parametrize("rows", [1, 12, 16])
def test_mul_into_randomized_tails(rows, k, n):
    w, q, scales, x = fixture(rows, k, n, rows * 100 + k * 10 + n)
    got, _ = run_mul_into(x, rows, w, k, n)
    xv = x.reshape(rows, k).astype(np.float64)
    prod = xv @ q.T.astype(np.float64)
    want = (prod * scales.astype(np.float64)).astype(np.float32)
    sum_abs = np.abs(xv) @ np.abs(q.T.astype(np.float64))
    bound = 1e-6 + (1.0 / 2048 + 1e-5) * sum_abs * np.abs(scales.astype(np.float64))
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)


def test_packed_activations_bit_exact_and_row_scales():
    import torch

    rng = np.random.default_rng(5)
    for k in [1, 2, 7, 8, 9, 16, 31, 33, 100, 4096]:
        for rows in [1, 5, 16]:
            x = (rng.standard_normal(rows * k) * np.exp2(rng.integers(-15, 15, rows * k))).astype(np.float32)
            x[rng.integers(0, x.size)] = 7e5  # a downscaled row
            ws = gphq.Workspace(k, rows)
            ws.pack(dev(x), rows, k)
            out = torch.zeros(rows * k, dtype=torch.int16, device="cuda")
            ws.activations(out)
            got = host(out).view(np.uint16).reshape(rows, k)
            want, s, inv = orc.f16_pack_rows(x, rows, k)
            assert np.array_equal(got, want), (k, rows)
            ds, di = torch.zeros(rows, device="cuda"), torch.zeros(rows, device="cuda")
            ws.row_scales(ds, di)
            assert np.array_equal(host(ds), s) and np.array_equal(host(di), inv)


@pytest.mark.parametrize("rows,k,n", [(12, 4096, 4096), (12, 4096, 1024), (12, 4096, 12288), (12, 12288, 4096)])
def test_matches_scalar_oracle_on_qwen3_8b_shapes(rows, k, n):
    w, q, scales, x = fixture(rows, k, n, rows * 100 + k * 10 + n)
    got, _ = run_mul_into(x, rows, w, k, n)
    act, _, inv = orc.f16_pack_rows(x, rows, k)
    want = orc.mul_panels(act, inv, q, scales, k, n).reshape(rows, n)
    tol = 2e-5 * math.sqrt(k)
    assert np.all(np.abs(got - want) <= tol * np.maximum(1.0, np.abs(want)))


def test_panel_ranges_and_stride():
    # q8gemm_test.go:114-153.
    rows, k, n, stride = 11, 257, 197, 211
    w, q, scales, x = fixture(rows, k, n, 7)
    full, _ = run_mul_into(x, rows, w, k, n)
    ws = gphq.Workspace(k, 16)
    ws.prepare(rows, k)
    for r in range(rows):
        ws.set_row_scale(r, orc.max_abs(x[r * k:(r + 1) * k]))
    dx = dev(x)
    for k0 in range(0, k, 50):
        ws.pack_range(dx, k, k0, min(k, k0 + 50))
    got = fill((rows - 1) * stride + n)
    for p in range(w.panels()):
        gphq.mul_panels(got, stride, ws, w, p, p + 1)
    out = host(got)
    for r in range(rows):
        assert np.array_equal(out[r * stride:r * stride + n].view(np.uint32), full[r].view(np.uint32))
        if r + 1 < rows:
            assert np.all(out[r * stride + n:(r + 1) * stride] == -7)


def test_row_scaling_handles_large_and_tiny_rows():
    # q8gemm_test.go:214-240.
    k, n = 96, 64
    w, q, scales, x = fixture(3, k, n, 11)
    x = x.reshape(3, k).copy()
    x[0] *= np.float32(1e6)
    x[1] *= np.float32(1e-7)
    x[2] *= np.float32(0.5)
    got, _ = run_mul_into(x.ravel(), 3, w, k, n)
    xv = x.astype(np.float64)
    want = (xv @ q.T.astype(np.float64)) * scales
    sum_abs = np.abs(xv) @ np.abs(q.T.astype(np.float64))
    assert np.all(np.abs(got - want) <= (1.0 / 2048) * sum_abs * scales)


def onehot_weights(w, k, n):
    """Reads back w[c, kk] * scale[c] through the product: x = identity rows."""
    eye = np.eye(k, dtype=np.float32)
    ws = gphq.Workspace(k, k)
    dst = fill(k * n)
    gphq.mul_into(dst, dev(eye), k, w, ws)
    return host(dst)[: k * n].reshape(k, n).T  # [n, k]


@pytest.mark.parametrize("rows,k,n", [(1, 7, 5), (12, 65, 129), (16, 256, 64)])
def test_f16_weights_hold_bf16_exactly(rows, k, n):
    rng = np.random.default_rng(k + n)
    v = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
    v[np.arange(n) * k + 3 % k] = 1.5  # one large outlier per row
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    w = gphq.Weights(k, n, f16=True)
    assert w.pack_bf16(bf) == 0
    back = onehot_weights(w, k, n)
    want = (bf.astype(np.uint32) << 16).view(np.float32).reshape(n, k)
    assert np.array_equal(back, want)
    # MulInto against float64 of the BF16 values.
    x = (rng.random(rows * k, dtype=np.float32) * 2 - 1).astype(np.float32)
    got, _ = run_mul_into(x, rows, w, k, n)
    xv = x.reshape(rows, k).astype(np.float64)
    exact = xv @ want.T.astype(np.float64)
    sum_abs = np.abs(xv) @ np.abs(want.T.astype(np.float64))
    assert np.all(np.abs(got - exact) <= 1e-6 + (1.0 / 2048 + 1e-5) * sum_abs)


def test_pack_bf16_golden_buffer_and_borrowed_storage():
    import torch

    g = np.load(os.path.join(GOLDEN, "f16_buffer.npz"))
    for k, n in [(3, 65), (32, 129)]:
        size = gphq.weights_f16_bytes(k, n)
        buf = torch.zeros(size, dtype=torch.uint8, device="cuda")
        borrowed = gphq.Weights(k, n, buffer=buf)
        owned = gphq.Weights(k, n, f16=True)
        assert borrowed.pack_bf16(g[f"bf16_{k}_{n}"]) == 0
        assert owned.pack_bf16(g[f"bf16_{k}_{n}"]) == 0
        want = orc.f16_to_f32(g[f"h_{k}_{n}"]).reshape(n, k) * g[f"scales_{k}_{n}"][:, None]
        assert np.array_equal(onehot_weights(borrowed, k, n), want)
        assert np.array_equal(onehot_weights(owned, k, n), want)
    short = gphq.weights_f16_bytes(3, 65) - 1
    with pytest.raises(gphq.GphqError, match="invalid dimensions"):
        gphq.Weights(3, 65, buffer=torch.zeros(short, dtype=torch.uint8, device="cuda"))


def reference_buffer(h_rows, scales, k, n):
    """The bytes of a reference NewWeightsF16Buffer after PackBF16: FP16 values
    in the panel layout [n/64][k/2][64][2] (packed.go:233-239), then n fp32
    row scales (packed.go:95-121)."""
    panels = orc.pack_panels(np.ascontiguousarray(h_rows, np.uint16).reshape(-1), k, n)
    return np.concatenate([panels.view(np.uint8), np.ascontiguousarray(scales, np.float32).view(np.uint8)])


def test_load_reference_f16_buffer_bytes():
    # A wcache-mapped buffer in the reference's own layout (weights.go:362-370)
    # loads into device weights equal to packing the same BF16 rows here.
    g = np.load(os.path.join(GOLDEN, "f16_buffer.npz"))
    lib = gphq.load()
    assert lib.gphq_q8gemm_reference_f16_bytes(3, 65) == 1284  # packed.go:78-93 for K = 3, N = 65
    for k, n in [(3, 65), (32, 129)]:
        ref = reference_buffer(g[f"h_{k}_{n}"], g[f"scales_{k}_{n}"], k, n)
        assert ref.size == lib.gphq_q8gemm_reference_f16_bytes(k, n)
        loaded = gphq.Weights(k, n, f16=True)
        loaded.load_reference(ref)
        packed = gphq.Weights(k, n, f16=True)
        packed.pack_bf16(g[f"bf16_{k}_{n}"])
        want = orc.f16_to_f32(g[f"h_{k}_{n}"]).reshape(n, k) * g[f"scales_{k}_{n}"][:, None]
        assert np.array_equal(onehot_weights(loaded, k, n), want)
        # Products through both are bit-identical.
        rng = np.random.default_rng(k)
        x = rng.standard_normal((5, k)).astype(np.float32)
        outs = []
        for w in (loaded, packed):
            ws = gphq.Workspace(k, 5)
            dst = fill(5 * n)
            gphq.mul_into(dst, dev(x), 5, w, ws)
            outs.append(host(dst).view(np.uint32))
        assert np.array_equal(outs[0], outs[1])
        with pytest.raises(gphq.GphqError, match="invalid dimensions"):
            loaded.load_reference(ref[:-1])
    bad = reference_buffer(g["h_3_65"], np.where(np.arange(65) == 7, np.inf, g["scales_3_65"]), 3, 65)
    with pytest.raises(gphq.GphqError, match="non-finite"):
        gphq.Weights(3, 65, f16=True).load_reference(bad)


def test_pack_bf16_counts_rounding_and_rejects_non_finite():
    k, n = 32, 4
    v = np.zeros(k * n, np.float32)
    v[0] = 1.0
    v[1] = 1.0 + 2.0 ** -7   # BF16 with 8 significant bits: exact in FP16 after the shift
    v[2] = 1.5 * 2.0 ** -38  # lands between FP16 subnormals after the shift: rounds
    v[k:] = 0.25
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    w = gphq.Weights(k, n, f16=True)
    want = orc.pack_bf16_rows(bf, k, n)[2]
    assert w.pack_bf16(bf) == want and want >= 1
    bad = bf.copy()
    bad[2 * k + 5] = 0x7F80  # +Inf in row 2
    with pytest.raises(gphq.GphqError, match="non-finite"):
        w.pack_bf16(bad)


def test_k_zero_and_sme_only_modes():
    w = gphq.Weights(0, 70)
    w.pack(np.zeros(0, np.int8), np.ones(70, np.float32))
    ws = gphq.Workspace(0, 4)
    ws.prepare(3, 0)
    dst = fill(3 * 70)
    gphq.mul_panels(dst, 70, ws, w, 0, w.panels())
    out = host(dst)
    assert np.all(out == 0) and not np.any(np.signbit(out))
    ws2 = gphq.Workspace(32, 16)
    for fn in (lambda: ws2.prepare_row_f16(32), lambda: ws2.prepare_rows_f16(2, 16)):
        with pytest.raises(gphq.GphqError, match="invalid dimensions"):
            fn()
    with pytest.raises(gphq.GphqError, match="non-finite"):
        gphq.Weights(4, 2).pack(np.zeros(8, np.int8), np.array([1, np.inf], np.float32))
