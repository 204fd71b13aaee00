"""GPU parity of the q8gemm int8 x int8 path (WeightsI8 / WorkspaceI8 /
MulPanelsI8 / MulStripsI8) through the C ABI. The bar is the reference's:
bit-for-bit equality with the exact integer oracle (int8_test.go:74-78,
167-171), for any panel/strip split.
"""
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


def int8_fixture(k, n, seed):
    # int8_test.go:12-30: weights in [-127, 127], scales (1..100)/997.
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, k * n).astype(np.int8)
    scales = (rng.integers(1, 101, n) / np.float32(997)).astype(np.float32)
    w = gphq.WeightsI8(k, n)
    w.pack(q, scales)
    return w, q.reshape(n, k), scales


def activations(rows, k, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(rows * k) * (1 + np.arange(rows * k) % 5)).astype(np.float32)
    if x.size:
        x[0] = 0  # an exact zero (int8_test.go:56)
    return x


def run_gpu(x, rows, k, w, n, stride=None, ws=None):
    stride = n if stride is None else stride
    ws = ws or gphq.WorkspaceI8(k, max(rows, 1))
    dx = dev(x)
    ws.pack(dx, rows, k)
    dst = fill((rows - 1) * stride + n if rows else 1)
    gphq.mul_panels_i8(dst, stride, ws, w, 0, w.panels())
    return host(dst), ws


def oracle_out(x, rows, k, q, scales, n):
    qa, rs, inv = orc.i8_pack_rows(x, rows, k)
    return orc.i8_mul_panels(qa, rs, q, scales, k, n), rs, inv


SHAPES = [(1, 4, 1), (3, 7, 17), (12, 64, 64), (16, 257, 129), (12, 4096, 1024), (5, 12288, 64), (1, 32, 64),
          (1, 4096, 1024), (1, 12288, 200), (1, 96, 5), (17, 100, 33), (64, 640, 96), (100, 512, 300),
          (200, 1024, 520),
          # the skinny kernel (17..256 rows, K a multiple of 256): one-stage K,
          # column tiles past N in a block, two row blocks
          (24, 256, 200), (48, 256, 500), (130, 1024, 64), (256, 2048, 77), (33, 12288, 48),
          # direct-to-LDS big tiles (129..512 rows), K not a multiple of 256
          (300, 640, 260), (512, 192, 200), (140, 64, 40),
          # K not a multiple of 256 from 65 rows (LDS kernel) and past 512 rows (big tiles)
          (100, 640, 200), (600, 320, 130)]


@pytest.mark.parametrize("rows,k,n", SHAPES, ids=[f"M{r}K{k}N{n}" for r, k, n in SHAPES])
def test_mul_panels_i8_bit_exact(rows, k, n):
    w, q, scales = int8_fixture(k, n, k * 31 + n)
    x = activations(rows, k, rows + k)
    got, ws = run_gpu(x, rows, k, w, n)
    want, rs, inv = oracle_out(x, rows, k, q, scales, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # The device row scales match the reference arithmetic bit for bit.
    import torch

    ds, di = torch.zeros(rows, device="cuda"), torch.zeros(rows, device="cuda")
    ws.row_scales(ds, di)
    assert np.array_equal(host(ds).view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(host(di).view(np.uint32), inv.view(np.uint32))


@pytest.mark.parametrize("m", [1, 16, 32, 64, 100, 128, 192, 256, 320, 512])
def test_config2_shapes_bit_exact(m):
    # Benchmark config 2: K = 4096, N = 12288; exact integer sums via a float64
    # product of the integer codes (every partial sum is an integer < 2^53, so
    # float64 accumulation is exact in any order).
    import torch

    k, n = 4096, 12288
    rng = np.random.default_rng(m)
    q = rng.integers(-127, 128, k * n).astype(np.int8)
    scales = (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float32)
    w = gphq.WeightsI8(k, n)
    w.pack(q, scales)
    x = rng.standard_normal(m * k).astype(np.float32)
    got, ws = run_gpu(x, m, k, w, n)
    qa, rs, _ = orc.i8_pack_rows(x, m, k)
    acc = (dev(qa.astype(np.float64)) @ dev(q.reshape(n, k).astype(np.float64)).T)
    acc = host(acc)
    assert np.all(acc == np.round(acc))
    want = (acc.astype(np.float32) * scales[None, :]).astype(np.float32) * rs[:, None]
    assert np.array_equal(got.reshape(m, n).view(np.uint32), want.astype(np.float32).view(np.uint32))
    if m <= 16:
        ref = orc.i8_mul_panels(qa, rs, q, scales, k, n, threads=8).reshape(m, n)
        assert np.array_equal(got.reshape(m, n).view(np.uint32), ref.view(np.uint32))
    del torch


def test_golden_tile():
    g = np.load(os.path.join(GOLDEN, "i8_tile.npz"))
    rows, k = g["x"].shape
    n = g["w"].shape[0]
    w = gphq.WeightsI8(k, n)
    w.pack(g["w"], g["scales"])
    got, _ = run_gpu(g["x"].ravel(), rows, k, w, n)
    assert np.array_equal(got.reshape(rows, n).view(np.uint32), g["want"].view(np.uint32))


@pytest.mark.parametrize("rows,k,n", [(1, 64, 64), (8, 128, 128), (12, 4096, 1024), (16, 257, 200), (5, 12288, 64),
                                      (3, 36, 30), (40, 300, 130), (24, 256, 330), (40, 512, 130), (120, 1024, 200),
                                      (200, 320, 200), (400, 256, 130)])
def test_strips_and_panels_bit_identical(rows, k, n):
    # int8_test.go:146-179: strips, panels, and per-panel calls all agree.
    w, q, scales = int8_fixture(k, n, k + 7 * n)
    x = activations(rows, k, rows * k)
    ws = gphq.WorkspaceI8(k, rows)
    ws.pack(dev(x), rows, k)
    full = fill(rows * n)
    gphq.mul_panels_i8(full, n, ws, w, 0, w.panels())
    strips = fill(rows * n, -1.0)
    gphq.mul_strips_i8(strips, n, ws, w, 0, w.strips())
    per = fill(rows * n, -2.0)
    for p in range(w.panels()):
        gphq.mul_panels_i8(per, n, ws, w, p, p + 1)
    mixed = fill(rows * n, -3.0)
    half = w.strips() // 2
    gphq.mul_strips_i8(mixed, n, ws, w, 0, half)
    gphq.mul_strips_i8(mixed, n, ws, w, half, w.strips())
    a = host(full).view(np.uint32)
    for other in (strips, per, mixed):
        assert np.array_equal(a, host(other).view(np.uint32))
    want, _, _ = oracle_out(x, rows, k, q, scales, n)
    assert np.array_equal(a, want.view(np.uint32))


def test_ranges_and_stride_leave_other_columns_untouched():
    # q8gemm_test.go:114-153 pattern for the int8 path.
    rows, k, n, stride = 11, 257, 197, 211
    w, q, scales = int8_fixture(k, n, 7)
    x = activations(rows, k, 3)
    ws = gphq.WorkspaceI8(k, 16)
    ws.pack(dev(x), rows, k)
    got = fill((rows - 1) * stride + n)
    gphq.mul_panels_i8(got, stride, ws, w, 1, 3)  # columns [64, 192)
    out = host(got)
    want, _, _ = oracle_out(x, rows, k, q, scales, n)
    want = want.reshape(rows, n)
    for r in range(rows):
        row = out[r * stride:r * stride + n]
        assert np.all(row[:64] == -7) and np.all(row[192:] == -7)
        assert np.array_equal(row[64:192].view(np.uint32), want[r, 64:192].view(np.uint32))
        if r + 1 < rows:
            assert np.all(out[r * stride + n:(r + 1) * stride] == -7)


def test_pack_range_with_host_row_scales_matches_fused_pack():
    rows, k, n = 6, 300, 70
    w, q, scales = int8_fixture(k, n, 11)
    x = activations(rows, k, 5)
    dx = dev(x)
    fused = gphq.WorkspaceI8(k, rows)
    fused.pack(dx, rows, k)
    a = fill(rows * n)
    gphq.mul_panels_i8(a, n, fused, w, 0, w.panels())
    split = gphq.WorkspaceI8(k, rows)
    split.prepare(rows, k)
    for r in range(rows):
        split.set_row_scale(r, orc.max_abs(x[r * k:(r + 1) * k]))
    for k0 in range(0, k, 52):  # multiples of 4; the last range ends at k
        split.pack_range(dx, k, k0, min(k, k0 + 52))
    b = fill(rows * n, -1.0)
    gphq.mul_panels_i8(b, n, split, w, 0, w.panels())
    assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32))


def test_set_row_scale_after_fused_pack_keeps_other_rows():
    # After a fused Pack (scales computed on the device), SetRowScale on one
    # row and a PackRange re-quantize that row only: the other rows keep the
    # scales Pack gave them (WorkspaceI8 keeps per-row state, int8.go:106-163).
    rows, k, n = 5, 256, 80
    w, q, scales = int8_fixture(k, n, 12)
    x = activations(rows, k, 6)
    dx = dev(x)
    ws = gphq.WorkspaceI8(k, rows)
    ws.pack(dx, rows, k)
    a = fill(rows * n)
    gphq.mul_panels_i8(a, n, ws, w, 0, w.panels())
    ws.set_row_scale(2, 2 * orc.max_abs(x[2 * k:3 * k]))
    ws.pack_range(dx, k, 0, k)
    b = fill(rows * n, -1.0)
    gphq.mul_panels_i8(b, n, ws, w, 0, w.panels())
    ha, hb = host(a).reshape(rows, n), host(b).reshape(rows, n)
    for r in (0, 1, 3, 4):
        assert np.array_equal(ha[r].view(np.uint32), hb[r].view(np.uint32)), r
    # Row 2 now uses the doubled scale: bit-equal to the oracle's quantizer
    # and product with that scale (int8.go:106-119, 163-168, 200-211).
    s2, inv2 = orc.i8_row_scale(np.float32(2 * orc.max_abs(x[2 * k:3 * k])))
    q2 = np.array([orc.i8_quantize(np.float32(v) * inv2) for v in x[2 * k:3 * k]], dtype=np.int8)
    want = orc.i8_mul_panels(q2.reshape(1, k), np.array([s2], np.float32), q, scales, k, n)
    assert np.array_equal(hb[2].view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(hb[2], ha[2])


def test_non_finite_rows_and_extremes():
    # NaN / Inf rows get scale 0 (int8.go:106-112); tiny and huge rows keep exact semantics.
    k, n = 96, 40
    w, q, scales = int8_fixture(k, n, 2)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, k)).astype(np.float32)
    x[0, 5] = np.nan
    x[1, 7] = np.inf
    x[2] *= np.float32(1e-38)  # max near the subnormal range
    x[3] *= np.float32(3e37)
    x[4] = 0
    x[5, ::2] = np.float32(2.5)  # ties at the rounding boundary after scaling
    got, _ = run_gpu(x.ravel(), 6, k, w, n)
    want, rs, _ = oracle_out(x.ravel(), 6, k, q, scales, n)
    assert rs[0] == 0 and rs[1] == 0 and rs[4] == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,k,stride", [(3, 16384, 16384), (4, 1024, 1028), (5, 992, 1000), (3, 1000, 1003),
                                           (2, 16, 20)])
def test_pack_row_stride_and_wide_rows(rows, k, stride):
    # Pack with a row stride, from K = 16 to 16384 (rows held in registers
    # where K is a multiple of 16 and rows are 16-byte aligned, the two-pass
    # quantizer otherwise), an infinite value in one row: the same bytes and
    # products as the oracle's quantizer.
    n = 40
    w, q, scales = int8_fixture(k, n, 4)
    rng = np.random.default_rng(k + stride)
    x = rng.standard_normal((rows - 1) * stride + k).astype(np.float32)
    x[stride + 3] = np.inf
    ws = gphq.WorkspaceI8(k, rows)
    ws.pack(dev(x), rows, k, stride=stride)
    got = fill(rows * n)
    gphq.mul_panels_i8(got, n, ws, w, 0, w.panels())
    xs = np.concatenate([x[r * stride:r * stride + k] for r in range(rows)])
    want, rs, _ = oracle_out(xs, rows, k, q, scales, n)
    assert rs[1] == 0
    assert np.array_equal(host(got).view(np.uint32), want.view(np.uint32))


def test_k_zero_clears_and_errors_match_reference():
    w = gphq.WeightsI8(0, 70)
    w.pack(np.zeros(0, np.int8), np.ones(70, np.float32))
    ws = gphq.WorkspaceI8(0, 4)
    ws.prepare(3, 0)
    dst = fill(3 * 70)
    gphq.mul_panels_i8(dst, 70, ws, w, 0, w.panels())
    out = host(dst)
    assert np.all(out == 0) and not np.any(np.signbit(out))
    # ws.k != w.k, bad panel ranges, short dst, non-finite weight scale.
    w2 = gphq.WeightsI8(64, 70)
    with pytest.raises(gphq.GphqError, match="invalid dimensions"):
        gphq.mul_panels_i8(dst, 70, ws, w2, 0, 1)
    ws2 = gphq.WorkspaceI8(64, 4)
    ws2.prepare(3, 64)
    with pytest.raises(gphq.GphqError, match="invalid dimensions"):
        gphq.mul_panels_i8(dst, 70, ws2, w2, 0, 3)
    with pytest.raises(gphq.GphqError, match="invalid dimensions"):
        gphq.mul_panels_i8(fill(10), 70, ws2, w2, 0, 1)
    with pytest.raises(gphq.GphqError, match="non-finite"):
        w2.pack(np.zeros(64 * 70, np.int8), np.full(70, np.nan, np.float32))
    with pytest.raises(gphq.GphqError, match="invalid dimensions"):
        ws2.prepare(5, 64)  # beyond the row capacity


def test_pack_rows_in_chunks_matches_pack():
    k, n = 130, 100
    rng = np.random.default_rng(4)
    q = rng.integers(-127, 128, k * n).astype(np.int8)
    scales = rng.random(n).astype(np.float32)
    whole = gphq.WeightsI8(k, n)
    whole.pack(q, scales)
    chunks = gphq.WeightsI8(k, n)
    for r0 in range(0, n, 30):  # chunks that split 16-row tiles
        r1 = min(n, r0 + 30)
        chunks.pack_rows(q[r0 * k:r1 * k], scales[r0:r1], r0)
    x = activations(4, k, 9)
    a, _ = run_gpu(x, 4, k, whole, n)
    b, _ = run_gpu(x, 4, k, chunks, n)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
