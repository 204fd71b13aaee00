"""GPU parity of the qwen3lm mm GEMM (Q8 / Q8B / Q4 with FP16 tiles) and of
the group-128 zero-point int4 variant, through the C ABI.

Reference semantics (gpu.metal:766-927): each K step's weights are FP16
(Q8 exact, Q8B half(code)*half(d), Q4 (half(nib)-8)*d), activations half(x),
fp32 accumulation. The oracle computes the same FP16 operands with float64
sums; the GPU may differ only by fp32 summation rounding, bounded by
K * 2^-23 * sum|a w| per output. The int4 variant is also held to the
relative 2e-3 against the un-rounded dequantized
weights (q - z) * s in float64.
"""
import numpy as np
import pytest

from gophonic_amd import gphq
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_mm(fmt, codes, scales, x, m, k, n, zeros=None, split=False):
    import torch

    nb = gphq.mm_split_workspace_bytes(m, k, n) if split else gphq.mm_workspace_bytes(m, k)
    work = torch.empty(max(1, nb), dtype=torch.uint8, device="cuda")
    y = torch.full((m * n,), float("nan"), device="cuda")
    gphq.mm(fmt, dev(codes), dev(scales), dev(x), y, m, k, n, work, zeros=None if zeros is None else dev(zeros))
    return host(y).reshape(m, n)


def weights(fmt, rng, n, k):
    if fmt == orc.FMT_Q8:
        return rng.integers(-127, 128, n * k).astype(np.int8), (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float32), None
    if fmt == orc.FMT_Q8B:
        return (rng.integers(-127, 128, n * k).astype(np.int8),
                (np.abs(rng.standard_normal(n * k // 32)) * 0.02).astype(np.float16).view(np.uint16), None)
    if fmt == orc.FMT_Q8B_F32:
        return (rng.integers(-127, 128, n * k).astype(np.int8),
                (np.abs(rng.standard_normal(n * k // 32)) * 0.02).astype(np.float32), None)
    if fmt == orc.FMT_Q4:
        return (rng.integers(0, 256, n * k // 2).astype(np.uint8),
                (np.abs(rng.standard_normal(n * k // 32)) * 0.02).astype(np.float16).view(np.uint16), None)
    # GPTQ4_G128: nibbles U[0,15] 8 per int32, fp16 scales |N|*0.01, zero points U[0,15].
    return (rng.integers(0, 2 ** 32, n * k // 8, dtype=np.uint64).astype(np.uint32),
            (np.abs(rng.standard_normal(n * k // 128)) * 0.01).astype(np.float16).view(np.uint16),
            rng.integers(0, 16, n * k // 128).astype(np.uint8))


FORMATS = [orc.FMT_Q8, orc.FMT_Q8B, orc.FMT_Q8B_F32, orc.FMT_Q4, orc.FMT_GPTQ4_G128]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("m,k,n", [(1, 128, 16), (3, 256, 50), (16, 512, 64), (17, 384, 100), (64, 1024, 96),
                                   (100, 640, 130), (33, 4096, 48)])
def test_mm_matches_fp16_tile_oracle(fmt, m, k, n):
    rng = np.random.default_rng(fmt * 7919 + m * 31 + k + n)
    codes, scales, zeros = weights(fmt, rng, n, k)
    x = rng.standard_normal(m * k).astype(np.float32)
    got = run_mm(fmt, codes, scales, x, m, k, n, zeros)
    want, absum = orc.mm_f64(fmt, codes, scales, x, m, k, n, zeros=zeros)
    assert np.isfinite(got).all()
    assert np.all(np.abs(got - want) <= k * 2.0 ** -23 * absum + 1e-30)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("m,k,n", [(100, 640, 130), (65, 4096, 200), (256, 4096, 512), (128, 12288, 256),
                                   (300, 1024, 1000)])
def test_mm_split_k_matches_fp16_tile_oracle(fmt, m, k, n):
    # With the split workspace, grids under 256 blocks split K; the splits are
    # added in order by a second kernel, so the bound is the unsplit one.
    rng = np.random.default_rng(fmt * 131 + m + k + n)
    codes, scales, zeros = weights(fmt, rng, n, k)
    x = rng.standard_normal(m * k).astype(np.float32)
    got = run_mm(fmt, codes, scales, x, m, k, n, zeros, split=True)
    want, absum = orc.mm_f64(fmt, codes, scales, x, m, k, n, zeros=zeros)
    assert np.isfinite(got).all()
    assert np.all(np.abs(got - want) <= k * 2.0 ** -23 * absum + 1e-30)
    again = run_mm(fmt, codes, scales, x, m, k, n, zeros, split=True)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))  # deterministic


def test_gptq_256_row_tiles_with_two_splits():
    # 129..256 rows over at least 96 column tiles: GPTQ takes 256 x 128 tiles
    # with two K splits; every output against the FP16-tile oracle, twice.
    m, k, n = 200, 512, 12288
    fmt = orc.FMT_GPTQ4_G128
    rng = np.random.default_rng(17)
    codes, scales, zeros = weights(fmt, rng, n, k)
    x = rng.standard_normal(m * k).astype(np.float32)
    got = run_mm(fmt, codes, scales, x, m, k, n, zeros, split=True)
    want, absum = orc.mm_f64(fmt, codes, scales, x, m, k, n, zeros=zeros)
    assert np.isfinite(got).all()
    assert np.all(np.abs(got - want) <= k * 2.0 ** -23 * absum + 1e-30)
    again = run_mm(fmt, codes, scales, x, m, k, n, zeros, split=True)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    # Each split is the unsplit product over its half of K (one K loop in the
    # same order), and the finish kernel's outputs are their fp32 sum, first
    # half + second.
    h = k // 2
    c2, s2, z2 = codes.reshape(n, k // 8), scales.reshape(n, k // 128), zeros.reshape(n, k // 128)
    x2 = x.reshape(m, k)
    halves = [run_mm(fmt, np.ascontiguousarray(c2[:, i * h // 8:(i + 1) * h // 8]).ravel(),
                     np.ascontiguousarray(s2[:, i * h // 128:(i + 1) * h // 128]).ravel(),
                     np.ascontiguousarray(x2[:, i * h:(i + 1) * h]).ravel(), m, h, n,
                     np.ascontiguousarray(z2[:, i * h // 128:(i + 1) * h // 128]).ravel()) for i in range(2)]
    assert np.array_equal(got.view(np.uint32), (halves[0] + halves[1]).view(np.uint32))


@pytest.mark.parametrize("k,n", [(2048, 37), (4096, 101), (6144, 9), (8192, 45), (12288, 77), (16384, 13),
                                 (4096, 1), (12288, 8)])
def test_gptq_one_row_every_k_step(k, n):
    # gphq_mm at m = 1 takes the GEMV for K a multiple of 2048 up to 16384, one
    # launch shape per K; row counts that do not fill the last row group must
    # not be written past N (the output is NaN-filled) and equal the float64
    # value with un-rounded weights within 1e-4 relative.
    rng = np.random.default_rng(k + n)
    codes, scales, zeros = weights(orc.FMT_GPTQ4_G128, rng, n, k)
    x = rng.standard_normal(k).astype(np.float16).astype(np.float32)
    got = run_mm(orc.FMT_GPTQ4_G128, codes, scales, x, 1, k, n, zeros)
    q = ((codes.reshape(n, k // 8)[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(n, k)
    z = np.repeat(zeros.reshape(n, k // 128).astype(np.float64), 128, axis=1)
    s = np.repeat(scales.reshape(n, k // 128).view(np.float16).astype(np.float64), 128, axis=1)
    ref = ((q.astype(np.float64) - z) * s) @ x.astype(np.float64)
    assert np.isfinite(got).all()
    rel = np.sqrt(((got[0] - ref) ** 2).sum() / (ref ** 2).sum())
    assert rel <= 1e-4


@pytest.mark.parametrize("m,split", [(1, False), (256, False), (256, True)])
@pytest.mark.parametrize("k,n", [(4096, 12288), (12288, 4096)])
def test_gptq_g128_config5_within_2e3(m, split, k, n):
    # Benchmark config 5 shapes. The north-star tolerance (2e-3 relative) is
    # checked against float64 with un-rounded weights on a sample of columns;
    # the FP16-tile oracle bounds the same sample tightly.
    rng = np.random.default_rng(m + k)
    codes, scales, zeros = weights(orc.FMT_GPTQ4_G128, rng, n, k)
    x = rng.standard_normal(m * k).astype(np.float16).astype(np.float32)  # fp16 activations
    got = run_mm(orc.FMT_GPTQ4_G128, codes, scales, x, m, k, n, zeros, split=split)
    cols = np.sort(rng.choice(n, 48, replace=False))
    rows = np.arange(m) if m <= 8 else np.sort(rng.choice(m, 8, replace=False))
    sub_codes = codes.reshape(n, k // 8)[cols]
    sub_scales = scales.reshape(n, k // 128)[cols]
    sub_zeros = zeros.reshape(n, k // 128)[cols]
    sub_x = x.reshape(m, k)[rows]
    want, absum = orc.mm_f64(orc.FMT_GPTQ4_G128, sub_codes, sub_scales, sub_x, len(rows), k, len(cols), zeros=sub_zeros)
    g = got[np.ix_(rows, cols)]
    # Un-rounded float64 reference.
    q = ((sub_codes[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(len(cols), k).astype(np.float64)
    z = np.repeat(sub_zeros.astype(np.float64), 128, axis=1)
    s = np.repeat(sub_scales.view(np.float16).astype(np.float64), 128, axis=1)
    ref = sub_x.astype(np.float64) @ ((q - z) * s).T
    rel = np.sqrt(((g - ref) ** 2).sum() / (ref ** 2).sum())
    assert rel <= 2e-3
    if m == 1:
        # The GEMV path keeps the weights un-rounded (fp32 sums of exact
        # products of (1024 + q) and half(x), then s * (dot - (1024 + z) * sum)):
        # far inside the tolerance against the un-rounded value.
        assert rel <= 1e-4
    else:
        # The mm path rounds each dequantized weight to FP16 (as the reference's
        # mm kernel does): the FP16-tile oracle bounds it tightly.
        assert np.all(np.abs(g - want) <= k * 2.0 ** -23 * absum + 1e-30)


def test_mm_rejects_bad_shapes():
    import torch

    t = torch.zeros(4096, device="cuda")
    work = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    with pytest.raises(gphq.GphqError):
        gphq.mm(orc.FMT_Q8B, t, t, t, t, 1, 48, 4, work)  # K % 32
    with pytest.raises(gphq.GphqError):
        gphq.mm(orc.FMT_GPTQ4_G128, t, t, t, t, 1, 64, 4, work, zeros=t)  # K % 128
    with pytest.raises(gphq.GphqError):
        gphq.mm(orc.FMT_Q8B, t, t, t, t, 64, 4096, 4, work)  # workspace too small
    with pytest.raises(gphq.GphqError):
        gphq.mm(3, t, t, t, t, 1, 64, 4, work)
