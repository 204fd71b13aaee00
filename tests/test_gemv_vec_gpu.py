"""GPU parity of the multi-vector GEMV (gphq_gemv_vec, the qwen3lm
gemvQ8BVector<V> contract): every lane agrees with the serial GEMV within the
reference's vector-vs-serial bound, max_abs <= 1e-4 and relative L2 <= 1e-5
(gpu_vector_batch_darwin_test.go:217-220, metric 338-361), and with float64
to relative L2 <= 1e-5.
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


def vector_error(want, got):
    want = np.asarray(want, np.float64)
    got = np.asarray(got, np.float64)
    finite = np.isfinite(want).all() and np.isfinite(got).all()
    d = want - got
    w2 = (want ** 2).sum()
    rel = np.sqrt((d ** 2).sum() / w2) if w2 else np.sqrt((d ** 2).sum())
    return np.abs(d).max(), rel, finite


def run_vec(fmt, codes, scales, x, lanes, k, n, x_stride=None, y_stride=None):
    import torch

    x_stride = k if x_stride is None else x_stride
    y_stride = n if y_stride is None else y_stride
    work = torch.empty(gphq.gemv_vec_workspace_bytes(lanes, k), dtype=torch.uint8, device="cuda")
    y = torch.full(((lanes - 1) * y_stride + n,), -7.0, device="cuda")
    gphq.gemv_vec(fmt, dev(codes), dev(scales), dev(x), y, lanes, k, n, work, x_stride=x_stride, y_stride=y_stride)
    return host(y)


def run_serial(fmt, codes, scales, x, k, n):
    import torch

    y = torch.empty(n, device="cuda")
    gphq.gemv(fmt, dev(codes), dev(scales), dev(x), y, k, n)
    return host(y)


@pytest.mark.parametrize("lanes", [1, 2, 4, 8, 16])
def test_reference_shape_vector_matches_serial(lanes):
    # gpu_vector_batch_darwin_test.go:57-110: k = 2048, n = 128, Q8B weights from
    # quantizeRowQ8B of N(0,1)*0.02 rows.
    k, n = 2048, 128
    rng = np.random.default_rng(311 * 821 + lanes)
    codes = np.zeros((n, k), np.int8)
    scales = np.zeros((n, k // 32), np.uint16)
    for r in range(n):
        codes[r], scales[r] = orc.quantize_row_q8b((rng.standard_normal(k) * 0.02).astype(np.float32))
    x = rng.standard_normal(lanes * k).astype(np.float32)
    got = run_vec(orc.FMT_Q8B, codes, scales, x, lanes, k, n).reshape(lanes, n)
    for v in range(lanes):
        want = run_serial(orc.FMT_Q8B, codes, scales, x[v * k:(v + 1) * k], k, n)
        max_abs, rel, finite = vector_error(want, got[v])
        assert finite and max_abs <= 1e-4 and rel <= 1e-5, (v, max_abs, rel)


def make_weights(fmt, rng, n, k):
    if fmt == orc.FMT_Q4:
        return rng.integers(0, 256, n * k // 2).astype(np.uint8), (np.abs(rng.standard_normal(n * k // 32)) * 0.01).astype(np.float16).view(np.uint16)
    codes = rng.integers(-127, 128, n * k).astype(np.int8)
    if fmt == orc.FMT_Q8B:
        return codes, (np.abs(rng.standard_normal(n * k // 32)) * 0.01).astype(np.float16).view(np.uint16)
    if fmt == orc.FMT_Q8B_F32:
        return codes, (np.abs(rng.standard_normal(n * k // 32)) * 0.01).astype(np.float32)
    return codes, (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float32)


@pytest.mark.parametrize("fmt", [orc.FMT_Q8, orc.FMT_Q8B, orc.FMT_Q8B_F32, orc.FMT_Q4])
@pytest.mark.parametrize("lanes", [1, 3, 8, 16, 32])
@pytest.mark.parametrize("k,n", [(1024, 80), (4096, 4096)])
def test_formats_lanes_against_float64_and_serial(fmt, lanes, k, n):
    rng = np.random.default_rng(fmt * 101 + lanes + k)
    codes, scales = make_weights(fmt, rng, n, k)
    x = rng.standard_normal(lanes * k).astype(np.float32)
    # Lanes of very different magnitudes: each is scaled on its own.
    x = (x.reshape(lanes, k) * np.exp2(np.arange(lanes) % 7 * 9 - 27)[:, None]).astype(np.float32).ravel()
    got = run_vec(fmt, codes, scales, x, lanes, k, n).reshape(lanes, n)
    check = range(lanes) if lanes <= 4 else [0, lanes // 2, lanes - 1]
    for v in check:
        xv = x[v * k:(v + 1) * k]
        y64, _ = orc.gemv_f64(fmt, codes, scales, xv, k, n)
        _, rel, finite = vector_error(y64, got[v])
        assert finite and rel <= 1e-5, (v, rel)
        serial = run_serial(fmt, codes, scales, xv, k, n)
        _, rel_s, _ = vector_error(serial, got[v])
        assert rel_s <= 1e-5, (v, rel_s)


def test_strides_leave_gaps_untouched():
    k, n, lanes, xs, ys = 512, 48, 5, 600, 64
    rng = np.random.default_rng(3)
    codes, scales = make_weights(orc.FMT_Q8B, rng, n, k)
    xfull = rng.standard_normal(lanes * xs).astype(np.float32)
    got = run_vec(orc.FMT_Q8B, codes, scales, xfull, lanes, k, n, x_stride=xs, y_stride=ys)
    for v in range(lanes):
        row = got[v * ys:v * ys + n]
        want, _ = orc.gemv_f64(orc.FMT_Q8B, codes, scales, xfull[v * xs:v * xs + k], k, n)
        assert vector_error(want, row)[1] <= 1e-5
        if v + 1 < lanes:
            assert np.all(got[v * ys + n:(v + 1) * ys] == -7.0)


def test_rejects_bad_arguments():
    import torch

    t = torch.zeros(1 << 16, device="cuda")
    work = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    with pytest.raises(gphq.GphqError):
        gphq.gemv_vec(orc.FMT_Q8B, t, t, t, t, 33, 64, 8, work)  # too many lanes
    with pytest.raises(gphq.GphqError):
        gphq.gemv_vec(orc.FMT_Q8B, t, t, t, t, 2, 48, 8, work)  # K % 32
    with pytest.raises(gphq.GphqError):
        gphq.gemv_vec(orc.FMT_Q8B, t, t, t, t, 16, 4096, 8, work[:100])  # workspace too small
