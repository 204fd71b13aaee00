"""Pins the CPU oracle (oracle/gphq_oracle.c) independently of itself: against
numpy's IEEE conversions and rounding, exact integer arithmetic, float64
bounds from the reference's own tests, and the committed golden fixtures.
"""
import math
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


# ---- FP16 conversion (q8gemm/gemm.go:297-341; q8gemm_test.go:189-212) -------

def test_f16_to_f32_exhaustive_matches_numpy():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    finite = ~np.isnan(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))


def test_f32_to_f16_round_trip_exhaustive():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = orc.f16_to_f32(h)
    back = orc.f32_to_f16(f)
    ok = np.isnan(f) | (back == h)
    assert ok.all()


def test_f32_to_f16_matches_numpy_nearest_even():
    rng = np.random.default_rng(3)
    # Every float16 value, its float32 neighbours and the exact midpoints
    # between consecutive float16 values, plus random magnitudes 2^-30..2^20.
    h = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16)
    base = h.view(np.float16).astype(np.float32)
    nxt = (h + 1).view(np.float16).astype(np.float32)
    mid = ((base.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    pts = np.concatenate([
        base, np.nextafter(base, np.float32(np.inf)), np.nextafter(base, np.float32(0)), mid,
        np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)),
        (rng.standard_normal(1_000_000) * np.exp2(rng.integers(-30, 20, 1_000_000))).astype(np.float32),
        np.array([65504, 65519.99, 65520, 1e6, np.inf, 5.96e-8, 2.98e-8, 2.99e-8, 1e-10], np.float32),
    ])
    pts = np.concatenate([pts, -pts])
    got = orc.f32_to_f16(pts)
    with np.errstate(over="ignore"):
        want = pts.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # NaN becomes the canonical quiet NaN with the input's sign.
    nan = np.array([np.nan, -np.nan], dtype=np.float32)
    nan[1] = -np.abs(nan[1])
    assert list(orc.f32_to_f16(nan)) == [0x7E00, 0xFE00]


def test_max_abs_propagates_nan_and_ignores_sign():
    assert orc.max_abs(np.array([1, -7, 3], np.float32)) == 7
    assert orc.max_abs(np.array([-0.0], np.float32)) == 0
    assert math.isnan(orc.max_abs(np.array([1, 2, np.nan] + list(range(3, 17)), np.float32)))
    assert orc.max_abs(np.zeros(0, np.float32)) == 0


# ---- q8gemv (q8gemv/scalar.go:8-17) ----------------------------------------

def test_q8gemv_known_answer_extremes():
    g = golden("q8gemv_extremes")
    got = orc.q8gemv_mul_into(g["x"], g["q"], g["scales"], int(g["k"]), int(g["n"]))
    assert np.array_equal(got.view(np.uint32), g["want"].view(np.uint32))


def test_q8gemv_nan_propagation():
    g = golden("q8gemv_nonfinite")
    got = orc.q8gemv_mul_into(g["x"], g["q"], g["scales"], int(g["k"]), int(g["n"]))
    assert np.isnan(got[0])


def test_q8gemv_k_zero_gives_signed_zero():
    got = orc.q8gemv_mul_into(np.zeros(0, np.float32), np.zeros(0, np.int8), np.array([2, -3], np.float32), 0, 2)
    assert got[0] == 0 and not np.signbit(got[0]) and np.signbit(got[1])


@pytest.mark.parametrize("k,n", [(1, 3), (17, 5), (257, 3), (4096, 3), (14336, 1)])
def test_q8gemv_within_fp32_bound_of_float64(k, n):
    rng = np.random.default_rng(k * 7 + n)
    x = ((rng.random(k, dtype=np.float32) * 2 - 1) * 4).astype(np.float32)
    q = rng.integers(-128, 128, k * n).astype(np.int8)
    s = ((rng.random(n, dtype=np.float32) * 2 - 1) * 0.1).astype(np.float32)
    for fma in (False, True):
        got = orc.q8gemv_mul_into(x, q, s, k, n, fma=fma)
        exact = (q.reshape(n, k).astype(np.float64) @ x.astype(np.float64)) * s.astype(np.float64)
        bound = (np.abs(q.reshape(n, k).astype(np.float64)) @ np.abs(x.astype(np.float64))) * np.abs(s) * k * 2.0 ** -23
        assert np.all(np.abs(got - exact) <= bound + 1e-30)
    # The two legal orders differ only by rounding.
    a = orc.q8gemv_mul_into(x, q, s, k, n)
    b = orc.q8gemv_mul_into(x, q, s, k, n, fma=True)
    assert np.allclose(a, b, rtol=1e-4, atol=1e-3)


# ---- qwen3lm block formats (gpu_darwin.go:582-658) --------------------------

def test_quantize_row_q8b_matches_projection_stream_golden():
    g = golden("q8b_stream")
    rows, cols = int(g["rows"]), int(g["cols"])
    for mi, m in enumerate(g["matrices"]):
        r = np.arange(rows)[:, None]
        c = np.arange(cols)[None, :]
        v = (((((r + int(m) * 13) * 3 + c * 7) % 101) - 50).astype(np.float32) * np.float32(0.001)).astype(np.float32)
        for row in (0, 1, rows - 1):
            q, sc = orc.quantize_row_q8b(v[row])
            assert np.array_equal(q, g["codes"][mi, row])
            assert np.array_equal(sc, g["scales"][mi, row])


def test_gemv_q8b_f64_matches_projection_stream_golden():
    g = golden("q8b_stream")
    rows, cols = int(g["rows"]), int(g["cols"])
    for mi in range(len(g["matrices"])):
        y64, _ = orc.gemv_f64(orc.FMT_Q8B, g["codes"][mi], g["scales"][mi], g["x"], cols, rows)
        assert np.allclose(y64, g["want"][mi], rtol=0, atol=1e-12)
        y = orc.gemv(orc.FMT_Q8B, g["codes"][mi], g["scales"][mi], g["x"], cols, rows)
        # gpu_projection_stream_darwin_test.go:98 tolerance.
        assert np.all(np.abs(y - g["want"][mi]) <= 1e-4 * (1 + np.abs(g["want"][mi])))


def test_gemv_q4_matches_pattern_golden():
    g = golden("q4_pattern")
    rows, k = int(g["rows"]), int(g["k"])
    y64, _ = orc.gemv_f64(orc.FMT_Q4, g["codes"], g["scales"], g["x"], k, rows)
    assert np.allclose(y64, g["want"], rtol=0, atol=1e-12)
    y = orc.gemv(orc.FMT_Q4, g["codes"], g["scales"], g["x"], k, rows)
    rel = np.sqrt(((y - g["want"]) ** 2).sum() / (g["want"] ** 2).sum())
    assert rel <= 1e-5  # gpu_darwin_test.go:94


def test_quantize_row_q8_properties():
    rng = np.random.default_rng(5)
    row = rng.standard_normal(4096).astype(np.float32)
    q, s = orc.quantize_row_q8(row)
    assert s == np.float32(np.abs(row).max()) / np.float32(127)
    want = np.clip(np.rint((row / s).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(q, want)
    q0, s0 = orc.quantize_row_q8(np.zeros(64, np.float32))
    assert s0 == 0 and not q0.any()


def test_quantize_row_q4_search_is_optimal_among_candidates():
    rng = np.random.default_rng(9)
    row = (rng.standard_normal(32 * 64) * 0.02).astype(np.float32)
    row[5] = 0.3  # an outlier block
    codes, sc = orc.quantize_row_q4(row)
    d = sc.view(np.float16).astype(np.float32)
    for b in range(64):
        v = row[b * 32:(b + 1) * 32].astype(np.float64)
        # Decode the chosen codes (split nibbles, stored +8).
        by = codes[b * 16:(b + 1) * 16]
        qv = np.concatenate([(by & 15).astype(np.int64), (by >> 4).astype(np.int64)]) - 8
        err = ((v - qv * float(d[b])) ** 2).sum()
        # Brute force over the 16 candidate scales in float64.
        peak = v[np.argmax(np.abs(v))]
        best = np.inf
        for step in range(16):
            cand = float(np.float32(np.float32(peak) / np.float32(-8) * (np.float32(1) - np.float32(0.02) * np.float32(step))))
            cand = float(np.float16(cand))
            if cand == 0:
                continue
            qq = np.clip(np.rint((v.astype(np.float32) / np.float32(cand)).astype(np.float32)), -8, 7)
            best = min(best, ((v - qq * cand) ** 2).sum())
        assert err <= best * (1 + 1e-5) + 1e-12
        # q4GroupScale (float64 error) picks a scale at least as good.
        g = float(orc.q4_group_scale(row[b * 32:(b + 1) * 32]))
        qg = np.clip(np.rint((v.astype(np.float32) / np.float32(g)).astype(np.float32)), -8, 7)
        assert ((v - qg * g) ** 2).sum() <= best * (1 + 1e-9) + 1e-15


# ---- q8gemm F16 path (gemm.go, packed.go, scalar.go) ------------------------

def test_f16_row_scale_places_max_in_2_14_2_15():
    for m in [1e-30, 3e-7, 0.5, 1.0, 1.5, 7.0, 65504.0, 1e6, 3e30]:
        s, inv = orc.f16_row_scale(np.float32(m))
        e = 15 - math.frexp(float(np.float32(m)))[1]
        e = min(max(e, -100), 100)
        assert s == np.float32(2.0 ** e) and inv == np.float32(2.0 ** -e)
        if -100 < 15 - math.frexp(float(np.float32(m)))[1] < 100:
            assert 2 ** 14 <= float(np.float32(m)) * float(s) < 2 ** 15
    for m in [0.0, np.inf, np.nan]:
        assert orc.f16_row_scale(np.float32(m)) == (1.0, 1.0)


def test_f16_pack_rows_matches_numpy_conversion():
    rng = np.random.default_rng(5)
    rows, k = 5, 100
    x = (rng.standard_normal(rows * k) * np.exp2(rng.integers(-15, 15, rows * k))).astype(np.float32)
    x[17] = 7e5
    h, s, inv = orc.f16_pack_rows(x, rows, k)
    for r in range(rows):
        want = (x[r * k:(r + 1) * k] * s[r]).astype(np.float16).view(np.uint16)
        assert np.array_equal(h[r], want)


def test_pack_bf16_matches_golden():
    g = golden("f16_buffer")
    for k, n in [(3, 65), (32, 129)]:
        h, sc, rounded = orc.pack_bf16_rows(g[f"bf16_{k}_{n}"], k, n)
        assert rounded == 0
        assert np.array_equal(h, g[f"h_{k}_{n}"])
        assert np.array_equal(sc, g[f"scales_{k}_{n}"])


def test_pack_bf16_rejects_non_finite():
    bf = np.array([0x3F80, 0x7F80, 0x3F80, 0x3F80], np.uint16)  # 1, +Inf, 1, 1
    assert orc.pack_bf16_rows(bf, 2, 2) is None


@pytest.mark.parametrize("rows,k,n", [(1, 7, 5), (12, 65, 129), (16, 257, 67), (3, 96, 64)])
def test_mul_panels_within_reference_bound(rows, k, n):
    # q8gemm_test.go:63-87 checkShape bound: (1/2048 + 1e-5) * sum|x w| * scale + 1e-6.
    rng = np.random.default_rng(rows * 100 + k * 10 + n)
    q = rng.integers(-127, 128, k * n).astype(np.int8).reshape(n, k)
    scales = (rng.integers(1, 101, n) / 1000).astype(np.float32)
    x = (rng.random(rows * k, dtype=np.float32) * 2 - 1).astype(np.float32)
    h, s, inv = orc.f16_pack_rows(x, rows, k)
    got = orc.mul_panels(h, inv, q, scales, k, n).reshape(rows, n)
    xv = x.reshape(rows, k).astype(np.float64)
    exact = (xv @ q.T.astype(np.float64)) * scales.astype(np.float64)
    bound = 1e-6 + (1 / 2048 + 1e-5) * (np.abs(xv) @ np.abs(q.T.astype(np.float64))) * scales
    assert np.all(np.abs(got - exact) <= bound)


def test_pack_panels_layout_round_trip():
    # packed.go:233-239 at(): index = (row/64)*pairs*128 + (k/2)*128 + (row%64)*2 + k%2.
    k, n = 7, 130
    src = np.arange(n * k, dtype=np.uint32).astype(np.uint16).reshape(n, k) + 1
    out = orc.pack_panels(src, k, n)
    pairs = (k + 1) // 2
    for row in range(n):
        for kk in range(k):
            assert out[(row // 64) * pairs * 128 + (kk // 2) * 128 + (row % 64) * 2 + kk % 2] == src[row, kk]
    assert np.count_nonzero(out) == n * k  # everything else is zero padding


# ---- q8gemm int8 path (int8.go) --------------------------------------------

def test_i8_quantize_matches_numpy_and_saturates():
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(100000) * 100).astype(np.float32)
    v = np.concatenate([v, np.array([0.5, 1.5, 2.5, -0.5, -2.5, 127.5, -128.5, 300, -300, np.inf, -np.inf], np.float32)])
    got = orc.i8_quantize_array(v)
    want = np.clip(np.rint(v), -128, 127).astype(np.int8)
    assert np.array_equal(got, want)
    assert orc.i8_quantize(np.float32(np.nan)) == 0


def test_i8_row_scale():
    assert orc.i8_row_scale(np.float32(127)) == (1.0, 1.0)
    s, inv = orc.i8_row_scale(np.float32(3.7))
    assert s == np.float32(3.7) / np.float32(127) and inv == np.float32(127) / np.float32(3.7)
    for m in [0.0, np.inf, np.nan]:
        assert orc.i8_row_scale(np.float32(m)) == (0.0, 0.0)


def test_i8_golden_tile_bit_exact():
    g = golden("i8_tile")
    rows, k = g["x"].shape
    n = g["w"].shape[0]
    qa, rs, inv = orc.i8_pack_rows(g["x"], rows, k)
    assert np.array_equal(qa, g["qa"])
    assert np.array_equal(rs, g["row_scale"])
    got = orc.i8_mul_panels(qa, rs, g["w"], g["scales"], k, n).reshape(rows, n)
    assert np.array_equal(got.view(np.uint32), g["want"].view(np.uint32))


@pytest.mark.parametrize("rows,k,n", [(1, 4, 1), (3, 7, 17), (12, 64, 64), (16, 257, 129), (5, 1000, 64)])
def test_i8_mul_panels_exact_integer_and_bound(rows, k, n):
    rng = np.random.default_rng(k * 31 + n)
    w = rng.integers(-127, 128, n * k).astype(np.int8).reshape(n, k)
    scales = (rng.integers(1, 101, n) / 997).astype(np.float32)
    x = (rng.standard_normal(rows * k) * (1 + np.arange(rows * k) % 5)).astype(np.float32)
    x[0] = 0
    qa, rs, inv = orc.i8_pack_rows(x, rows, k)
    got = orc.i8_mul_panels(qa, rs, w, scales, k, n).reshape(rows, n)
    acc = qa.astype(np.int64) @ w.astype(np.int64).T
    want = (acc.astype(np.float32) * scales[None, :]).astype(np.float32) * rs[:, None]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    # int8_test.go:83-96: error vs float64 is at most half a step per element.
    xv = x.reshape(rows, k).astype(np.float64)
    wv = w.astype(np.float64) * scales[:, None].astype(np.float64)
    exact = xv @ wv.T
    bound = 0.5 * rs[:, None].astype(np.float64) * np.abs(wv).sum(axis=1)[None, :]
    assert np.all(np.abs(got - exact) <= bound * 1.001 + 1e-4)
    # Panel splits give identical bits (int8_test.go:146-179 invariant).
    split = np.zeros(rows * n, np.float32)
    for p in range((n + 63) // 64):
        orc.i8_mul_panels(qa, rs, w, scales, k, n, p0=p, p1=p + 1, dst=split)
    assert np.array_equal(split.view(np.uint32), got.ravel().view(np.uint32))


def test_i8_multithreaded_matches_single():
    rng = np.random.default_rng(1)
    rows, k, n = 4, 128, 300
    w = rng.integers(-127, 128, n * k).astype(np.int8).reshape(n, k)
    scales = rng.random(n).astype(np.float32)
    qa = rng.integers(-128, 128, rows * k).astype(np.int8).reshape(rows, k)
    rs = rng.random(rows).astype(np.float32)
    a = orc.i8_mul_panels(qa, rs, w, scales, k, n)
    b = orc.i8_mul_panels(qa, rs, w, scales, k, n, threads=3)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_pack_panels_quads_layout():
    k, n = 9, 70
    src = (np.arange(n * k) % 120 + 1).astype(np.int8).reshape(n, k)
    out = orc.pack_panels_quads(src, k, n)
    quads = (k + 3) // 4
    for row in range(n):
        for kk in range(k):
            assert out[(row // 64) * quads * 256 + (kk // 4) * 256 + (row % 64) * 4 + kk % 4] == src[row, kk]
    assert np.count_nonzero(out) == n * k


@pytest.mark.parametrize("fmt", [orc.FMT_Q8, orc.FMT_Q8B, orc.FMT_Q8B_F32, orc.FMT_Q4, orc.FMT_GPTQ4_G128])
def test_mm_f64_matches_numpy_fp16_tiles(fmt):
    """The mm oracle's FP16 operands (gpu.metal:836-861 tile dequantization,
    activations half(x)) rebuilt with numpy's float16 rounding and nibble
    unpacking, summed in float64."""
    rng = np.random.default_rng(fmt)
    m, k, n = 3, 256, 5
    x = rng.standard_normal(m * k).astype(np.float32)
    # Values chosen so the fp16 rounding matters: scales with full fp32 / fp16 mantissas.
    if fmt == orc.FMT_Q4:
        codes = rng.integers(0, 256, n * k // 2).astype(np.uint8)
        sc = (np.abs(rng.standard_normal(n * k // 32)) * 0.02).astype(np.float16)
        b = codes.reshape(n, k // 32, 16)
        q = np.concatenate([b & 15, b >> 4], axis=2).astype(np.float32) - 8
        w = (q * sc.astype(np.float32).reshape(n, k // 32, 1)).astype(np.float16).reshape(n, k)
        scales = sc.view(np.uint16)
    elif fmt == orc.FMT_GPTQ4_G128:
        codes = rng.integers(0, 2 ** 32, n * k // 8, dtype=np.uint64).astype(np.uint32)
        sc = (np.abs(rng.standard_normal(n * k // 128)) * 0.01).astype(np.float16)
        zeros = rng.integers(0, 16, n * k // 128).astype(np.uint8)
        q = ((codes.reshape(n, k // 8, 1) >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(n, k).astype(np.float32)
        z = np.repeat(zeros.reshape(n, k // 128), 128, axis=1).astype(np.float32)
        w = ((q - z) * np.repeat(sc.reshape(n, k // 128), 128, axis=1).astype(np.float32)).astype(np.float16)
        scales = sc.view(np.uint16)
    else:
        codes = rng.integers(-127, 128, n * k).astype(np.int8)
        c = codes.reshape(n, k).astype(np.float32)
        if fmt == orc.FMT_Q8:
            scales = (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float32)
            w = c.astype(np.float16)
        elif fmt == orc.FMT_Q8B:
            sc = (np.abs(rng.standard_normal(n * k // 32)) * 0.02).astype(np.float16)
            w = (c * np.repeat(sc.reshape(n, k // 32), 32, axis=1).astype(np.float32)).astype(np.float16)
            scales = sc.view(np.uint16)
        else:
            scales = (np.abs(rng.standard_normal(n * k // 32)) * 0.02).astype(np.float32)
            hs = scales.astype(np.float16).astype(np.float32)
            w = (c * np.repeat(hs.reshape(n, k // 32), 32, axis=1)).astype(np.float16)
    xh = x.astype(np.float16).astype(np.float64).reshape(m, k)
    want = xh @ w.astype(np.float64).T
    if fmt == orc.FMT_Q8:
        want = want * scales.astype(np.float64)[None, :]
    got, absum = orc.mm_f64(fmt, codes, scales, x, m, k, n, zeros=zeros if fmt == orc.FMT_GPTQ4_G128 else None)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    assert np.all(absum >= np.abs(got) * (1 - 1e-12))
