"""GPU parity of the batched pass's int8 route (gphq_prefill_set_arith
GPHQ_PASS_INT8), through the C ABI.

The route is the CPU provider's int8 arithmetic (qwen3lm/ops.go:96-147,
198-215) over Q8 layers: every projection input row is quantized with
WorkspaceI8's per-row rule (int8.go:106-168) and multiplied exactly in int32
with MulPanelsI8's scaling (float32(sum) * weight scale) * row scale
(int8.go:170-211), on int8 MFMA.

* One projection (gphq_prefill_project) whose input is not normalized (O and
  down, residual add) is bit-exact: the pinned C rotation for down's input
  (orc.rotation_apply_f32, hadamard.go:51-58), the pinned C quantizer
  (orc.i8_pack_rows), exact int64 sums, float32 scaling and the float32 add.
* Normalized inputs (QKV, gate/up with SwiGLU) and whole passes are held to
  the float64 oracle with the same per-row quantization (DecodeOracle.int8).
  The device normalizes in float32, so an input value within rounding of a
  code boundary may take the neighbouring code. One flipped code k moves an
  output row by (max|x| / 127) * |W[:, k]|, relative (max/rms) / (127 sqrt(K))
  of the row: about 9e-4 at K = 1024, doubled by SwiGLU's product. Rows are
  held to relative L2 5e-3 (a flip or two) and 95% of them to 1e-5 (no
  flip: a wrong scale, order or gate/up pairing fails every row).
* Whole passes: past the first projection, inputs differ from the oracle's
  by the FP16 attention's rounding (about 1e-3 relative), and quantizing
  them turns that into code flips in a few percent of the values, as large
  as the quantization error itself. The reference holds its int8 weights to
  cosine 0.999 against float64 on its test checkpoint (qwen3lm/
  embeds_test.go:43-46, weights_test.go:117); on these random-init models
  exact int8 arithmetic alone (the oracle with int8 = True) is about that far
  from float64, since the attention output enters the O projection
  unrotated. So the last state's distance (1 - cosine) from float64 and from
  the int8 oracle is held to twice the exact int8 arithmetic's distance from
  float64; the first layer's K/V rows, whose input is the exact embedding
  rows, to the int8 oracle at the batched pass's 0.99999
  (gpu_official_darwin_test.go:86). That the route quantizes at all, and
  exactly, is what the single-projection tests and the FP16-route
  comparison below establish.
"""
import numpy as np
import pytest

from gophonic_amd import gphq
from oracle import lm_oracle as lo
from oracle import oracle as orc
from tests import lm_common as lc
from tests.test_lm_decode_gpu import _read_dev_floats, setup
from tests.test_lm_prefill_gpu import cosine, run_prefill

pytestmark = pytest.mark.gpu

COS = 0.99999


def rel_rows(want, got):
    want, got = np.asarray(want, np.float64), np.asarray(got, np.float64)
    assert np.isfinite(got).all()
    return np.linalg.norm(want - got, axis=1) / np.maximum(np.linalg.norm(want, axis=1), 1e-30)


def test_set_arith_validation():
    _, _, lm8b = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    ws = gphq.Prefill(lm8b, 16)
    assert ws.arith == gphq.PASS_FP16
    with pytest.raises(gphq.GphqError) as e:
        ws.set_arith(gphq.PASS_INT8)
    assert e.value.status == gphq.ERR_UNSUPPORTED
    assert ws.arith == gphq.PASS_FP16
    _, _, lm8 = setup(lc.GPU_SHAPE, lo.FMT_Q8, seed=5)
    ws = gphq.Prefill(lm8, 16)
    with pytest.raises(gphq.GphqError) as e:
        ws.set_arith(2)
    assert e.value.status == gphq.ERR_UNSUPPORTED
    ws.set_arith(gphq.PASS_INT8)
    assert ws.arith == gphq.PASS_INT8
    ws.set_arith(gphq.PASS_FP16)
    assert ws.arith == gphq.PASS_FP16


def _layer_weights(model, proj):
    """(codes [n][k] int8, scales [n] float32, n, k) of one projection of layer 0."""
    g = model["geom"]
    L = model["layers"][0]
    n, k, (codes, sc) = {
        0: (g.qd + 2 * g.kvd, g.hidden, L.qkv),
        1: (g.hidden, g.qd, L.o),
        2: (2 * g.inter, g.hidden, L.gu),
        3: (g.hidden, g.inter, L.down),
    }[proj]
    return np.asarray(codes, np.int8).reshape(n, k), np.asarray(sc, np.float32), n, k


@pytest.mark.parametrize("geom", [lc.GPU_SHAPE, lc.SMALL_06B], ids=["gpu_shape", "qwen3_06b"])
@pytest.mark.parametrize("proj", [1, 3])
@pytest.mark.parametrize("rows", [1, 7, 300])
def test_project_int8_residual_add_bit_exact(geom, proj, rows):
    import torch

    model, _, lm = setup(geom, lo.FMT_Q8, seed=6)
    W, sw, n, k = _layer_weights(model, proj)
    rng = np.random.default_rng(100 * proj + rows)
    x = rng.standard_normal((rows, k)).astype(np.float32) * 3
    x[rows // 2] *= 1e-30  # a tiny-scale row
    if rows > 2:
        x[1] = 0.0  # no finite positive maximum: scale 0
        x[2, 5] = np.nan  # SetRowScale(NaN): the row quantizes to zero
    if rows > 4:
        x[3, 7] = np.inf  # an infinite maximum: scale 0
        x[4] *= np.float32(1e-38)  # subnormal values: 127 / max overflows, products clamp
    y0 = rng.standard_normal((rows, n)).astype(np.float32)
    ws = gphq.Prefill(lm, max(rows, 16))
    ws.set_arith(gphq.PASS_INT8)
    xd = torch.from_numpy(x).cuda()
    yd = torch.from_numpy(y0).cuda()
    print(f"project int8 proj={proj} rows={rows} k={k} n={n}", flush=True)
    ws.project(0, proj, xd, rows, yd)
    got = yd.cpu().numpy()
    xin = x
    if proj == 3:  # Q8 down input: the intermediate rotation, in float32
        rot = lo.rotation(k)
        xin = np.stack([orc.rotation_apply_f32(row, rot) for row in x])
    qa, sa, _ = orc.i8_pack_rows(xin, rows, k)
    sums = qa.astype(np.int64) @ W.astype(np.int64).T
    assert np.abs(sums).max() < 2**31
    v = (sums.astype(np.float32) * sw[None, :]) * sa[:, None]
    want = y0 + v
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("proj", [0, 2])
@pytest.mark.parametrize("rows", [1, 64, 257])
def test_project_int8_normalized_inputs(proj, rows):
    import torch

    model, oracle, lm = setup(lc.SMALL_06B, lo.FMT_Q8, seed=6)
    W, sw, n, k = _layer_weights(model, proj)
    g = model["geom"]
    rng = np.random.default_rng(7 * proj + rows)
    x = (rng.standard_normal((rows, k)) * rng.uniform(0.01, 30, (rows, 1))).astype(np.float32)
    ws = gphq.Prefill(lm, max(rows, 16))
    ws.set_arith(gphq.PASS_INT8)
    width = n if proj == 0 else n // 2
    yd = torch.full((rows, width), 5.0, device="cuda")
    print(f"project int8 proj={proj} rows={rows}", flush=True)
    ws.project(0, proj, torch.from_numpy(x).cuda(), rows, yd)
    got = yd.cpu().numpy()
    o = lo.DecodeOracle.__new__(lo.DecodeOracle)
    o.g, o.int8 = g, True
    wq = W.astype(np.float64) * sw.astype(np.float64)[:, None]
    y = o._mm(o._norm_rows(x.astype(np.float64)), wq)
    if proj == 2:
        gate, up = y[:, 0::2], y[:, 1::2]
        y = gate / (1.0 + np.exp(-gate)) * up
    err = rel_rows(y, got)
    print(f"  max row rel {err.max():.3g}, median {np.median(err):.3g}")
    assert err.max() <= 5e-3, err.max()
    assert np.mean(err <= 1e-5) >= 0.95, np.sort(err)[-10:]


@pytest.mark.parametrize("rows", [64, 16, 1], ids=["one_pass", "passes_of_16", "one_token_passes"])
def test_prefill_int8_matches_oracle(rows):
    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(31)
    n = 45 if rows > 1 else 9
    tokens = list(rng.integers(0, g.vocab, n))
    ws = gphq.Prefill(lm, rows)
    ws.set_arith(gphq.PASS_INT8)
    kv = gphq.Prefix(lm, 64)
    got = run_prefill(ws, kv, 0, tokens, g)
    want, _ = oracle.finish_rows(oracle.prefill(oracle.new_cache(64), 0, tokens, last_only=True))
    oracle.int8 = True
    try:
        cache = oracle.new_cache(64)
        want8, _ = oracle.finish_rows(oracle.prefill(cache, 0, tokens, last_only=True))
    finally:
        oracle.int8 = False
    c, c8, e8 = cosine(want[0], got), cosine(want8[0], got), 1.0 - cosine(want[0], want8[0])
    print(f"int8 pass rows={rows}: cosine {c:.9f} to float64 (exact int8: {1 - e8:.9f}), {c8:.9f} to the int8 oracle")
    assert 1.0 - c <= 2.0 * e8 and 1.0 - c8 <= 2.0 * e8, (c, c8, e8)
    kc, vc, cap = kv.kv()
    for base, want_rows in ((kc, cache[0][0]), (vc, cache[0][1])):
        got_rows = _read_dev_floats(base, n * g.kvd).reshape(n, g.kvd)
        for r in range(n):
            assert cosine(want_rows[r], got_rows[r]) >= COS, r


def test_prefill_int8_differs_from_fp16_route():
    # The two routes quantize differently (int8 rows against FP16 tiles), so
    # their states differ by about the int8 quantization error (1 - cosine
    # near 1e-3 on this model), not bit for bit: the switch takes effect.
    import torch

    model, _, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8, seed=5)
    g = model["geom"]
    tokens = list(np.random.default_rng(3).integers(0, g.vocab, 20))
    outs = []
    for arith in (gphq.PASS_FP16, gphq.PASS_INT8):
        ws = gphq.Prefill(lm, 32)
        ws.set_arith(arith)
        kv = gphq.Prefix(lm, 32)
        outs.append(run_prefill(ws, kv, 0, tokens, g))
    assert not np.array_equal(outs[0], outs[1])
    assert cosine(outs[0], outs[1]) >= 0.995
    torch.cuda.synchronize()
