"""Pins the GPTQ producer oracle (oracle/gptq_oracle.py) without retyping it:

* inverse_factor against scipy's Cholesky of H^-1 (the unique upper factor
  with a positive diagonal, reached without the reversal trick) and the
  reference's own check H U^T U = I (gptq_linalg_test.go:14-67);
* round_rows (Cholesky form) against round_rows_obs (optimal-brain-surgeon
  updates with the downdated H^-1), which must choose the same codes;
* the reference's property that GPTQ beats round-to-nearest in output error
  on correlated inputs (gptq_linalg_test.go:72-148), for 8 and 4 bits.
"""
import numpy as np
import pytest
import scipy.linalg

from oracle import gptq_oracle as go
from oracle import oracle as orc


def spd(n, seed, rows=None):
    rng = np.random.default_rng(seed)
    rows = rows or n + 17
    x = rng.standard_normal((rows, n))
    return x.T @ x / rows + np.eye(n)


@pytest.mark.parametrize("n", [1, 7, 128, 300])
def test_inverse_factor_matches_scipy_and_inverts(n):
    h = spd(n, n)
    u = go.inverse_factor(h)
    assert np.array_equal(u, np.triu(u))
    ref = scipy.linalg.cholesky(np.linalg.inv(h), lower=False)
    assert np.allclose(u, ref, rtol=1e-9, atol=1e-12 * np.abs(ref).max())
    assert np.abs(h @ (u.T @ u) - np.eye(n)).max() <= 1e-9


def test_damp_marks_dead_channels():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((40, 6))
    x[:, 2] = 0
    h, dead = go.damp(go.hessian(x))
    assert dead.tolist() == [False, False, True, False, False, False]
    raw = x.T @ x
    mean = np.trace(raw) / 6
    assert h[2, 2] == pytest.approx(1 + 0.01 * mean)
    assert h[0, 0] == pytest.approx(raw[0, 0] + 0.01 * mean)


@pytest.mark.parametrize("bits", [8, 4])
def test_cholesky_form_equals_obs_form(bits):
    rng = np.random.default_rng(bits)
    rows, k, n = 200, 96, 6
    base = rng.standard_normal((rows, 1))
    x = base + 0.5 * rng.standard_normal((rows, k))
    h, _ = go.damp(go.hessian(x))
    w = rng.standard_normal((n, k)).astype(np.float32)
    codes, scales, _ = go.round_rows(w, go.inverse_factor(h), bits)
    q_obs = go.round_rows_obs(w, np.linalg.inv(h), bits)
    if bits == 8:
        q = codes.astype(np.int64)
    else:
        nib = codes.reshape(n, k // 32, 16)
        q = (np.concatenate([nib & 15, nib >> 4], axis=2).astype(np.int64) - 8).reshape(n, k)
    assert (q == q_obs).mean() >= 0.99  # float64 reassociation can move a code at a tie


@pytest.mark.parametrize("bits", [8, 4])
def test_gptq_beats_round_to_nearest(bits):
    rng = np.random.default_rng(56)
    rows, k, n = 512, 256, 16
    base = rng.standard_normal((rows, 1))
    x = (base + 0.5 * rng.standard_normal((rows, k))).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    h, _ = go.damp(go.hessian(x))
    _, _, g = go.round_rows(w, go.inverse_factor(h), bits)
    nearest = w.astype(np.float64).copy()
    for o in range(n):
        if bits == 8:
            s = np.float32(np.abs(w[o]).max() / np.float32(127))
            nearest[o] = np.rint(w[o] / s) * np.float64(s)
        else:
            for b in range(0, k, 32):
                d = np.float32(orc.q4_group_scale(w[o, b:b + 32]))
                nearest[o, b:b + 32] = np.clip(np.rint(w[o, b:b + 32] / d), -8, 7) * np.float64(d)
    err = lambda q: float(((x.astype(np.float64) @ (w.astype(np.float64) - q).T) ** 2).sum())
    assert err(g) < err(nearest)


# ---- the calibration pass (gptq.go:330-600) ----------------------------------

from oracle import lm_oracle as lo  # noqa: E402
from tests import lm_common as lc  # noqa: E402

CAL_G = lo.Geometry(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=96, max_pos=320)
PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
        "mlp.up_proj", "mlp.down_proj")


def cal_checkpoint(g, seed):
    """BF16 bits of a random Qwen3 checkpoint with lmtest's distributions
    (lmtest/lmtest.go:64-90), as the calibration pass reads it."""
    rng = np.random.default_rng(seed)
    bits = lambda off, sc, *shape: lc.bf16_bits((off + sc * rng.standard_normal(shape)).astype(np.float32))
    shapes = [(g.qd, g.hidden), (g.kvd, g.hidden), (g.kvd, g.hidden), (g.hidden, g.qd), (g.inter, g.hidden),
              (g.inter, g.hidden), (g.hidden, g.inter)]
    layers = []
    for _ in range(g.layers):
        layers.append(dict(proj=[bits(0, 0.1, *s) for s in shapes], attn=bits(1, 0.1, g.hidden),
                           mlp=bits(1, 0.1, g.hidden), qn=bits(1, 0.1, g.head_dim), kn=bits(1, 0.1, g.head_dim)))
    return bits(0, 1, g.vocab, g.hidden), layers


def f32(bits):
    return lo.bf16_to_f64(bits).astype(np.float32)


def test_calibration_weights_keep_each_projection_in_the_rotated_basis():
    # calibration.weights stores W.diag(norm).R_in^T, then R_out on the left:
    # for any x, W' (R_in x) = R_out (W diag(norm) x). The rotations are the
    # hidden / intermediate ones and the per-head one (hadamard.go, pinned to
    # scipy's Hadamard in tests/test_oracle_lm.py). Their scale is the float32
    # 1/sqrt(block), inexact for blocks 128 and 512, so R^T R = (1 + 3.4e-8) I
    # there (as in the reference): the bound is 1e-7 of the result.
    g = CAL_G
    embed, layers = cal_checkpoint(g, 1)
    cal = go.CalibrationOracle(g, embed, [[1, 2, 3]])
    L = layers[0]
    mats = cal.weights(L["proj"], f32(L["attn"]), f32(L["mlp"]))
    rng = np.random.default_rng(2)
    norm = {"attn": f32(L["attn"]).astype(np.float64), "mlp": f32(L["mlp"]).astype(np.float64), None: 1.0}
    for p, (nm, rin, rout) in enumerate(go._WEIGHT_SPEC):
        w = lo.bf16_to_f64(L["proj"][p]).reshape(mats[p].shape)
        x = rng.standard_normal(w.shape[1])
        got = mats[p] @ lo.rot_apply(x, cal.rot[rin])
        want = w @ (norm[nm] * x)
        if rout is not None:
            want = lo.rot_apply(want, cal.rot[rout])
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-7 * np.abs(want).max())


def test_calibration_pass_without_rounding_equals_the_batched_oracle():
    # With the rounding left out, calibration.layer is the model's forward
    # pass in the GPU basis, sequence by sequence: each sequence's residual
    # rows after every layer equal DecodeOracle.prefill of that sequence alone
    # (a fresh cache at position 0) over the same GPU-basis matrices
    # (DecodeOracle is pinned to transformers' Qwen3 in tests/test_oracle_lm.py).
    g = CAL_G
    embed, layers = cal_checkpoint(g, 3)
    rng = np.random.default_rng(4)
    seqs = [rng.integers(0, g.vocab, n).tolist() for n in (9, 1, 17)]
    cal = go.CalibrationOracle(g, embed, seqs)
    h = cal.h
    W = []
    for li, L in enumerate(layers):
        mats = cal.weights(L["proj"], f32(L["attn"]), f32(L["mlp"]))
        out = cal.layer(mats, f32(L["qn"]), f32(L["kn"]), h=h)
        h = out["residual"]
        gu = np.empty((2 * g.inter, g.hidden))
        gu[0::2], gu[1::2] = mats[4], mats[5]
        W.append(dict(qkv=np.vstack(mats[:3]), o=mats[3], gu=gu, down=mats[6],
                      qn=f32(L["qn"]).astype(np.float64), kn=f32(L["kn"]).astype(np.float64)))
        dec = lo.DecodeOracle(g, lo.FMT_Q8, [], embed, np.ones(g.hidden, np.float32),
                              (np.zeros(g.head_rows * g.hidden, np.int8),
                               np.zeros(g.head_rows * g.hidden // 32, np.uint16)))
        dec.W = list(W)
        for sl, s in zip(cal.seq_slices, seqs):
            want = dec.prefill(dec.new_cache(len(s)), 0, s)
            np.testing.assert_allclose(h[sl], want, rtol=0, atol=1e-9 * np.abs(want).max(), err_msg=f"layer {li}")


@pytest.mark.parametrize("bits", [8, 4])
def test_calibration_rounds_each_group_over_its_own_inputs(bits):
    # With rounding, each group is rounded against the inputs of the pass so
    # far (round_group over the layer's attention input, context, MLP input and
    # down input), the next projections use the rounded matrices, and GPTQ
    # beats round-to-nearest on every projection's own inputs
    # (gptq_linalg_test.go:72-148).
    g = CAL_G
    embed, layers = cal_checkpoint(g, 5)
    rng = np.random.default_rng(6)
    seqs = [rng.integers(0, g.vocab, n).tolist() for n in (40, 25)]
    cal = go.CalibrationOracle(g, embed, seqs)
    L = layers[0]
    mats = cal.weights(L["proj"], f32(L["attn"]), f32(L["mlp"]))
    out = cal.layer(mats, f32(L["qn"]), f32(L["kn"]), bits=bits)
    inputs = ["attn_input"] * 3 + ["context", "mlp_input", "mlp_input", "down_input"]
    for p in range(7):
        x = out[inputs[p]]
        codes, scales = out["rounded"][p]
        q = out["mats"][p]
        k = q.shape[1]
        if bits == 8:
            s = scales.astype(np.float64)[:, None]
            np.testing.assert_array_equal(q, codes.astype(np.float64) * s)
            near = np.rint(mats[p].astype(np.float32) / scales[:, None]).clip(-127, 127) * s
        else:
            q4 = np.concatenate([codes.reshape(-1, k // 32, 16) & 15, codes.reshape(-1, k // 32, 16) >> 4], axis=2)
            d = scales.view(np.float16).astype(np.float64)[:, :, None]
            np.testing.assert_array_equal(q, ((q4.astype(np.float64) - 8) * d).reshape(q.shape))
            near = np.empty_like(q)
            w32 = mats[p].astype(np.float32)
            for r in range(q.shape[0]):
                for b in range(0, k, 32):
                    dd = np.float32(orc.q4_group_scale(w32[r, b:b + 32]))
                    near[r, b:b + 32] = np.clip(np.rint(w32[r, b:b + 32] / dd), -8, 7) * np.float64(dd)
        err = lambda qv: float(((x @ (mats[p] - qv).T) ** 2).sum())
        assert err(q) < err(near), p
    # The residual advanced through the rounded matrices, not the float ones.
    ref = cal.layer(out["mats"], f32(L["qn"]), f32(L["kn"]))
    np.testing.assert_allclose(out["residual"], ref["residual"], rtol=0, atol=1e-12 * np.abs(ref["residual"]).max())
