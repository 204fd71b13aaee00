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
