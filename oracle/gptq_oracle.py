"""float64 restatement of the GPTQ producer's core (cmd/qwen3-gptq ->
qwen3lm quantizeGroup / gptqInverseFactor / gptqRound, gptq.go:604-796,
gptq_linalg.go:185-223), for parity tests.

TEST INFRASTRUCTURE. Only tests/ may import this module; the product
library never does.

* hessian(x): H = X^T X of the calibration rows (gptq.go:606-622; the 2/rows
  factor of the comment is not applied by the code and cancels in GPTQ).
* damp(h): dead channels (H[i][i] == 0) get H[i][i] = 1, then every diagonal
  entry gains 0.01 * mean(diag) (gptq.go:623-637).
* inverse_factor(h): U upper triangular with H^-1 = U^T U, computed as the
  reference does, U = J chol(J H J)^-1 J with J the reversal.
* round_rows(w, u, bits): column by column, code = clamp(rne(w/s)), error
  e = (w - q s) / U[c][c], later columns w[j] -= e U[c][j]; 8-bit: one scale
  max|row|/127 per row taken before rounding; 4-bit: q4GroupScale of the
  current 32 values at each group start (gptq.go:703-796). float64 except the
  scale search and the code division, which follow the reference's float32.

Pinned in tests/test_gptq_oracle.py by: scipy's Cholesky of H^-1 (an
independent route to the same unique factor) and H U^T U = I
(gptq_linalg_test.go:14-67); the Hinv-downdate form of GPTQ (optimal brain
surgeon updates with H^-1 and its Schur complements, Frantar et al. 2022),
which must give the same codes; and the reference's own property that GPTQ
beats round-to-nearest in output error (gptq_linalg_test.go:72-148).
"""
import numpy as np

from . import oracle as orc

GPTQ_DAMP = 0.01
GROUP = 32


def hessian(x):
    x = np.asarray(x, np.float64)
    return x.T @ x


def damp(h):
    h = np.array(h, np.float64, copy=True)
    k = h.shape[0]
    mean = np.trace(h) / k
    dead = np.diag(h) == 0
    h[np.arange(k), np.arange(k)] = np.where(dead, 1.0, np.diag(h)) + GPTQ_DAMP * mean
    return h, dead


def inverse_factor(h):
    h = np.asarray(h, np.float64)
    a = h[::-1, ::-1]
    L = np.linalg.cholesky(a)
    X = np.linalg.inv(L)
    return np.triu(X[::-1, ::-1])


def q4_group_scale(v):
    """gptq.go:764-791 (the C oracle's restatement, float64 error sums)."""
    return float(orc.q4_group_scale(np.asarray(v, np.float32)))


def round_rows(w, u, bits):
    """GPTQ rounding of w [n][k] against U: (codes, scales, rounded values
    float64 [n][k]). codes: int8 [n][k] (bits 8) or the GPU Q4 bytes [n][k/2]
    (bits 4); scales: float32 [n] or float16 bits [n][k/32]."""
    w = np.array(w, np.float64, copy=True)
    n, k = w.shape
    u = np.asarray(u, np.float64)
    q = np.zeros((n, k), np.int64)
    if bits == 8:
        s32 = (np.abs(w.astype(np.float32)).max(axis=1) / np.float32(127)).astype(np.float32)
        scales = s32
    else:
        scales = np.zeros((n, k // GROUP), np.uint16)
        s32 = np.zeros(n, np.float32)
    for c in range(k):
        if bits == 4 and c % GROUP == 0:
            for r in range(n):
                s32[r] = q4_group_scale(w[r, c:c + GROUP].astype(np.float32))
            scales[:, c // GROUP] = s32.astype(np.float16).view(np.uint16)
        lo, hi = (-127, 127) if bits == 8 else (-8, 7)
        with np.errstate(divide="ignore", invalid="ignore"):
            ratio = (w[:, c].astype(np.float32) / s32).astype(np.float64)
        code = np.where(s32 != 0, np.clip(np.rint(ratio), lo, hi), 0).astype(np.int64)
        qv = code * s32.astype(np.float64)
        e = (w[:, c] - qv) / u[c, c]
        w[:, c] = qv
        w[:, c + 1:] -= e[:, None] * u[c, c + 1:][None, :]
        q[:, c] = code
    if bits == 8:
        codes = q.astype(np.int8)
    else:
        nib = (q + 8).astype(np.uint8).reshape(n, k // GROUP, GROUP)
        codes = (nib[:, :, :16] | (nib[:, :, 16:] << 4)).reshape(n, k // 2)
    return codes, scales, w


def round_rows_obs(w, hinv, bits):
    """The same rounding in its optimal-brain-surgeon form: after quantizing
    column c, w[j] -= (w_c - q_c) / Hinv[c][c] * Hinv[c][j], then Hinv loses
    row and column c by its Schur complement. Returns the codes (the scales
    are chosen as in round_rows). Independent of the Cholesky factor."""
    w = np.array(w, np.float64, copy=True)
    hv = np.array(hinv, np.float64, copy=True)
    n, k = w.shape
    q = np.zeros((n, k), np.int64)
    s32 = (np.abs(w.astype(np.float32)).max(axis=1) / np.float32(127)).astype(np.float32) if bits == 8 \
        else np.zeros(n, np.float32)
    for c in range(k):
        if bits == 4 and c % GROUP == 0:
            for r in range(n):
                s32[r] = q4_group_scale(w[r, c:c + GROUP].astype(np.float32))
        lo, hi = (-127, 127) if bits == 8 else (-8, 7)
        with np.errstate(divide="ignore", invalid="ignore"):
            ratio = (w[:, c].astype(np.float32) / s32).astype(np.float64)
        code = np.where(s32 != 0, np.clip(np.rint(ratio), lo, hi), 0).astype(np.int64)
        qv = code * s32.astype(np.float64)
        d = (w[:, c] - qv) / hv[c, c]
        w[:, c] = qv
        w[:, c + 1:] -= d[:, None] * hv[c, c + 1:][None, :]
        hv = hv - np.outer(hv[:, c], hv[c, :]) / hv[c, c]
        q[:, c] = code
    return q
