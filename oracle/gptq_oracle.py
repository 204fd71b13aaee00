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

* CalibrationOracle: the calibration pass of QuantizeGPTQ (newCalibration,
  calibration.weights / layer / attention, normalizedRows, project;
  gptq.go:330-600) in float64: the calibration rows' residual stream in the
  GPU basis, advanced layer by layer through the GPTQ-rounded projections,
  each group rounded against the inputs the layers before it produce.

Pinned in tests/test_gptq_oracle.py by: scipy's Cholesky of H^-1 (an
independent route to the same unique factor) and H U^T U = I
(gptq_linalg_test.go:14-67); the Hinv-downdate form of GPTQ (optimal brain
surgeon updates with H^-1 and its Schur complements, Frantar et al. 2022),
which must give the same codes; the reference's own property that GPTQ
beats round-to-nearest in output error (gptq_linalg_test.go:72-148); and,
for the calibration pass, the GPU-basis weights preserving each projection's
product under the rotations, and the unrounded pass equal to the batched
decode oracle's prefill of each sequence (DecodeOracle.prefill, itself
pinned to transformers' Qwen3).
"""
import numpy as np

from . import lm_oracle as lo
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


MAX_SEQ = 256  # gptqMaxSeq (gptq.go:40)

# calibration.weights' rotations per projection (gptq.go:404-417): the folded
# norm ("attn", "mlp" or None), the input rotation and the output rotation.
_WEIGHT_SPEC = (("attn", "hidden", None), ("attn", "hidden", None), ("attn", "hidden", "head_v"),
                (None, "head_o", "hidden"), ("mlp", "hidden", None), ("mlp", "hidden", None),
                (None, "inter", "hidden"))


def round_group(x, mats, bits):
    """quantizeGroup (gptq.go:602-665) of the matrices sharing inputs x:
    [(codes, scales, rounded float64 matrix)] with dead channels zeroed."""
    h, dead = damp(hessian(x))
    u = inverse_factor(h)
    out = []
    for m in mats:
        m = np.array(m, np.float64, copy=True)
        m[:, dead] = 0
        out.append(round_rows(m.astype(np.float32), u, bits))
    return out


class CalibrationOracle:
    """float64 calibration pass over token-id sequences (newCalibration,
    gptq.go:344-383): self.h [rows][hidden] is the residual stream, each row
    the hidden rotation of its BF16 embedding row; positions count from 0 in
    each sequence, and a row attends to the rows of its sequence up to itself."""

    def __init__(self, geom, embed_bf16, sequences):
        g = self.g = geom
        self.rot = {"hidden": lo.rotation(g.hidden), "inter": lo.rotation(g.inter),
                    "head_v": lo.head_rotation(g.head_dim, g.kvd), "head_o": lo.head_rotation(g.head_dim, g.qd)}
        ids = np.concatenate([np.asarray(s, np.int64) for s in sequences])
        self.pos = np.concatenate([np.arange(len(s)) for s in sequences])
        self.seq_slices = []
        r = 0
        for s in sequences:
            self.seq_slices.append(slice(r, r + len(s)))
            r += len(s)
        embed = np.asarray(embed_bf16, np.uint16).reshape(g.vocab, g.hidden)
        self.h = lo.rot_apply(lo.bf16_to_f64(embed[ids]).reshape(len(ids), g.hidden), self.rot["hidden"])
        cos, sin = lo.rope_table(g, MAX_SEQ)
        self.cos, self.sin = cos.astype(np.float64), sin.astype(np.float64)

    def weights(self, bf16, attn_norm, mlp_norm):
        """calibration.weights (gptq.go:386-433) of the seven projections
        (BF16 bits [n][k] each, file order): the norm folded into the columns,
        R_in along each row, R_out across the rows: float64 [n][k] each."""
        norms = {"attn": np.asarray(attn_norm, np.float64), "mlp": np.asarray(mlp_norm, np.float64), None: None}
        out = []
        for raw, (norm, rin, rout) in zip(bf16, _WEIGHT_SPEC):
            w = lo.bf16_to_f64(raw).reshape(np.asarray(raw).shape)
            if norms[norm] is not None:
                w = w * norms[norm][None, :]
            w = lo.rot_apply(w, self.rot[rin]).reshape(w.shape)
            if rout is not None:
                w = lo.rot_apply(w.T, self.rot[rout]).reshape(w.T.shape).T
            out.append(np.ascontiguousarray(w))
        return out

    def _norm_rows(self, v, w=None):
        inv = 1.0 / np.sqrt((v * v).sum(axis=1, keepdims=True) / v.shape[1] + self.g.eps)
        return v * inv if w is None else v * inv * w

    def _rope(self, v, pos):
        half = self.g.head_dim // 2
        c, s = self.cos[pos][:, None, :], self.sin[pos][:, None, :]
        a, b = v[..., :half], v[..., half:]
        return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)

    def attention(self, q, k, v, q_norm, k_norm):
        """calibration.attention (gptq.go:529-571): head RMSNorm and RoPE at
        each row's position, causal softmax attention within each sequence."""
        g = self.g
        hd, rows = g.head_dim, q.shape[0]
        qn = np.asarray(q_norm, np.float64)
        kn = np.asarray(k_norm, np.float64)
        qh = q.reshape(rows, g.heads, hd)
        kh = k.reshape(rows, g.kv_heads, hd)
        qh = qh / np.sqrt((qh * qh).mean(axis=2, keepdims=True) + g.eps) * qn
        kh = kh / np.sqrt((kh * kh).mean(axis=2, keepdims=True) + g.eps) * kn
        qh, kh = self._rope(qh, self.pos), self._rope(kh, self.pos)
        vh = v.reshape(rows, g.kv_heads, hd)
        grp = g.heads // g.kv_heads
        scale = 1.0 / np.sqrt(hd)
        ctx = np.empty((rows, g.heads, hd))
        for sl in self.seq_slices:
            n = sl.stop - sl.start
            causal = np.tril(np.ones((n, n), bool))
            for h in range(g.heads):
                s = qh[sl, h] @ kh[sl, h // grp].T * scale
                s = np.where(causal, s, -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                ctx[sl, h] = (p / p.sum(axis=1, keepdims=True)) @ vh[sl, h // grp]
        return ctx.reshape(rows, g.qd)

    def layer(self, mats, q_norm, k_norm, bits=None, h=None):
        """calibration.layer (gptq.go:437-524) from residual h (self.h by
        default): with bits, each group is GPTQ-rounded over its inputs before
        its projection (round_group); without, the matrices are used as given.
        Returns dict(attn_input, context, mlp_input, down_input, residual,
        mats (as used), rounded ([(codes, scales)] per projection, or None))."""
        g = self.g
        h = self.h if h is None else np.asarray(h, np.float64)
        mats = [np.asarray(m, np.float64) for m in mats]
        rounded = [None] * 7
        out = {}

        def group(x, ps):
            if bits is None:
                return
            for p, (codes, scales, w) in zip(ps, round_group(x, [mats[p] for p in ps], bits)):
                mats[p] = w
                rounded[p] = (codes, scales)

        x = out["attn_input"] = self._norm_rows(h)
        group(x, (0, 1, 2))
        ctx = out["context"] = self.attention(x @ mats[0].T, x @ mats[1].T, x @ mats[2].T, q_norm, k_norm)
        group(ctx, (3,))
        h = h + ctx @ mats[3].T
        x = out["mlp_input"] = self._norm_rows(h)
        group(x, (4, 5))
        gate, up = x @ mats[4].T, x @ mats[5].T
        with np.errstate(over="ignore"):
            act = gate / (1.0 + np.exp(-gate)) * up
        act = out["down_input"] = lo.rot_apply(act, self.rot["inter"]).reshape(act.shape)
        group(act, (6,))
        out["residual"] = h + act @ mats[6].T
        out["mats"], out["rounded"] = mats, rounded if bits is not None else None
        return out
