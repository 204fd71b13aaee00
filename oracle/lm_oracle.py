"""float64 restatement of one qwen3lm GPU decode step (the lane API's
DecodeBatchInto / DecodeBatchGreedyInto), for parity tests.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product library never does.

What is restated (reference paths are relative to the gophonic tree):

* The residual stream lives in the hidden rotation's basis R = scale*H*diag(s)
  (qwen3lm/hadamard.go:13-86, gpu_darwin.go:57-61). The token's BF16
  embedding row is rotated on entry (gpu_darwin.go:1170-1175).
* Per layer (gpu_darwin.go:1193-1235, kernels gpu.metal:68-162, 339-466):
  QKV GEMV over the RMS-normalized residual (PRO_NORM: the input RMSNorm
  weight is folded into the stored rows), attend1 (head RMSNorm with q_norm /
  k_norm, RoPE from a float32 table, K/V append at row `pos`, softmax over
  rows 0..pos), O GEMV added to the residual (EPI_ADD), gate/up GEMV over the
  normalized residual with interleaved gate/up rows and SwiGLU (EPI_SWIGLU),
  the down input's online Hadamard for Q8 and Q4 weights (rotate, skipped for
  Q8B, gpu_darwin.go:209-215), down GEMV added to the residual.
* After the layers (gpu_darwin.go:1241-1280): R^T, final RMSNorm with the
  final norm weight (ops.go:251-254) -> the hidden output; R again; the Q8B
  head GEMV over vocab rows; first-maximum argmax (decode_batch.go:182-191).

Everything is float64 on the dequantized weights (the kernels' per-block
scaling is exact in float64), so this is the precision target the fp32 device
path is measured against. Pinned against Hugging Face transformers' Qwen3 in
float64 (tests/test_oracle_lm.py), with the unrotated weights the stored ones
imply.
"""
from dataclasses import dataclass

import numpy as np

from . import oracle as orc

FMT_Q4, FMT_Q8, FMT_Q8B, FMT_Q8B_F32 = 4, 8, 9, 10


@dataclass(frozen=True)
class Geometry:
    """A dense Qwen3 decoder's shape (lmtest.Geometry, lmtest/lmtest.go:22-24)."""

    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    max_pos: int
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def qd(self):
        return self.heads * self.head_dim

    @property
    def kvd(self):
        return self.kv_heads * self.head_dim

    @property
    def head_rows(self):
        # gpuModel.loadHead pads the vocabulary to 16 rows (gpu_darwin.go:343).
        return (self.vocab + 15) // 16 * 16


def rotation(k):
    """hadamard.go:24-47 newRotation: (signs float32[k], block, scale)."""
    signs = np.empty(k, np.float32)
    scale = np.zeros(1, np.float32)
    block = orc.lib().orc_rotation(k, orc._p(signs, orc._f32p), orc._p(scale, orc._f32p))
    return signs, int(block), float(scale[0])


def hadamard_f64(v, block):
    """Unnormalized Walsh-Hadamard transform of each `block` run of the last
    axis, in natural order (the network of hadamard.go:62-78), float64."""
    v = np.array(v, dtype=np.float64, copy=True)
    shape = v.shape
    v = v.reshape(-1, block)
    h = 1
    while h < block:
        w = v.reshape(v.shape[0], -1, 2, h)
        a, b = w[:, :, 0, :].copy(), w[:, :, 1, :].copy()
        w[:, :, 0, :] = a + b
        w[:, :, 1, :] = a - b
        h *= 2
    return v.reshape(shape)


def rot_apply(x, rot):
    signs, block, scale = rot
    return hadamard_f64(np.asarray(x, np.float64) * scale * signs, block)


def rot_unapply(x, rot):
    signs, block, scale = rot
    return hadamard_f64(x, block) * scale * signs


def head_rotation(head_dim, length):
    """The per-head rotation of value rows and o inputs (gpu_darwin.go:217-221):
    newRotation(head_dim)'s signs repeated over `length` values."""
    signs, block, scale = rotation(head_dim)
    return np.tile(signs, length // head_dim), block, scale


def rot_matrix(rot):
    """The dense orthogonal matrix R with R @ x == rot_apply(x, rot)."""
    signs, block, scale = rot
    k = len(signs)
    return rot_apply(np.eye(k), rot).T


def bf16_to_f64(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def dequant(fmt, codes, scales, n, k):
    """float64 [n][k] of a qwen3lm weight matrix (gpu.metal:46-61 formats)."""
    if fmt == FMT_Q4:
        b = np.asarray(codes, np.uint8).reshape(n, k // 32, 16)
        v = np.concatenate([(b & 15), (b >> 4)], axis=2).astype(np.float64) - 8.0
        d = np.asarray(scales, np.uint16).view(np.float16).astype(np.float64).reshape(n, k // 32, 1)
        return (v * d).reshape(n, k)
    q = np.asarray(codes, np.int8).reshape(n, k).astype(np.float64)
    if fmt == FMT_Q8:
        return q * np.asarray(scales, np.float32).astype(np.float64).reshape(n, 1)
    if fmt == FMT_Q8B:
        d = np.asarray(scales, np.uint16).view(np.float16).astype(np.float64)
    elif fmt == FMT_Q8B_F32:
        d = np.asarray(scales, np.float32).astype(np.float64)
    else:
        raise ValueError(f"format {fmt}")
    return (q.reshape(n, k // 32, 32) * d.reshape(n, k // 32, 1)).reshape(n, k)


def rope_table(geom, positions):
    """gpu_darwin.go:232-241: float32(cos/sin(pos * invFreq[d])) with
    invFreq[d] = 1/theta^(2d/headDim) in float64 (weights.go:685-688)."""
    half = geom.head_dim // 2
    inv = 1.0 / np.power(geom.theta, (2.0 * np.arange(half)) / geom.head_dim)
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@dataclass
class Layer:
    """One layer's stored projections (gpuLayer, gpu_darwin.go:45-56):
    (codes, scales) of the fused QKV rows [qd+2kvd][hidden], O [hidden][qd],
    interleaved gate/up [2*inter][hidden] (row 2i gate, 2i+1 up) and down
    [hidden][inter]; q_norm / k_norm float32[head_dim]."""

    qkv: tuple
    o: tuple
    gu: tuple
    down: tuple
    q_norm: np.ndarray
    k_norm: np.ndarray


class DecodeOracle:
    """float64 single-token decode over stored qwen3lm GPU weights."""

    def __init__(self, geom, fmt, layers, embed_bf16, final_norm, head):
        g = geom
        self.g, self.fmt = g, fmt
        self.hrot, self.irot = rotation(g.hidden), rotation(g.inter)
        self.embed = np.asarray(embed_bf16, np.uint16).reshape(g.vocab, g.hidden)
        self.final_norm = np.asarray(final_norm, np.float32).astype(np.float64)
        self.W = []
        for L in layers:
            self.W.append(dict(
                qkv=dequant(fmt, *L.qkv, g.qd + 2 * g.kvd, g.hidden),
                o=dequant(fmt, *L.o, g.hidden, g.qd),
                gu=dequant(fmt, *L.gu, 2 * g.inter, g.hidden),
                down=dequant(fmt, *L.down, g.hidden, g.inter),
                qn=np.asarray(L.q_norm, np.float32).astype(np.float64),
                kn=np.asarray(L.k_norm, np.float32).astype(np.float64),
            ))
        self._head_codes = np.asarray(head[0], np.int8).reshape(g.head_rows, g.hidden)[: g.vocab]
        self._head_scales = np.asarray(head[1], np.uint16).reshape(g.head_rows, g.hidden // 32)[: g.vocab]
        self._head = None
        cos, sin = rope_table(g, g.max_pos)
        self.cos, self.sin = cos.astype(np.float64), sin.astype(np.float64)

    @property
    def head(self):
        """float64 [vocab][hidden] of the Q8B head (dequantized on first use)."""
        if self._head is None:
            self._head = dequant(FMT_Q8B, self._head_codes, self._head_scales, self.g.vocab, self.g.hidden)
        return self._head

    HEAD_CHUNK = 8192  # rows per dequantized chunk
    DENSE_HEAD_MAX = 1 << 26  # head values kept dense in float64 (512 MiB)

    def head_rows(self, x):
        """head @ x_r for each row of x [rows][hidden] -> [rows][vocab]. A
        full-size head (151,936 x 4096 is 5 GB in float64) is dequantized in
        row chunks instead of being kept; each logit is the same float64 dot
        product either way."""
        g = self.g
        x = np.atleast_2d(np.asarray(x, np.float64))
        if self._head is not None or g.vocab * g.hidden <= self.DENSE_HEAD_MAX:
            return x @ self.head.T
        out = np.empty((x.shape[0], g.vocab))
        for r in range(0, g.vocab, self.HEAD_CHUNK):
            e = min(g.vocab, r + self.HEAD_CHUNK)
            w = dequant(FMT_Q8B, self._head_codes[r:e], self._head_scales[r:e], e - r, g.hidden)
            out[:, r:e] = x @ w.T
        return out

    def new_cache(self, capacity):
        g = self.g
        return [(np.zeros((capacity, g.kvd)), np.zeros((capacity, g.kvd))) for _ in range(g.layers)]

    def _norm(self, v, w=None):
        inv = 1.0 / np.sqrt(np.dot(v, v) / len(v) + self.g.eps)
        return v * inv if w is None else v * inv * w

    def _rope(self, v, pos):
        half = self.g.head_dim // 2
        c, s = self.cos[pos], self.sin[pos]
        a, b = v[:half].copy(), v[half:].copy()
        return np.concatenate([a * c - b * s, b * c + a * s])

    def embed_row(self, token):
        """The rotated input row (gpu_darwin.go:1172-1174)."""
        return rot_apply(bf16_to_f64(self.embed[token]), self.hrot)

    def layers(self, cache, pos, h):
        """Runs every layer on residual h (rotated basis) at position pos,
        appending K/V to cache; returns the new residual."""
        g = self.g
        grp = g.heads // g.kv_heads
        scale = 1.0 / np.sqrt(g.head_dim)
        hd = g.head_dim
        for li, W in enumerate(self.W):
            qkv = W["qkv"] @ self._norm(h)
            kc, vc = cache[li]
            for kh in range(g.kv_heads):
                k = qkv[g.qd + kh * hd: g.qd + (kh + 1) * hd]
                v = qkv[g.qd + g.kvd + kh * hd: g.qd + g.kvd + (kh + 1) * hd]
                kc[pos, kh * hd:(kh + 1) * hd] = self._rope(self._norm(k, W["kn"]), pos)
                vc[pos, kh * hd:(kh + 1) * hd] = v
            ctx = np.empty(g.qd)
            for qh in range(g.heads):
                kh = qh // grp
                q = self._rope(self._norm(qkv[qh * hd:(qh + 1) * hd], W["qn"]), pos) * scale
                s = kc[: pos + 1, kh * hd:(kh + 1) * hd] @ q
                p = np.exp(s - s.max())
                ctx[qh * hd:(qh + 1) * hd] = (p / p.sum()) @ vc[: pos + 1, kh * hd:(kh + 1) * hd]
            h = h + W["o"] @ ctx
            gu = W["gu"] @ self._norm(h)
            gate, up = gu[0::2], gu[1::2]
            with np.errstate(over="ignore"):  # exp(-gate) = inf gives act = -0, as in float32
                act = gate / (1.0 + np.exp(-gate)) * up
            if self.fmt != FMT_Q8B:
                act = rot_apply(act, self.irot)
            h = h + W["down"] @ act
        return h

    def _norm_rows(self, v, w=None):
        inv = 1.0 / np.sqrt((v * v).sum(axis=1, keepdims=True) / v.shape[1] + self.g.eps)
        return v * inv if w is None else v * inv * w

    def _rope_rows(self, v, pos):
        half = self.g.head_dim // 2
        c, s = self.cos[pos], self.sin[pos]
        a, b = v[:, :half], v[:, half:]
        return np.concatenate([a * c - b * s, b * c + a * s], axis=1)

    def _mm(self, x, w):
        """x [rows][k] @ w^T in float64; with int8 activations (the CPU
        provider's int8 route, qwen3lm/ops.go:96-147, 198-215) each row of x is
        first replaced by its WorkspaceI8 quantization s * q (int8.go:106-168:
        s = max|x|/127, q = round-half-even(x * 127/max|x|) saturated to
        [-128, 127]; a row with no finite positive maximum gives zeros)."""
        if not self.int8:
            return x @ w.T
        m = np.abs(x).max(axis=1, keepdims=True)
        ok = np.isfinite(m) & (m > 0)
        safe = np.where(ok, m, 1.0)
        q = np.clip(np.rint(x * (127.0 / safe)), -128, 127)
        return np.where(ok, q * (safe / 127.0), 0.0) @ w.T

    int8 = False

    def prefill(self, cache, base, tokens, last_only=False, embeds=None, tail=None):
        """All rows of tokens at positions base.. at once (the batched pass,
        gpu_darwin.go:1703-1764: each row attends cache rows 0..its own
        position): appends K/V and returns the residual rows [T][hidden]. The
        same float64 math as stepping layers() token by token.

        tail: the last layer still appends every row's K/V but finishes only
        the final `tail` rows (the rows HiddenTail*/HiddenLast* return), and
        the result is those rows' residuals [tail][hidden]; last_only is
        tail=1. For a one-layer model this skips the other rows' attention
        and MLP.

        embeds: (token, rows [occurrences][hidden]) -- Embeds
        (evaluator.go:150-163, gpu_darwin.go:1582-1590): the i-th occurrence
        of token takes row i (float32, unrotated like an embedding row)
        instead of the embedding table's row.

        With int8 = True every projection multiplies per-row int8-quantized
        inputs (_mm), the arithmetic of the int8 route."""
        g = self.g
        T = len(tokens)
        hd = g.head_dim
        grp = g.heads // g.kv_heads
        scale = 1.0 / np.sqrt(hd)
        pos = base + np.arange(T)
        ids = np.asarray(tokens, np.int64)
        raw = bf16_to_f64(self.embed[ids]).reshape(T, g.hidden)
        if embeds is not None:
            at = np.nonzero(ids == embeds[0])[0]
            rows_in = np.asarray(embeds[1], np.float32).reshape(-1, g.hidden)
            assert len(rows_in) == len(at), "one Embeds row per placeholder"
            raw[at] = rows_in.astype(np.float64)
        h = rot_apply(raw, self.hrot).reshape(T, g.hidden)
        mask = np.arange(base + T)[None, :] <= pos[:, None]
        tail = 1 if last_only and tail is None else tail
        for li, W in enumerate(self.W):
            rows = slice(T - tail, T) if tail is not None and li == len(self.W) - 1 else slice(0, T)
            hn = self._norm_rows(h)
            kv = self._mm(hn, W["qkv"][g.qd:])
            qs = self._mm(hn[rows], W["qkv"][: g.qd])
            kc, vc = cache[li]
            for kh in range(g.kv_heads):
                k = kv[:, kh * hd:(kh + 1) * hd]
                v = kv[:, g.kvd + kh * hd: g.kvd + (kh + 1) * hd]
                kc[pos, kh * hd:(kh + 1) * hd] = self._rope_rows(self._norm_rows(k, W["kn"]), pos)
                vc[pos, kh * hd:(kh + 1) * hd] = v
            prow = pos[rows]
            ctx = np.empty((len(prow), g.qd))
            for qh in range(g.heads):
                kh = qh // grp
                q = self._rope_rows(self._norm_rows(qs[:, qh * hd:(qh + 1) * hd], W["qn"]), prow) * scale
                s = np.where(mask[rows], q @ kc[: base + T, kh * hd:(kh + 1) * hd].T, -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                ctx[:, qh * hd:(qh + 1) * hd] = (p / p.sum(axis=1, keepdims=True)) @ vc[: base + T, kh * hd:(kh + 1) * hd]
            h = h[rows] + self._mm(ctx, W["o"])
            gu = self._mm(self._norm_rows(h), W["gu"])
            gate, up = gu[:, 0::2], gu[:, 1::2]
            with np.errstate(over="ignore"):
                act = gate / (1.0 + np.exp(-gate)) * up
            if self.fmt != FMT_Q8B:
                act = rot_apply(act, self.irot).reshape(act.shape)
            h = h + self._mm(act, W["down"])
        return h

    def finish(self, h):
        """(hidden, logits): R^T, final RMSNorm, R, head (first vocab rows)."""
        hidden, logits = self.finish_rows(np.asarray(h, np.float64)[None, :])
        return hidden[0], logits[0]

    def finish_rows(self, h):
        """finish() of each residual row of h [rows][hidden], with one pass
        over the head for all rows: (hidden [rows][hidden], logits [rows][vocab])."""
        h = np.atleast_2d(np.asarray(h, np.float64))
        hu = rot_unapply(h, self.hrot).reshape(h.shape)
        hidden = self._norm_rows(hu, self.final_norm)
        logits = self.head_rows(rot_apply(hidden, self.hrot).reshape(h.shape))
        return hidden, logits

    def step(self, cache, pos, token):
        """One decode step for one lane: (hidden, logits, next_token)."""
        h = self.layers(cache, pos, self.embed_row(token))
        hidden, logits = self.finish(h)
        return hidden, logits, greedy_argmax(logits)


def greedy_argmax(values):
    """decode_batch.go:182-191: strict greater-than scan from index 0; ties
    keep the first index; NaNs never replace the best."""
    best, at = values[0], 0
    for i in range(1, len(values)):
        if values[i] > best:
            best, at = values[i], i
    return at


def greedy_argmax_np(values):
    """The same rule, vectorized (NaN at index 0 keeps index 0)."""
    v = np.asarray(values)
    if np.isnan(v[0]):
        return 0
    w = np.where(np.isnan(v), -np.inf, v)
    return int(np.argmax(w))


def quantize_rows_i8(x):
    """WorkspaceI8's per-row quantization (int8.go:106-168) in float64, as the
    dequantized values s * q: s = max|x| / 127, q = round-half-even(x * 127 /
    max|x|) saturated to [-128, 127]; a row with no finite positive maximum
    gives zeros."""
    x = np.atleast_2d(np.asarray(x, np.float64))
    m = np.abs(x).max(axis=1, keepdims=True)
    ok = np.isfinite(m) & (m > 0)
    safe = np.where(ok, m, 1.0)
    q = np.clip(np.rint(x * (127.0 / safe)), -128, 127)
    return np.where(ok, q * (safe / 127.0), 0.0)


class CpuInt8Oracle:
    """float64 restatement of the reference CPU provider's int8 decode step
    (qwen3lm/ops.go:96-254 over WeightsInt8 rows, weights.go:314-349,
    738-831): the residual stream is not rotated; each projection input is
    RMS-normalized with its norm weight, rotated by the projection's input
    rotation (newRotation of the hidden width for q/k/v/gate/up and the head,
    of q_dim for o, of the intermediate width for down), quantized per row
    (quantize_rows_i8) and multiplied by the int8 rows times their per-row
    scales (the rows store W R^T, quantizeRotatedRows). Head RMSNorm and RoPE,
    softmax attention over the K/V cache, SwiGLU and the residual adds as in
    the GPU step. With quantize=False the activations are used unquantized and
    the step is the model's own forward pass (pinned against DecodeOracle in
    tests/test_cpu_baseline.py).

    layers: dicts with w (seven [n][k] arrays: q, k, v, o, gate, up, down),
    s (seven per-row scales, or None for float rows), attn_norm, mlp_norm,
    q_norm, k_norm; head (w, s) likewise."""

    def __init__(self, geom, layers, final_norm, head, quantize=True):
        g = self.g = geom
        self.rot = {"h": rotation(g.hidden), "c": rotation(g.qd), "i": rotation(g.inter)}
        f64 = lambda v: np.asarray(v, np.float64)
        deq = lambda w, s: f64(w) if s is None else f64(w) * f64(s)[:, None]
        self.L = [dict(w=[deq(w, s) for w, s in zip(L["w"], L["s"])], attn=f64(L["attn_norm"]),
                       mlp=f64(L["mlp_norm"]), qn=f64(L["q_norm"]), kn=f64(L["k_norm"])) for L in layers]
        self.final_norm = f64(final_norm)
        self.head = deq(*head)
        self.quantize = quantize

    def _norm(self, v, w=None):
        inv = 1.0 / np.sqrt(np.dot(v, v) / len(v) + self.g.eps)
        return v * inv if w is None else v * inv * w

    def _proj(self, x, rot, w):
        x = rot_apply(x, self.rot[rot])
        if self.quantize:
            x = quantize_rows_i8(x)[0]
        return w @ x

    def step(self, h, kc, vc, pos, cos, sin):
        """One token at position pos: h (the embedding row, unrotated) ->
        (residual, post-final-norm state, logits); appends K/V at pos of each
        layer's cache (kc[l], vc[l]: [cap][kv_dim]); cos / sin: the RoPE row."""
        g = self.g
        hd, half, grp = g.head_dim, g.head_dim // 2, g.heads // g.kv_heads
        h = np.array(h, np.float64)
        c, s = np.asarray(cos, np.float64), np.asarray(sin, np.float64)
        rope = lambda v: np.concatenate([v[:half] * c - v[half:] * s, v[half:] * c + v[:half] * s])
        scale = 1.0 / np.sqrt(hd)
        for li, L in enumerate(self.L):
            W = L["w"]
            x = self._norm(h, L["attn"])
            q, k, v = self._proj(x, "h", W[0]), self._proj(x, "h", W[1]), self._proj(x, "h", W[2])
            for kh in range(g.kv_heads):
                kc[li][pos, kh * hd:(kh + 1) * hd] = rope(self._norm(k[kh * hd:(kh + 1) * hd], L["kn"]))
                vc[li][pos, kh * hd:(kh + 1) * hd] = v[kh * hd:(kh + 1) * hd]
            ctx = np.empty(g.qd)
            for qh in range(g.heads):
                kh = qh // grp
                qv = rope(self._norm(q[qh * hd:(qh + 1) * hd], L["qn"]))
                sc = kc[li][: pos + 1, kh * hd:(kh + 1) * hd] @ qv * scale
                p = np.exp(sc - sc.max())
                ctx[qh * hd:(qh + 1) * hd] = (p / p.sum()) @ vc[li][: pos + 1, kh * hd:(kh + 1) * hd]
            h = h + self._proj(ctx, "c", W[3])
            x = self._norm(h, L["mlp"])
            gate, up = self._proj(x, "h", W[4]), self._proj(x, "h", W[5])
            with np.errstate(over="ignore"):
                act = gate / (1.0 + np.exp(-gate)) * up
            h = h + self._proj(act, "i", W[6])
        hidden = self._norm(h, self.final_norm)
        return h, hidden, self._proj(hidden, "h", self.head)
