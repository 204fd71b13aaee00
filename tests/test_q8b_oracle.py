"""Pins the block-32 int8 oracle (oracle.q8b_quantize / q8b_gemm), the
benchmark configuration-2 variant with no counterpart in the reference:

* the quantizer equals the pinned per-row quantizer (WorkspaceI8,
  int8.go:106-168, pinned in test_oracle.py) applied to every 32-value block
  as a row of its own;
* the GEMM's block products equal exact int64 sums (numpy), its result is
  within fp32 accumulation of the float64 sum of scaled block products, and on
  inputs where every operation is exact (power-of-two scales, small codes) it
  equals that float64 sum bit for bit.
"""
import numpy as np

from oracle import oracle as orc


def test_quantize_is_the_row_rule_per_block():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((6, 160)) * rng.choice([1e-3, 1.0, 300.0], size=(6, 1))).astype(np.float32)
    x[1, 32:64] = 0.0
    x[2, 70] = np.nan
    x[3, 100] = np.inf
    q, d = orc.q8b_quantize(x, 6, 160)
    for r in range(6):
        for b in range(5):
            qr, s, _ = orc.i8_pack_rows(x[r, 32 * b:32 * b + 32].reshape(1, 32), 1, 32)
            assert np.array_equal(q[r, 32 * b:32 * b + 32], qr[0]), (r, b)
            assert d[r, b].view(np.uint32) == s[0].view(np.uint32), (r, b)
    assert (d[1, 1] == 0) and not q[1, 32:64].any()
    assert d[2, 2] == 0 and not q[2, 64:96].any()
    assert d[3, 3] == 0 and not q[3, 96:128].any()


def block_sums(qa, da, qw, dw):
    m, k = qa.shape
    n = qw.shape[0]
    kb = k // 32
    dots = np.einsum("mbi,nbi->mnb", qa.reshape(m, kb, 32).astype(np.int64), qw.reshape(n, kb, 32).astype(np.int64))
    return dots, dots.astype(np.float64) * (da[:, None, :].astype(np.float64) * dw[None, :, :].astype(np.float64))


def test_gemm_within_fp32_accumulation_of_float64():
    rng = np.random.default_rng(4)
    m, k, n = 7, 320, 13
    qa = rng.integers(-128, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    da = (np.abs(rng.standard_normal((m, k // 32))) * 0.02).astype(np.float32)
    dw = (np.abs(rng.standard_normal((n, k // 32))) * 0.01).astype(np.float32)
    y = orc.q8b_gemm(qa, da, qw, dw, m, k, n).astype(np.float64)
    _, terms = block_sums(qa, da, qw, dw)
    want = terms.sum(axis=2)
    bound = np.abs(terms).sum(axis=2) * (k // 32 + 2) * 2.0 ** -23
    assert (np.abs(y - want) <= bound).all()
    # Plausible mistakes do not fit the bound: the weight scales of the wrong
    # block, or one scale per weight row instead of per block.
    _, shifted = block_sums(qa, da, qw, np.roll(dw, 1, axis=1))
    assert not (np.abs(y - shifted.sum(axis=2)) <= bound).all()
    _, per_row = block_sums(qa, da, qw, np.repeat(dw[:, :1], k // 32, axis=1))
    assert not (np.abs(y - per_row.sum(axis=2)) <= bound).all()


def test_gemm_exact_on_exact_inputs():
    rng = np.random.default_rng(5)
    m, k, n = 4, 256, 9
    qa = rng.integers(-8, 9, (m, k)).astype(np.int8)
    qw = rng.integers(-8, 9, (n, k)).astype(np.int8)
    da = (2.0 ** rng.integers(-6, 3, (m, k // 32))).astype(np.float32)
    dw = (2.0 ** rng.integers(-6, 3, (n, k // 32))).astype(np.float32)
    y = orc.q8b_gemm(qa, da, qw, dw, m, k, n)
    _, terms = block_sums(qa, da, qw, dw)
    assert np.array_equal(y.astype(np.float64), terms.sum(axis=2))
