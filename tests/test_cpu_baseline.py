"""The CPU baseline's decode step (oracle/gphq_oracle.c orc_lm_step_i8, timed
by bench.py beside the GPU decode). It carries no parity claim; these checks
hold it to what a timing baseline must do: the same work whatever the worker
count, finite output, and the residual really updated by every layer."""
import ctypes

import numpy as np

from oracle import cpu_baseline as cb
from oracle import oracle as orc

GEOM = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, intermediate=512, vocab=300)


def run_step(threads, layers=None):
    lib = orc.lib()
    lib.orc_lm_step_i8.restype = None
    lib.orc_lm_step_i8.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] + [ctypes.c_void_p] * 7 + [ctypes.c_int]
    g = dict(GEOM)
    H, I, hd = g["hidden"], g["intermediate"], g["head_dim"]
    qd, kvd = g["heads"] * hd, g["kv_heads"] * hd
    L = g["layers"] if layers is None else layers
    rng = np.random.default_rng(5)
    keep = []
    arr = (cb._Layer * max(L, 1))()
    for li in range(L):
        for p, (n, k) in enumerate([(qd, H), (kvd, H), (kvd, H), (H, qd), (I, H), (I, H), (H, I)]):
            w = rng.integers(-127, 128, n * k, dtype=np.int8)
            s = (np.abs(rng.standard_normal(n)) * 0.002).astype(np.float32)
            keep += [w, s]
            arr[li].w[p], arr[li].s[p] = w.ctypes.data, s.ctypes.data
        for name, n in (("attn_norm", H), ("mlp_norm", H), ("q_norm", hd), ("k_norm", hd)):
            v = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
            keep.append(v)
            setattr(arr[li], name, v.ctypes.data)
    ctx, cap = 5, 8
    geom = cb._Geom(H, g["heads"], g["kv_heads"], hd, I, g["vocab"], L, cap, 1e-6)
    kc = rng.standard_normal(max(L, 1) * cap * kvd).astype(np.float32)
    vc = rng.standard_normal(max(L, 1) * cap * kvd).astype(np.float32)
    inv = 1.0 / np.power(1e6, (2.0 * np.arange(hd // 2)) / hd)
    cosv, sinv = np.cos(ctx * inv).astype(np.float32), np.sin(ctx * inv).astype(np.float32)
    head = rng.integers(-127, 128, g["vocab"] * H, dtype=np.int8)
    head_s = (np.abs(rng.standard_normal(g["vocab"])) * 0.002).astype(np.float32)
    fnorm = np.ones(H, np.float32)
    h = rng.standard_normal(H).astype(np.float32)
    h0 = h.copy()
    logits = np.zeros(g["vocab"], np.float32)
    lib.orc_lm_step_i8(ctypes.byref(geom), arr, kc.ctypes.data, vc.ctypes.data, ctx, cosv.ctypes.data,
                       sinv.ctypes.data, fnorm.ctypes.data, head.ctypes.data, head_s.ctypes.data, h.ctypes.data,
                       logits.ctypes.data, threads)
    return h0, h, logits, kc, vc


def test_step_independent_of_workers():
    ref = run_step(1)
    for t in (2, 3, 7):
        got = run_step(t)
        for a, b in zip(ref, got):
            np.testing.assert_array_equal(a, b)


def test_step_updates_residual_and_cache():
    h0, h, logits, kc, vc = run_step(2)
    assert np.all(np.isfinite(h)) and np.all(np.isfinite(logits))
    assert not np.array_equal(h0, h)
    assert np.abs(logits).max() > 0
    # No layers: the residual passes through and only the head runs.
    h0z, hz, lz, _, _ = run_step(2, layers=0)
    np.testing.assert_array_equal(h0z, hz)
    assert np.abs(lz).max() > 0
