"""The CPU baseline's decode step (oracle/gphq_oracle.c orc_lm_step_i8, timed
by bench.py beside the GPU decode for configurations 3 and 4b): the
reference's CPU int8 path (qwen3lm/ops.go:96-254 over WeightsInt8 rows).

Pinned in two steps:
* the float64 CpuInt8Oracle (oracle/lm_oracle.py) with its activations left
  unquantized is the model's own forward pass: on the same BF16 model it gives
  the hidden state and logits of DecodeOracle.step (the GPU-basis decode
  oracle, pinned to transformers' Qwen3 in tests/test_oracle_lm.py), whose
  weights are stored in the other basis (norms folded, residual rotated);
* the C step equals CpuInt8Oracle with int8 activations to relative L2 1e-5
  (residual, logits and the appended K/V rows), so the quantization points,
  the rotations and the int8 products are the reference's.
Besides: the same work whatever the worker count, and the residual passing
through unchanged with no layers."""
import ctypes

import numpy as np

from oracle import cpu_baseline as cb
from oracle import gptq_oracle as go
from oracle import lm_oracle as lo
from oracle import oracle as orc
from tests import lm_common as lc

GEOM = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, intermediate=512, vocab=300)
G = lo.Geometry(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=300, max_pos=64)


def make_inputs(layers=None, seed=5):
    g = dict(GEOM)
    H, I, hd = g["hidden"], g["intermediate"], g["head_dim"]
    qd, kvd = g["heads"] * hd, g["kv_heads"] * hd
    L = g["layers"] if layers is None else layers
    rng = np.random.default_rng(seed)
    lay = []
    for _ in range(L):
        d = dict(w=[], s=[])
        for n, k in [(qd, H), (kvd, H), (kvd, H), (H, qd), (I, H), (I, H), (H, I)]:
            d["w"].append(rng.integers(-127, 128, (n, k), dtype=np.int8))
            d["s"].append((np.abs(rng.standard_normal(n)) * 0.002).astype(np.float32))
        for name, n in (("attn_norm", H), ("mlp_norm", H), ("q_norm", hd), ("k_norm", hd)):
            d[name] = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
        lay.append(d)
    ctx, cap = 5, 8
    kc = rng.standard_normal((max(L, 1), cap, kvd)).astype(np.float32)
    vc = rng.standard_normal((max(L, 1), cap, kvd)).astype(np.float32)
    inv = 1.0 / np.power(1e6, (2.0 * np.arange(hd // 2)) / hd)
    cosv, sinv = np.cos(ctx * inv).astype(np.float32), np.sin(ctx * inv).astype(np.float32)
    head = (rng.integers(-127, 128, (g["vocab"], H), dtype=np.int8),
            (np.abs(rng.standard_normal(g["vocab"])) * 0.002).astype(np.float32))
    fnorm = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
    h = rng.standard_normal(H).astype(np.float32)
    return dict(layers=lay, kc=kc, vc=vc, pos=ctx, cap=cap, cos=cosv, sin=sinv, head=head, fnorm=fnorm, h=h)


def run_step(threads, layers=None, inputs=None):
    lib = orc.lib()
    lib.orc_lm_step_i8.restype = None
    lib.orc_lm_step_i8.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] + [ctypes.c_void_p] * 7 + [ctypes.c_int]
    d = make_inputs(layers) if inputs is None else inputs
    g = GEOM
    L = len(d["layers"])
    arr = (cb._Layer * max(L, 1))()
    for li, lay in enumerate(d["layers"]):
        for p in range(7):
            arr[li].w[p], arr[li].s[p] = lay["w"][p].ctypes.data, lay["s"][p].ctypes.data
        for name in ("attn_norm", "mlp_norm", "q_norm", "k_norm"):
            setattr(arr[li], name, lay[name].ctypes.data)
    geom = cb._Geom(g["hidden"], g["heads"], g["kv_heads"], g["head_dim"], g["intermediate"], g["vocab"], L, d["cap"],
                    1e-6)
    kc, vc, h = d["kc"].copy(), d["vc"].copy(), d["h"].copy()
    logits = np.zeros(g["vocab"], np.float32)
    lib.orc_lm_step_i8(ctypes.byref(geom), arr, kc.ctypes.data, vc.ctypes.data, d["pos"], d["cos"].ctypes.data,
                       d["sin"].ctypes.data, d["fnorm"].ctypes.data, d["head"][0].ctypes.data,
                       d["head"][1].ctypes.data, h.ctypes.data, logits.ctypes.data, threads)
    return d["h"], h, logits, kc, vc


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


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


def test_c_step_equals_the_float64_int8_step():
    d = make_inputs()
    h0, h, logits, kc, vc = run_step(3, inputs=d)
    orc8 = lo.CpuInt8Oracle(G, d["layers"], d["fnorm"], d["head"])
    kc64, vc64 = d["kc"].astype(np.float64), d["vc"].astype(np.float64)
    want_h, _, want_logits = orc8.step(d["h"], kc64, vc64, d["pos"], d["cos"], d["sin"])
    assert rel_l2(h, want_h) <= 1e-5
    assert rel_l2(logits, want_logits) <= 1e-5
    for got, want in ((kc, kc64), (vc, vc64)):
        np.testing.assert_allclose(got[:, d["pos"]], want[:, d["pos"]], rtol=0,
                                   atol=1e-5 * np.abs(want[:, d["pos"]]).max())
        np.testing.assert_array_equal(np.delete(got, d["pos"], axis=1), np.delete(want, d["pos"], axis=1))


def test_float64_int8_step_is_the_model_in_the_cpu_basis():
    # The same BF16 model stored both ways: the CPU provider's rows W R_in^T
    # with the norms applied to the activations (CpuInt8Oracle, unquantized),
    # and the GPU basis with the norms folded and the residual rotated
    # (calibration.weights' transform, DecodeOracle). Both must give the
    # model's hidden state and logits; the float32 rotation scale makes R^T R
    # = (1 + 3.4e-8) I for blocks 128 and 512, so the bound is 1e-6.
    g = G
    from tests.test_gptq_oracle import cal_checkpoint, f32

    embed, layers = cal_checkpoint(g, 9)
    rng = np.random.default_rng(10)
    head = lc.bf16_bits((0.02 * rng.standard_normal((g.vocab, g.hidden))).astype(np.float32))
    fnorm = f32(lc.bf16_bits((1 + 0.1 * rng.standard_normal(g.hidden)).astype(np.float32)))
    cal = go.CalibrationOracle(g, embed, [[0]])
    cpu_layers, W = [], []
    for L in layers:
        raw = [lo.bf16_to_f64(p).reshape(p.shape) for p in L["proj"]]
        # The CPU rows: each weight row rotated by its input rotation; o's is
        # newRotation(q_dim), not the GPU basis' per-head one.
        rot_cpu = [lo.rotation(g.hidden)] * 3 + [lo.rotation(g.qd)] + [lo.rotation(g.hidden)] * 2 + \
                  [lo.rotation(g.inter)]
        cpu_layers.append(dict(w=[lo.rot_apply(w, r).reshape(w.shape) for w, r in zip(raw, rot_cpu)], s=[None] * 7,
                               attn_norm=f32(L["attn"]), mlp_norm=f32(L["mlp"]), q_norm=f32(L["qn"]),
                               k_norm=f32(L["kn"])))
        m = cal.weights(L["proj"], f32(L["attn"]), f32(L["mlp"]))
        gu = np.empty((2 * g.inter, g.hidden))
        gu[0::2], gu[1::2] = m[4], m[5]
        W.append(dict(qkv=np.vstack(m[:3]), o=m[3], gu=gu, down=m[6], qn=f32(L["qn"]).astype(np.float64),
                      kn=f32(L["kn"]).astype(np.float64)))
    head64 = lo.bf16_to_f64(head).reshape(g.vocab, g.hidden)
    cpu = lo.CpuInt8Oracle(g, cpu_layers, fnorm, (lo.rot_apply(head64, lo.rotation(g.hidden)).reshape(head64.shape),
                                                  None), quantize=False)
    dec = lo.DecodeOracle(g, lo.FMT_Q8, [], embed, fnorm, (np.zeros(g.head_rows * g.hidden, np.int8),
                                                           np.zeros(g.head_rows * g.hidden // 32, np.uint16)))
    dec.W = W
    dec._head = lo.rot_apply(head64, lo.rotation(g.hidden)).reshape(head64.shape)
    cache = dec.new_cache(8)
    kc = [np.zeros((8, g.kvd)) for _ in range(g.layers)]
    vc = [np.zeros((8, g.kvd)) for _ in range(g.layers)]
    cos, sin = lo.rope_table(g, 8)
    vrot = lo.head_rotation(g.head_dim, g.kvd)
    for pos, tok in enumerate([3, 77, 150, 299]):
        want_hidden, want_logits, _ = dec.step(cache, pos, tok)
        _, hidden, logits = cpu.step(lo.bf16_to_f64(embed.reshape(g.vocab, g.hidden)[tok]), kc, vc, pos, cos[pos],
                                     sin[pos])
        assert rel_l2(hidden, want_hidden) <= 1e-6, pos
        assert rel_l2(logits, want_logits) <= 1e-6, pos
        for li in range(g.layers):
            # The GPU basis keeps value rows per-head rotated.
            np.testing.assert_allclose(lo.rot_apply(vc[li][pos], vrot), cache[li][1][pos], rtol=0, atol=1e-6)
            np.testing.assert_allclose(kc[li][pos], cache[li][0][pos], rtol=0, atol=1e-6)
