"""GPU parity of the GPTQ calibration pass (gphq_gptq_calibration_* and
gphq_gptq_quantize: QuantizeGPTQ and its calibration, qwen3lm/gptq.go:191-600)
through the C ABI, against the float64 oracle (oracle/gptq_oracle.py
CalibrationOracle, pinned by tests/test_gptq_oracle.py).

Each layer is checked in two parts, so that fp32 rounding on one side cannot
hide a mistake on the other:
* the forward pass: from the device's residual at the layer's start and the
  rounded matrices the device wrote (codes times scales, exactly the values
  its projections used), the oracle's float64 layer gives every set of rows
  the device keeps (attention input, context, MLP input, down input, the new
  residual) to relative L2 1e-5;
* the rounding: the oracle's GPTQ over the device's own inputs of each group
  (float64 factor, its own float64 GPU-basis matrices) picks the device's codes
  for >= 99% (8 bits) or 97% (4 bits, whose code boundaries lie 16 times
  closer) of the values of sampled rows, and the two roundings' output
  errors on those inputs agree to 2%: the factors differ by fp32 rounding, a
  value within that of a code boundary may go either way, and GPTQ's error
  feedback then carries the difference along the row (so codes may differ by
  more than one step there; with one shared factor they never do,
  tests/test_gptq_gpu.py); 8-bit row scales agree to 1e-6; GPTQ's output
  error on the device's inputs is below round-to-nearest's for every
  projection (gptq_linalg_test.go:72-148).
The whole producer (gphq_gptq_quantize) writes a GPHQ0001 file whose bytes
equal the layer-by-layer calls', which formats.load_lm places and decodes
like the float64 oracle over the placed bytes.
"""
import json

import numpy as np
import pytest

from gophonic_amd import formats as fm
from gophonic_amd import gphq
from oracle import gptq_oracle as go
from oracle import lm_oracle as lo
from tests import lm_common as lc
from tests.test_gptq_oracle import PROJ, cal_checkpoint, f32

pytestmark = pytest.mark.gpu

# Qwen3-0.6B's widths with 8 heads, two layers and a small vocabulary.
G = lo.Geometry(hidden=1024, layers=2, heads=8, kv_heads=4, head_dim=128, inter=2048, vocab=512, max_pos=512)
SAMPLE = 32  # rows per projection checked against the oracle's rounding


def cfg_of(g, fmt=gphq.FMT_Q8):
    return gphq.lm_config(hidden=g.hidden, layers=g.layers, heads=g.heads, kv_heads=g.kv_heads, head_dim=g.head_dim,
                          intermediate=g.inter, vocab=g.vocab, max_positions=g.max_pos, fmt=fmt, eps=g.eps,
                          rope_theta=g.theta)


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def shapes(g):
    return [(g.qd, g.hidden), (g.kvd, g.hidden), (g.kvd, g.hidden), (g.hidden, g.qd), (g.inter, g.hidden),
            (g.inter, g.hidden), (g.hidden, g.inter)]


def outputs(g, bits):
    import torch

    codes, scales = [], []
    for n, k in shapes(g):
        cb, sb = fm.gptq_row_bytes(bits, k)
        codes.append(torch.zeros(n * cb, dtype=torch.uint8, device="cuda"))
        scales.append(torch.zeros(n * sb, dtype=torch.uint8, device="cuda"))
    return codes, scales


def rounded(codes, scales, bits, n, k):
    """The rounded matrix the device used: float32(code * scale)."""
    if bits == 8:
        q = codes.view(np.int8).reshape(n, k).astype(np.float32)
        return (q * scales.view(np.float32)[:, None]).astype(np.float64)
    nib = codes.reshape(n, k // 32, 16)
    q = (np.concatenate([nib & 15, nib >> 4], axis=2).astype(np.float32) - 8)
    d = scales.view(np.float16).reshape(n, k // 32, 1).astype(np.float32)
    return (q * d).reshape(n, k).astype(np.float64)


def codes_of(codes, bits, n, k):
    if bits == 8:
        return codes.view(np.int8).reshape(n, k).astype(np.int64)
    nib = codes.reshape(n, k // 32, 16)
    return (np.concatenate([nib & 15, nib >> 4], axis=2).astype(np.int64) - 8).reshape(n, k)


def rel_l2(got, want):
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def sequences(g, lens, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, g.vocab, n).astype(np.int32).tolist() for n in lens]


@pytest.mark.parametrize("bits", [8, 4])
def test_calibration_layers_match_float64(bits):
    import torch

    g = G
    embed, layers = cal_checkpoint(g, 11 + bits)
    seqs = sequences(g, (37, 64, 1, 90), bits)
    print(f"gptq calibration bits={bits} rows={sum(map(len, seqs))} hidden={g.hidden}", flush=True)
    cal = gphq.GptqCalibration(cfg_of(g), seqs, dev(embed.view(np.int16)))
    orc = go.CalibrationOracle(g, embed, seqs)
    h0 = cal.rows(gphq.CAL_RESIDUAL).cpu().numpy().astype(np.float64)
    assert rel_l2(h0, orc.h) <= 1e-6
    keys = {gphq.CAL_ATTN_INPUT: "attn_input", gphq.CAL_CONTEXT: "context", gphq.CAL_MLP_INPUT: "mlp_input",
            gphq.CAL_DOWN_INPUT: "down_input", gphq.CAL_RESIDUAL: "residual"}
    inputs = [gphq.CAL_ATTN_INPUT] * 3 + [gphq.CAL_CONTEXT, gphq.CAL_MLP_INPUT, gphq.CAL_MLP_INPUT,
                                          gphq.CAL_DOWN_INPUT]
    for li, L in enumerate(layers):
        h_in = cal.rows(gphq.CAL_RESIDUAL).cpu().numpy().astype(np.float64)
        codes, scales = outputs(g, bits)
        srcs = [dev(p.view(np.int16)) for p in L["proj"]]
        print(f"  layer {li}", flush=True)
        cal.layer(srcs, f32(L["attn"]), f32(L["mlp"]), f32(L["qn"]), f32(L["kn"]), bits, codes, scales)
        torch.cuda.synchronize()
        got = {w: cal.rows(w).cpu().numpy().astype(np.float64) for w in keys}
        cs = [(c.cpu().numpy(), s.cpu().numpy()) for c, s in zip(codes, scales)]
        used = [rounded(c, s, bits, n, k) for (c, s), (n, k) in zip(cs, shapes(g))]
        # The forward pass through the device's rounded matrices.
        ref = orc.layer(used, f32(L["qn"]), f32(L["kn"]), h=h_in)
        for w, name in keys.items():
            e = rel_l2(got[w], ref[name])
            assert e <= 1e-5, (li, name, e)
        # The rounding of each projection over the device's inputs of its group.
        mats = orc.weights(L["proj"], f32(L["attn"]), f32(L["mlp"]))
        factors = {}
        for p, ((c, s), (n, k)) in enumerate(zip(cs, shapes(g))):
            x = got[inputs[p]]
            if inputs[p] not in factors:
                hh, dead = go.damp(go.hessian(x))
                factors[inputs[p]] = (go.inverse_factor(hh), dead)
            u, dead = factors[inputs[p]]
            w0 = mats[p].astype(np.float32)
            w0[:, dead] = 0
            rows = np.linspace(0, n - 1, SAMPLE).astype(int)
            want_codes, want_scales, want_w = go.round_rows(w0[rows], u, bits)
            q = codes_of(c, bits, n, k)[rows]
            wq = codes_of(want_codes.view(np.uint8), bits, len(rows), k)
            same = (q == wq).mean()
            w64 = w0[rows].astype(np.float64)
            e_dev = float(((x @ (w64 - used[p][rows]).T) ** 2).sum())
            e_orc = float(((x @ (w64 - want_w).T) ** 2).sum())
            print(f"    {PROJ[p]}: codes equal {same:.4f}, output error {e_dev / e_orc:.4f} of the oracle's",
                  flush=True)
            assert same >= (0.99 if bits == 8 else 0.97), (li, PROJ[p], same)
            assert abs(e_dev - e_orc) <= 0.02 * e_orc, (li, PROJ[p], e_dev, e_orc)
            if bits == 8:
                np.testing.assert_allclose(s.view(np.float32)[rows], want_scales, rtol=1e-6)
            # GPTQ beats round-to-nearest on its own inputs.
            if bits == 8:
                sc = np.abs(w0).max(axis=1) / np.float32(127)
                near = (np.rint(w0 / sc[:, None]).clip(-127, 127) * sc[:, None]).astype(np.float64)
            else:
                near = np.empty((n, k))
                for r in range(n):
                    for b in range(0, k, 32):
                        d = np.float32(go.q4_group_scale(w0[r, b:b + 32]))
                        near[r, b:b + 32] = np.clip(np.rint(w0[r, b:b + 32] / d), -8, 7) * np.float64(d)
            err = lambda qv: float(((x @ (w0.astype(np.float64) - qv).T) ** 2).sum())
            assert err(used[p]) < err(near), (li, PROJ[p])
    cal.close()


def test_calibration_validates_like_the_reference():
    import torch

    g = G
    embed = torch.zeros(g.vocab * g.hidden, dtype=torch.int16, device="cuda")
    with pytest.raises(gphq.GphqError) as e:
        gphq.GptqCalibration(cfg_of(g), [], embed)
    assert e.value.status == gphq.ERR_CALIBRATION_EMPTY and str(e.value) == "qwen3: empty calibration set"
    for lens in ((257,), (256,) * 16 + (1,), (3, 0)):
        with pytest.raises(gphq.GphqError) as e:
            gphq.GptqCalibration(cfg_of(g), [[1] * n for n in lens], embed)
        assert e.value.status == gphq.ERR_CALIBRATION_SHAPE
    with pytest.raises(gphq.GphqError) as e:
        gphq.GptqCalibration(cfg_of(g), [[1, g.vocab]], embed)
    assert e.value.status == gphq.ERR_TOKEN_VOCAB
    cal = gphq.GptqCalibration(cfg_of(g), [[1, 2, 3]], embed)
    codes, scales = outputs(g, 8)
    srcs = [torch.zeros(n * k, dtype=torch.int16, device="cuda") for n, k in shapes(g)]
    one = np.ones(g.hidden, np.float32)
    with pytest.raises(gphq.GphqError) as e:
        cal.layer(srcs, one, one, one[:128], one[:128], 3, codes, scales)
    assert e.value.status == gphq.ERR_UNSUPPORTED
    cal.close()


# ---- the whole producer: checkpoint in, GPHQ0001 file out ---------------------------

# The reference requires projection widths that are multiples of 4096
# (gptq.go:211-213): Qwen3-8B's hidden and head widths, one 4096-wide MLP block.
G8 = lo.Geometry(hidden=4096, layers=2, heads=32, kv_heads=8, head_dim=128, inter=4096, vocab=256, max_pos=512)


def write_checkpoint(path, g, seed):
    import torch
    from safetensors.torch import save_file

    embed, layers = cal_checkpoint(g, seed)
    rng = np.random.default_rng(seed + 1)
    t = {"model.embed_tokens.weight": embed,
         "model.norm.weight": lc.bf16_bits((1 + 0.1 * rng.standard_normal(g.hidden)).astype(np.float32)),
         "lm_head.weight": lc.bf16_bits((0.02 * rng.standard_normal((g.vocab, g.hidden))).astype(np.float32))}
    for i, L in enumerate(layers):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = L["attn"]
        t[p + "post_attention_layernorm.weight"] = L["mlp"]
        t[p + "self_attn.q_norm.weight"] = L["qn"]
        t[p + "self_attn.k_norm.weight"] = L["kn"]
        for name, bits in zip(PROJ, L["proj"]):
            t[p + name + ".weight"] = bits
    out = {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16).copy()).view(torch.bfloat16)
           for k, v in t.items()}
    save_file(out, str(path / "model.safetensors"))
    (path / "config.json").write_text(json.dumps({"hidden_size": g.hidden}))
    return embed, layers, t


@pytest.mark.parametrize("fmt", ["gpu", "gpu-q4"])
def test_quantize_writes_the_file_load_lm_places_and_decodes(tmp_path, fmt):
    import torch

    from tests.test_prepare_gpu import stored_layers

    g = G8
    bits = 8 if fmt == "gpu" else 4
    lfmt = gphq.FMT_Q8 if bits == 8 else gphq.FMT_Q4
    ck = tmp_path / "ckpt"
    ck.mkdir()
    embed, layers, tensors = write_checkpoint(ck, g, 21)
    texts = sequences(g, (300, 50, 7), 22)  # 300 tokens are cut into 256 + 44
    seq_lens = gphq.gptq_calibration_sequences([len(t) for t in texts])
    assert seq_lens.tolist() == [256, 44, 50, 7]
    seen = []
    print(f"gptq quantize {fmt} hidden={g.hidden} layers={g.layers}", flush=True)
    gphq.gptq_quantize(ck, fmt, cfg_of(g, lfmt), texts, progress=lambda l, n: seen.append((l, n)))
    assert seen == [(1, 2), (2, 2)]
    raw = open(fm.gptq_path(ck, fmt), "rb").read()
    assert raw[:8] == b"GPHQ0001" and int.from_bytes(raw[8:16], "little") == bits
    assert int.from_bytes(raw[16:24], "little") == fm.gptq_fingerprint(ck)
    # The same bytes as the layer-by-layer calls over the same sequences.
    flat = np.concatenate([np.asarray(t, np.int32) for t in texts])
    seqs, off = [], 0
    for n in seq_lens:
        seqs.append(flat[off:off + n].tolist())
        off += n
    cal = gphq.GptqCalibration(cfg_of(g), seqs, dev(embed.view(np.int16)))
    at = 24
    for L in layers:
        codes, scales = outputs(g, bits)
        cal.layer([dev(p.view(np.int16)) for p in L["proj"]], f32(L["attn"]), f32(L["mlp"]), f32(L["qn"]),
                  f32(L["kn"]), bits, codes, scales)
        for c, s in zip(codes, scales):
            for part in (c, s):
                b = part.cpu().numpy().tobytes()
                assert raw[at:at + len(b)] == b, at
                at += len(b)
    assert at == len(raw)
    cal.close()
    # load_lm places every projection from the file, and the model decodes
    # like the float64 oracle over the placed bytes.
    geom = dict(hidden=g.hidden, layers=g.layers, heads=g.heads, kv_heads=g.kv_heads, head_dim=g.head_dim,
                intermediate=g.inter, vocab=g.vocab, max_positions=g.max_pos, eps=g.eps, rope_theta=g.theta)
    lm, stats = fm.load_lm(ck, geom, lfmt, cache_dir=tmp_path / "cache")
    assert stats["gptq_placed"] == 7 * g.layers
    stored, head = stored_layers(lm, g, lfmt)
    for L, S in zip(layers, stored):
        S.q_norm, S.k_norm = f32(L["qn"]), f32(L["kn"])
    oracle = lo.DecodeOracle(g, lfmt, stored, embed, f32(tensors["model.norm.weight"]), head)
    cache = oracle.new_cache(16)
    ws = gphq.DecodeBatch(lm, 1)
    kv = gphq.Prefix(lm, 16)
    hidden = torch.empty((1, g.hidden), device="cuda")
    logits = torch.empty((1, g.vocab), device="cuda")
    for pos, tok in enumerate([5, 17, 200, 3]):
        ws.into([kv], [pos], [tok], hidden, logits)
        _, want, _ = oracle.step(cache, pos, tok)
        assert rel_l2(logits.cpu().numpy()[0].astype(np.float64), want) <= 1e-5, pos
    ws.check()


def test_quantize_rejects_like_the_reference(tmp_path):
    g = G8
    with pytest.raises(gphq.GphqError, match='GPTQ supports "gpu" and "gpu-q4", not "gpu-q8"'):
        gphq.gptq_quantize(tmp_path, "gpu-q8", cfg_of(g), [[1, 2]])
    narrow = lo.Geometry(hidden=1024, layers=1, heads=8, kv_heads=4, head_dim=128, inter=4096, vocab=256, max_pos=64)
    with pytest.raises(gphq.GphqError) as e:
        gphq.gptq_quantize(tmp_path, "gpu", cfg_of(narrow), [[1, 2]])
    assert e.value.status == gphq.ERR_GPTQ_WIDTH
    assert str(e.value) == "qwen3: GPTQ needs projection widths that are multiples of 4096"
    with pytest.raises(gphq.GphqError) as e:
        gphq.gptq_quantize(tmp_path, "gpu", cfg_of(g), [[], []])
    assert e.value.status == gphq.ERR_CALIBRATION_EMPTY
    with pytest.raises(gphq.GphqError) as e:  # no checkpoint in the directory
        gphq.gptq_quantize(tmp_path, "gpu", cfg_of(g), [[1, 2]])
    assert e.value.status == gphq.ERR_IO
    assert not list(tmp_path.iterdir())  # no file left behind
