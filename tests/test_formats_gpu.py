"""GPU tests of the checkpoint loader (formats.load_lm, the reference's
loadGPU + loadHead, qwen3lm/gpu_darwin.go:161-373): a BF16 safetensors
checkpoint prepared on the device into cache entries, then mapped and
uploaded as it is; the GPTQ file's rows placed where it holds a projection.

The prepared bytes are held to gphq.prepare_lm over the same tensors (itself
bit-exact with the C oracle and decoding like transformers' Qwen3,
tests/test_prepare_gpu.py): every byte of every layer buffer and of the
head equal, from a fresh entry and from a committed one.
"""
import json

import numpy as np
import pytest

from gophonic_amd import formats as fm
from gophonic_amd import gphq
from tests import lm_common as lc
from tests.test_prepare_gpu import lmtest_checkpoint

pytestmark = pytest.mark.gpu

G = lc.GPU_SHAPE
GEOM = dict(hidden=G.hidden, layers=G.layers, heads=G.heads, kv_heads=G.kv_heads, head_dim=G.head_dim,
            intermediate=G.inter, vocab=G.vocab, max_positions=G.max_pos, eps=G.eps, rope_theta=G.theta)


def write_ckpt(path, tensors):
    import torch
    from safetensors.torch import save_file

    out = {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16).copy()).view(torch.bfloat16)
           for k, v in tensors.items()}
    save_file(out, str(path / "model.safetensors"))
    (path / "config.json").write_text(json.dumps({"hidden_size": G.hidden}))


def device_bytes(lm):
    """Every bound buffer of lm: the layer buffers, then the embedding, then the head."""
    return [b.view(-1).cpu().numpy().view(np.uint8) for b in lm._keep]


@pytest.mark.parametrize("fmt", [gphq.FMT_Q8B, gphq.FMT_Q4])
def test_loader_fresh_then_cached_equals_prepare(tmp_path, fmt):
    ck = tmp_path / "ckpt"
    ck.mkdir()
    tensors = lmtest_checkpoint(G, seed=17)
    write_ckpt(ck, tensors)
    want = device_bytes(gphq.prepare_lm(GEOM, fmt, tensors))
    cache = tmp_path / "cache"
    lm1, s1 = fm.load_lm(ck, GEOM, fmt, cache_dir=cache)
    assert s1["layers_fresh"] and s1["head_fresh"] and s1["gptq_placed"] == 0
    lm2, s2 = fm.load_lm(ck, GEOM, fmt, cache_dir=cache)
    assert not s2["layers_fresh"] and not s2["head_fresh"]
    for got in (device_bytes(lm1), device_bytes(lm2)):
        assert len(got) == len(want)
        for i, (a, b) in enumerate(zip(got, want)):
            assert np.array_equal(a, b), i
    # The two models decode alike, bit for bit.
    import torch

    outs = []
    for lm in (lm1, lm2):
        ws = gphq.DecodeBatch(lm, 1)
        kv = gphq.Prefix(lm, 16)
        out = torch.full((6, 1), -1, dtype=torch.int32, device="cuda")
        ws.greedy_run([kv], [0], [5], 6, out)
        ws.check()
        outs.append(out.cpu().numpy())
    np.testing.assert_array_equal(outs[0], outs[1])


def test_loader_places_gptq_rows(tmp_path):
    # gptq.go:170-190 place and gpu_darwin.go:438-485: a GPTQ file matching
    # the checkpoint replaces round-to-nearest for every projection it holds;
    # gate and up rows interleave (step 2).
    ck = tmp_path / "ckpt"
    ck.mkdir()
    tensors = lmtest_checkpoint(G, seed=18)
    write_ckpt(ck, tensors)
    cfg = gphq.lm_config(fmt=gphq.FMT_Q8, **GEOM)
    rng = np.random.default_rng(3)
    shapes = [(G.qd, G.hidden), (G.kvd, G.hidden), (G.kvd, G.hidden), (G.hidden, G.qd), (G.inter, G.hidden),
              (G.inter, G.hidden), (G.hidden, G.inter)]
    rows = {}
    w = fm.GptqWriter(ck, "gpu")
    for layer in range(G.layers):
        for name, (n, k) in zip(gphq.LAYER_PROJECTIONS, shapes):
            codes = rng.integers(-127, 128, (n, k), dtype=np.int8)
            scales = (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float32)
            w.write(codes)
            w.write(scales)
            rows[(layer, name)] = (codes, scales)
    w.commit()
    lm, stats = fm.load_lm(ck, GEOM, gphq.FMT_Q8, cache_dir=tmp_path / "cache")
    assert stats["gptq_placed"] == 7 * G.layers
    desc, _ = gphq.lm_layer_layout(cfg)
    bufs = device_bytes(lm)
    for layer in range(G.layers):
        b = bufs[layer]
        qkv = np.concatenate([rows[(layer, n)][0] for n in gphq.LAYER_PROJECTIONS[:3]])
        qkv_s = np.concatenate([rows[(layer, n)][1] for n in gphq.LAYER_PROJECTIONS[:3]])
        gate, up = rows[(layer, "mlp.gate_proj")], rows[(layer, "mlp.up_proj")]
        gu = np.empty((2 * G.inter, G.hidden), np.int8)
        gu[0::2], gu[1::2] = gate[0], up[0]
        gu_s = np.empty(2 * G.inter, np.float32)
        gu_s[0::2], gu_s[1::2] = gate[1], up[1]
        o, d = rows[(layer, "self_attn.o_proj")], rows[(layer, "mlp.down_proj")]
        for off, soff, codes, scales in ((desc.qkv, desc.qkv_scale, qkv, qkv_s), (desc.o, desc.o_scale, *o),
                                         (desc.gu, desc.gu_scale, gu, gu_s), (desc.d, desc.d_scale, *d)):
            assert np.array_equal(b[off:off + codes.size].view(np.int8), codes.reshape(-1))
            assert np.array_equal(b[soff:soff + 4 * scales.size].view(np.float32), scales)
