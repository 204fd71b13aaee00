"""CPU tests of the file formats behind the C ABI: safetensors checkpoints
(internal/safetensors), the GPTQ weight file (qwen3lm/gptq.go) and the
prepared-weight cache (internal/wcache).

Files are written by independent code: the safetensors package (Hugging
Face's own writer), numpy, and the byte layouts the reference documents;
hashes are checked against hashlib (SHA-256) and the published FNV-1a basis.
The wcache tests follow the reference's wcache_test.go.
"""
import hashlib
import json
import os
import threading
import time

import numpy as np
import pytest

from gophonic_amd import formats as fm
from gophonic_amd import gphq

torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")


def write_checkpoint(path, tensors, name="model.safetensors", metadata=None):
    st_torch.save_file({k: v.contiguous() for k, v in tensors.items()}, os.path.join(path, name),
                       metadata=metadata)


def bf16_bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.fixture
def ckpt(tmp_path):
    g = torch.Generator().manual_seed(3)
    t = {
        "model.embed_tokens.weight": torch.randn(8, 64, generator=g).to(torch.bfloat16),
        "model.layers.0.self_attn.q_proj.weight": torch.randn(32, 64, generator=g).to(torch.bfloat16),
        "model.norm.weight": torch.randn(64, generator=g).to(torch.float16),
        "lm_head.weight": torch.randn(8, 64, generator=g),
    }
    write_checkpoint(tmp_path, t, metadata={"format": "pt"})
    return tmp_path, t


def test_safetensors_read_bf16_f16_f32(ckpt):
    path, t = ckpt
    c = fm.Checkpoint(path)
    assert c.has("model.norm.weight") and not c.has("model.norm")
    assert c.info("model.layers.0.self_attn.q_proj.weight") == ("BF16", (32, 64))
    assert c.lookup("lm_head.weight", 8, 64) == "F32"
    q = c.bf16("model.layers.0.self_attn.q_proj.weight", 32, 64)
    np.testing.assert_array_equal(q, bf16_bits(t["model.layers.0.self_attn.q_proj.weight"]))
    # ReadBits from an element offset (safetensors.go:203-213).
    np.testing.assert_array_equal(c.read_bits("model.embed_tokens.weight", 70, 100),
                                  bf16_bits(t["model.embed_tokens.weight"]).reshape(-1)[100:170])
    # Float32 widens each dtype exactly.
    np.testing.assert_array_equal(c.float32("model.norm.weight", 64), t["model.norm.weight"].float().numpy())
    np.testing.assert_array_equal(c.float32("lm_head.weight", 8, 64), t["lm_head.weight"].numpy())
    np.testing.assert_array_equal(c.float32("model.embed_tokens.weight", 8, 64),
                                  t["model.embed_tokens.weight"].float().numpy())
    bits, release = c.map_bf16("model.embed_tokens.weight", 8, 64)
    np.testing.assert_array_equal(bits, bf16_bits(t["model.embed_tokens.weight"]))
    release()
    c.close()


def test_safetensors_errors_carry_the_reference_messages(ckpt):
    path, _ = ckpt
    c = fm.Checkpoint(path)
    cases = [
        (lambda: c.lookup("nope", 1), gphq.ERR_TENSOR_MISSING, "checkpoint is missing nope"),
        (lambda: c.lookup("lm_head.weight", 8, 65), gphq.ERR_TENSOR_SHAPE, "lm_head.weight has shape [8 64], want [8 65]"),
        (lambda: c.lookup("lm_head.weight", 512), gphq.ERR_TENSOR_SHAPE, "lm_head.weight has shape [8 64], want [512]"),
        (lambda: c.bf16("lm_head.weight", 8, 64), gphq.ERR_TENSOR_DTYPE,
         "lm_head.weight is F32; the loader expects the official BF16 checkpoint"),
        (lambda: c.read_bits("model.norm.weight", 10, 60), gphq.ERR_READ_RANGE, "read outside the tensor"),
    ]
    for fn, status, msg in cases:
        with pytest.raises(gphq.GphqError) as e:
            fn()
        assert e.value.status == status and str(e.value) == msg


def test_safetensors_rejects_non_finite_and_bad_files(tmp_path):
    write_checkpoint(tmp_path, {"w": torch.tensor([1.0, float("inf")], dtype=torch.bfloat16)})
    c = fm.Checkpoint(tmp_path)
    with pytest.raises(gphq.GphqError, match="w has a non-finite value"):
        c.float32("w", 2)
    c.close()
    bad = tmp_path / "bad"
    bad.mkdir()
    (bad / "model.safetensors").write_bytes((10 ** 9).to_bytes(8, "little") + b"{}")
    with pytest.raises(gphq.GphqError, match="invalid safetensors header length") as e:
        fm.Checkpoint(bad)
    assert e.value.status == gphq.ERR_FORMAT
    header = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 64]}}).encode()
    (bad / "model.safetensors").write_bytes(len(header).to_bytes(8, "little") + header + bytes(16))
    with pytest.raises(gphq.GphqError, match="tensor x has invalid data offsets"):
        fm.Checkpoint(bad)
    with pytest.raises(gphq.GphqError) as e:
        fm.Checkpoint(tmp_path / "missing")
    assert e.value.status == gphq.ERR_IO


def test_safetensors_f16_widening_is_exact_for_every_finite_value(tmp_path):
    # safetensors.go:255-270 F16ToF32 against numpy's IEEE conversion.
    h = np.arange(65536, dtype=np.uint16)
    finite = h[np.isfinite(h.view(np.float16))]
    write_checkpoint(tmp_path, {"h": torch.from_numpy(finite.view(np.int16).copy()).view(torch.float16)})
    c = fm.Checkpoint(tmp_path)
    got = c.float32("h", finite.size)
    np.testing.assert_array_equal(got.view(np.uint32), finite.view(np.float16).astype(np.float32).view(np.uint32))


def test_safetensors_sharded_index(tmp_path):
    a = {"a.weight": torch.arange(6, dtype=torch.float32).reshape(2, 3).to(torch.bfloat16)}
    b = {"b.weight": torch.ones(4, dtype=torch.float32)}
    write_checkpoint(tmp_path, a, "model-00001-of-00002.safetensors")
    write_checkpoint(tmp_path, b, "model-00002-of-00002.safetensors")
    index = {"metadata": {"total_size": 28}, "weight_map": {"a.weight": "model-00001-of-00002.safetensors",
                                                           "b.weight": "model-00002-of-00002.safetensors"}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    c = fm.Checkpoint(tmp_path)
    np.testing.assert_array_equal(c.bf16("a.weight", 2, 3), bf16_bits(a["a.weight"]))
    np.testing.assert_array_equal(c.float32("b.weight", 4), np.ones(4, np.float32))
    index["weight_map"]["b.weight"] = "../x.safetensors"
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    with pytest.raises(gphq.GphqError, match="is not a plain file name"):
        fm.Checkpoint(tmp_path)


# ---- GPTQ file --------------------------------------------------------------------

def fnv1a64(data):
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & (2 ** 64 - 1)
    return h


def test_gptq_fingerprint_is_fnv1a_over_the_snapshot_listing(tmp_path):
    assert fm.gptq_fingerprint(tmp_path) == 0xCBF29CE484222325  # FNV-1a 64 of nothing: the offset basis
    (tmp_path / "model-00001.safetensors").write_bytes(b"abc")
    (tmp_path / "config.json").write_text("{}")
    (tmp_path / "tokenizer.json").write_text("{}")  # not part of the snapshot
    lines = ""
    for n in sorted(["model-00001.safetensors", "config.json"]):
        s = os.stat(tmp_path / n)
        lines += f"{n} {s.st_size} {s.st_mtime_ns}\n"
    assert fm.gptq_fingerprint(tmp_path) == fnv1a64(lines.encode())
    assert fm.gptq_path(tmp_path, "gpu-q4") == os.path.join(str(tmp_path), "gophonic-gptq-gpu-q4.bin")


def tiny_cfg(fmt=gphq.FMT_Q8):
    return gphq.lm_config(hidden=256, layers=2, heads=2, kv_heads=1, head_dim=128, intermediate=512, vocab=96,
                          max_positions=64, fmt=fmt)


PROJ = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
        "mlp.up_proj", "mlp.down_proj"]


def proj_shapes(cfg):
    h, qd, kv, i = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim, cfg.intermediate
    return [(qd, h), (kv, h), (kv, h), (h, qd), (i, h), (i, h), (h, i)]


def write_gptq(path, fmt, cfg, seed=0):
    """A GPTQ file for cfg with random rows; returns {name: (codes, scales)}."""
    bits = 8 if fmt == "gpu" else 4
    rng = np.random.default_rng(seed)
    w = fm.GptqWriter(path, fmt)
    want = {}
    for layer in range(cfg.layers):
        for name, (n, k) in zip(PROJ, proj_shapes(cfg)):
            cb, sb = fm.gptq_row_bytes(bits, k)
            codes = rng.integers(0, 256, n * cb, dtype=np.uint8)
            scales = rng.integers(0, 256, n * sb, dtype=np.uint8)
            w.write(codes)
            w.write(scales)
            want[f"layers.{layer}.{name}.weight"] = (codes, scales)
    w.commit()
    return want


@pytest.mark.parametrize("fmt", ["gpu", "gpu-q4"])
def test_gptq_file_round_trip_and_offsets(tmp_path, fmt):
    (tmp_path / "model.safetensors").write_bytes(b"weights")
    cfg = tiny_cfg(gphq.FMT_Q8 if fmt == "gpu" else gphq.FMT_Q4)
    want = write_gptq(tmp_path, fmt, cfg)
    raw = open(fm.gptq_path(tmp_path, fmt), "rb").read()
    bits = 8 if fmt == "gpu" else 4
    assert raw[:8] == b"GPHQ0001" and int.from_bytes(raw[8:16], "little") == bits
    assert int.from_bytes(raw[16:24], "little") == fm.gptq_fingerprint(tmp_path)
    g = fm.GptqFile.open(tmp_path, fmt, cfg)
    assert g is not None and g.bits == bits
    for name, (codes, scales) in want.items():
        c0, s0 = g.projection(name)
        assert raw[c0:c0 + codes.size] == codes.tobytes() and raw[s0:s0 + scales.size] == scales.tobytes()
    assert g.projection("layers.2.mlp.up_proj.weight") is None  # past the layers
    assert g.projection("layers.0.mlp.gate.weight") is None
    assert g.projection("embed_tokens.weight") is None
    g.close()
    other = "gpu-q4" if fmt == "gpu" else "gpu"
    assert fm.GptqFile.open(tmp_path, other, cfg) is None  # no file for the other format


def test_gptq_file_ignored_when_stale_or_truncated(tmp_path):
    (tmp_path / "model.safetensors").write_bytes(b"v1")
    cfg = tiny_cfg()
    write_gptq(tmp_path, "gpu", cfg)
    assert fm.GptqFile.open(tmp_path, "gpu", cfg) is not None
    bigger = gphq.lm_config(hidden=256, layers=3, heads=2, kv_heads=1, head_dim=128, intermediate=512, vocab=96,
                            max_positions=64, fmt=gphq.FMT_Q8)
    assert fm.GptqFile.open(tmp_path, "gpu", bigger) is None  # size of another model
    time.sleep(0.01)
    (tmp_path / "model.safetensors").write_bytes(b"v2")  # the checkpoint changed
    assert fm.GptqFile.open(tmp_path, "gpu", cfg) is None
    with pytest.raises(gphq.GphqError, match='GPTQ supports "gpu" and "gpu-q4", not "gpu-q8"'):
        fm.GptqWriter(tmp_path, "gpu-q8")


@pytest.mark.parametrize("fmt", ["gpu", "gpu-q4"])
def test_gptq_place_rejects_a_shape_other_than_the_files(tmp_path, fmt):
    # place reads n rows of the projection's row bytes from the file's own
    # offsets, so n and k must be the projection's shape under the file's
    # configuration; anything else would read the next projection's bytes.
    # The check comes before any device work, so a host buffer stands in.
    import torch

    (tmp_path / "model.safetensors").write_bytes(b"weights")
    cfg = tiny_cfg(gphq.FMT_Q8 if fmt == "gpu" else gphq.FMT_Q4)
    write_gptq(tmp_path, fmt, cfg)
    g = fm.GptqFile.open(tmp_path, fmt, cfg)
    buf = torch.zeros(1 << 20, dtype=torch.uint8)
    name = "layers.1.mlp.up_proj.weight"
    n, k = proj_shapes(cfg)[5]
    for bad_n, bad_k in [(n, k + 32), (n, k - 32), (n + 1, k), (n - 1, k)]:
        with pytest.raises(gphq.GphqError) as e:
            g.place(name, bad_n, bad_k, buf, 0, 1 << 19)
        assert e.value.status == gphq.ERR_DIMENSIONS
        assert f"is {n}x{k} in the file, not {bad_n}x{bad_k}" in str(e.value)
    assert not buf.any()
    g.close()


# ---- weight cache -----------------------------------------------------------------

def test_sha256_known_answers():
    assert fm.sha256(b"").hex() == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    assert fm.sha256(b"abc").hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    rng = np.random.default_rng(1)
    for n in (55, 56, 63, 64, 65, 1000, 4099):
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert fm.sha256(data) == hashlib.sha256(data).digest(), n


def test_key_hashes_path_parts_and_files(tmp_path):
    ck = tmp_path / "Qwen3 8B.é"
    ck.mkdir()
    (ck / "model.safetensors").write_bytes(b"v1")
    (ck / "config.json").write_text("{}")
    os.symlink(ck / "config.json", ck / "link.json")  # not a regular file: left out
    key = fm.wcache_key(ck, "gpu-q8", "v1", "opt")
    h = hashlib.sha256()
    for p in ("v1", "opt"):
        h.update(p.encode() + b"\0")
    for n in sorted(os.listdir(ck)):
        s = os.lstat(ck / n)
        if os.path.islink(ck / n):
            continue
        h.update(f"{n}\0{s.st_size}\0{s.st_mtime_ns}\0".encode())
    where = hashlib.sha256(str(ck).encode()).hexdigest()[:8]
    assert key == f"Qwen3_8B__-{where}.gpu-q8.{h.hexdigest()[:24]}"
    assert fm.wcache_round_up(0) == fm.WCACHE_ALIGN and fm.wcache_round_up(fm.WCACHE_ALIGN + 1) == 2 * fm.WCACHE_ALIGN


def test_fresh_then_mapped(tmp_path):
    # wcache_test.go:13-70 TestFreshThenMapped.
    cache = tmp_path / "cache"
    ck = tmp_path / "ckpt"
    ck.mkdir()
    (ck / "model.safetensors").write_bytes(b"v1")
    key = fm.wcache_key(ck, "gpu", "v1")
    A = fm.WCACHE_ALIGN

    def regions():
        lay = fm.Layout()
        return lay.take(10), lay.take(A + 1)

    f = fm.WcacheFile(cache, key, 3 * A)
    assert f.fresh
    (a0, a1), (b0, b1) = regions()
    assert (a1, b1) == (A, 2 * A)
    p = f.payload()
    p[a0], p[b0 + b1 - 1] = 7, 9
    f.done(a0, a1)
    f.commit()
    f.close()
    f = fm.WcacheFile(cache, key, 3 * A)
    assert not f.fresh
    p = f.payload()
    assert p[a0] == 7 and p[b0 + b1 - 1] == 9
    raw = open(os.path.join(cache, key + ".bin"), "rb").read(24)
    assert raw[:8] == b"GPHWCACH" and int.from_bytes(raw[8:16], "little") == 4 * A and raw[16] == 1
    f.close()
    # A changed checkpoint gets a new entry, which replaces the old one.
    time.sleep(0.01)
    (ck / "model.safetensors").write_bytes(b"v2!")
    key2, other = fm.wcache_key(ck, "gpu", "v1"), fm.wcache_key(ck, "gpu-q4", "v1")
    assert key2 != key
    for k in (other, key2):
        f = fm.WcacheFile(cache, k, A)
        assert f.fresh
        f.commit()
        f.close()
    names = sorted(n for n in os.listdir(cache) if ".bin" in n)
    assert names == sorted([key2 + ".bin", other + ".bin"]), names


def test_uncommitted_is_discarded(tmp_path):
    # wcache_test.go:72-88 TestUncommittedIsDiscarded.
    cache = tmp_path / "cache"
    (tmp_path / "ck").mkdir()
    key = fm.wcache_key(tmp_path / "ck", "gpu")
    f = fm.WcacheFile(cache, key, fm.WCACHE_ALIGN)
    f.close()
    assert not [n for n in os.listdir(cache) if ".bin" in n]
    f = fm.WcacheFile(cache, key, fm.WCACHE_ALIGN)
    assert f.fresh
    f.close()


def test_no_directory():
    # wcache_test.go:90-100 TestNoDirectory.
    f = fm.WcacheFile("", "x.gpu.00", 5)
    assert f.fresh and f.payload().size == fm.WCACHE_ALIGN
    f.payload()[0] = 1
    f.commit()
    f.close()


def test_one_preparer(tmp_path):
    # wcache_test.go:102-121 TestOnePreparer: a second Open waits for the
    # first entry to be committed and maps it.
    cache = tmp_path / "cache"
    (tmp_path / "ck").mkdir()
    key = fm.wcache_key(tmp_path / "ck", "gpu")
    first = fm.WcacheFile(cache, key, fm.WCACHE_ALIGN)
    assert first.fresh
    out = {}
    t = threading.Thread(target=lambda: out.setdefault("f", fm.WcacheFile(cache, key, fm.WCACHE_ALIGN)))
    t.start()
    first.payload()[0] = 42
    time.sleep(0.05)
    assert t.is_alive()  # waiting on the preparer's lock
    first.commit()
    t.join(10)
    f = out["f"]
    assert not f.fresh and f.payload()[0] == 42
    f.close()
    first.close()


def test_gptq_calibration_sequences_cut_like_the_reference():
    # calibrationSequences' add (gptq.go:275-287): each text's tokens in
    # pieces of at most 256 (gptqMaxSeq) until 4096 (gptqMaxRows) are taken;
    # empty texts give nothing.
    assert gphq.gptq_calibration_sequences([]).tolist() == []
    assert gphq.gptq_calibration_sequences([0, 5, 0]).tolist() == [5]
    assert gphq.gptq_calibration_sequences([600, 3]).tolist() == [256, 256, 88, 3]
    got = gphq.gptq_calibration_sequences([1000] * 5)
    assert got.sum() == 4096 and got.max() == 256
    assert got.tolist() == [256, 256, 256, 232] * 4 + [96]
    assert gphq.gptq_calibration_sequences([4096, 10]).tolist() == [256] * 16
