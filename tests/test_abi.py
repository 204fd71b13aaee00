"""CPU checks of the C ABI: the library loads, exports every symbol that
include/gphq.h declares, maps status codes to the reference's messages, and
rejects bad arguments before touching a device (so these run without a GPU).
"""
import ctypes
import os
import re

import pytest

from gophonic_amd import gphq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in os.listdir(os.path.join(ROOT, "include")):
        if h.endswith(".h"):
            text = open(os.path.join(ROOT, "include", h)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(gphq_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = gphq.load()
    names = declared_functions()
    assert names, "no declarations found"
    for name in names:
        assert hasattr(lib, name), name
        assert name in gphq.SIGNATURES, f"{name} has no ctypes signature"


def test_error_strings_are_the_reference_messages():
    assert gphq.error_string(gphq.ERR_INVALID_DIMENSIONS) == "q8gemv: invalid dimensions"  # q8gemv.go:20
    assert gphq.error_string(gphq.ERR_INVALID_WEIGHT_LENGTH) == "q8gemv: invalid weight length"  # q8gemv.go:24,27
    assert gphq.error_string(gphq.ERR_DIMENSIONS) == "q8gemm: invalid dimensions or buffer length"  # packed.go:26
    assert gphq.error_string(gphq.ERR_NON_FINITE) == "q8gemm: non-finite row scale"  # packed.go:27
    assert gphq.error_string(gphq.OK) == ""


# q8gemv_test.go:91-117 shape cases: (x_len, q_len, s_len, dst_len, k, n) -> status.
SHAPE_CASES = [
    ("negative-k", 0, 0, 0, 0, -1, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("negative-n", 0, 0, 0, 0, 0, -1, gphq.ERR_INVALID_DIMENSIONS),
    ("activation-length", 1, 0, 0, 0, 0, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("scale-length", 0, 0, 1, 0, 0, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("output-length", 0, 0, 0, 1, 0, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("weights-length", 1, 1, 2, 2, 1, 2, gphq.ERR_INVALID_WEIGHT_LENGTH),
    ("k0-with-weights", 0, 3, 2, 2, 0, 2, gphq.ERR_INVALID_WEIGHT_LENGTH),
    ("ragged-weights", 4, 7, 2, 2, 4, 2, gphq.ERR_INVALID_WEIGHT_LENGTH),
]


@pytest.mark.parametrize("name,xl,ql,sl,dl,k,n,want", SHAPE_CASES, ids=[c[0] for c in SHAPE_CASES])
def test_q8gemv_shape_checks_before_any_device_work(name, xl, ql, sl, dl, k, n, want):
    lib = gphq.load()
    # Non-null dummy pointers: validation must fail before any dereference.
    p = ctypes.c_void_p(16)
    got = lib.gphq_q8gemv_mul_into(p, xl, p, ql, p, sl, p, dl, k, n, None)
    assert got == want


def test_q8gemv_empty_output_is_a_no_op():
    lib = gphq.load()
    assert lib.gphq_q8gemv_mul_into(None, 0, None, 0, None, 0, None, 0, 0, 0, None) == gphq.OK
    assert lib.gphq_q8gemv_mul_into(None, 5, None, 0, None, 0, None, 0, 5, 0, None) == gphq.OK


def test_gemv_rejects_bad_formats_and_shapes():
    lib = gphq.load()
    p = ctypes.c_void_p(256)
    assert lib.gphq_gemv(3, p, p, p, p, 64, 4, None) == gphq.ERR_UNSUPPORTED
    assert lib.gphq_gemv(gphq.FMT_Q8B, p, p, p, p, 48, 4, None) == gphq.ERR_DIMENSIONS  # K % 32
    assert lib.gphq_gemv(gphq.FMT_Q4, p, p, p, p, 40, 4, None) == gphq.ERR_DIMENSIONS
    assert lib.gphq_gemv(gphq.FMT_Q8B, p, p, p, p, -32, 4, None) == gphq.ERR_DIMENSIONS
    assert lib.gphq_gemv(gphq.FMT_Q8B, ctypes.c_void_p(8), p, p, p, 64, 4, None) == gphq.ERR_DIMENSIONS  # alignment
    assert lib.gphq_gemv(gphq.FMT_Q8B, p, p, p, p, 64, 0, None) == gphq.OK  # nothing to do


def _lm_cfg(**kw):
    base = dict(hidden=4096, layers=36, heads=32, kv_heads=8, head_dim=128, intermediate=12288, vocab=151936,
                max_positions=40960, fmt=gphq.FMT_Q8B)
    base.update(kw)
    return gphq.lm_config(**base)


def test_lm_layer_layout_qwen3_8b_q8b():
    # gpu_darwin.go:251-283 place(): codes then scales, 256-byte aligned regions.
    L, n = gphq.lm_layer_layout(_lm_cfg())
    qkv_rows = 4096 + 2 * 1024
    assert (L.qkv, L.qkv_scale) == (0, qkv_rows * 4096)
    assert L.o == qkv_rows * 4096 + 2 * qkv_rows * 128
    assert L.gu_scale - L.gu == 24576 * 4096
    assert L.d_scale - L.d == 4096 * 12288
    assert n == L.d_scale + 2 * 4096 * 384 == 204996608
    # Q8 keeps one fp32 scale per row; Q4 halves the codes.
    L8, n8 = gphq.lm_layer_layout(_lm_cfg(fmt=gphq.FMT_Q8))
    assert L8.o - L8.qkv_scale == 4 * qkv_rows
    L4, _ = gphq.lm_layer_layout(_lm_cfg(fmt=gphq.FMT_Q4))
    assert L4.qkv_scale == qkv_rows * 2048


def test_lm_head_layout_pads_vocab_to_16():
    rows, so, n = gphq.lm_head_layout(_lm_cfg(vocab=151937))
    assert rows == 151952 and so == (151952 * 4096 + 255) // 256 * 256 and n == so + 2 * 151952 * 128


@pytest.mark.parametrize("kw", [dict(head_dim=64, heads=64), dict(heads=72, kv_heads=8), dict(hidden=4000),
                                dict(intermediate=12320), dict(heads=30, kv_heads=8), dict(eps=0.0),
                                dict(intermediate=96 * 5)])
def test_lm_new_rejects_geometry_before_device_work(kw):
    # gpu_darwin.go:116-129 gpuGeometry and weights.go:678-680.
    lib = gphq.load()
    h = ctypes.c_void_p()
    assert lib.gphq_lm_new(ctypes.byref(_lm_cfg(**kw)), ctypes.byref(h)) == gphq.ERR_GEOMETRY
    assert not h.value


def test_decode_entry_points_reject_null_workspace():
    lib = gphq.load()
    p = ctypes.c_void_p(256)
    assert lib.gphq_decode_batch_into(None, None, 1, p, p, p, 1, p, 1, None) == gphq.ERR_FOREIGN_WORKSPACE
    assert lib.gphq_decode_batch_new(None, 1, ctypes.byref(ctypes.c_void_p())) == gphq.ERR_FOREIGN_WORKSPACE
    assert lib.gphq_decode_batch_logits(None, p, 1, p, 1, None) == gphq.ERR_FOREIGN_WORKSPACE
    assert gphq.error_string(gphq.ERR_PREFIX_FULL) == "qwen3: decode prefix has no room for another token"


def test_gemv_vec_rejects_misaligned_vectors():
    lib = gphq.load()
    p = ctypes.c_void_p(256)
    big = 1 << 30
    # x_stride not a multiple of 4, then x not 16-byte aligned: rejected before any device work.
    assert lib.gphq_gemv_vec(gphq.FMT_Q8B, p, p, p, 66, p, 64, 2, 64, 64, p, big, None) == gphq.ERR_DIMENSIONS
    assert lib.gphq_gemv_vec(gphq.FMT_Q8B, p, p, ctypes.c_void_p(260), 64, p, 64, 2, 64, 64, p, big, None) == \
        gphq.ERR_DIMENSIONS


@pytest.mark.parametrize("fmt", [gphq.FMT_Q8B, gphq.FMT_Q8, gphq.FMT_Q4])
def test_prepare_layer_jobs_are_prepare_gpus_list(fmt):
    # gpu_darwin.go:400-415: q, k, v, o, gate, up, down with their norms,
    # rotations, destination rows and layer-buffer offsets (no device work).
    import numpy as np

    cfg = _lm_cfg(fmt=fmt)
    L, _ = gphq.lm_layer_layout(cfg)
    an, mn = np.full(4096, 2.0, np.float32), np.full(4096, 3.0, np.float32)
    jobs, (a, m) = gphq.prepare_layer_jobs(cfg, an, mn)
    h, qd, kv, inter, hd = 4096, 4096, 1024, 12288, 128
    down_in = (0, 0) if fmt == gphq.FMT_Q8B else (inter, 0)
    want = [  # n, k, norm, in, out, base, sc, step, row0
        (qd, h, a, (h, 0), (0, 0), L.qkv, L.qkv_scale, 1, 0),
        (kv, h, a, (h, 0), (0, 0), L.qkv, L.qkv_scale, 1, qd),
        (kv, h, a, (h, 0), (0, hd), L.qkv, L.qkv_scale, 1, qd + kv),
        (h, qd, None, (0, hd), (h, 0), L.o, L.o_scale, 1, 0),
        (inter, h, m, (h, 0), (0, 0), L.gu, L.gu_scale, 2, 0),
        (inter, h, m, (h, 0), (0, 0), L.gu, L.gu_scale, 2, 1),
        (h, inter, None, down_in, (h, 0), L.d, L.d_scale, 1, 0),
    ]
    for j, (n, k, norm, rin, rout, base, sc, step, row0) in zip(jobs, want):
        assert (j.n, j.k, j.base, j.sc, j.step, j.row0, j.fmt) == (n, k, base, sc, step, row0, fmt)
        assert (j.in_rot.width, j.in_rot.tile) == rin and (j.out_rot.width, j.out_rot.tile) == rout
        assert j.norm_host == (None if norm is None else norm.ctypes.data)
        assert j.scale_mul == 1.0 and not j.src_bf16_dev


def test_prepare_head_jobs_chunk_the_vocabulary():
    # gpu_darwin.go:432-436: chunks of max(inter, 4096) rows, Q8B, hidden input rotation.
    lib = gphq.load()
    cfg = _lm_cfg(vocab=151936)
    chunk = lib.gphq_prepare_head_chunk_rows(ctypes.byref(cfg))
    assert chunk == 12288
    rows, so, _ = gphq.lm_head_layout(cfg)
    seen = 0
    for r in range(0, 151936, chunk):
        j = gphq.PrepareJob()
        assert lib.gphq_prepare_head_job(ctypes.byref(cfg), r, None, 0, ctypes.byref(j)) == gphq.OK
        assert (j.n, j.k, j.fmt, j.row0, j.step, j.base, j.sc) == (min(chunk, 151936 - r), 4096, gphq.FMT_Q8B, r,
                                                                      1, 0, so)
        assert (j.in_rot.width, j.out_rot.width, j.out_rot.tile) == (4096, 0, 0)
        seen += j.n
    assert seen == 151936
    assert lib.gphq_prepare_head_job(ctypes.byref(cfg), 151936, None, 0, ctypes.byref(j)) == gphq.ERR_DIMENSIONS
    need = lib.gphq_prepare_lm_work_bytes(ctypes.byref(cfg))
    assert need == max(lib.gphq_prepare_work_bytes(n, k) for n, k in
                       [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (12288, 4096)])
