"""Pins the decode oracle (oracle/lm_oracle.py and the rotation functions of
oracle/gphq_oracle.c) without retyping its formulas:

* splitmix64 against the published first outputs of the generator;
* the rotation against the dense matrix scale*H*diag(signs) built from
  scipy's Sylvester Hadamard, orthogonality and dot-product preservation
  (qwen3lm/kernels_test.go:73-111), and the block rule of that test;
* the float64 decode step against Hugging Face transformers' Qwen3 (an
  independent implementation of the same architecture) in float64, with the
  unrotated weights that the stored, rotated ones imply;
* the RoPE table against transformers' own rotary embedding.
"""
import numpy as np
import pytest
import scipy.linalg

from oracle import lm_oracle as lo
from oracle import oracle as orc
from tests import lm_common as lc


def test_splitmix64_published_outputs():
    # The first outputs of splitmix64 from state 0 (Vigna's reference
    # generator, also java.util.SplittableRandom's mixing function).
    got = orc.splitmix64_outputs(0, 3)
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


@pytest.mark.parametrize("k", [8, 96, 136, 1024, 3072, 4096, 12288])
def test_rotation_block_rule(k):
    # kernels_test.go:75-78: block = min(4096, k & -k).
    signs, block, scale = lo.rotation(k)
    assert block == min(4096, k & -k)
    assert scale == np.float32(1 / np.sqrt(block))
    assert set(np.unique(signs)) <= {-1.0, 1.0}
    # Signs are not degenerate: roughly half are negative.
    assert 0.3 < np.mean(signs < 0) < 0.7 or k < 64


@pytest.mark.parametrize("k", [96, 1024, 3072])
def test_rotation_matches_dense_hadamard(k):
    signs, block, scale = rot = lo.rotation(k)
    H = scipy.linalg.hadamard(block).astype(np.float64)
    R = np.zeros((k, k))
    for b in range(0, k, block):
        R[b:b + block, b:b + block] = scale * H @ np.diag(signs[b:b + block].astype(np.float64))
    rng = np.random.default_rng(k)
    x = rng.standard_normal(k).astype(np.float32)
    want = R @ x.astype(np.float64)
    np.testing.assert_allclose(lo.rot_apply(x, rot), want, rtol=0, atol=1e-12 * np.abs(want).max())
    got32 = orc.rotation_apply_f32(x, rot).astype(np.float64)
    assert np.abs(got32 - want).max() <= 1e-6 * np.abs(want).max()
    # The inverse is the transpose.
    back = orc.rotation_unapply_f32(got32.astype(np.float32), rot).astype(np.float64)
    assert np.abs(back - x).max() <= 1e-6 * np.abs(x).max()
    np.testing.assert_allclose(lo.rot_unapply(want, rot), x, atol=1e-12 * np.abs(x).max())
    np.testing.assert_allclose(lo.rot_matrix(rot), R, atol=1e-15)


@pytest.mark.parametrize("k", [8, 96, 136, 4096, 12288])
def test_rotation_orthogonal_as_reference(k):
    # kernels_test.go:80-110, the same vectors and bounds.
    rot = lo.rotation(k)
    i = np.arange(k)
    x = (np.sin(i * 1.7).astype(np.float32) * (1 + i % 9).astype(np.float32)).astype(np.float32)
    norm = float(np.dot(x.astype(np.float64), x))
    y = orc.rotation_apply_f32(x, rot)
    rotated = float(np.dot(y.astype(np.float64), y))
    assert abs(rotated - norm) <= 1e-5 * norm
    w = np.cos(i).astype(np.float32)
    dot = float(np.dot(w.astype(np.float64), x))
    rw = orc.rotation_apply_f32(w, rot)
    got = float(np.dot(rw.astype(np.float64), y))
    assert abs(got - dot) <= 1e-4 * np.sqrt(norm) * np.sqrt(k)


def test_fwht_float32_network_matches_float64():
    # The float32 network agrees with the float64 transform to rounding.
    rng = np.random.default_rng(3)
    v = rng.standard_normal(4096).astype(np.float32)
    a = v.copy()
    orc.lib().orc_fwht(orc._p(a, orc._f32p), len(a))
    want = lo.hadamard_f64(v, 4096)
    assert np.abs(a - want).max() <= 64 * 2 ** -24 * np.abs(want).max() * 12


def _hf_model(model):
    """transformers Qwen3ForCausalLM in float64 holding the unrotated weights
    that the stored ones imply (stored = W.R^T for q/k/v/gate/up and the head;
    R.W (Q8B down) or R.W.Ri^T (Q8/Q4 down) and R.W for o)."""
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    g, fmt = model["geom"], model["fmt"]
    cfg = tr.Qwen3Config(
        vocab_size=g.vocab, hidden_size=g.hidden, intermediate_size=g.inter, num_hidden_layers=g.layers,
        num_attention_heads=g.heads, num_key_value_heads=g.kv_heads, head_dim=g.head_dim,
        max_position_embeddings=g.max_pos, rms_norm_eps=g.eps,
        rope_parameters={"rope_type": "default", "rope_theta": g.theta},
        tie_word_embeddings=False, attention_bias=False)
    cfg._attn_implementation = "eager"
    m = tr.Qwen3ForCausalLM(cfg).double().eval()
    R = lo.rot_matrix(lo.rotation(g.hidden))
    Ri = lo.rot_matrix(lo.rotation(g.inter))
    sd = {"model.embed_tokens.weight": lo.bf16_to_f64(model["embed"]).reshape(g.vocab, g.hidden),
          "model.norm.weight": model["final_norm"].astype(np.float64),
          "lm_head.weight": lo.dequant(lo.FMT_Q8B, *model["head"], g.head_rows, g.hidden)[: g.vocab] @ R}
    for li, L in enumerate(model["layers"]):
        p = f"model.layers.{li}."
        qkv = lo.dequant(fmt, *L.qkv, g.qd + 2 * g.kvd, g.hidden) @ R
        gu = lo.dequant(fmt, *L.gu, 2 * g.inter, g.hidden) @ R
        down = R.T @ lo.dequant(fmt, *L.down, g.hidden, g.inter)
        if fmt != lo.FMT_Q8B:
            down = down @ Ri
        sd.update({
            p + "self_attn.q_proj.weight": qkv[: g.qd],
            p + "self_attn.k_proj.weight": qkv[g.qd: g.qd + g.kvd],
            p + "self_attn.v_proj.weight": qkv[g.qd + g.kvd:],
            p + "self_attn.o_proj.weight": R.T @ lo.dequant(fmt, *L.o, g.hidden, g.qd),
            p + "self_attn.q_norm.weight": L.q_norm.astype(np.float64),
            p + "self_attn.k_norm.weight": L.k_norm.astype(np.float64),
            p + "input_layernorm.weight": np.ones(g.hidden),
            p + "post_attention_layernorm.weight": np.ones(g.hidden),
            p + "mlp.gate_proj.weight": gu[0::2],
            p + "mlp.up_proj.weight": gu[1::2],
            p + "mlp.down_proj.weight": down,
        })
    state = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}
    missing, unexpected = m.load_state_dict(state, strict=False)
    assert not unexpected and not [k for k in missing if "rotary" not in k]
    return m


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q8, lo.FMT_Q4])
def test_decode_oracle_matches_transformers_qwen3(fmt):
    torch = pytest.importorskip("torch")
    model = lc.random_model(lc.GPU_SHAPE, fmt, seed=11 + fmt)
    g = model["geom"]
    orc_ = lc.oracle_for(model)
    hf = _hf_model(model)
    tokens = [5, 17, 3, 90, 44, 44, 0]
    with torch.no_grad():
        ids = torch.tensor([tokens])
        hid = hf.model(ids).last_hidden_state[0].numpy()
        logits = hf.lm_head(torch.from_numpy(hid)).numpy()
    cache = orc_.new_cache(16)
    for pos, t in enumerate(tokens):
        hidden, lg, nxt = orc_.step(cache, pos, t)
        # transformers computes RMSNorm, RoPE angles and softmax in float32,
        # so agreement is to float32 rounding, far below any structural error.
        rel_h = np.linalg.norm(hidden - hid[pos]) / np.linalg.norm(hid[pos])
        rel_l = np.linalg.norm(lg - logits[pos]) / np.linalg.norm(logits[pos])
        assert rel_h < 2e-5 and rel_l < 2e-5, (pos, rel_h, rel_l)
        assert nxt == int(np.argmax(logits[pos])) or np.sort(logits[pos])[-1] - np.sort(logits[pos])[-2] < 1e-3


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q8])
def test_batched_prefill_oracle_matches_stepping_and_transformers(fmt):
    """The batched-pass restatement (DecodeOracle.prefill) against the
    token-by-token step and against transformers' own batched causal pass,
    with the prompt split into two passes (the second continuing the cache)."""
    torch = pytest.importorskip("torch")
    model = lc.random_model(lc.GPU_SHAPE, fmt, seed=21 + fmt)
    g = model["geom"]
    orc_ = lc.oracle_for(model)
    tokens = [7, 1, 88, 88, 30, 2, 64, 11, 5, 93, 40]
    split = 4
    c1 = orc_.new_cache(16)
    h1 = np.concatenate([orc_.prefill(c1, 0, tokens[:split]), orc_.prefill(c1, split, tokens[split:])])
    c2 = orc_.new_cache(16)
    for pos, t in enumerate(tokens):
        h2 = orc_.layers(c2, pos, orc_.embed_row(t))
        assert np.abs(h1[pos] - h2).max() <= 1e-9 * np.abs(h2).max(), pos
    for (k1, v1), (k2, v2) in zip(c1, c2):
        assert np.abs(k1 - k2).max() <= 1e-9 * np.abs(k2).max()
        assert np.abs(v1 - v2).max() <= 1e-9 * np.abs(v2).max()
    hf = _hf_model(model)
    with torch.no_grad():
        hid = hf.model(torch.tensor([tokens])).last_hidden_state[0].numpy()
    for pos in range(len(tokens)):
        hidden, _ = orc_.finish(h1[pos])
        assert np.linalg.norm(hidden - hid[pos]) / np.linalg.norm(hid[pos]) < 2e-5, pos


@pytest.mark.parametrize("layers", [1, 2])
def test_prefill_last_only_equals_full_pass(layers):
    """prefill(last_only=True), used at workload size, against the pinned full
    pass: the final row's residual and every appended K/V row agree."""
    g = lo.Geometry(hidden=256, layers=layers, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=96, max_pos=64)
    model = lc.random_model(g, lo.FMT_Q8B, seed=70 + layers)
    orc_ = lc.oracle_for(model)
    rng = np.random.default_rng(layers)
    tokens = list(rng.integers(0, g.vocab, 23))
    c_full, c_last = orc_.new_cache(40), orc_.new_cache(40)
    orc_.prefill(c_full, 0, tokens[:5])
    orc_.prefill(c_last, 0, tokens[:5])
    full = orc_.prefill(c_full, 5, tokens[5:])
    last = orc_.prefill(c_last, 5, tokens[5:], last_only=True)
    assert last.shape == (1, g.hidden)
    assert np.abs(last[0] - full[-1]).max() <= 1e-12 * np.abs(full[-1]).max()
    for (k1, v1), (k2, v2) in zip(c_full, c_last):
        assert np.abs(k1 - k2).max() <= 1e-12 * np.abs(k1).max()
        assert np.abs(v1 - v2).max() <= 1e-12 * np.abs(v1).max()


def test_prefill_embeds_and_tail():
    """Embeds rows that equal the embedding table's rows (as float32) give the
    plain pass exactly; the tail rows equal the full pass's last rows."""
    g = lo.Geometry(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=96, max_pos=64)
    model = lc.random_model(g, lo.FMT_Q8B, seed=81)
    orc_ = lc.oracle_for(model)
    tokens = [5, 90, 7, 90, 90, 3, 11, 90, 1]
    ph = 90
    rows = lo.bf16_to_f64(model["embed"][ph]).astype(np.float32)
    occ = tokens.count(ph)
    c1, c2, c3 = orc_.new_cache(16), orc_.new_cache(16), orc_.new_cache(16)
    plain = orc_.prefill(c1, 0, tokens)
    spliced = orc_.prefill(c2, 0, tokens, embeds=(ph, np.tile(rows, (occ, 1))))
    np.testing.assert_array_equal(spliced, plain)
    tail = orc_.prefill(c3, 0, tokens, tail=4)
    assert tail.shape == (4, g.hidden)
    assert np.abs(tail - plain[-4:]).max() <= 1e-12 * np.abs(plain).max()
    for (k1, v1), (k3, v3) in zip(c1, c3):
        assert np.abs(k1 - k3).max() <= 1e-12 * np.abs(k1).max()


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q8])
def test_prefill_embeds_match_transformers_inputs_embeds(fmt):
    """The spliced pass against transformers' Qwen3 fed inputs_embeds with the
    same rows at the placeholders (and embedding rows elsewhere)."""
    torch = pytest.importorskip("torch")
    model = lc.random_model(lc.GPU_SHAPE, fmt, seed=31 + fmt)
    g = model["geom"]
    orc_ = lc.oracle_for(model)
    tokens = [4, 60, 60, 9, 60, 22, 7]
    ph = 60
    rng = np.random.default_rng(8)
    rows = rng.standard_normal((tokens.count(ph), g.hidden)).astype(np.float32)
    h = orc_.prefill(orc_.new_cache(16), 0, tokens, embeds=(ph, rows))
    emb = lo.bf16_to_f64(model["embed"]).reshape(g.vocab, g.hidden)[tokens]
    emb[np.array(tokens) == ph] = rows.astype(np.float64)
    hf = _hf_model(model)
    with torch.no_grad():
        hid = hf.model(inputs_embeds=torch.from_numpy(emb)[None]).last_hidden_state[0].numpy()
    for pos in range(len(tokens)):
        hidden, _ = orc_.finish(h[pos])
        assert np.linalg.norm(hidden - hid[pos]) / np.linalg.norm(hid[pos]) < 2e-5, pos


def test_chunked_head_equals_dense_head():
    """head_rows over row chunks (the path a 151,936-row head takes) gives the
    dense head's logits; the chunk boundary falls inside the vocabulary."""
    g = lo.Geometry(hidden=256, layers=1, heads=2, kv_heads=1, head_dim=128, inter=512, vocab=1000, max_pos=8)
    model = lc.random_model(g, lo.FMT_Q8B, seed=3)
    orc_ = lc.oracle_for(model)
    x = np.random.default_rng(0).standard_normal((3, g.hidden))
    dense = x @ orc_.head.T
    chunked = lc.oracle_for(model)
    chunked.HEAD_CHUNK, chunked.DENSE_HEAD_MAX = 384, 0  # force the chunked path
    got = chunked.head_rows(x)
    assert chunked._head is None
    np.testing.assert_allclose(got, dense, rtol=1e-13, atol=1e-13 * np.abs(dense).max())
    hid, lg = orc_.finish_rows(x)
    for i in range(3):
        h1, l1 = orc_.finish(x[i])
        np.testing.assert_allclose(h1, hid[i], rtol=1e-13)
        np.testing.assert_allclose(l1, lg[i], rtol=1e-12, atol=1e-12 * np.abs(l1).max())


def test_rope_table_matches_transformers():
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    g = lc.GPU_SHAPE
    cfg = tr.Qwen3Config(hidden_size=g.hidden, num_attention_heads=g.heads, num_key_value_heads=g.kv_heads,
                         head_dim=g.head_dim, max_position_embeddings=g.max_pos,
                         rope_parameters={"rope_type": "default", "rope_theta": g.theta})
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    emb = Qwen3RotaryEmbedding(cfg)
    pos = torch.arange(64)[None, :]
    cos, sin = emb(torch.zeros(1, dtype=torch.float32), pos)
    c, s = lo.rope_table(g, 64)
    half = g.head_dim // 2
    # transformers forms the angle in float32; positions < 64 keep it within 1e-5.
    np.testing.assert_allclose(cos[0, :, :half].numpy(), c, atol=1e-5)
    np.testing.assert_allclose(cos[0, :, half:].numpy(), c, atol=1e-5)
    np.testing.assert_allclose(sin[0, :, :half].numpy(), s, atol=1e-5)


def test_greedy_argmax_rules():
    # decode_batch.go:182-191: first maximum, NaN never wins, NaN at 0 keeps 0.
    nan = float("nan")
    assert lo.greedy_argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert lo.greedy_argmax([nan, 5.0, 6.0]) == 0
    assert lo.greedy_argmax([1.0, nan, 0.5, 7.0]) == 3
    assert lo.greedy_argmax([-0.0, 0.0]) == 0
    for v in ([1.0, 3.0, 3.0, 2.0], [nan, 5.0, 6.0], [1.0, nan, 0.5, 7.0], [-np.inf, -np.inf]):
        assert lo.greedy_argmax_np(v) == lo.greedy_argmax(v)


@pytest.mark.parametrize("n,k,rot_k,tile", [(256, 8, 256, 0), (1024, 3, 1024, 0), (256, 5, 0, 128)])
def test_rotation_apply_rows_matches_dense(n, k, rot_k, tile):
    # hadamard.go:88-104: applyRows(a) == R @ a, rotating along the row index.
    rot = lo.head_rotation(tile, n) if tile else lo.rotation(rot_k)
    R = lo.rot_matrix(rot)
    rng = np.random.default_rng(n + k)
    a = rng.standard_normal((n, k)).astype(np.float32)
    got = orc.rotation_apply_rows_f32(a, rot).astype(np.float64)
    want = R @ a.astype(np.float64)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    # Rows of the identity become the columns of R.
    np.testing.assert_allclose(orc.rotation_apply_rows_f32(np.eye(n, dtype=np.float32), rot), R, atol=1e-6)


def test_prepare_projection_oracle_roundtrip():
    # A prepared job dequantizes back to R_out . (W diag(norm)) . R_in^T within the
    # quantizer's bound: every stored row is the rotated row to half a step.
    g = lc.GPU_SHAPE
    rng = np.random.default_rng(4)
    n, k = g.hidden, g.qd
    w = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
    bf = lc.bf16_bits(w)
    wf = lo.bf16_to_f64(bf).reshape(n, k)
    hin = lo.head_rotation(g.head_dim, k)
    hout = lo.rotation(g.hidden)
    dst = np.zeros(n * k + n * (k // 32) * 2, np.uint8)
    orc.prepare_projection(bf, n, k, lo.FMT_Q8B, dst, 0, n * k, in_rot=hin, out_rot=hout)
    deq = lo.dequant(lo.FMT_Q8B, dst[:n * k], dst[n * k:].view(np.uint16), n, k)
    want = lo.rot_matrix(hout) @ wf @ lo.rot_matrix(hin).T
    step = np.abs(want).reshape(n, k // 32, 32).max(axis=2, keepdims=True) / 127
    err = np.abs(deq - want).reshape(n, k // 32, 32)
    assert (err <= 0.5 * step * 1.01 + 1e-6).all()


def test_int8_route_quantization_matches_pinned_quantizer():
    """The int8 mode's per-row quantization (DecodeOracle._mm) against the
    pinned C quantizer of WorkspaceI8 (orc.i8_pack_rows, bit-exact with
    int8.go:106-168): on float32 rows the codes agree except where float32's
    x * (127/max) and float64's land on opposite sides of a rounding boundary
    (then by one step), and the step s = max/127 equals the C scale to float32
    rounding. Rows of zeros, a NaN and an infinity quantize to zero."""
    rng = np.random.default_rng(8)
    rows, k = 64, 1024
    x = (rng.standard_normal((rows, k)) * rng.uniform(1e-3, 1e3, (rows, 1))).astype(np.float32)
    x[3] = 0.0
    x[4, 7] = np.nan
    x[5, 9] = np.inf
    x[6, :8] = [127.0, -127.0, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5]  # exact ties at max 127
    x[6, 8:] = 0.0
    o = lo.DecodeOracle.__new__(lo.DecodeOracle)
    o.int8 = True
    x64 = x.astype(np.float64)
    deq = o._mm(x64, np.eye(k))  # the quantized rows s * q themselves
    q_c, s_c, _ = orc.i8_pack_rows(x, rows, k)
    for r in range(rows):
        if r in (3, 4, 5):
            assert not deq[r].any() and not q_c[r].any() and s_c[r] == 0
            continue
        s = np.abs(x64[r]).max() / 127.0
        assert abs(s - float(s_c[r])) <= 2 * np.spacing(np.float32(s_c[r])), r
        q = np.rint(deq[r] / s)
        diff = q - q_c[r].astype(np.float64)
        assert np.abs(diff).max() <= 1, r
        assert np.mean(diff == 0) >= 0.999, r
    # Ties round to even, saturation at -128..127 as the C quantizer.
    assert np.array_equal(np.rint(deq[6, :8] / (127.0 / 127.0)), [127, -127, 64, -64, 0, -0, 2, -2])
    assert np.array_equal(q_c[6, :8], [127, -127, 64, -64, 0, 0, 2, -2])
    o.int8 = False
    y = rng.standard_normal((3, k))
    w = rng.standard_normal((5, k))
    assert np.array_equal(o._mm(y, w), y @ w.T)
