"""GPU parity of the qwen3lm batched pass (gphq_prefill_*), through the C ABI,
against the float64 oracle's batched pass (oracle/lm_oracle.py
DecodeOracle.prefill, itself pinned to stepping and to transformers' Qwen3).

The bound is the reference's batched-vs-token-by-token check
(gpu_official_darwin_test.go:63-87): cosine >= 0.99999 between the last
token's post-final-norm states. The batched pass multiplies FP16 weight and
activation tiles (the reference mm's arithmetic) and runs attention on FP16
tiles, so it is not bit-identical to the fp32 decode step; K/V rows are held
to the same cosine per row, and a decode step that reads a prefilled cache to
the same bound.
"""
import numpy as np
import pytest

from gophonic_amd import gphq
from oracle import lm_oracle as lo
from tests import lm_common as lc
from tests.test_lm_decode_gpu import QWEN3_8B_LAYER, _read_dev_floats, geom_kwargs, setup

pytestmark = pytest.mark.gpu

COS = 0.99999


def cosine(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    assert np.isfinite(b).all()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def run_prefill(ws, kv, keep, tokens, g):
    import torch

    hidden = torch.full((g.hidden,), -7.0, device="cuda")
    print(f"prefill keep={keep} n={len(tokens)} rows={ws.rows}", flush=True)
    ws.extend(kv, keep, tokens, hidden)
    ws.check()
    return hidden.cpu().numpy()


def check_cache(oracle_cache, kv, g, rows):
    """Cosine of every appended K/V row (first and last layer) with the oracle's."""
    kc, vc, cap = kv.kv()
    for layer in (0, g.layers - 1):
        for base, want in ((kc, oracle_cache[layer][0]), (vc, oracle_cache[layer][1])):
            got = _read_dev_floats(base + layer * cap * g.kvd * 4, rows * g.kvd).reshape(rows, g.kvd)
            for r in range(rows):
                assert cosine(want[r], got[r]) >= COS, (layer, r)


@pytest.mark.parametrize("fmt", lc.FMTS)
def test_prefill_matches_oracle(fmt):
    model, oracle, lm = setup(lc.GPU_SHAPE, fmt, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(31)
    tokens = list(rng.integers(0, g.vocab, 45))
    ws = gphq.Prefill(lm, 64)
    kv = gphq.Prefix(lm, 64)
    got = run_prefill(ws, kv, 0, tokens, g)
    cache = oracle.new_cache(64)
    h = oracle.prefill(cache, 0, tokens)
    want, _ = oracle.finish(h[-1])
    assert cosine(want, got) >= COS
    check_cache(cache, kv, g, len(tokens))


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q8])
def test_passes_extension_and_decode_after_prefill(fmt):
    # 20 tokens in passes of 16 + 4, then 13 more continuing the cache at
    # keep = 20 (16 + ... rows per pass), then one decode step on the result.
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, fmt, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(32)
    first, second = list(rng.integers(0, g.vocab, 20)), list(rng.integers(0, g.vocab, 13))
    ws = gphq.Prefill(lm, 16)
    kv = gphq.Prefix(lm, 48)
    run_prefill(ws, kv, 0, first, g)
    got = run_prefill(ws, kv, 20, second, g)
    cache = oracle.new_cache(48)
    oracle.prefill(cache, 0, first)
    h = oracle.prefill(cache, 20, second)
    want, _ = oracle.finish(h[-1])
    assert cosine(want, got) >= COS
    check_cache(cache, kv, g, 33)
    dec = gphq.DecodeBatch(lm, 1)
    tok = int(rng.integers(0, g.vocab))
    hidden = torch.empty((1, g.hidden), device="cuda")
    logits = torch.empty((1, g.vocab), device="cuda")
    dec.into([kv], [33], [tok], hidden, logits)
    dec.check()
    wh, wl, _ = oracle.step(cache, 33, tok)
    assert cosine(wh, hidden.cpu().numpy()[0]) >= COS
    assert cosine(wl, logits.cpu().numpy()[0]) >= COS


def test_one_token_pass_and_rewrite():
    # A one-token pass takes the GEMV path; extending at a smaller keep
    # overwrites the stored suffix (evaluator.go:223 truncates the tokens).
    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B_F32, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(33)
    toks = list(rng.integers(0, g.vocab, 12))
    ws = gphq.Prefill(lm, 32)
    kv = gphq.Prefix(lm, 32)
    run_prefill(ws, kv, 0, toks, g)
    alt = list(rng.integers(0, g.vocab, 6))
    run_prefill(ws, kv, 5, alt, g)  # rows 5..10 rewritten
    got = run_prefill(ws, kv, 11, [int(toks[3])], g)
    cache = oracle.new_cache(32)
    oracle.prefill(cache, 0, toks[:5] + alt)
    h = oracle.prefill(cache, 11, [int(toks[3])])
    want, _ = oracle.finish(h[-1])
    assert cosine(want, got) >= COS
    check_cache(cache, kv, g, 12)


def test_prefill_06b_widths():
    # Qwen3-0.6B widths (16 query / 8 KV heads, hidden 1024): several 32-row
    # attention blocks per KV head, keys over several tiles.
    model, oracle, lm = setup(lc.SMALL_06B, lo.FMT_Q8B, seed=7)
    g = model["geom"]
    rng = np.random.default_rng(34)
    tokens = list(rng.integers(0, g.vocab, 150))
    ws = gphq.Prefill(lm, 128)
    kv = gphq.Prefix(lm, 160)
    got = run_prefill(ws, kv, 0, tokens, g)
    cache = oracle.new_cache(160)
    h = oracle.prefill(cache, 0, tokens)
    want, _ = oracle.finish(h[-1])
    assert cosine(want, got) >= COS
    check_cache(cache, kv, g, len(tokens))


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B_F32, lo.FMT_Q8])
def test_prefill_8b_widths(fmt):
    # One layer at Qwen3-8B widths: GEMM tiles at K = 4096 and 12288, four
    # query heads per KV head.
    model, oracle, lm = setup(QWEN3_8B_LAYER, fmt, seed=21)
    g = model["geom"]
    rng = np.random.default_rng(35)
    tokens = list(rng.integers(0, g.vocab, 40))
    ws = gphq.Prefill(lm, 64)
    kv = gphq.Prefix(lm, 64)
    got = run_prefill(ws, kv, 0, tokens, g)
    cache = oracle.new_cache(64)
    h = oracle.prefill(cache, 0, tokens)
    want, _ = oracle.finish(h[-1])
    assert cosine(want, got) >= COS
    check_cache(cache, kv, g, len(tokens))


@pytest.mark.parametrize("group", [1, 3, 5, 8])
def test_prefill_query_groups(group):
    # Query heads per KV head other than the 2 and 4 above: the attention
    # kernel's block shape changes with the group (one or two 32-row halves).
    geom = lo.Geometry(hidden=256, layers=1, heads=group, kv_heads=1, head_dim=128, inter=512, vocab=96,
                       max_pos=320)
    model, oracle, lm = setup(geom, lo.FMT_Q8B, seed=40 + group)
    g = model["geom"]
    rng = np.random.default_rng(36 + group)
    tokens = list(rng.integers(0, g.vocab, 100))
    ws = gphq.Prefill(lm, 128)
    kv = gphq.Prefix(lm, 128)
    got = run_prefill(ws, kv, 0, tokens, g)
    cache = oracle.new_cache(128)
    h = oracle.prefill(cache, 0, tokens)
    want, _ = oracle.finish(h[-1])
    assert cosine(want, got) >= COS
    check_cache(cache, kv, g, len(tokens))


def test_prefill_validation_errors():
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    ws = gphq.Prefill(lm, 8)
    kv = gphq.Prefix(lm, 8)
    hid = torch.empty(g.hidden, device="cuda")

    def status(fn):
        try:
            fn()
        except gphq.GphqError as e:
            return e.status
        return gphq.OK

    other = gphq.lm_from_stored(geom_kwargs(g), lo.FMT_Q8B, model["layers"], model["embed"], model["final_norm"],
                                model["head"])
    assert status(lambda: ws.extend(gphq.Prefix(other, 8), 0, [1], hid)) == gphq.ERR_FOREIGN_PREFIX
    assert status(lambda: ws.extend(None, 0, [1], hid)) == gphq.ERR_FOREIGN_PREFIX
    assert status(lambda: ws.extend(kv, -1, [1], hid)) == gphq.ERR_KEEP_RANGE
    assert status(lambda: ws.extend(kv, 6, [1, 2, 3], hid)) == gphq.ERR_PREFIX_CAPACITY
    assert status(lambda: ws.extend(kv, 0, [], hid)) == gphq.ERR_EMPTY_SEQUENCE
    assert status(lambda: ws.extend(kv, 0, [1], torch.empty(g.hidden + 1, device="cuda"))) == gphq.ERR_DEST_WIDTH
    assert status(lambda: ws.extend(kv, 0, [1, g.vocab], hid)) == gphq.ERR_TOKEN_VOCAB
    assert status(lambda: ws.extend(kv, 0, [-1], hid)) == gphq.ERR_TOKEN_VOCAB
    long_kv = gphq.Prefix(lm, g.max_pos + 8)
    assert status(lambda: ws.extend(long_kv, g.max_pos - 1, [1, 2], hid)) == gphq.ERR_CONTEXT
    # Nothing was enqueued by the rejected calls: the prefix is untouched.
    kc, vc, cap = kv.kv()
    assert not _read_dev_floats(kc, g.kvd * cap).any()
    assert status(lambda: gphq.Prefill(lm, 0)) == gphq.ERR_DIMENSIONS
    bare = gphq.Lm(gphq.lm_config(fmt=lo.FMT_Q8B, **geom_kwargs(g)))
    assert status(lambda: gphq.Prefill(bare, 4)) == gphq.ERR_MODEL_INCOMPLETE


def oracle_last(oracle, prefix, seq, capacity=128):
    """The oracle's last-token state of seq evaluated after `prefix` tokens."""
    cache = oracle.new_cache(capacity)
    if prefix:
        oracle.prefill(cache, 0, prefix)
    h = oracle.prefill(cache, len(prefix), seq)
    want, _ = oracle.finish(h[-1])
    return want


def run_batch(ws, seqs, g, shared=None, past=0):
    import torch

    hidden = torch.full((len(seqs), g.hidden), -7.0, device="cuda")
    print(f"batch lens={[len(q) for q in seqs]} past={past} rows={ws.rows}", flush=True)
    ws.batch(seqs, hidden, shared=shared, past=past)
    ws.check()
    return hidden.cpu().numpy()


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q4])
def test_batch_matches_separate_sequences(fmt):
    # HiddenLastBatchInto: four sequences packed into passes of 24 rows
    # (5 + 17 + 1, then 9), and a batch of one single-token sequence (the GEMV
    # path); each result against the oracle's separate evaluation.
    model, oracle, lm = setup(lc.GPU_SHAPE, fmt, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(41)
    seqs = [list(rng.integers(0, g.vocab, n)) for n in (5, 17, 1, 9)]
    ws = gphq.Prefill(lm, 24)
    got = run_batch(ws, seqs, g)
    for i, q in enumerate(seqs):
        assert cosine(oracle_last(oracle, [], q), got[i]) >= COS, i
    one = [[int(rng.integers(0, g.vocab))]]
    got = run_batch(ws, one, g)
    assert cosine(oracle_last(oracle, [], one[0]), got[0]) >= COS


def test_batch_shared_prefix_is_read_only():
    # HiddenLastSharedInto: three continuations of a 12-token prefix, packed
    # in one pass; the prefix's cache rows are unchanged afterwards.
    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(42)
    prefix = list(rng.integers(0, g.vocab, 12))
    ws = gphq.Prefill(lm, 32)
    kv = gphq.Prefix(lm, 40)
    run_prefill(ws, kv, 0, prefix, g)
    kc, vc, cap = kv.kv()
    before = [_read_dev_floats(base, g.layers * cap * g.kvd) for base in (kc, vc)]
    seqs = [list(rng.integers(0, g.vocab, n)) for n in (7, 1, 20)]
    got = run_batch(ws, seqs, g, shared=kv, past=12)
    for i, q in enumerate(seqs):
        assert cosine(oracle_last(oracle, prefix, q), got[i]) >= COS, i
    after = [_read_dev_floats(base, g.layers * cap * g.kvd) for base in (kc, vc)]
    assert all(np.array_equal(a, b) for a, b in zip(before, after))
    # The prefix still serves a plain extension afterwards.
    more = list(rng.integers(0, g.vocab, 3))
    assert cosine(oracle_last(oracle, prefix, more), run_prefill(ws, kv, 12, more, g)) >= COS


@pytest.mark.parametrize("group", [3, 8])
def test_batch_query_groups(group):
    # Packed rows at other query groups (one 32-row half per block above 4).
    geom = lo.Geometry(hidden=256, layers=1, heads=group, kv_heads=1, head_dim=128, inter=512, vocab=96,
                       max_pos=320)
    model, oracle, lm = setup(geom, lo.FMT_Q8B, seed=40 + group)
    g = model["geom"]
    rng = np.random.default_rng(46 + group)
    seqs = [list(rng.integers(0, g.vocab, n)) for n in (40, 3, 70, 33)]
    ws = gphq.Prefill(lm, 160)
    got = run_batch(ws, seqs, g)
    for i, q in enumerate(seqs):
        assert cosine(oracle_last(oracle, [], q, 160), got[i]) >= COS, i


def test_batch_validation_errors():
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    ws = gphq.Prefill(lm, 8)
    kv = gphq.Prefix(lm, 8)
    other = gphq.lm_from_stored(geom_kwargs(g), lo.FMT_Q8B, model["layers"], model["embed"], model["final_norm"],
                                model["head"])
    hid = torch.empty((2, g.hidden), device="cuda")

    def status(f):
        try:
            f()
        except gphq.GphqError as e:
            return e.status
        return gphq.OK

    assert status(lambda: ws.batch([[1], [2]], hid, shared=gphq.Prefix(other, 8), past=0)) == gphq.ERR_FOREIGN_PREFIX
    assert status(lambda: ws.batch([[1], [2]], hid, shared=kv, past=9)) == gphq.ERR_KEEP_RANGE
    assert status(lambda: ws.batch([[1], [2]], hid, past=1)) == gphq.ERR_KEEP_RANGE
    assert status(lambda: ws.batch([], hid)) == gphq.ERR_SEQUENCE_COUNT
    assert status(lambda: ws.batch([[1], []], hid)) == gphq.ERR_EMPTY_SEQUENCE
    assert status(lambda: ws.batch([[1], [2] * (g.max_pos + 1)], hid)) == gphq.ERR_CONTEXT
    assert status(lambda: ws.batch([[1]], hid)) == gphq.ERR_DEST_WIDTH
    assert status(lambda: ws.batch([[1], [g.vocab]], hid)) == gphq.ERR_TOKEN_VOCAB
    assert status(lambda: ws.batch([[1], [2] * 9], hid)) == gphq.ERR_PASS_ROWS


# ---- Embeds, tail states and the reuse contract (gphq_prefill_extend_embed) ----

def run_embed(ws, kv, stored, keep, tokens, k, g, ph=0, rows=None, reuse=0):
    import torch

    tail = torch.full((k, g.hidden), -7.0, device="cuda")
    dev_rows = None if rows is None else torch.from_numpy(np.ascontiguousarray(rows, np.float32)).cuda()
    print(f"extend_embed stored={stored} keep={keep} n={len(tokens)} k={k} rows={ws.rows}", flush=True)
    ws.extend_embed(kv, stored, keep, tokens, tail, embeds_token=ph, embeds_rows=dev_rows, reuse=reuse)
    ws.check()
    return tail.cpu().numpy()


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q4])
def test_embeds_splice_and_tail_match_oracle(fmt):
    # qwen3asr's splice (transcriber.go:481-551): audio rows at the
    # placeholder positions, spread over two passes, and the last 12 states
    # (HiddenTailExtendEmbedInto). 25 tokens in passes of 16 would leave 9 of
    # the 12 tail rows for the second pass, so the passes are 13 + 12
    # (gpu_darwin.go:1473-1479: the last pass holds the whole tail).
    model, oracle, lm = setup(lc.GPU_SHAPE, fmt, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(51)
    ph = 77
    tokens = [int(t) if t != ph else 3 for t in rng.integers(0, g.vocab, 25)]
    for i in (0, 4, 5, 6, 12, 13, 18, 24):
        tokens[i] = ph
    occ = tokens.count(ph)
    rows = rng.standard_normal((occ, g.hidden)).astype(np.float32)
    ws = gphq.Prefill(lm, 16)
    kv = gphq.Prefix(lm, 48)
    k = 12
    got = run_embed(ws, kv, 0, 0, tokens, k, g, ph, rows)
    cache = oracle.new_cache(48)
    h = oracle.prefill(cache, 0, tokens, embeds=(ph, rows), tail=k)
    want, _ = oracle.finish_rows(h)
    for i in range(k):
        assert cosine(want[i], got[i]) >= COS, i
    check_cache(cache, kv, g, len(tokens))


def test_embeds_of_table_rows_equal_plain_tokens_bitwise():
    # Splice rows that are the embedding table's own rows (as float32) give
    # the bits of the unspliced pass: the splice changes only the source row.
    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(52)
    tokens = [int(t) for t in rng.integers(0, g.vocab, 23)]
    ph = tokens[3]
    occ = tokens.count(ph)
    table = lo.bf16_to_f64(model["embed"][ph]).astype(np.float32)
    ws = gphq.Prefill(lm, 32)
    a = run_embed(ws, gphq.Prefix(lm, 32), 0, 0, tokens, 5, g, ph, np.tile(table, (occ, 1)))
    b = run_embed(ws, gphq.Prefix(lm, 32), 0, 0, tokens, 5, g)
    np.testing.assert_array_equal(a, b)
    # The tail's last row is HiddenLastExtendInto's state.
    last = run_prefill(ws, gphq.Prefix(lm, 32), 0, tokens, g)
    np.testing.assert_array_equal(b[-1], last)


def test_continue_with_reuse_recomputes_every_row():
    # HiddenLastContinueEmbedInto: a declared reuse passes the reference's
    # checks and changes nothing (the GPU path recomputes every row,
    # evaluator.go:197-199), including at a kept anchor inside the cache.
    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B_F32, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(53)
    first = [int(t) for t in rng.integers(0, g.vocab, 20)]
    ws = gphq.Prefill(lm, 32)
    kv = gphq.Prefix(lm, 48)
    run_embed(ws, kv, 0, 0, first, 1, g)
    ids = first[6:] + [int(t) for t in rng.integers(0, g.vocab, 4)]
    a = run_embed(ws, kv, 20, 6, ids, 3, g, reuse=14)
    kv2 = gphq.Prefix(lm, 48)
    run_embed(ws, kv2, 0, 0, first, 1, g)
    b = run_embed(ws, kv2, 20, 6, ids, 3, g, reuse=0)
    np.testing.assert_array_equal(a, b)
    cache = oracle.new_cache(48)
    oracle.prefill(cache, 0, first[:6])
    h = oracle.prefill(cache, 6, ids, tail=3)
    want, _ = oracle.finish_rows(h)
    for i in range(3):
        assert cosine(want[i], a[i]) >= COS, i


def test_embed_extend_validation_errors():
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    ws = gphq.Prefill(lm, 8)
    kv = gphq.Prefix(lm, 16)
    rows = torch.zeros((2, g.hidden), device="cuda")

    def status(fn):
        try:
            fn()
        except gphq.GphqError as e:
            return e.status
        return gphq.OK

    t1 = torch.full((1, g.hidden), -7.0, device="cuda")
    t3 = torch.full((3, g.hidden), -7.0, device="cuda")
    ok = [1, 2, 3, 4]
    # Tail shape (evaluator.go:298-301): empty, ragged, more rows than tokens, beyond maxTail.
    assert status(lambda: ws.extend_embed(kv, 0, 0, ok, t1.view(-1)[:0])) == gphq.ERR_TAIL_SHAPE
    assert status(lambda: ws.extend_embed(kv, 0, 0, ok, t3.view(-1)[: g.hidden + 5])) == gphq.ERR_TAIL_SHAPE
    assert status(lambda: ws.extend_embed(kv, 0, 0, [1, 2], t3)) == gphq.ERR_TAIL_SHAPE
    big = torch.zeros((257, g.hidden), device="cuda")
    assert status(lambda: ws.extend_embed(kv, 0, 0, list(range(300)), big)) == gphq.ERR_TAIL_SHAPE
    # Prefix and anchor (evaluator.go:182-196).
    other = gphq.lm_from_stored(geom_kwargs(g), lo.FMT_Q8B, model["layers"], model["embed"], model["final_norm"],
                                model["head"])
    assert status(lambda: ws.extend_embed(gphq.Prefix(other, 16), 0, 0, ok, t1)) == gphq.ERR_FOREIGN_PREFIX
    assert status(lambda: ws.extend_embed(kv, 2, 3, ok, t1)) == gphq.ERR_KEEP_RANGE
    assert status(lambda: ws.extend_embed(kv, 14, 14, ok, t1)) == gphq.ERR_PREFIX_CAPACITY
    assert status(lambda: ws.extend_embed(kv, 6, 2, ok, t1, reuse=5)) == gphq.ERR_REUSE
    assert status(lambda: ws.extend_embed(kv, 9, 2, ok, t1, reuse=5)) == gphq.ERR_REUSE
    # One row per placeholder (evaluator.go:200-211).
    assert status(lambda: ws.extend_embed(kv, 0, 0, [1, 5, 5, 5], t1, embeds_token=5, embeds_rows=rows)) == \
        gphq.ERR_EMBED_ROWS
    # The batch checks (evaluator.go:540-560).
    assert status(lambda: ws.extend_embed(kv, 0, 0, [], t1)) == gphq.ERR_EMPTY_SEQUENCE
    assert status(lambda: ws.extend_embed(kv, 0, 0, [1, g.vocab], t1)) == gphq.ERR_TOKEN_VOCAB
    # A tail taller than one pass.
    t9 = torch.zeros((9, g.hidden), device="cuda")
    assert status(lambda: ws.extend_embed(kv, 0, 0, list(range(12)), t9)) == gphq.ERR_PASS_ROWS
    torch.cuda.synchronize()
    assert (t1 == -7.0).all() and (t3 == -7.0).all()
    kc, _, cap = kv.kv()
    assert not _read_dev_floats(kc, g.kvd * cap).any()
