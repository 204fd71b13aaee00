"""GPU parity of the qwen3lm decode provider (gphq_lm / gphq_prefix /
gphq_decode_*), through the C ABI, against the float64 oracle
(oracle/lm_oracle.py, itself pinned to transformers' Qwen3).

Bounds are the reference GPU decode test's (gpu_decode_batch_darwin_test.go:
121-131: hidden relative 1e-5, logits relative 1e-5), applied as relative L2
against float64, plus a max-abs bound scaled to the vector's magnitude (the
reference's absolute 1e-4 / 2e-4 assume real-checkpoint magnitudes of about
1; these random-weight models run at about 30-100x that).
"""
import numpy as np
import pytest

from gophonic_amd import gphq
from oracle import lm_oracle as lo
from tests import lm_common as lc

pytestmark = pytest.mark.gpu

REL = 1e-5


def geom_kwargs(g):
    return dict(hidden=g.hidden, layers=g.layers, heads=g.heads, kv_heads=g.kv_heads, head_dim=g.head_dim,
                intermediate=g.inter, vocab=g.vocab, max_positions=g.max_pos, eps=g.eps, rope_theta=g.theta)


def device_model(model):
    return gphq.lm_from_stored(geom_kwargs(model["geom"]), model["fmt"], model["layers"], model["embed"],
                               model["final_norm"], model["head"])


def err(want, got):
    want, got = np.asarray(want, np.float64), np.asarray(got, np.float64)
    assert np.isfinite(got).all()
    d = want - got
    return float(np.sqrt((d ** 2).sum() / (want ** 2).sum())), float(np.abs(d).max() / np.abs(want).max())


def top_gap(logits):
    s = np.sort(np.asarray(logits, np.float64))
    return s[-1] - s[-2]


_CACHE = {}


def setup(geom, fmt, seed):
    key = (geom, fmt, seed)
    if key not in _CACHE:
        model = lc.random_model(geom, fmt, seed)
        _CACHE.clear()
        _CACHE[key] = (model, lc.oracle_for(model), device_model(model))
    return _CACHE[key]


def prefill(oracle, ws, kvs, prompts):
    """Extends each lane by its prompt (teacher-forced), on the device and in
    the oracle; returns the oracle caches and positions."""
    caches = [oracle.new_cache(kv.capacity) for kv in kvs]
    lanes = len(kvs)
    pos = [0] * lanes
    steps = max(len(p) for p in prompts)
    for t in range(steps):
        active = [i for i in range(lanes) if t < len(prompts[i])]
        if not active:
            continue
        ws.extend([kvs[i] for i in active], [pos[i] for i in active], [[prompts[i][t] for i in active]])
        for i in active:
            oracle.layers(caches[i], pos[i], oracle.embed_row(prompts[i][t]))
            pos[i] += 1
    return caches, pos


@pytest.mark.parametrize("fmt", lc.FMTS)
@pytest.mark.parametrize("lanes", [1, 3])
def test_decode_batch_into_matches_oracle(fmt, lanes):
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, fmt, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(100 + lanes)
    ws = gphq.DecodeBatch(lm, 4)
    kvs = [gphq.Prefix(lm, 64) for _ in range(lanes)]
    prompts = [list(rng.integers(0, g.vocab, n)) for n in (0, 5, 17)[:lanes]]
    caches, pos = prefill(oracle, ws, kvs, prompts)
    tokens = list(rng.integers(0, g.vocab, lanes))
    hidden = torch.full((lanes, g.hidden), -5.0, device="cuda")
    logits = torch.full((lanes, g.vocab), -5.0, device="cuda")
    ws.into(kvs, pos, tokens, hidden, logits)
    ws.check()
    hid, lg = hidden.cpu().numpy(), logits.cpu().numpy()
    for i in range(lanes):
        wh, wl, _ = oracle.step(caches[i], pos[i], tokens[i])
        rh, ah = err(wh, hid[i])
        rl, al = err(wl, lg[i])
        assert rh <= REL and rl <= REL, (i, rh, rl)
        assert ah <= 10 * REL and al <= 10 * REL, (i, ah, al)
        # The appended K/V row equals the oracle's (the cache the next step reads).
        kc, vc, cap = kvs[i].kv()
        for layer in (0, g.layers - 1):
            for name, base, want in (("k", kc, caches[i][layer][0]), ("v", vc, caches[i][layer][1])):
                got = _read_dev_floats(base + ((layer * cap + pos[i]) * g.kvd) * 4, g.kvd)
                r, _ = err(want[pos[i]], got)
                assert r <= REL, (name, layer, r)


def _read_dev_floats(addr, n):
    """Copies n floats from a raw device address (a prefix's cache)."""
    import ctypes

    import torch

    out = torch.empty(n, dtype=torch.float32, device="cuda")
    # The HIP runtime torch loaded (same soname), so device addresses agree.
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    torch.cuda.synchronize()
    assert hip.hipMemcpy(out.data_ptr(), addr, n * 4, 3) == 0  # hipMemcpyDeviceToDevice
    return out.cpu().numpy()


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q8])
def test_decode_06b_widths_long_context(fmt):
    # Qwen3-0.6B widths (16 query / 8 KV heads, hidden 1024, inter 3072) with a
    # 300-token context: many attention splits and more than one block per
    # split's key range.
    import torch

    model, oracle, lm = setup(lc.SMALL_06B, fmt, seed=9)
    g = model["geom"]
    rng = np.random.default_rng(7)
    ws = gphq.DecodeBatch(lm, 2)
    kvs = [gphq.Prefix(lm, 400), gphq.Prefix(lm, 320)]
    prompts = [list(rng.integers(0, g.vocab, 300)), list(rng.integers(0, g.vocab, 41))]
    caches, pos = prefill(oracle, ws, kvs, prompts)
    for lanes in (1, 2):
        tokens = list(rng.integers(0, g.vocab, lanes))
        hidden = torch.empty((lanes, g.hidden), device="cuda")
        logits = torch.empty((lanes, g.vocab), device="cuda")
        ws.into(kvs[:lanes], pos[:lanes], tokens, hidden, logits)
        hid, lg = hidden.cpu().numpy(), logits.cpu().numpy()
        for i in range(lanes):
            wh, wl, _ = oracle.step(caches[i], pos[i], tokens[i])
            rh, _ = err(wh, hid[i])
            rl, _ = err(wl, lg[i])
            assert rh <= REL and rl <= REL, (lanes, i, rh, rl)
            pos[i] += 1


@pytest.mark.parametrize("group", [1, 3, 5, 8])
def test_decode_query_groups(group):
    # Query heads per KV head other than 2 and 4: the attention kernel's
    # per-lane query registers and keys per step change with the group. Two
    # lanes at ragged contexts of 150 and 37 keys (several splits, a partial
    # last step, the new key in the last block).
    import torch

    geom = lo.Geometry(hidden=256, layers=2, heads=group, kv_heads=1, head_dim=128, inter=512, vocab=96,
                       max_pos=320)
    model, oracle, lm = setup(geom, lo.FMT_Q8B, seed=50 + group)
    g = model["geom"]
    rng = np.random.default_rng(60 + group)
    ws = gphq.DecodeBatch(lm, 2)
    kvs = [gphq.Prefix(lm, 200), gphq.Prefix(lm, 64)]
    prompts = [list(rng.integers(0, g.vocab, 150)), list(rng.integers(0, g.vocab, 37))]
    caches, pos = prefill(oracle, ws, kvs, prompts)
    tokens = list(rng.integers(0, g.vocab, 2))
    hidden = torch.empty((2, g.hidden), device="cuda")
    logits = torch.empty((2, g.vocab), device="cuda")
    ws.into(kvs, pos, tokens, hidden, logits)
    hid, lg = hidden.cpu().numpy(), logits.cpu().numpy()
    for i in range(2):
        wh, wl, _ = oracle.step(caches[i], pos[i], tokens[i])
        rh, _ = err(wh, hid[i])
        rl, _ = err(wl, lg[i])
        assert rh <= REL and rl <= REL, (group, i, rh, rl)


@pytest.mark.parametrize("lanes", [1, 2, 5])
def test_greedy_into_and_run_match_oracle(lanes):
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(31 + lanes)
    ws = gphq.DecodeBatch(lm, 8)
    steps = 12
    kvs = [gphq.Prefix(lm, 80) for _ in range(lanes)]
    prompts = [list(rng.integers(0, g.vocab, 3 + 4 * i)) for i in range(lanes)]
    caches, pos0 = prefill(oracle, ws, kvs, prompts)
    # Copies of the prefixes for the chained run.
    kvs2 = [gphq.Prefix(lm, 80) for _ in range(lanes)]
    for a, b in zip(kvs2, kvs):
        a.copy_from(b, max(pos0))
    first = list(rng.integers(0, g.vocab, lanes))
    # Step by step through greedy_into.
    hidden = torch.empty((lanes, g.hidden), device="cuda")
    nxt = torch.empty(lanes, dtype=torch.int32, device="cuda")
    toks, pos, seq = list(first), list(pos0), []
    for _ in range(steps):
        ws.greedy_into(kvs, pos, toks, hidden, nxt)
        toks = nxt.cpu().numpy().tolist()
        seq.append(toks)
        pos = [p + 1 for p in pos]
    hid_step = hidden.cpu().numpy()
    # The chained run on the copies gives the same tokens and hidden states.
    out = torch.full((steps, lanes), -1, dtype=torch.int32, device="cuda")
    hidden2 = torch.empty((lanes, g.hidden), device="cuda")
    ws.greedy_run(kvs2, pos0, first, steps, out, hidden2)
    ws.check()
    assert out.cpu().numpy().tolist() == seq
    np.testing.assert_array_equal(hidden2.cpu().numpy(), hid_step)
    # Each chosen token is the oracle's argmax, teacher-forced with the GPU's
    # choices (a near tie within the bound may go either way).
    for i in range(lanes):
        t = first[i]
        for s in range(steps):
            _, wl, want = oracle.step(caches[i], pos0[i] + s, t)
            got = seq[s][i]
            assert got == want or wl[want] - wl[got] <= 1e-4 * np.abs(wl).max(), (i, s, got, want)
            t = got


def test_lanes_together_match_lanes_alone():
    # gpu_vector_batch_darwin_test.go:217-220: batched lanes agree with
    # single-lane decodes to max_abs 1e-4 (scaled) and relative 1e-5.
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(77)
    lanes = 6
    ws = gphq.DecodeBatch(lm, lanes)
    prompts = [list(rng.integers(0, g.vocab, 2 + i)) for i in range(lanes)]
    tokens = list(rng.integers(0, g.vocab, lanes))
    kvs_a = [gphq.Prefix(lm, 32) for _ in range(lanes)]
    kvs_b = [gphq.Prefix(lm, 32) for _ in range(lanes)]
    _, pos = prefill(oracle, ws, kvs_a, prompts)
    for a, b in zip(kvs_b, kvs_a):
        a.copy_from(b, max(pos))
    hid = torch.empty((lanes, g.hidden), device="cuda")
    lg = torch.empty((lanes, g.vocab), device="cuda")
    ws.into(kvs_a, pos, tokens, hid, lg)
    for i in range(lanes):
        h1 = torch.empty((1, g.hidden), device="cuda")
        l1 = torch.empty((1, g.vocab), device="cuda")
        ws.into([kvs_b[i]], [pos[i]], [tokens[i]], h1, l1)
        rh, ah = err(h1.cpu().numpy()[0], hid.cpu().numpy()[i])
        rl, al = err(l1.cpu().numpy()[0], lg.cpu().numpy()[i])
        assert rh <= REL and rl <= REL and ah <= 10 * REL and al <= 10 * REL, (i, rh, rl, ah, al)


def test_validation_errors():
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    ws = gphq.DecodeBatch(lm, 2)
    a, b = gphq.Prefix(lm, 4), gphq.Prefix(lm, 4)
    hid = torch.empty((3, g.hidden), device="cuda")
    nxt = torch.empty(3, dtype=torch.int32, device="cuda")

    def status(fn):
        try:
            fn()
        except gphq.GphqError as e:
            return e.status
        return gphq.OK

    assert status(lambda: ws.greedy_into([a, b, gphq.Prefix(lm, 4)], [0, 0, 0], [1, 1, 1], hid, nxt)) == \
        gphq.ERR_LANE_CAPACITY
    assert status(lambda: ws.greedy_into([a, a], [0, 0], [1, 1], hid, nxt)) == gphq.ERR_DUPLICATE_PREFIX
    assert status(lambda: ws.greedy_into([a], [4], [1], hid, nxt)) == gphq.ERR_PREFIX_FULL
    assert status(lambda: ws.greedy_into([a], [0], [g.vocab], hid, nxt)) == gphq.ERR_TOKEN_RANGE
    assert status(lambda: ws.greedy_into([a], [0], [-1], hid, nxt)) == gphq.ERR_TOKEN_RANGE
    other = gphq.lm_from_stored(geom_kwargs(g), lo.FMT_Q8B, model["layers"], model["embed"], model["final_norm"],
                                model["head"])
    assert status(lambda: ws.greedy_into([gphq.Prefix(other, 4)], [0], [1], hid, nxt)) == gphq.ERR_FOREIGN_PREFIX
    assert status(lambda: ws.greedy_run([a], [2], [1], 3, torch.empty(3, dtype=torch.int32, device="cuda"))) == \
        gphq.ERR_PREFIX_FULL
    # Nothing was enqueued by the rejected calls: the prefixes are untouched.
    kc, vc, cap = a.kv()
    assert not _read_dev_floats(kc, g.kvd * cap).any()
    # A model without a head cannot make a workspace.
    bare = gphq.Lm(gphq.lm_config(fmt=lo.FMT_Q8B, **geom_kwargs(g)))
    assert status(lambda: gphq.DecodeBatch(bare, 1)) == gphq.ERR_MODEL_INCOMPLETE


def test_run_graph_replays_match_eager_launches():
    # The chained run replays one captured step as a HIP graph. Several runs,
    # with eager decode work and synchronizations between them and a
    # recapture for new prefixes, must each equal the eager launches.
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(5)
    lanes, steps = 3, 7
    ws = gphq.DecodeBatch(lm, 4)
    base = [gphq.Prefix(lm, 40) for _ in range(lanes)]
    prompts = [list(rng.integers(0, g.vocab, 4 + i)) for i in range(lanes)]
    _, pos = prefill(oracle, ws, base, prompts)
    first = list(rng.integers(0, g.vocab, lanes))

    def run(graph, kvs):
        for a, b in zip(kvs, base):
            a.copy_from(b, max(pos))
        ws.set_graph(graph)
        out = torch.full((steps, lanes), -1, dtype=torch.int32, device="cuda")
        hid = torch.empty((lanes, g.hidden), device="cuda")
        ws.greedy_run(kvs, pos, first, steps, out, hid)
        torch.cuda.synchronize()
        return out.cpu().numpy(), hid.cpu().numpy()

    kv1 = [gphq.Prefix(lm, 40) for _ in range(lanes)]
    kv2 = [gphq.Prefix(lm, 40) for _ in range(lanes)]
    want_t, want_h = run(False, kv1)
    other = gphq.Prefix(lm, 40)
    for rep in range(3):
        got_t, got_h = run(True, kv1 if rep < 2 else kv2)
        np.testing.assert_array_equal(got_t, want_t)
        np.testing.assert_array_equal(got_h, want_h)
        # Eager work on the same workspace between replays.
        h1 = torch.empty((1, g.hidden), device="cuda")
        l1 = torch.empty((1, g.vocab), device="cuda")
        ws.into([other], [rep], [int(first[0])], h1, l1)
        torch.cuda.synchronize()


def test_run_graph_recaptured_after_prefix_free_and_rebind():
    # The captured step holds the lanes' K/V addresses and the bound weight
    # addresses. A prefix freed and replaced by a new one (whose host object
    # may reuse the freed one's address, with other K/V buffers and another
    # capacity), or a layer rebound to other weights, must not replay the
    # stale graph: each chained run equals the eager launches.
    import torch

    model = lc.random_model(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    lm = device_model(model)  # rebound below: not the shared cached model
    g = model["geom"]
    rng = np.random.default_rng(12)
    lanes, steps = 2, 5
    ws = gphq.DecodeBatch(lm, 2)
    base = [gphq.Prefix(lm, 40) for _ in range(lanes)]
    prompts = [list(rng.integers(0, g.vocab, 6 + i)) for i in range(lanes)]
    _, pos = prefill(lc.oracle_for(model), ws, base, prompts)
    first = list(rng.integers(0, g.vocab, lanes))

    def run(graph, kvs):
        for a, b in zip(kvs, base):
            a.copy_from(b, max(pos))
        ws.set_graph(graph)
        out = torch.full((steps, lanes), -1, dtype=torch.int32, device="cuda")
        hid = torch.empty((lanes, g.hidden), device="cuda")
        ws.greedy_run(kvs, pos, first, steps, out, hid)
        torch.cuda.synchronize()
        return out.cpu().numpy(), hid.cpu().numpy()

    kv1 = [gphq.Prefix(lm, 40) for _ in range(lanes)]
    run(True, kv1)  # captures a graph over kv1
    addrs = [p.h.value for p in kv1]
    for p in kv1:
        p.close()
    kv2 = [gphq.Prefix(lm, 24 + 8 * i) for i in range(lanes)]
    reused = sum(p.h.value in addrs for p in kv2)
    got_t, got_h = run(True, kv2)
    want_t, want_h = run(False, kv2)
    np.testing.assert_array_equal(got_t, want_t)
    np.testing.assert_array_equal(got_h, want_h)
    print(f"prefix host addresses reused: {reused} of {lanes}")
    # Rebind layer 0 to another model's weights after a capture.
    run(True, kv2)
    other_model = lc.random_model(lc.GPU_SHAPE, lo.FMT_Q8B, seed=6)
    other = device_model(other_model)
    desc, _ = gphq.lm_layer_layout(lm.cfg)
    L0 = other_model["layers"][0]
    lm.bind_layer(0, other._keep[0], desc, L0.q_norm, L0.k_norm)
    got_t, got_h = run(True, kv2)
    want2_t, want2_h = run(False, kv2)
    np.testing.assert_array_equal(got_t, want2_t)
    np.testing.assert_array_equal(got_h, want2_h)
    assert not np.array_equal(want2_h, want_h)  # the rebind changed the model


# One layer at Qwen3-8B widths: the GEMVs take the K = 4096 shapes with two
# and four K slices (the norm prologue's cross-slice sum included) and
# down's K = 12288 in six slices.
QWEN3_8B_LAYER = lo.Geometry(hidden=4096, layers=1, heads=32, kv_heads=8, head_dim=128, inter=12288, vocab=1000,
                             max_pos=64)


@pytest.mark.parametrize("fmt", [lo.FMT_Q8B, lo.FMT_Q8])
def test_decode_8b_widths(fmt):
    import torch

    model, oracle, lm = setup(QWEN3_8B_LAYER, fmt, seed=21)
    g = model["geom"]
    rng = np.random.default_rng(8)
    ws = gphq.DecodeBatch(lm, 2)
    kvs = [gphq.Prefix(lm, 32), gphq.Prefix(lm, 32)]
    caches, pos = prefill(oracle, ws, kvs, [list(rng.integers(0, g.vocab, 9)), list(rng.integers(0, g.vocab, 4))])
    for lanes in (1, 2):
        tokens = list(rng.integers(0, g.vocab, lanes))
        hidden = torch.empty((lanes, g.hidden), device="cuda")
        logits = torch.empty((lanes, g.vocab), device="cuda")
        ws.into(kvs[:lanes], pos[:lanes], tokens, hidden, logits)
        hid, lg = hidden.cpu().numpy(), logits.cpu().numpy()
        for i in range(lanes):
            wh, wl, _ = oracle.step(caches[i], pos[i], tokens[i])
            rh, ah = err(wh, hid[i])
            rl, al = err(wl, lg[i])
            assert rh <= REL and rl <= REL, (lanes, i, rh, rl)
            assert ah <= 10 * REL and al <= 10 * REL, (lanes, i, ah, al)
            pos[i] += 1


def test_decode_8b_widths_16_lanes():
    # 16 lanes through the stationary-activation multi-vector GEMVs at Qwen3-8B
    # widths, the down projection (K = 12288) on its K-split path.
    import torch

    model, oracle, lm = setup(QWEN3_8B_LAYER, lo.FMT_Q8B_F32, seed=23)
    g = model["geom"]
    rng = np.random.default_rng(9)
    lanes = 16
    ws = gphq.DecodeBatch(lm, lanes)
    kvs = [gphq.Prefix(lm, 16) for _ in range(lanes)]
    caches, pos = prefill(oracle, ws, kvs, [list(rng.integers(0, g.vocab, 1 + i % 5)) for i in range(lanes)])
    tokens = list(rng.integers(0, g.vocab, lanes))
    hidden = torch.empty((lanes, g.hidden), device="cuda")
    logits = torch.empty((lanes, g.vocab), device="cuda")
    ws.into(kvs, pos, tokens, hidden, logits)
    hid, lg = hidden.cpu().numpy(), logits.cpu().numpy()
    for i in range(lanes):
        wh, wl, _ = oracle.step(caches[i], pos[i], tokens[i])
        rh, _ = err(wh, hid[i])
        rl, _ = err(wl, lg[i])
        assert rh <= REL and rl <= REL, (i, rh, rl)


def head_oracle(oracle, hidden):
    """LogitsInto on float64: the head times R applied to each post-final-norm state."""
    h = np.asarray(hidden, np.float64)
    return np.stack([oracle.head @ lo.rot_apply(row, oracle.hrot) for row in h])


@pytest.mark.parametrize("lanes", [1, 3])
def test_logits_of_step_hidden_equal_step_logits(lanes):
    """The head over a step's hidden states reproduces that step's logits bit
    for bit (same rotation and the same GEMV for the same row count)."""
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(40 + lanes)
    ws = gphq.DecodeBatch(lm, 4)
    kvs = [gphq.Prefix(lm, 32) for _ in range(lanes)]
    prompts = [list(rng.integers(0, g.vocab, n)) for n in (4, 9, 2)[:lanes]]
    _, pos = prefill(oracle, ws, kvs, prompts)
    hidden = torch.empty((lanes, g.hidden), device="cuda")
    logits = torch.empty((lanes, g.vocab), device="cuda")
    ws.into(kvs, pos, list(rng.integers(0, g.vocab, lanes)), hidden, logits)
    again = torch.full((lanes, g.vocab), -7.0, device="cuda")
    ws.logits(hidden, again)
    torch.cuda.synchronize()
    assert torch.equal(again, logits)
    rl, al = err(head_oracle(oracle, hidden.cpu().numpy()), again.cpu().numpy())
    assert rl <= REL and al <= 10 * REL, (rl, al)


@pytest.mark.parametrize("rows,capacity", [(1, 1), (2, 4), (11, 4), (256, 32)])
def test_logits_rows_match_oracle(rows, capacity):
    """LogitsRowsInto over row counts that span several workspace chunks
    (11 rows through 4 lanes: 4 + 4 + 3) up to the reference's maxTail (256)."""
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    rng = np.random.default_rng(rows)
    hid = (rng.standard_normal((rows, g.hidden)) * 2).astype(np.float32)
    ws = gphq.DecodeBatch(lm, capacity)
    out = torch.full((rows, g.vocab), -7.0, device="cuda")
    ws.logits(torch.from_numpy(hid).cuda(), out)
    got = out.cpu().numpy()
    want = head_oracle(oracle, hid)
    for r in range(rows):
        rl, al = err(want[r], got[r])
        assert rl <= REL and al <= 10 * REL, (r, rl, al)
    # A row's logits do not depend on the rows beside it beyond the GEMV
    # variant: one row alone agrees to the same bound.
    one = torch.empty((1, g.vocab), device="cuda")
    ws.logits(torch.from_numpy(hid[-1:]).cuda(), one)
    rl, _ = err(want[-1], one.cpu().numpy()[0])
    assert rl <= REL


def test_logits_validation_errors():
    import torch

    model, oracle, lm = setup(lc.GPU_SHAPE, lo.FMT_Q8B, seed=5)
    g = model["geom"]
    ws = gphq.DecodeBatch(lm, 2)

    def status(fn):
        try:
            fn()
        except gphq.GphqError as e:
            return e.status
        return gphq.OK

    hid = torch.zeros((3, g.hidden), device="cuda")
    out = torch.full((3, g.vocab), -7.0, device="cuda")
    assert status(lambda: ws.logits(hid[:0], out[:0])) == gphq.ERR_LOGITS_SHAPE
    assert status(lambda: ws.logits(hid.view(-1)[: g.hidden + 1], out[:1])) == gphq.ERR_LOGITS_SHAPE
    assert status(lambda: ws.logits(hid, out[:2])) == gphq.ERR_LOGITS_SHAPE
    assert status(lambda: ws.logits(hid, out.view(-1)[: 3 * g.vocab - 1])) == gphq.ERR_LOGITS_SHAPE
    big = torch.zeros((257, g.hidden), device="cuda")
    assert status(lambda: ws.logits(big, torch.empty((257, g.vocab), device="cuda"))) == gphq.ERR_LOGITS_SHAPE
    both = torch.zeros(4 * g.hidden, device="cuda")
    assert status(lambda: ws.logits(both[: g.hidden], both[g.hidden - 4: g.hidden - 4 + g.vocab])) == \
        gphq.ERR_OVERLAP
    torch.cuda.synchronize()
    assert (out == -7.0).all()
    assert gphq.error_string(gphq.ERR_LOGITS_SHAPE).startswith("qwen3: logits")


# A small model with a long RoPE table, for contexts of a few thousand keys.
LONG = lo.Geometry(hidden=256, layers=2, heads=2, kv_heads=1, head_dim=128, inter=512, vocab=96, max_pos=4096)


def test_attention_ranges_follow_the_context_not_the_capacity():
    # The attention blocks take their key ranges from the lane's context
    # alone. A prefix with twice the rows it needs (the reference's callers
    # double capacity, qwen3/chat.go:760-769) decodes the same bits as one
    # sized to the need, step by step, eagerly, or replayed from one captured
    # step; here the run crosses a change of range (2560 keys over 32 splits
    # take 80 keys each, 2561 take 96), so a replayed step first loads the
    # range the capture expected and then its own. The first step matches the
    # float64 oracle over the same cache rows.
    import torch

    g = LONG
    model = lc.random_model(g, lo.FMT_Q8B, 23)
    oracle = lc.oracle_for(model)
    lm = device_model(model)
    rng = np.random.default_rng(8)
    ctx, steps = 2552, 16
    src = gphq.Prefix(lm, ctx + steps + 1)
    pf = gphq.Prefill(lm, 512)
    pf.extend(src, 0, list(rng.integers(0, g.vocab, ctx)), torch.empty(g.hidden, device="cuda"))
    pf.check()
    first = int(rng.integers(0, g.vocab))
    ws = gphq.DecodeBatch(lm, 1)

    def fresh(cap):
        kv = gphq.Prefix(lm, cap)
        kv.copy_from(src, ctx)
        return kv

    # The oracle's first step over the prefilled rows.
    kc, vc, cap = src.kv()
    rows = _read_dev_floats(kc, g.layers * cap * g.kvd).reshape(g.layers, cap, g.kvd)
    vrows = _read_dev_floats(vc, g.layers * cap * g.kvd).reshape(g.layers, cap, g.kvd)
    cache = [(rows[i].astype(np.float64).copy(), vrows[i].astype(np.float64).copy()) for i in range(g.layers)]
    want_h, want_l, _ = oracle.step(cache, ctx, first)
    kv = fresh(ctx + steps + 1)
    h1 = torch.empty((1, g.hidden), device="cuda")
    l1 = torch.empty((1, g.vocab), device="cuda")
    ws.into([kv], [ctx], [first], h1, l1)
    rh, _ = err(want_h, h1.cpu().numpy()[0])
    rl, _ = err(want_l, l1.cpu().numpy()[0])
    assert rh <= REL and rl <= REL, (rh, rl)

    def step_by_step(cap):
        kv = fresh(cap)
        hid = torch.empty((1, g.hidden), device="cuda")
        nxt = torch.empty(1, dtype=torch.int32, device="cuda")
        tok, toks = first, []
        for s in range(steps):
            ws.greedy_into([kv], [ctx + s], [tok], hid, nxt)
            tok = int(nxt.cpu().numpy()[0])
            toks.append(tok)
        return np.array(toks), hid.cpu().numpy()

    def run(cap, graph):
        kv = fresh(cap)
        ws.set_graph(graph)
        out = torch.full((steps, 1), -1, dtype=torch.int32, device="cuda")
        hid = torch.empty((1, g.hidden), device="cuda")
        ws.greedy_run([kv], [ctx], [first], steps, out, hid)
        torch.cuda.synchronize()
        return out.cpu().numpy()[:, 0], hid.cpu().numpy()

    want_t, want_hid = step_by_step(ctx + steps + 1)
    for cap in (ctx + steps + 1, 2 * (ctx + steps)):
        for got_t, got_hid in (step_by_step(cap), run(cap, False), run(cap, True)):
            np.testing.assert_array_equal(got_t, want_t)
            np.testing.assert_array_equal(got_hid, want_hid)
    ws.check()
