"""Random qwen3lm GPU-format models for the decode tests (numpy, seeded).

Value distributions follow the benchmark's decode configurations: int8 codes
uniform in [-127, 127], block (or row) scales |N(0,1)|*0.02, Q4 bytes uniform,
norm weights 1 + N(0, 0.02), BF16 embeddings N(0, 1), and a Q8B head whose
rows are padded to a multiple of 16 with zeros (gpu_darwin.go:343-346).
"""
import numpy as np

from oracle import lm_oracle as lo

FMTS = (lo.FMT_Q8B, lo.FMT_Q8B_F32, lo.FMT_Q8, lo.FMT_Q4)

# lmtest.GPUShape (lmtest/lmtest.go:34): the smallest geometry the GPU backend runs.
GPU_SHAPE = lo.Geometry(hidden=256, layers=2, heads=2, kv_heads=1, head_dim=128, inter=512, vocab=96, max_pos=320)
# Qwen3-0.6B widths with fewer layers and a smaller vocabulary.
SMALL_06B = lo.Geometry(hidden=1024, layers=3, heads=16, kv_heads=8, head_dim=128, inter=3072, vocab=1000, max_pos=640)


def rand_matrix(rng, fmt, n, k, scale=0.02):
    """(codes, scales) of an n x k stored matrix in format fmt."""
    if fmt == lo.FMT_Q4:
        codes = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
        sc = (np.abs(rng.standard_normal(n * k // 32)) * scale).astype(np.float16).view(np.uint16)
        return codes, sc
    codes = rng.integers(-127, 128, n * k, dtype=np.int8)
    if fmt == lo.FMT_Q8:
        sc = (np.abs(rng.standard_normal(n)) * scale).astype(np.float32)
    elif fmt == lo.FMT_Q8B:
        sc = (np.abs(rng.standard_normal(n * k // 32)) * scale).astype(np.float16).view(np.uint16)
    else:
        sc = (np.abs(rng.standard_normal(n * k // 32)) * scale).astype(np.float32)
    return codes, sc


def bf16_bits(x):
    """Round-to-nearest-even BF16 bits of float32 values."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def random_model(geom, fmt, seed):
    """dict(layers=[lo.Layer], embed=bf16 bits, final_norm, head=(codes, scales))."""
    g = geom
    rng = np.random.default_rng(seed)
    layers = []
    for _ in range(g.layers):
        layers.append(lo.Layer(
            qkv=rand_matrix(rng, fmt, g.qd + 2 * g.kvd, g.hidden),
            o=rand_matrix(rng, fmt, g.hidden, g.qd),
            gu=rand_matrix(rng, fmt, 2 * g.inter, g.hidden),
            down=rand_matrix(rng, fmt, g.hidden, g.inter),
            q_norm=(1 + 0.02 * rng.standard_normal(g.head_dim)).astype(np.float32),
            k_norm=(1 + 0.02 * rng.standard_normal(g.head_dim)).astype(np.float32),
        ))
    embed = bf16_bits(rng.standard_normal((g.vocab, g.hidden)).astype(np.float32))
    final_norm = (1 + 0.02 * rng.standard_normal(g.hidden)).astype(np.float32)
    hc, hs = rand_matrix(rng, lo.FMT_Q8B, g.head_rows, g.hidden)
    hc = hc.reshape(g.head_rows, g.hidden)
    hc[g.vocab:] = 0
    hs = hs.reshape(g.head_rows, g.hidden // 32)
    hs[g.vocab:] = 0
    return dict(geom=g, fmt=fmt, layers=layers, embed=embed, final_norm=final_norm,
                head=(hc.reshape(-1), hs.reshape(-1)))


def oracle_for(model):
    return lo.DecodeOracle(model["geom"], model["fmt"], model["layers"], model["embed"], model["final_norm"],
                           model["head"])
