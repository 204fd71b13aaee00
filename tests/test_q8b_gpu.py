"""GPU parity of the block-32 int8 path (gphq_q8b_quantize / gphq_q8b_gemm),
through the C ABI, bit-exact against the oracle (oracle.q8b_quantize /
q8b_gemm, pinned in tests/test_q8b_oracle.py): codes and scales equal, and every
output equals the oracle's block-ordered fmaf sum bit for bit."""
import numpy as np
import pytest

from gophonic_amd import gphq
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def quantize_dev(x):
    import torch

    rows, k = x.shape
    q = torch.empty((rows, k), dtype=torch.int8, device="cuda")
    d = torch.empty((rows, k // 32), dtype=torch.float32, device="cuda")
    gphq.q8b_quantize(dev(x), rows, k, q, d)
    return q, d


def test_quantize_bit_exact_with_special_blocks():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((9, 224)) * rng.choice([1e-6, 1.0, 1e4], size=(9, 1))).astype(np.float32)
    x[0, :32] = 0.0
    x[1, 40] = np.nan
    x[2, 100] = -np.inf
    x[3, 3] = np.float32(2.0 ** -130)  # subnormal maximum of its block
    x[4, 64:96] = np.float32(127.0) / 2 * np.sign(rng.standard_normal(32))  # every value a tie of the rule
    print("q8b quantize 9x224", flush=True)
    q, d = quantize_dev(x)
    wq, wd = orc.q8b_quantize(x, 9, 224)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), wd.view(np.uint32))


@pytest.mark.parametrize("m,k,n", [(1, 64, 96), (5, 4096, 200), (37, 160, 130), (128, 4096, 384), (300, 1024, 257),
                                   (1, 4096, 1001), (16, 2048, 301), (3, 8192, 77), (2, 1024, 3), (17, 1024, 64),
                                   (32, 4096, 130), (24, 96, 50), (33, 4096, 96), (255, 512, 100), (256, 160, 97),
                                   (1, 2048, 37), (1, 8192, 100), (1, 12288, 45), (1, 4096, 3)])
def test_gemm_bit_exact(m, k, n):
    import torch

    rng = np.random.default_rng(m + k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    dw = (np.abs(rng.standard_normal((n, k // 32))) * 0.01).astype(np.float32)
    q, d = quantize_dev(x)
    y = torch.empty((m, n), device="cuda")
    print(f"q8b gemm m={m} k={k} n={n}", flush=True)
    gphq.q8b_gemm(q, d, dev(qw), dev(dw), y, m, k, n)
    want = orc.q8b_gemm(q.cpu().numpy(), d.cpu().numpy(), qw, dw, m, k, n)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m", [1, 16, 128, 512])
def test_config2_shape_rows_bit_exact(m):
    # Benchmark configuration 2 (K = 4096, N = 12288) at each bench M: sampled
    # rows against the oracle (rows are independent).
    import torch

    k, n = 4096, 12288
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn((m, k), device="cuda", generator=g)
    qw = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
    dw = torch.randn((n, k // 32), device="cuda", generator=g).abs() * 0.01
    q = torch.empty((m, k), dtype=torch.int8, device="cuda")
    d = torch.empty((m, k // 32), device="cuda")
    gphq.q8b_quantize(x, m, k, q, d)
    y = torch.empty((m, n), device="cuda")
    print(f"q8b gemm config 2 m={m}", flush=True)
    gphq.q8b_gemm(q, d, qw, dw, y, m, k, n)
    rows = sorted({0, min(m - 1, 131), min(m - 1, 255), min(m - 1, 256), m - 1})
    qh, dh = q.cpu().numpy()[rows], d.cpu().numpy()[rows]
    want = orc.q8b_gemm(qh, dh, qw.cpu().numpy(), dw.cpu().numpy(), len(rows), k, n)
    assert np.array_equal(y.cpu().numpy()[rows].view(np.uint32), want.view(np.uint32))
    wq, wd = orc.q8b_quantize(x.cpu().numpy()[rows], len(rows), k)
    assert np.array_equal(qh, wq) and np.array_equal(dh.view(np.uint32), wd.view(np.uint32))
