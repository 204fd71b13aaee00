"""gphq_gemv_vec_noalloc (the multi-vector GEMV on the library's static
scratch, for callers that cannot allocate) against gphq_gemv_vec with a
caller workspace: the same kernels, so the same bits, through the C ABI.
Two calls in a row, the second with a smaller input, so the second runs on
the scratch the first left behind; then a request beyond the static array;
then, in a fresh process, a first call made under HIP graph capture.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

from gophonic_amd import gphq

pytestmark = pytest.mark.gpu


def weights(fmt, rng, n, k):
    if fmt == gphq.FMT_Q4:
        codes = rng.integers(0, 256, n * k // 2).astype(np.uint8)
        scales = (np.abs(rng.standard_normal(n * k // 32)) * 0.01).astype(np.float16).view(np.uint16)
    elif fmt == gphq.FMT_Q8B:
        codes = rng.integers(-127, 128, n * k).astype(np.int8)
        scales = (np.abs(rng.standard_normal(n * k // 32)) * 0.01).astype(np.float16).view(np.uint16)
    elif fmt == gphq.FMT_Q8B_F32:
        codes = rng.integers(-127, 128, n * k).astype(np.int8)
        scales = (np.abs(rng.standard_normal(n * k // 32)) * 0.01).astype(np.float32)
    else:
        codes = rng.integers(-127, 128, n * k).astype(np.int8)
        scales = (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float32)
    return codes, scales


def both(fmt, lanes, k, n, seed):
    """(noalloc output, workspace output) as uint32 bit patterns."""
    import torch

    rng = np.random.default_rng(seed)
    codes, scales = weights(fmt, rng, n, k)
    dc, ds = torch.from_numpy(codes).cuda(), torch.from_numpy(scales).cuda()
    x = torch.from_numpy(rng.standard_normal(lanes * k).astype(np.float32)).cuda()
    y0 = torch.full((lanes * n,), -7.0, device="cuda")
    gphq.gemv_vec_noalloc(fmt, dc, ds, x, y0, lanes, k, n)
    work = torch.empty(gphq.gemv_vec_workspace_bytes(lanes, k), dtype=torch.uint8, device="cuda")
    y1 = torch.full((lanes * n,), -9.0, device="cuda")
    gphq.gemv_vec(fmt, dc, ds, x, y1, lanes, k, n, work)
    torch.cuda.synchronize()
    return y0.cpu().numpy().view(np.uint32), y1.cpu().numpy().view(np.uint32)


# (first call, second smaller call): the stationary-activation path (8-bit,
# K a multiple of 512 up to 4096, 2-16 lanes), its K-split form is not used
# here (no split buffer), and the per-block path (Q4, more than 16 lanes).
PAIRS = [
    ((gphq.FMT_Q8B, 16, 4096, 4096), (gphq.FMT_Q8B, 3, 1024, 200)),
    ((gphq.FMT_Q8B_F32, 8, 4096, 1536), (gphq.FMT_Q8, 2, 2048, 96)),
    ((gphq.FMT_Q4, 32, 12288, 512), (gphq.FMT_Q4, 5, 4096, 64)),
    ((gphq.FMT_Q8B, 32, 16384, 256), (gphq.FMT_Q8B, 1, 96, 17)),
]


@pytest.mark.parametrize("first,second", PAIRS, ids=[f"pair{i}" for i in range(len(PAIRS))])
def test_noalloc_equals_workspace_entry(first, second):
    for seed, (fmt, lanes, k, n) in enumerate((first, second)):
        assert gphq.gemv_vec_workspace_bytes(lanes, k) <= gphq.GEMV_VEC_NOALLOC_BYTES
        got, want = both(fmt, lanes, k, n, 1000 * seed + lanes + k)
        assert np.array_equal(got, want), (fmt, lanes, k, n)


def test_noalloc_rejects_more_than_its_scratch():
    import torch

    lanes, k, n = 32, 32768, 16
    assert gphq.gemv_vec_workspace_bytes(lanes, k) > gphq.GEMV_VEC_NOALLOC_BYTES
    codes = torch.zeros(n * k, dtype=torch.int8, device="cuda")
    scales = torch.zeros(n * k // 32, dtype=torch.float16, device="cuda")
    x = torch.zeros(lanes * k, device="cuda")
    y = torch.full((lanes * n,), -7.0, device="cuda")
    with pytest.raises(gphq.GphqError) as e:
        gphq.gemv_vec_noalloc(gphq.FMT_Q8B, codes, scales, x, y, lanes, k, n)
    assert e.value.status == gphq.ERR_SCRATCH_LIMIT
    torch.cuda.synchronize()
    assert (y == -7.0).all()


# Run in a fresh process, so that the scratch address is first looked up
# while the stream is being captured (torch.cuda.graph's default global
# capture mode). Each replay follows eager work on the same inputs and is
# checked bit for bit against gphq_gemv_vec with a caller workspace.
CAPTURE_CHILD = r"""
import sys
import numpy as np
import torch
from gophonic_amd import gphq

fmt, lanes, k, n = gphq.FMT_Q8B, 4, 4096, 1024
rng = np.random.default_rng(11)
codes = torch.from_numpy(rng.integers(-127, 128, n * k).astype(np.int8)).cuda()
scales = torch.from_numpy((np.abs(rng.standard_normal(n * k // 32)) * 0.01).astype(np.float16)).cuda()
x = torch.zeros(lanes * k, device="cuda")
y = torch.full((lanes * n,), -7.0, device="cuda")
work = torch.empty(gphq.gemv_vec_workspace_bytes(lanes, k), dtype=torch.uint8, device="cuda")
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    gphq.gemv_vec_noalloc(fmt, codes, scales, x, y, lanes, k, n)
for rep in range(3):
    x.copy_(torch.from_numpy(rng.standard_normal(lanes * k).astype(np.float32)).cuda())
    y.fill_(-7.0)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    want = torch.full((lanes * n,), -9.0, device="cuda")
    gphq.gemv_vec(fmt, codes, scales, x, want, lanes, k, n, work)
    torch.cuda.synchronize()
    same = np.array_equal(y.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32))
    print(f"replay {rep}: {'equal' if same else 'DIFFERENT'}", flush=True)
    if not same:
        sys.exit(1)
print("capture ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    res = subprocess.run([sys.executable, "-c", CAPTURE_CHILD], cwd=root, env=env, capture_output=True, text=True,
                         timeout=240)
    assert res.returncode == 0 and "capture ok" in res.stdout, res.stdout + res.stderr
