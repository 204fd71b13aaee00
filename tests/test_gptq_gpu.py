"""GPU parity of the GPTQ producer (gphq_gptq_factor / gphq_gptq_round),
through the C ABI, against the float64 oracle (oracle/gptq_oracle.py, pinned
by tests/test_gptq_oracle.py).

The device works in fp32 as the reference does (fp32 products and storage,
float64 inside the small substitutions), so it is held to fp32-level bounds:
U within 1e-3 of the float64 factor relative to its largest entry and
H U^T U = I to 1e-3 on calibration rows with a strong common component (an
ill-conditioned H), and to the reference's own 1e-4 on its well-conditioned
H = X^T X / rows + I at k = 1, 7, 128 and 300 (gptq_linalg_test.go:14-67);
rounding against the same U picks the
oracle's codes except where a value sits within fp32 rounding of a code
boundary (>= 99% equal, never more than one step apart), and keeps the
reference's property that GPTQ beats round-to-nearest
(gptq_linalg_test.go:72-148).
"""
import numpy as np
import pytest

from gophonic_amd import gphq
from oracle import gptq_oracle as go
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def calib(rows, k, seed, dead=()):
    rng = np.random.default_rng(seed)
    base = rng.standard_normal((rows, 1))
    x = (base + 0.5 * rng.standard_normal((rows, k))).astype(np.float32)
    for d in dead:
        x[:, d] = 0
    return x


def factor(x):
    import torch

    rows, k = x.shape
    u = torch.empty((k, k), device="cuda")
    dead = torch.empty(k, dtype=torch.uint8, device="cuda")
    print(f"gptq factor rows={rows} k={k}", flush=True)
    gphq.gptq_factor(dev(x), rows, k, u, dead)
    return u.cpu().numpy(), dead.cpu().numpy().astype(bool)


@pytest.mark.parametrize("rows,k", [(40, 7), (200, 128), (300, 300), (1100, 1024)])
def test_factor_matches_float64(rows, k):
    x = calib(rows, k, k, dead=(3,))
    u, dead = factor(x)
    h, want_dead = go.damp(go.hessian(x))
    assert np.array_equal(dead, want_dead)
    want = go.inverse_factor(h)
    assert np.array_equal(u, np.triu(u))
    assert np.abs(u - want).max() <= 1e-3 * np.abs(want).max()
    u64 = u.astype(np.float64)
    assert np.abs(h @ (u64.T @ u64) - np.eye(k)).max() <= 1e-3


@pytest.mark.parametrize("k", [1, 7, 128, 300])
def test_factor_meets_the_reference_bound(k):
    # The reference's own check (gptq_linalg_test.go:14-67): H = X^T X / rows
    # + I for X ~ N(0, 1) with rows = k + 17, max |H (U^T U) - I| <= 1e-4 in
    # float64 sums over the fp32 U. The device takes calibration rows, not H,
    # so the rows are X / sqrt(rows) stacked on the identity (whose Gram
    # matrix is X^T X / rows + I); the device then damps H by 0.01 of its mean
    # diagonal, which keeps the reference's conditioning (every eigenvalue at
    # least 1). H below is that damped Hessian in float64.
    rows = k + 17
    rng = np.random.default_rng(3 * k + 1)
    x = rng.standard_normal((rows, k))
    xs = np.vstack([x / np.sqrt(rows), np.eye(k)]).astype(np.float32)
    u, dead = factor(xs)
    assert not dead.any()
    assert np.array_equal(u, np.triu(u))
    h, _ = go.damp(go.hessian(xs))
    u64 = u.astype(np.float64)
    worst = np.abs(h @ (u64.T @ u64) - np.eye(k)).max()
    assert worst <= 1e-4, worst


def test_factor_rejects_non_finite_hessian():
    import torch

    x = calib(32, 16, 2)
    x[5, 7] = np.nan
    u = torch.empty((16, 16), device="cuda")
    dead = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(gphq.GphqError) as e:
        gphq.gptq_factor(dev(x), 32, 16, u, dead)
    assert e.value.status == gphq.ERR_NOT_POSITIVE_DEFINITE


def round_dev(w, u, dead, bits):
    import torch

    n, k = w.shape
    wd = dev(w)
    codes = torch.zeros(n * k if bits == 8 else n * k // 2, dtype=torch.uint8, device="cuda")
    scales = torch.zeros(n * 4 if bits == 8 else n * (k // 32) * 2, dtype=torch.uint8, device="cuda")
    print(f"gptq round n={n} k={k} bits={bits}", flush=True)
    gphq.gptq_round(wd, n, k, dev(u), dev(dead.astype(np.uint8)), bits, codes, scales)
    return wd.cpu().numpy(), codes.cpu().numpy(), scales.cpu().numpy()


def q_of(codes, bits, n, k):
    if bits == 8:
        return codes.view(np.int8).reshape(n, k).astype(np.int64)
    nib = codes.reshape(n, k // 32, 16)
    return (np.concatenate([nib & 15, nib >> 4], axis=2).astype(np.int64) - 8).reshape(n, k)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("n,k", [(16, 256), (37, 320), (64, 1024)])
def test_round_matches_float64(bits, n, k):
    rng = np.random.default_rng(n + k + bits)
    x = calib(4 * k, k, k + 1, dead=(5,))
    u, dead = factor(x)
    w = rng.standard_normal((n, k)).astype(np.float32)
    got_w, codes, scales = round_dev(w, u, dead, bits)
    w0 = w.copy()
    w0[:, dead] = 0
    want_codes, want_scales, want_w = go.round_rows(w0, u.astype(np.float64), bits)
    q, wq = q_of(codes, bits, n, k), q_of(want_codes.view(np.uint8), bits, n, k)
    same = (q == wq).mean()
    assert same >= 0.99, same
    assert np.abs(q - wq).max() <= 1
    if bits == 8:
        assert np.array_equal(scales.view(np.float32), want_scales)
    else:
        assert (scales.view(np.uint16).reshape(n, k // 32) == want_scales).mean() >= 0.99
    assert np.isfinite(got_w).all()
    # The rounded values are the codes times their scales.
    if bits == 8:
        s = scales.view(np.float32)[:, None].astype(np.float64)
    else:
        s = np.repeat(scales.view(np.float16).reshape(n, k // 32).astype(np.float64), 32, axis=1)
    assert np.array_equal(got_w.astype(np.float64), (q * s).astype(np.float32).astype(np.float64))
    # GPTQ beats round-to-nearest with the same inputs (gptq_linalg_test.go:72-148).
    near = np.zeros_like(w0, dtype=np.float64)
    for o in range(n):
        if bits == 8:
            sc = np.float32(np.abs(w0[o]).max() / np.float32(127))
            near[o] = np.rint(w0[o] / sc) * np.float64(sc)
        else:
            for b in range(0, k, 32):
                d = np.float32(orc.q4_group_scale(w0[o, b:b + 32]))
                near[o, b:b + 32] = np.clip(np.rint(w0[o, b:b + 32] / d), -8, 7) * np.float64(d)
    x64 = x.astype(np.float64)
    err = lambda qv: float(((x64 @ (w0.astype(np.float64) - qv).T) ** 2).sum())
    assert err(got_w.astype(np.float64)) < err(near)


@pytest.mark.parametrize("bits", [8, 4])
def test_full_size_group_properties(bits):
    """Qwen3-8B's hidden size with the reference's 4096 calibration rows
    (gptqMaxRows, gptq.go:39): H U^T U = I and the rounding's properties,
    checked in float64 on the device."""
    import torch

    k, rows, n = 4096, 4096, 512
    g = torch.Generator(device="cuda").manual_seed(bits)
    x = (torch.randn(rows, 1, device="cuda", generator=g)
         + 0.5 * torch.randn(rows, k, device="cuda", generator=g)).contiguous()
    x[:, 9] = 0
    u = torch.empty((k, k), device="cuda")
    dead = torch.empty(k, dtype=torch.uint8, device="cuda")
    print(f"gptq factor rows={rows} k={k}", flush=True)
    gphq.gptq_factor(x, rows, k, u, dead)
    assert dead.nonzero().flatten().tolist() == [9]
    h = x.double().T @ x.double()
    diag = h.diagonal()
    mean = diag.mean()
    diag[9] = 1
    diag += 0.01 * mean
    ud = u.double()
    eye = torch.eye(k, device="cuda", dtype=torch.float64)
    assert torch.equal(u, u.triu())
    assert (h @ (ud.T @ ud) - eye).abs().max().item() <= 1e-3
    w = torch.randn(n, k, device="cuda", generator=g)
    w0 = w.clone()
    w0[:, 9] = 0
    codes = torch.empty(n * k if bits == 8 else n * k // 2, dtype=torch.uint8, device="cuda")
    scales = torch.empty(n * 4 if bits == 8 else n * (k // 32) * 2, dtype=torch.uint8, device="cuda")
    print(f"gptq round n={n} k={k} bits={bits}", flush=True)
    gphq.gptq_round(w, n, k, u, dead, bits, codes, scales)
    if bits == 8:
        q = codes.view(torch.int8).reshape(n, k).double()
        s = scales.view(torch.float32)[:, None].double()
        near = torch.round(w0 / (w0.abs().amax(1, keepdim=True) / 127)) * (w0.abs().amax(1, keepdim=True) / 127)
    else:
        nib = codes.reshape(n, k // 32, 16).long()
        q = (torch.cat([nib & 15, nib >> 4], dim=2) - 8).reshape(n, k).double()
        s = scales.view(torch.float16).reshape(n, k // 32).double().repeat_interleave(32, dim=1)
        near = None
    assert torch.equal(w.double(), (q * s).float().double())
    assert torch.all(q[:, 9] == 0)
    err = lambda qv: ((x.double() @ (w0.double() - qv).T) ** 2).sum().item()
    if near is None:  # 4-bit round-to-nearest with the GPU's own group scales
        near = torch.clamp(torch.round(w0.double() / s), -8, 7) * s
    assert err(w.double()) < 0.9 * err(near.double())
