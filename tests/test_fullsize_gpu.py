"""Parity at the full BASELINE sizes (configs C2, C3 and C5's optimizer) through the C-ABI.

The kernels run on the whole input; the NumPy oracle checks them where it finishes in
seconds: row-independent outputs (GELU/SiLU/softmax/LayerNorm dx) on a random sample
of rows, and the outputs that depend on every row (LayerNorm dgamma/dbeta,
BatchNorm dx/dgamma/dbeta) in full, in float64.  Tolerance rtol 1e-5 (fp32), with the
rms-scaled absolute term of conftest.assert_close.  GPU only."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F32, assert_close

pytestmark = pytest.mark.gpu


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def rows_of(t, idx):
    return t[torch.as_tensor(idx, device=t.device)].double().cpu().numpy()


def sample(n, k, seed):
    return np.sort(np.random.default_rng(seed).choice(n, size=k, replace=False))


@pytest.mark.parametrize("kind", ["gelu", "silu"])
def test_c2_activation_bwd_full(cuda, kind):
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(8192, 8192, device="cuda", generator=g)
    dy = torch.randn(8192, 8192, device="cuda", generator=g)
    dx = torch.empty_like(x)
    L().act_bwd(kind, x, dy, dx, False)
    idx = sample(8192, 48, 1)
    ref = (O.gelu_bwd if kind == "gelu" else O.silu_bwd)(rows_of(x, idx), rows_of(dy, idx))
    assert_close(rows_of(dx, idx), ref, RTOL_F32, f"{kind} dx rows")
    # the last rows hold the grid's final blocks
    ref = (O.gelu_bwd if kind == "gelu" else O.silu_bwd)(rows_of(x, [8191]), rows_of(dy, [8191]))
    assert_close(rows_of(dx, [8191]), ref, RTOL_F32, f"{kind} dx last row")


def test_c2_softmax_bwd_full(cuda):
    g = torch.Generator(device="cuda").manual_seed(12)
    logits = torch.randn(16384, 4096, device="cuda", generator=g) * 2
    y = L().softmax_fwd(logits)
    dy = torch.randn(16384, 4096, device="cuda", generator=g)
    dx = torch.empty_like(y)
    L().softmax_bwd(y, dy, dx, False)
    idx = np.concatenate([sample(16383, 40, 2), [16383]])
    assert_close(rows_of(y, idx), O.softmax_fwd(rows_of(logits, idx)), RTOL_F32, "softmax y")
    assert_close(rows_of(dx, idx), O.softmax_bwd(rows_of(y, idx), rows_of(dy, idx)), RTOL_F32,
                 "softmax dx rows")


def test_c2_layernorm_bwd_full(cuda):
    R, C = 16384, 4096
    g = torch.Generator(device="cuda").manual_seed(13)
    x = torch.randn(R, C, device="cuda", generator=g)
    gam = 1 + 0.02 * torch.randn(C, device="cuda", generator=g)
    bet = 0.02 * torch.randn(C, device="cuda", generator=g)
    dy = torch.randn(R, C, device="cuda", generator=g)
    _, mean, rstd = L().layernorm_fwd(x, gam, bet, 1e-5)
    dx = torch.empty_like(x)
    dg, db = torch.empty_like(gam), torch.empty_like(bet)
    L().layernorm_bwd(x, mean, rstd, gam, dy, dx, dg, db, False, False)
    g64 = gam.double().cpu().numpy()
    idx = np.concatenate([sample(R - 1, 40, 3), [R - 1]])
    _, xh, _, var = O.layernorm_fwd(rows_of(x, idx), g64, bet.double().cpu().numpy())
    dxr, _, _ = O.layernorm_bwd(xh, var, g64, rows_of(dy, idx))
    assert_close(rows_of(dx, idx), dxr, RTOL_F32, "layernorm dx rows")
    # dgamma, dbeta need every row: float64 sums over row chunks
    dgr = np.zeros(C)
    dbr = np.zeros(C)
    for r0 in range(0, R, 2048):
        xs = x[r0:r0 + 2048].double().cpu().numpy()
        ds = dy[r0:r0 + 2048].double().cpu().numpy()
        _, xh, _, var = O.layernorm_fwd(xs, g64, 0.0)
        _, a, b = O.layernorm_bwd(xh, var, g64, ds)
        dgr += a
        dbr += b
    assert_close(dg, dgr, RTOL_F32, "layernorm dgamma")
    assert_close(db, dbr, RTOL_F32, "layernorm dbeta")


def test_c3_bn_relu_bwd_nhwc_full(cuda):
    N, H, W, C = 64, 56, 56, 256
    g = torch.Generator(device="cuda").manual_seed(14)
    x = torch.randn(N, H, W, C, device="cuda", generator=g)
    gam = 1 + 0.1 * torch.randn(C, device="cuda", generator=g)
    bet = 0.1 * torch.randn(C, device="cuda", generator=g)
    dy = torch.randn(N, H, W, C, device="cuda", generator=g)
    rm, rv = torch.zeros(C, device="cuda"), torch.ones(C, device="cuda")
    _, mean, rstd, _ = L().batchnorm_fwd_train(x, gam, bet, 1e-5, 0.1, rm, rv, True, L().NHWC)
    dx = torch.empty_like(x)
    dg, db = torch.empty_like(gam), torch.empty_like(bet)
    L().batchnorm_bwd(x, mean, rstd, gam, bet, dy, dx, dg, db, True, False, False, L().NHWC)
    # The statistics and the ReLU mask are first checked against the oracle's float64
    # forward: mean and rstd per channel at the fp32 bar, and the mask wherever the
    # float64 pre-activation is farther from 0 than fp32 rounding of its terms reaches.
    x32 = x.cpu().numpy()
    g32, b32 = gam.cpu().numpy(), bet.cpu().numpy()
    x64 = x32.astype(np.float64)
    _, cache = O.batchnorm_relu_fwd_nhwc(x64, g32.astype(np.float64), b32.astype(np.float64),
                                         1e-5, relu=False)
    assert_close(mean, cache[5], RTOL_F32, "bn mean")
    assert_close(rstd, 1.0 / np.sqrt(cache[6] + 1e-5), RTOL_F32, "bn rstd")
    pre = cache[4].transpose(0, 2, 3, 1)  # float64 gamma*xhat + beta, NHWC
    band = 1e-5 * (np.abs(g32) * np.abs(cache[0].transpose(0, 2, 3, 1)) + np.abs(b32))
    # the mask as the kernel forms it: fp32, ((x - mean) * rstd) * gamma + beta > 0 in
    # that order without contraction (NumPy does not fuse), from its own statistics
    m32, r32 = mean.cpu().numpy(), rstd.cpu().numpy()
    on = (g32 * ((x32 - m32) * r32) + b32) > 0
    del x32
    differ = on != (pre > 0)
    assert not (differ & (np.abs(pre) > band)).any(), "ReLU mask differs from the oracle's"
    assert int(differ.sum()) <= 1000, int(differ.sum())
    del pre, band, differ
    # the oracle's backward then runs without ReLU on the gradient masked as the kernel
    # masked it (the few elements inside the rounding band would otherwise move dgamma
    # and dbeta by one element's contribution)
    dym = dy.cpu().numpy().astype(np.float64) * on
    del on
    dxr, dgr, dbr = O.batchnorm_relu_bwd_nhwc(dym, g32.astype(np.float64), cache, relu=False)
    assert_close(dg, dgr, RTOL_F32, "bn dgamma")
    assert_close(db, dbr, RTOL_F32, "bn dbeta")
    assert_close(dx, dxr, RTOL_F32, "bn dx")


NPARAM = 83_200_000  # C5's parameter count, as 48 tensors


def _c5_sizes():
    return [NPARAM // 48] * 47 + [NPARAM - 47 * (NPARAM // 48)]


def test_c5_adamw_full(cuda):
    """AdamW (lr 3e-4, wd 0.1) over 83.2M parameters in 48 tensors, two steps; every
    element is independent, so sampled elements of every tensor (and each tensor's
    last element) are checked against the oracle."""
    sizes = _c5_sizes()
    g = torch.Generator(device="cuda").manual_seed(15)
    ps = [torch.randn(n, device="cuda", generator=g) for n in sizes]
    p0 = [p.clone() for p in ps]
    ms = [torch.zeros(n, device="cuda") for n in sizes]
    vs = [torch.zeros(n, device="cuda") for n in sizes]
    grads = [[torch.randn(n, device="cuda", generator=g) * 1e-3 for n in sizes] for _ in range(2)]
    for t in (1, 2):
        L().adam_step(ps, grads[t - 1], ms, vs, None, 3e-4, 0.9, 0.999, 1e-8, 0.1,
                      1 - 0.9 ** t, 1 - 0.999 ** t)
    for i, n in enumerate(sizes):
        idx = np.append(sample(n - 1, 64, 100 + i), n - 1)
        p, m, v = rows_of(p0[i], idx), np.zeros(len(idx)), np.zeros(len(idx))
        for t in (1, 2):
            p, m, v, _ = O.adam_step(p, rows_of(grads[t - 1][i], idx), m, v, t, lr=3e-4,
                                     weight_decay=0.1)
        assert_close(rows_of(ps[i], idx), p, RTOL_F32, f"adamw p[{i}]")
        assert_close(rows_of(ms[i], idx), m, RTOL_F32, f"adamw m[{i}]")
        assert_close(rows_of(vs[i], idx), v, RTOL_F32, f"adamw v[{i}]")


def test_c5_unscale_full_bit_exact(cuda):
    """GradScaler unscale over 83.2M fp32 gradients: per-tensor non-finite flags are
    exact (an inf in the last element of the last tensor, a NaN in the middle of
    another; bits 0 and 1: non-finite before and after scaling), and unscaled values
    equal the fp32 product bit for bit on sampled elements."""
    sizes = _c5_sizes()
    g = torch.Generator(device="cuda").manual_seed(16)
    gs = [torch.randn(n, device="cuda", generator=g) * 1e3 for n in sizes]
    gs[47][-1] = float("inf")
    gs[3][sizes[3] // 2] = float("nan")
    before = [x.clone() for x in gs]
    inv = np.float32(1.0 / 65536.0)
    flags = L().unscale_check(gs, float(inv))
    want = [0] * 48
    want[47] = 3
    want[3] = 3
    assert flags == want
    for i, n in enumerate(sizes):
        idx = np.append(sample(n - 1, 64, 200 + i), n - 1)
        b = before[i][torch.as_tensor(idx, device="cuda")].cpu().numpy()
        a = gs[i][torch.as_tensor(idx, device="cuda")].cpu().numpy()
        fin = np.isfinite(b)
        assert np.array_equal(a[fin], (b[fin] * inv).astype(np.float32)), f"unscale tensor {i}"


def test_c5_cross_entropy_full(cuda):
    """Fused cross-entropy over C5's fp16 logits [8192, 32000]: rows are independent, so
    sampled rows (and the last) of the loss, LSE and gradient are checked against the
    oracle on the same fp16 logits (loss/LSE rtol 1e-5 relative to fp32 arithmetic
    over fp16 inputs: 1e-4; gradient compared after rounding to fp16, rtol 1e-2)."""
    N, C = 8192, 32000
    g = torch.Generator(device="cuda").manual_seed(17)
    x = (torch.randn(N, C, device="cuda", generator=g) * 3).half()
    y = torch.randint(0, C, (N,), device="cuda", generator=g)
    lse, loss = L().cross_entropy_fwd(x, y)
    grad = torch.empty_like(x)
    L().cross_entropy_bwd(x, y, lse, grad, 1.0 / N, False)
    idx = np.append(sample(N - 1, 24, 4), N - 1)
    xs = rows_of(x, idx)
    ys = y[torch.as_tensor(idx, device="cuda")].cpu().numpy().astype(np.int64)
    rows, probs = O.cross_entropy_fwd(xs, ys, 0.0, "none")
    assert_close(loss[torch.as_tensor(idx, device="cuda")], rows, 1e-4, "ce loss rows")
    want = O.cross_entropy_bwd(probs, ys, 0.0, "sum") / N
    assert_close(rows_of(grad, idx), torch.tensor(want).half().double().numpy(), 1e-2,
                 "ce grad rows")
