"""Parity at the full BASELINE sizes (configs C2, C3 and C5's optimizer) through the C-ABI.

The kernels run on the whole input and the NumPy oracle checks every element of every
output in float64, over chunks of rows (row-independent outputs chunk by chunk; the
outputs that depend on every row, LayerNorm dgamma/dbeta and BatchNorm dgamma/dbeta,
from float64 sums over the chunks).  Tolerance rtol 1e-5 (fp32), with the
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


def rows(t, r0, r1):
    return t[r0:r1].double().cpu().numpy()


CHUNK = 1024  # rows per float64 comparison chunk (64 MiB of float64 at 8192 columns)


@pytest.mark.parametrize("kind", ["gelu", "silu"])
def test_c2_activation_bwd_full(cuda, kind):
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(8192, 8192, device="cuda", generator=g)
    dy = torch.randn(8192, 8192, device="cuda", generator=g)
    dx = torch.empty_like(x)
    L().act_bwd(kind, x, dy, dx, False)
    ref_fn = O.gelu_bwd if kind == "gelu" else O.silu_bwd
    for r0 in range(0, 8192, CHUNK):
        ref = ref_fn(rows(x, r0, r0 + CHUNK), rows(dy, r0, r0 + CHUNK))
        assert_close(rows(dx, r0, r0 + CHUNK), ref, RTOL_F32, f"{kind} dx rows {r0}..")


def test_c2_softmax_bwd_full(cuda):
    g = torch.Generator(device="cuda").manual_seed(12)
    logits = torch.randn(16384, 4096, device="cuda", generator=g) * 2
    y = L().softmax_fwd(logits)
    dy = torch.randn(16384, 4096, device="cuda", generator=g)
    dx = torch.empty_like(y)
    L().softmax_bwd(y, dy, dx, False)
    for r0 in range(0, 16384, 2 * CHUNK):
        r1 = r0 + 2 * CHUNK
        yr = rows(y, r0, r1)
        assert_close(yr, O.softmax_fwd(rows(logits, r0, r1)), RTOL_F32, f"softmax y {r0}..")
        assert_close(rows(dx, r0, r1), O.softmax_bwd(yr, rows(dy, r0, r1)), RTOL_F32,
                     f"softmax dx rows {r0}..")


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
    # every row's dx, and dgamma, dbeta as float64 sums over the row chunks
    dgr = np.zeros(C)
    dbr = np.zeros(C)
    for r0 in range(0, R, 2 * CHUNK):
        r1 = r0 + 2 * CHUNK
        _, xh, _, var = O.layernorm_fwd(rows(x, r0, r1), g64, 0.0)
        dxr, a, b = O.layernorm_bwd(xh, var, g64, rows(dy, r0, r1))
        assert_close(rows(dx, r0, r1), dxr, RTOL_F32, f"layernorm dx rows {r0}..")
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
    element is independent; every element of every tensor is checked against the
    oracle in float64."""
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
    f64 = lambda t: t.double().cpu().numpy()  # noqa: E731
    for i, n in enumerate(sizes):
        p, m, v = f64(p0[i]), np.zeros(n), np.zeros(n)
        for t in (1, 2):
            p, m, v, _ = O.adam_step(p, f64(grads[t - 1][i]), m, v, t, lr=3e-4,
                                     weight_decay=0.1)
        assert_close(ps[i], p, RTOL_F32, f"adamw p[{i}]")
        assert_close(ms[i], m, RTOL_F32, f"adamw m[{i}]")
        assert_close(vs[i], v, RTOL_F32, f"adamw v[{i}]")


def test_c5_unscale_full_bit_exact(cuda):
    """GradScaler unscale over 83.2M fp32 gradients: per-tensor non-finite flags are
    exact (an inf in the last element of the last tensor, a NaN in the middle of
    another; bits 0 and 1: non-finite before and after scaling), and unscaled values
    equal the fp32 product bit for bit on every finite element."""
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
    for i in range(48):
        b = before[i].cpu().numpy()
        a = gs[i].cpu().numpy()
        fin = np.isfinite(b)
        assert np.array_equal(a[fin], b[fin] * inv), f"unscale tensor {i}"


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
