"""Fused cross-entropy kernels (tg_cross_entropy_fwd/bwd) vs the oracle restatement
of CrossEntropyLoss (_nn.py:1128-1185).  GPU only.

Tolerance: per-row losses and gradients rtol 1e-5 for fp32 logits; for fp16/bf16
logits the reference is evaluated on the same rounded logits, and the gradient is
compared after rounding to the logits dtype (rtol 1e-2 / 3e-2)."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, RTOL_F32, assert_close

pytestmark = pytest.mark.gpu
RT = {torch.float32: RTOL_F32, torch.float16: RTOL_F16, torch.bfloat16: 3e-2}


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def f64(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("N,C", [(32, 10), (7, 4097), (64, 32000), (3, 1)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("smooth", [0.0, 0.1])
def test_ce_kernels_vs_oracle(cuda, N, C, dt, smooth):
    g = torch.Generator(device="cuda").manual_seed(N * 7 + C)
    x = (torch.randn(N, C, device="cuda", generator=g) * 3).to(dt)
    y = torch.randint(0, C, (N,), device="cuda", generator=g)
    lse, loss = L().cross_entropy_fwd(x, y, smooth)
    rows, probs = O.cross_entropy_fwd(f64(x), f64(y).astype(np.int64), smooth, "none")
    if C == 1:  # p = 1: the loss is -log(1 + 1e-10) ~ -1e-10, 0 in fp32
        assert np.abs(f64(loss)).max() <= 1e-6  # a few fp32 ulps of log(1)
    else:
        assert_close(loss, rows, RTOL_F32 if dt == torch.float32 else 1e-4, "loss rows")
    lse_ref = np.log(np.exp(f64(x) - f64(x).max(1, keepdims=True)).sum(1)) + f64(x).max(1)
    assert_close(lse, lse_ref, RTOL_F32, "lse")
    want = O.cross_entropy_bwd(probs, f64(y).astype(np.int64), smooth, "mean")
    grad = torch.empty_like(x)
    L().cross_entropy_bwd(x, y, lse, grad, 1.0 / N, False, smooth)
    want_t = torch.tensor(want).to(dt).double().numpy()  # as stored in the logits dtype
    acc = torch.ones(N, C, device="cuda")
    L().cross_entropy_bwd(x, y, lse, acc, 1.0 / N, True, smooth)  # fp32, accumulating
    if C == 1:  # exact gradient 0; exp rounding leaves |p - 1| ~ 1e-7
        assert np.abs(f64(grad)).max() <= 1e-6 and np.abs(f64(acc) - 1.0).max() <= 1e-6
        return
    assert_close(grad, want_t, RT[dt], "grad")
    assert_close(acc, want + 1.0, RTOL_F32, "grad accumulate")


def test_ce_module_matches_oracle_and_ignores_upstream(cuda):
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(3)
    x_np = rng.standard_normal((16, 50)).astype(np.float32) * 2
    y = rng.integers(0, 50, 16)
    for red in ("mean", "sum", "none"):
        x = tg.Tensor(x_np, requires_grad=True)
        loss = tg.CrossEntropyLoss(reduction=red, label_smoothing=0.05)(x, y)
        lo, probs = O.cross_entropy_fwd(x_np.astype(np.float64), y, 0.05, red)
        assert_close(loss.data, np.asarray(lo), RTOL_F32, f"loss {red}")
        (loss * 3.0).sum().backward() if red == "none" else (loss * 3.0).backward()
        # the reference backward never reads the upstream gradient (x3 is ignored)
        assert_close(x.grad, O.cross_entropy_bwd(probs, y, 0.05, red), RTOL_F32, f"grad {red}")


def test_ce_noncontiguous_grad_target_falls_back(cuda):
    """A gradient buffer that is not a contiguous [N, C] tensor takes the
    temporary-buffer path; the result must match the fused path."""
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(4)
    x_np = rng.standard_normal((8, 12)).astype(np.float32)
    y = rng.integers(0, 12, 8)
    a = tg.Tensor(x_np, requires_grad=True)
    tg.CrossEntropyLoss()(a, y).backward()
    b = tg.Tensor(x_np, requires_grad=True)
    b.grad = np.zeros((12, 8), np.float32).T  # transposed view: non-contiguous
    tg.CrossEntropyLoss()(b, y).backward()
    assert_close(b.grad, f64(a.grad), RTOL_F32, "fallback path")


def test_ce_target_range(cuda):
    import tensor_gpu_v2 as tg
    x = tg.Tensor(np.zeros((2, 3), np.float32), requires_grad=True)
    with pytest.raises(IndexError):
        tg.CrossEntropyLoss()(x, np.array([0, 3]))
    # device targets are not checked on the host: the kernel reports NaN for the row
    lse, loss = L().cross_entropy_fwd(x.data, torch.tensor([0, 5], device="cuda"))
    out = loss.cpu().numpy()
    assert np.isfinite(out[0]) and np.isnan(out[1])


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.float64])
def test_ce_negative_targets_wrap(cuda, tg, dt):
    """Targets in [-C, 0) count from the end (NumPy indexing, as in the reference) in
    every kernel: host and device targets give the wrapped targets' loss and gradient
    bit for bit, through the one-pass, the two-pass and the fp64 paths."""
    rng = np.random.default_rng(5)
    N, C = 16, 40
    xv = rng.standard_normal((N, C)) * 2
    yw = rng.integers(0, C, N)
    yn = np.where(np.arange(N) % 2 == 0, yw - C, yw)  # half of them negative
    npdt = {torch.float32: np.float32, torch.float16: np.float16, torch.float64: np.float64}[dt]
    out = {}
    for name, y in (("wrapped", yw), ("host", yn), ("device", torch.as_tensor(yn).cuda())):
        for gif in (True, False):
            x = tg.Tensor(xv.astype(npdt), requires_grad=True)
            loss = tg.CrossEntropyLoss(grad_in_forward=gif)(x, y)
            loss.backward()
            out[(name, gif)] = (loss.data.double().cpu(), x.grad.double().cpu())
    for k, (l, g) in out.items():
        assert torch.equal(l, out[("wrapped", k[1])][0]), k
        assert torch.equal(g, out[("wrapped", k[1])][1]), k
    # below -C: NaN on the device path
    lse, loss = L().cross_entropy_fwd(torch.zeros(2, 3, device="cuda"),
                                      torch.tensor([-3, -4], device="cuda"))
    o = loss.cpu().numpy()
    assert np.isfinite(o[0]) and np.isnan(o[1])


@pytest.mark.parametrize("N,C", [(32, 16), (7, 4096), (64, 32000), (5, 32768), (9, 8)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_ce_fwd_grad_equals_fwd_then_bwd(cuda, N, C, dt):
    """tg_cross_entropy_fwd_grad (one read of the logits) against tg_cross_entropy_fwd
    followed by tg_cross_entropy_bwd: bit-identical lse, loss and gradient, also for an
    out-of-range target (NaN loss, no target term); the oracle pins the pair."""
    if not L().cross_entropy_fwd_grad_ok(torch.empty(1, C, dtype=dt, device="cuda")):
        assert dt == torch.float32 and C > 16384
        return
    g = torch.Generator(device="cuda").manual_seed(N + C)
    x = (torch.randn(N, C, device="cuda", generator=g) * 3).to(dt)
    y = torch.randint(0, C, (N,), device="cuda", generator=g)
    y[N // 2] = C  # outside [0, C)
    lse, loss = L().cross_entropy_fwd(x, y)
    ref = torch.empty_like(x)
    L().cross_entropy_bwd(x, y, lse, ref, 1.0 / N, False)
    lse2, loss2, grad = L().cross_entropy_fwd_grad(x, y, 1.0 / N)
    assert torch.equal(lse2, lse)
    assert torch.equal(torch.nan_to_num(loss2, nan=-7.0), torch.nan_to_num(loss, nan=-7.0))
    assert torch.isnan(loss2[N // 2])
    assert torch.equal(grad, ref)


def test_ce_module_gradient_formed_in_forward(cuda):
    """CrossEntropyLoss with a backward to follow takes the one-pass kernel: the logits'
    gradient (adopted from the forward, then accumulated on a second backward) equals
    the two-pass path's (under no_grad-free eval it is not formed at all)."""
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(3)
    x_np = (rng.standard_normal((64, 4096)) * 2).astype(np.float32)
    y_np = rng.integers(0, 4096, 64)
    grads = []
    for smoothing in (0.0, 1e-12):  # any smoothing takes the two-pass path
        x = tg.Tensor(x_np)
        ce = tg.CrossEntropyLoss(label_smoothing=smoothing)
        for _ in range(2):
            ce(x, y_np).backward()
        grads.append(x.grad.clone())
    assert_close(grads[0], f64(grads[1]), 1e-6, "one-pass vs two-pass CE gradient")
    x = tg.Tensor(x_np)
    with tg.no_grad():
        loss = tg.CrossEntropyLoss()(x, y_np)
    assert loss.data.numel() == 1


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_ce_grad_in_forward_switch(cuda, tg, dt):
    """CrossEntropyLoss(grad_in_forward=False) forms the gradient only inside
    backward (the reference's order) and gives the same loss and gradient bit for bit
    as the default one-pass mode."""
    rng = np.random.default_rng(3)
    x_np = (3 * rng.standard_normal((64, 3000))).astype(np.float32)
    y_np = rng.integers(0, 3000, 64)
    out = []
    for gf in (True, False):
        x = tg.Tensor(torch.as_tensor(x_np).to(dt).cuda())
        loss = tg.CrossEntropyLoss(grad_in_forward=gf)(x, y_np)
        loss.backward()
        out.append((loss.data.float().cpu(), x.grad.float().cpu()))
    assert torch.equal(out[0][0], out[1][0])
    assert torch.equal(out[0][1], out[1][1])
