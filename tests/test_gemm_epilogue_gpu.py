"""Fused GEMM epilogues (tg_gemm_epilogue) against the separate kernels they replace,
bit for bit, and the Linear / GELU / residual compositions that use them.  GPU only.

GELU backward: (G @ W^T) rounded to the dtype, times gelu'(h), (+ C), equals
tg_gemm into a 16-bit buffer followed by tg_gelu_bwd.  GELU forward: the GEMM+bias
output and gelu of it equal tg_gemm_bias followed by tg_gelu_fwd.  Residual: the
GEMM+bias output plus r equals tg_gemm_bias followed by a 16-bit add.  The closures'
results are then compared between the fused and the separate compositions (module
gradients bit-identical), and the GELU-backward fusion is checked against the float64
oracle of the pair (rtol 1e-2 under fp16)."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, assert_close

pytestmark = pytest.mark.gpu


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def rnd(shape, dt, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, device="cuda", generator=g) * scale).to(dt)


SHAPES = [(512, 1024, 256), (1000, 520, 128), (4096, 4096, 1024)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_gelu_bwd_epilogue_bit_exact(cuda, M, N, K, dt, beta):
    G = rnd((M, K), dt, 1)
    W = rnd((N, K), dt, 2, 0.05)   # a Linear weight [N_in, K_out]: dA = G @ W^T
    h = rnd((M, N), dt, 3, 2.0)
    c0 = rnd((M, N), dt, 4)
    fused = c0.clone()
    assert L().gemm_epilogue("gelu_bwd", G, W, h, fused, beta=beta)
    da = L().matmul2d(G, W, trans_b=True)  # fp16 output, as the separate path stores it
    assert da.dtype == dt
    ref = c0.clone()
    L().act_bwd("gelu", h, da, ref, beta != 0.0)
    assert torch.equal(fused, ref)


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bias", [True, False])
def test_gelu_fwd_and_residual_epilogues_bit_exact(cuda, M, N, K, dt, bias):
    A = rnd((M, K), dt, 5)
    W = rnd((K, N), dt, 6, 0.05)
    b = rnd((N,), torch.float32, 7) if bias else None
    h, act = torch.empty(M, N, dtype=dt, device="cuda"), torch.empty(M, N, dtype=dt, device="cuda")
    assert L().gemm_epilogue("gelu_fwd", A, W, act, h, b)
    if bias:
        ref_h = torch.empty_like(h)
        L().gemm_bias(A, W, b, ref_h)
    else:
        ref_h = L().matmul2d(A, W)
    assert torch.equal(h, ref_h)
    assert torch.equal(act, L().act_fwd("gelu", ref_h))
    r = rnd((M, N), dt, 8)
    out = torch.empty_like(h)
    assert L().gemm_epilogue("residual", A, W, r, out, b)
    assert torch.equal(out, r + ref_h)


def test_epilogue_unsupported_shape_falls_back(cuda):
    A = rnd((100, 96), torch.float16, 9)  # K = 96: not a multiple of the kernel's k-step
    W = rnd((96, 128), torch.float16, 10)
    x = torch.empty(100, 128, dtype=torch.float16, device="cuda")
    assert L().gemm_epilogue("residual", A, W, x, torch.empty_like(x)) is False
    assert L().gemm_epilogue("gelu_fwd", A.float(), W.float(), x.float(), x.float()) is False


def _mlp(tg, fused, seed=0):
    """x -> LN -> fc1 -> GELU -> fc2 -> + x under fp16 autocast; returns (loss, grads)."""
    rng = np.random.default_rng(seed)
    d, f = 256, 1024
    xv = rng.standard_normal((4, 128, d)).astype(np.float32)
    np.random.seed(seed)
    fc1, fc2 = tg.Linear(d, f), tg.Linear(f, d)
    for lin, s in ((fc1, 1), (fc2, 2)):
        lin.b.data = tg.Tensor(rng.standard_normal(lin.b.shape).astype(np.float32) * 0.1).data
    x = tg.Tensor(xv)
    with tg.autocast():
        xh = x * 1.0
        if fused:
            y = fc2(fc1(xh, activation="gelu"), residual=xh)
        else:
            y = xh + fc2(fc1(xh).gelu())
        loss = (y * y).mean()
    loss.backward()
    grads = [p.grad.float().cpu() for p in (fc1.w, fc1.b, fc2.w, fc2.b)] + [x.grad.float().cpu()]
    return loss.data.float().cpu(), grads, (fc1, fc2, xv)


@pytest.mark.parametrize("fuse_bwd", [True, False])
def test_fused_mlp_equals_separate_ops(cuda, tg, fuse_bwd):
    """Linear(activation="gelu") and Linear(residual=) give the same loss and the same
    parameter and input gradients, bit for bit, as the separate Linear / gelu / +
    composition; the GELU-backward fusion (config switch) does not change them."""
    from tensor_gpu_v2 import _config as cfg
    old = cfg.fuse_gelu_backward
    try:
        cfg.fuse_gelu_backward = fuse_bwd
        l1, g1, _ = _mlp(tg, True)
        cfg.fuse_gelu_backward = False
        l0, g0, _ = _mlp(tg, False)
    finally:
        cfg.fuse_gelu_backward = old
    assert torch.equal(l1, l0)
    for a, b in zip(g1, g0):
        assert torch.equal(a, b)


def test_gelu_backward_fusion_vs_oracle_and_intermediate(cuda, tg):
    """fp16 Linear -> gelu -> Linear: the first layer's weight gradient against the
    float64 oracle of the pair at the fp16 bar; with the fusion on the GELU output's
    own gradient is not formed (zeros), with it off it holds dA."""
    from tensor_gpu_v2 import _config as cfg
    rng = np.random.default_rng(3)
    xv = rng.standard_normal((256, 128)).astype(np.float16)
    w1 = (rng.standard_normal((128, 512)) * 0.1).astype(np.float16)
    w2 = (rng.standard_normal((512, 64)) * 0.1).astype(np.float16)
    dy = rng.standard_normal((256, 64)).astype(np.float16)
    out = {}
    old = cfg.fuse_gelu_backward
    try:
        for fuse in (True, False):
            cfg.fuse_gelu_backward = fuse
            l1, l2 = tg.Linear(128, 512, bias=False), tg.Linear(512, 64, bias=False)
            l1.w.data = torch.as_tensor(w1).cuda()
            l2.w.data = torch.as_tensor(w2).cuda()
            x = tg.Tensor(xv, requires_grad=False)
            g = l1(x).gelu()
            y = l2(g)
            y.backward(dy)
            out[fuse] = (l1.w.grad.float().cpu(), g.grad.float().cpu())
    finally:
        cfg.fuse_gelu_backward = old
    x64, w164, w264, dy64 = (t.astype(np.float64) for t in (xv, w1, w2, dy))
    h64 = x64 @ w164
    dgate = O.gelu_bwd(h64, dy64 @ w264.T)
    assert_close(out[True][0], x64.T @ dgate, RTOL_F16, "dW1 (fused)")
    assert torch.equal(out[True][0], out[False][0])
    assert float(out[True][1].abs().max()) == 0.0
    assert_close(out[False][1], dy64 @ w264.T, RTOL_F16, "gelu output grad (unfused)")
