"""fp64 paths: float64 data keeps its dtype in the reference (_core.py:173-193) and its
CuPy / NumPy arithmetic runs in float64, so fp64 tensors are computed in double here.
Each kernel is checked against the NumPy oracle in float64 (tolerance 1e-11: the
difference is summation order only), and the composed C1 MLP step with float64 input
against the oracle's float64 step.  GPU only."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F32, assert_close

pytestmark = pytest.mark.gpu

RTOL_F64 = 1e-11


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def dev(a):
    return torch.tensor(np.asarray(a, dtype=np.float64), device="cuda")


def host(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("M,N,K,ta,tb", [(1, 1, 1, False, False), (64, 64, 16, False, False),
                                         (100, 37, 53, True, False), (33, 129, 200, False, True),
                                         (257, 65, 31, True, True), (512, 384, 1024, False, False)])
def test_gemm_f64(cuda, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 7 + N + K)
    a = rng.standard_normal((K, M) if ta else (M, K))
    b = rng.standard_normal((N, K) if tb else (K, N))
    want = (a.T if ta else a) @ (b.T if tb else b)
    out = L().matmul2d(dev(a), dev(b), trans_a=ta, trans_b=tb)
    assert out.dtype == torch.float64
    assert_close(out, want, RTOL_F64, f"gemm f64 {M}x{N}x{K}")
    # alpha / beta and a batch with a broadcast operand (stride 0)
    c0 = rng.standard_normal((3, M, N))
    C = dev(c0)
    A = dev(np.stack([a] * 3))
    L().gemm(A, dev(b), C, ta, tb, 0.5, 2.0, M, N, K, a.shape[1], b.shape[1], N,
             a.size, 0, M * N, 3)
    assert_close(C, 0.5 * want[None] + 2.0 * c0, RTOL_F64, "gemm f64 alpha/beta batched")


@pytest.mark.parametrize("kind", ["gelu", "silu"])
@pytest.mark.parametrize("acc", [False, True])
def test_activation_f64(cuda, kind, acc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(10007) * 3
    dy = rng.standard_normal(10007)
    fwd, bwd = (O.gelu_fwd, O.gelu_bwd) if kind == "gelu" else (O.silu_fwd, O.silu_bwd)
    y = L().act_fwd(kind, dev(x))
    assert_close(y, fwd(x), RTOL_F64, f"{kind} fwd f64")
    base = rng.standard_normal(10007)
    dx = dev(base) if acc else torch.empty(10007, dtype=torch.float64, device="cuda")
    L().act_bwd(kind, dev(x), dev(dy), dx, acc)
    assert_close(dx, bwd(x, dy) + (base if acc else 0), RTOL_F64, f"{kind} bwd f64")


def test_axpby_fill_f64(cuda):
    rng = np.random.default_rng(4)
    x, y = rng.standard_normal(5000), rng.standard_normal(5000)
    z = L().axpbyz(dev(x), dev(y), 1.0 / 3.0, -2.5)
    np.testing.assert_allclose(host(z), x / 3.0 - 2.5 * y, rtol=1e-15, atol=1e-15)
    y32 = torch.tensor(y.astype(np.float32), device="cuda")
    L().axpby(dev(x), y32, 1.0, 1.0)  # fp64 into an fp32 buffer: rounded once
    np.testing.assert_array_equal(host(y32), (x + y.astype(np.float32)).astype(np.float32))
    f = torch.empty(1000, dtype=torch.float64, device="cuda")
    L().fill(f, 0.25)
    assert np.all(host(f) == 0.25)


@pytest.mark.parametrize("rows,cols", [(1, 1), (37, 1000), (300, 64)])
def test_softmax_f64(cuda, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)) * 2
    dy = rng.standard_normal((rows, cols))
    y = L().softmax_fwd(dev(x))
    yr = O.softmax_fwd(x)
    assert_close(y, yr, RTOL_F64, "softmax fwd f64")
    dx = torch.empty_like(y)
    L().softmax_bwd(y, dev(dy), dx, False)
    assert_close(dx, O.softmax_bwd(yr, dy), RTOL_F64, "softmax bwd f64")


@pytest.mark.parametrize("rows,cols,acc", [(5, 3, False), (300, 1024, True), (2049, 96, False)])
def test_layernorm_f64(cuda, rows, cols, acc):
    rng = np.random.default_rng(rows)
    x = rng.standard_normal((rows, cols)) * 1.5 + 0.3
    dy = rng.standard_normal((rows, cols))
    g = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.02 * rng.standard_normal(cols)).astype(np.float32)
    gd, bd = torch.tensor(g, device="cuda"), torch.tensor(b, device="cuda")
    y, mean, rstd = L().layernorm_fwd(dev(x), gd, bd, 1e-5)
    assert mean.dtype == torch.float64
    yr, xh, _, var = O.layernorm_fwd(x, g.astype(np.float64), b.astype(np.float64))
    assert_close(y, yr, RTOL_F64, "layernorm fwd f64")
    dxr, dgr, dbr = O.layernorm_bwd(xh, var, g.astype(np.float64), dy)
    base = rng.standard_normal((rows, cols))
    dx = dev(base) if acc else torch.empty(rows, cols, dtype=torch.float64, device="cuda")
    dg = torch.empty(cols, device="cuda")
    db = torch.empty(cols, device="cuda")
    L().layernorm_bwd(dev(x), mean, rstd, gd, dev(dy), dx, dg, db, acc, False)
    assert_close(dx, dxr + (base if acc else 0), RTOL_F64, "layernorm dx f64")
    # the parameters are fp32: their gradients are the fp64 sums rounded once
    np.testing.assert_array_equal(host(dg), dgr.astype(np.float32))
    np.testing.assert_array_equal(host(db), dbr.astype(np.float32))


def test_reduce_rows_f64(cuda):
    rng = np.random.default_rng(6)
    g = rng.standard_normal((4099, 300))
    out = torch.empty(300, dtype=torch.float64, device="cuda")
    L().reduce_rows(dev(g), out, False)
    assert_close(out, g.sum(0), RTOL_F64, "reduce_rows f64")
    base = rng.standard_normal(300).astype(np.float32)
    o32 = torch.tensor(base, device="cuda")
    L().reduce_rows(dev(g), o32, True)
    np.testing.assert_array_equal(host(o32), (base.astype(np.float64) + g.sum(0)).astype(np.float32))


@pytest.mark.parametrize("smooth", [0.0, 0.1])
def test_cross_entropy_f64(cuda, smooth):
    rng = np.random.default_rng(7)
    N, C = 64, 1000
    x = rng.standard_normal((N, C)) * 3
    t = rng.integers(0, C, N)
    lse, loss = L().cross_entropy_fwd(dev(x), torch.tensor(t, device="cuda"), smooth)
    rows, probs = O.cross_entropy_fwd(x, t, smooth, reduction="none")
    assert loss.dtype == torch.float64
    assert_close(loss, rows, RTOL_F64, "ce loss f64")
    g = torch.empty(N, C, dtype=torch.float64, device="cuda")
    L().cross_entropy_bwd(dev(x), torch.tensor(t, device="cuda"), lse, g, 1.0 / N, False, smooth)
    assert_close(g, O.cross_entropy_bwd(probs, t, smooth), RTOL_F64, "ce grad f64")


def test_adam_f64(cuda):
    rng = np.random.default_rng(8)
    p, g = rng.standard_normal(777), rng.standard_normal(777) * 1e-3
    m, v, vm = rng.standard_normal(777) * 1e-3, rng.random(777) * 1e-6, rng.random(777) * 1e-6
    P, M_, V, VM = dev(p), dev(m), dev(v), dev(vm)
    t = 3
    L().adam_step([P], [dev(g)], [M_], [V], [VM], 1e-3, 0.9, 0.999, 1e-8, 0.1,
                  1 - 0.9 ** t, 1 - 0.999 ** t)
    pr, mr, vr, vmr = O.adam_step(p, g, m, v, t, lr=1e-3, weight_decay=0.1, amsgrad=True,
                                  v_max=vm)
    for got, want, n in ((P, pr, "p"), (M_, mr, "m"), (V, vr, "v"), (VM, vmr, "v_max")):
        assert_close(got, want, 1e-13, f"adam f64 {n}")


def test_unscale_and_norm_f64(cuda):
    g1 = dev([3.0, 4.0, 0.5])
    g2 = dev([np.inf, 1.0])
    flags = L().unscale_check([g1, g2], 0.5)
    assert flags == [0, 3]
    np.testing.assert_array_equal(host(g1), [1.5, 2.0, 0.25])
    v, fl = L().grad_norm([g1], 0)
    assert v == 1.5 ** 2 + 2.0 ** 2 + 0.25 ** 2 and fl == [0]
    v, fl = L().grad_norm([g1, g2], 1)
    assert v == 2.0 and fl == [0, 1]
    L().zero_nonfinite([g2])
    assert host(g2)[0] == 0.0


def test_mlp_step_float64_input(cuda):
    """The C1 MLP fed a float64 array (np.random.randn without a cast): the reference
    promotes x @ w (float32 weights) to float64, so the loss and every intermediate are
    float64; the parameter gradients are float64 values rounded once to the float32
    gradient buffers, and Adam updates the float32 parameters."""
    import tensor_gpu_v2 as tg
    np.random.seed(0)
    x = np.random.randn(32, 784)
    l1, l2 = tg.Linear(784, 256), tg.Linear(256, 10)
    w1, w2 = l1.w.numpy().copy(), l2.w.numpy().copy()
    xt = tg.Tensor(x, requires_grad=False)
    assert xt.data.dtype == torch.float64
    loss = l2(l1(xt).gelu()).mean()
    assert loss.data.dtype == torch.float64
    loss.backward()
    ref = O.mlp_step(x, w1, np.zeros(256), w2, np.zeros(10), dtype=np.float64)
    assert abs(loss.item() - ref["loss"]) <= 1e-12 * abs(ref["loss"])
    for p, k in ((l1.w, "dw1"), (l1.b, "db1"), (l2.w, "dw2"), (l2.b, "db2")):
        assert p.grad.dtype == torch.float32
        np.testing.assert_allclose(p.grad.cpu().numpy(), ref[k].astype(np.float32),
                                   rtol=1e-6, atol=1e-6 * np.abs(ref[k]).max())
    opt = tg.Adam([l1.w, l1.b, l2.w, l2.b], lr=1e-3)
    opt.step()
    assert_close(l1.w.data, ref["w1"], RTOL_F32, "w1 after Adam")


def test_float64_parameter_adam(cuda):
    """A parameter made from a float64 array is float64 in the reference; its gradient
    and Adam state stay float64 and the update runs in double."""
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(9)
    p0 = rng.standard_normal((50, 7))
    p = tg.Tensor(p0)
    assert p.data.dtype == torch.float64
    ((p * p).sum() * 0.5).backward()  # grad = p
    np.testing.assert_allclose(p.grad.cpu().numpy(), p0, rtol=1e-15)
    opt = tg.AdamW([p], lr=1e-2, weight_decay=0.1)
    opt.step()
    pr, _, _, _ = O.adam_step(p0, p0, np.zeros_like(p0), np.zeros_like(p0), 1, lr=1e-2,
                              weight_decay=0.1)
    assert p.data.dtype == torch.float64
    assert_close(p.data, pr, 1e-13, "fp64 AdamW")


def test_float64_softmax_layernorm_ce_autograd(cuda):
    """float64 activations through LayerNorm, softmax and CrossEntropyLoss (the loss's
    logits float64, its gradient float64) against float64 torch autograd."""
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(10)
    x0 = rng.standard_normal((16, 40))
    t = rng.integers(0, 40, 16)
    ln = tg.LayerNorm(40)
    x = tg.Tensor(x0)
    h = ln(x)
    s = h.softmax()
    loss = tg.CrossEntropyLoss()(s * 3.0, t)
    assert loss.data.dtype == torch.float64
    loss.backward()
    xt = torch.tensor(x0, requires_grad=True)
    ht = torch.nn.functional.layer_norm(xt, (40,), eps=1e-5)
    st = torch.softmax(ht, -1) * 3.0
    lt = torch.nn.functional.cross_entropy(st, torch.tensor(t))
    # the reference's loss adds 1e-10 inside the log: within 1e-9 of torch's
    assert abs(loss.item() - lt.item()) < 1e-8
    lt.backward()
    assert_close(x.grad, xt.grad.numpy(), 1e-8, "fp64 LN-softmax-CE input gradient")


@pytest.mark.parametrize("n,V,acc", [(300, 40, False), (8192, 1000, True), (9000, 64, False)])
def test_embedding_bwd_f64_rows_into_fp32(cuda, n, V, acc):
    """An fp64 output gradient scattered into the fp32 embedding gradient: np.add.at on
    a float32 array adds each float64 row in double and rounds at every step; the kernel
    does the same, so the result is bit-exact (one launch up to 8192 tokens, the sorted
    path beyond)."""
    rng = np.random.default_rng(n)
    idx = rng.integers(0, V, n)
    idx[: n // 4] = idx[0]
    d = rng.standard_normal((n, 24))
    want = np.zeros((V, 24), np.float32)
    np.add.at(want, idx, d)
    base = rng.standard_normal((V, 24)).astype(np.float32)
    grad = torch.tensor(base if acc else np.zeros_like(base), device="cuda")
    L().embedding_bwd(dev(d), torch.tensor(idx, device="cuda"), grad, acc)
    exp = (base + want) if acc else want
    np.testing.assert_array_equal(host(grad), exp)


@pytest.mark.parametrize("B,H,Sq,Sk,D,causal,layout", [
    (2, 3, 70, 70, 40, False, 0), (2, 3, 70, 70, 40, True, 0),
    (1, 2, 33, 65, 16, True, 0),   # fewer queries than keys
    (1, 2, 65, 33, 24, True, 0),   # more queries than keys
    (2, 4, 48, 48, 32, True, 1),   # (B, S, H, D) memory, the head split of a projection
    (1, 1, 300, 257, 8, False, 0),
])
def test_flash_attention_f64(cuda, B, H, Sq, Sk, D, causal, layout):
    """fp64 forward (o, natural-log lse) and backward (the reference's row term
    rowsum(P*dP)) against the float64 oracle; accumulate adds to existing gradients."""
    rng = np.random.default_rng(B * 100 + Sq + Sk + D + causal)
    q = rng.standard_normal((B, H, Sq, D))
    k = rng.standard_normal((B, H, Sk, D))
    v = rng.standard_normal((B, H, Sk, D))
    do = rng.standard_normal((B, H, Sq, D))
    scale = D ** -0.5
    o_ref, lse_ref = O.flash_attention_fwd(q, k, v, causal, scale)
    dq_ref, dk_ref, dv_ref = O.flash_attention_bwd(q, k, v, do, causal, scale)

    def put(a):  # layout 1: (B, S, H, D) memory viewed as (B, H, S, D)
        t = dev(a)
        return t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3) if layout else t

    qt, kt, vt, dot = put(q), put(k), put(v), put(do)
    o, lse = L().flash_attn_fwd(qt, kt, vt, scale, causal, layout)
    assert o.dtype == torch.float64 and lse.dtype == torch.float64
    assert_close(o, o_ref, RTOL_F64, "fp64 attention o")
    assert_close(lse, lse_ref, RTOL_F64, "fp64 attention lse")
    grads = [L().fa_empty(B, H, s, D, torch.float64, qt.device, layout) for s in (Sq, Sk, Sk)]
    for g in grads:
        g.fill_(0.5)
    L().flash_attn_bwd(qt, kt, vt, o, dot, lse, *grads, scale, causal, True, layout)
    for g, ref, n in zip(grads, (dq_ref, dk_ref, dv_ref), ("dq", "dk", "dv")):
        assert_close(g, ref + 0.5, 1e-10, f"fp64 attention {n}")


def test_flash_attention_f64_autograd_3d(cuda):
    """tg.flash_attention on float64 (B, L, D) tensors: values and gradients stay
    float64 and match the oracle."""
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((3, 50, 24)) for _ in range(3))
    g = rng.standard_normal((3, 50, 24))
    Q, K, V = tg.Tensor(q), tg.Tensor(k), tg.Tensor(v)
    out = tg.flash_attention(Q, K, V, is_causal=True)
    assert out.data.dtype == torch.float64
    out.backward(tg.Tensor(g))
    o_ref, _ = O.flash_attention_fwd(q, k, v, True)
    assert_close(out.data, o_ref, RTOL_F64, "o")
    for t, ref in zip((Q, K, V), O.flash_attention_bwd(q, k, v, g, True)):
        assert t.grad.dtype == torch.float64
        assert_close(t.grad, ref, 1e-10, "3-D fp64 attention grad")


@pytest.mark.parametrize("fmt", ["NCHW", "NHWC"])
@pytest.mark.parametrize("relu", [True, False])
def test_batchnorm_f64_module(cuda, fmt, relu):
    """FusedBatchNormReLU / BatchNorm2D on float64 data: output, batch statistics in the
    running-stat update (float64 buffers, as the reference's update promotes them), dx in
    double, dgamma/dbeta rounded into the fp32 parameter gradients — against the
    oracle's float64 training forward/backward."""
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(11 + relu)
    N, C, Hh, W = 4, 6, 5, 7
    x_nchw = rng.standard_normal((N, C, Hh, W)) * 1.5 + 0.3
    dy_nchw = rng.standard_normal((N, C, Hh, W))
    mod = (tg.FusedBatchNormReLU if relu else tg.BatchNorm2D)(C, data_format=fmt)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    mod.gamma.data.copy_(torch.tensor(g))
    mod.beta.data.copy_(torch.tensor(b))
    to = (lambda a: a.transpose(0, 2, 3, 1).copy()) if fmt == "NHWC" else (lambda a: a)
    x = tg.Tensor(to(x_nchw))
    y = mod(x)
    assert y.data.dtype == torch.float64
    y.backward(tg.Tensor(to(dy_nchw)))
    y_ref, cache = O.batchnorm_relu_fwd(x_nchw, g.astype(np.float64), b.astype(np.float64),
                                        1e-5, relu)
    dx_ref, dg_ref, db_ref = O.batchnorm_relu_bwd(dy_nchw, g.astype(np.float64), cache, relu)
    assert_close(y.data, to(y_ref), RTOL_F64, "fp64 BN output")
    assert x.grad.dtype == torch.float64
    assert_close(x.grad, to(dx_ref), 1e-10, "fp64 BN dx")
    assert mod.gamma.grad.dtype == torch.float32
    assert_close(mod.gamma.grad, dg_ref, 1e-6, "BN dgamma (fp32 buffer)")
    assert_close(mod.beta.grad, db_ref, 1e-6, "BN dbeta (fp32 buffer)")
    assert mod.running_mean.dtype == torch.float64
    assert_close(mod.running_mean, 0.1 * cache[5], RTOL_F64, "running mean")
    assert_close(mod.running_var, 0.9 + 0.1 * cache[6], RTOL_F64, "running var")


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("fmt", ["NCHW", "NHWC"])
def test_batchnorm2d_eval_mode_gradient(cuda, dt, fmt):
    """BatchNorm2D in eval mode normalises with the running statistics and still
    differentiates, with the training formula applied to those statistics (reference
    _nn.py:706-736): against the oracle's eval forward and its backward on that cache."""
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(21)
    N, C, Hh, W = 3, 5, 4, 6
    x_nchw = (rng.standard_normal((N, C, Hh, W)) * 2).astype(dt)
    dy_nchw = rng.standard_normal((N, C, Hh, W)).astype(dt)
    rm = (0.5 * rng.standard_normal(C)).astype(np.float32)
    rv = (0.5 + rng.random(C)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    mod = tg.BatchNorm2D(C, data_format=fmt)
    mod.gamma.data.copy_(torch.tensor(g))
    mod.beta.data.copy_(torch.tensor(b))
    mod.running_mean.copy_(torch.tensor(rm))
    mod.running_var.copy_(torch.tensor(rv))
    mod.eval()
    to = (lambda a: a.transpose(0, 2, 3, 1).copy()) if fmt == "NHWC" else (lambda a: a)
    x = tg.Tensor(to(x_nchw))
    y = mod(x)
    y.backward(tg.Tensor(to(dy_nchw)))
    # the reference's parameters and running statistics are float32 arrays: std_inv is
    # formed in float32 and meets the data's dtype after that (NumPy promotion), so the
    # oracle gets them as float32 too
    y_ref, cache = O.batchnorm_eval_fwd(x_nchw, g, b, rm, rv, 1e-5)
    dx_ref, dg_ref, db_ref = O.batchnorm_relu_bwd(dy_nchw, g, cache, False)
    tol = RTOL_F64 if dt == np.float64 else RTOL_F32
    assert_close(y.data, to(y_ref), tol, "eval BN output")
    # dx: every sum in double here; the reference rounds std_inv**3 in float32, so
    # the float64 result agrees to float32 rounding of that factor (1e-6)
    assert_close(x.grad, to(dx_ref), 1e-6 if dt == np.float64 else RTOL_F32, "eval BN dx")
    assert_close(mod.gamma.grad, dg_ref, 1e-6, "eval BN dgamma")
    assert_close(mod.beta.grad, db_ref, 1e-6, "eval BN dbeta")


@pytest.mark.parametrize("R,C", [(64, 128), (70, 33)])
def test_transpose_add_f64(cuda, R, C):
    """sync_tied_gradients' source.grad += param.grad.T (_training.py:264-284) with a
    float64 side: added in double, cast once to the destination (bit-exact with NumPy)."""
    rng = np.random.default_rng(R + C)
    src = rng.standard_normal((R, C))
    d64 = rng.standard_normal((C, R))
    out = dev(d64)
    L().transpose_add(dev(src), out)
    assert np.array_equal(host(out), d64 + src.T)
    d32 = rng.standard_normal((C, R)).astype(np.float32)
    out32 = torch.tensor(d32, device="cuda")
    L().transpose_add(dev(src), out32)
    assert np.array_equal(out32.cpu().numpy(), (d32.astype(np.float64) + src.T).astype(np.float32))
    s32 = rng.standard_normal((R, C)).astype(np.float32)
    out = dev(d64)
    L().transpose_add(torch.tensor(s32, device="cuda"), out)
    assert np.array_equal(host(out), d64 + s32.astype(np.float64).T)
