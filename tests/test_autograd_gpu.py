"""The tensor_gpu_v2 API (Tensor.backward, modules, optimizers, GradScaler,
clipping, autocast) on the MI355X, compared with the oracle and with the
reference test-suite's known answers.  GPU only."""
import os

import numpy as np
import pytest
import torch

import oracle as O
from conftest import GOLDEN, RTOL_F16, RTOL_F32, RTOL_F32_MM, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture
def tg(cuda):
    import tensor_gpu_v2
    return tensor_gpu_v2


def npf(a):
    return np.asarray(a, dtype=np.float32)


# ------------------------------------------------------------------ C1: README MLP
def test_mlp_c1_step_matches_golden(tg):
    f = np.load(os.path.join(GOLDEN, "mlp_c1.npz"), allow_pickle=False)
    np.random.seed(0)
    x = tg.Tensor(np.random.randn(32, 784).astype(np.float32), requires_grad=False)
    l1, l2 = tg.Linear(784, 256), tg.Linear(256, 10)
    loss = l2(l1(x).gelu()).mean()
    loss.backward()
    assert abs(loss.item() - float(f["loss"])) <= 1e-5 * abs(float(f["loss"]))
    assert_close(l2.w.grad, f["dw2"], RTOL_F32_MM, "dw2")
    assert_close(l2.b.grad, f["db2"], RTOL_F32, "db2")
    assert_close(l1.b.grad, f["db1"], RTOL_F32, "db1")
    dw1 = l1.w.grad.cpu().numpy().reshape(-1)
    assert_close(dw1[f["dw1_idx"]], f["dw1_sel"], RTOL_F32_MM, "dw1 sample")
    assert abs(dw1.astype(np.float64).sum() - float(f["dw1_sum"])) < 1e-4 * np.sqrt(float(f["dw1_sq"]))
    opt = tg.Adam([l1.w, l1.b, l2.w, l2.b], lr=1e-3)
    opt.step()
    assert_close(l2.w.data, f["w2"], RTOL_F32, "w2 after Adam")
    assert_close(l1.w.data.reshape(-1)[torch.as_tensor(f["dw1_idx"]).cuda()], f["w1_sel"],
                 RTOL_F32, "w1 sample after Adam")


# ------------------------------------------------------------------ matmul backward
MATMUL_CASES = [((2, 4, 5), (5, 3)), ((2, 4, 5), (1, 5, 3)), ((3, 2, 4, 5), (5, 3)),
                ((5,), (5,)), ((5,), (5, 3)), ((2, 5), (5,)), ((2, 1, 5), (5,)),
                ((5,), (2, 5, 3)), ((64, 96), (96, 48)), ((3, 37, 64), (64, 20))]


@pytest.mark.parametrize("ash,bsh", MATMUL_CASES)
def test_matmul_backward_broadcast(tg, ash, bsh):
    # the reference's cases (test_autograd_regressions_phase6.py:86-95) in fp32
    rng = np.random.default_rng(123)
    a_np = rng.standard_normal(ash).astype(np.float32)
    b_np = rng.standard_normal(bsh).astype(np.float32)
    a = tg.Tensor(a_np)
    b = tg.Tensor(b_np)
    y = a @ b
    dy = rng.standard_normal(y.shape).astype(np.float32)
    y.backward(dy)
    da, db = O.matmul_bwd(a_np.astype(np.float64), b_np.astype(np.float64), dy.astype(np.float64))
    assert tuple(a.grad.shape) == ash and tuple(b.grad.shape) == bsh
    assert_close(y.data, a_np.astype(np.float64) @ b_np.astype(np.float64), RTOL_F32_MM, "y")
    assert_close(a.grad, da, RTOL_F32_MM, "da")
    assert_close(b.grad, db, RTOL_F32_MM, "db")


def test_matmul_backward_validation(tg):
    # (test_autograd_regressions_phase6.py:481-515)
    a = tg.Tensor(np.arange(6.0, dtype=np.float32).reshape(2, 3))
    b = tg.Tensor(np.arange(12.0, dtype=np.float32).reshape(3, 4))
    y = a @ b
    y.grad = torch.ones(3, 4, device="cuda")
    with pytest.raises(ValueError):
        y._backward()
    ai = tg.Tensor(np.arange(6, dtype=np.int32).reshape(2, 3))
    bf = tg.Tensor(np.ones((3, 2), dtype=np.float32))
    y2 = ai @ bf
    y2.grad = torch.ones_like(y2.data)
    with pytest.raises(TypeError):
        y2._backward()


def test_unbroadcast_validation(tg):
    t = tg.Tensor(np.zeros((2, 3), np.float32), requires_grad=False)
    with pytest.raises(ValueError):
        t._unbroadcast(torch.ones(2, 3, device="cuda"), (2, 3, 1))
    with pytest.raises(ValueError):
        t._unbroadcast(torch.ones(2, 3, device="cuda"), (2, 4))
    r = t._unbroadcast(torch.ones(2, 3, 4, device="cuda"), (1, 3, 1))
    assert tuple(r.shape) == (1, 3, 1) and torch.all(r == 8.0)
    r = t._unbroadcast(torch.ones(7, 5, 3, device="cuda"), (3,))
    assert torch.all(r == 35.0)


# ------------------------------------------------------------------ elementwise / softmax ops
@pytest.mark.parametrize("op", ["gelu", "silu", "softmax"])
def test_activation_ops_backward(tg, op):
    rng = np.random.default_rng(4)
    x_np = rng.standard_normal((33, 257)).astype(np.float32) * 2
    dy = rng.standard_normal((33, 257)).astype(np.float32)
    x = tg.Tensor(x_np)
    y = getattr(x, op)()
    y.backward(dy)
    xd, dyd = x_np.astype(np.float64), dy.astype(np.float64)
    if op == "gelu":
        want, ywant = O.gelu_bwd(xd, dyd), O.gelu_fwd(xd)
    elif op == "silu":
        want, ywant = O.silu_bwd(xd, dyd), O.silu_fwd(xd)
    else:
        ywant = O.softmax_fwd(xd)
        want = O.softmax_bwd(y.data.double().cpu().numpy(), dyd)
    assert_close(y.data, ywant, RTOL_F32, f"{op} forward")
    assert_close(x.grad, want, RTOL_F32, f"{op} backward")


def test_softmax_other_axis_and_accumulation(tg):
    rng = np.random.default_rng(5)
    x_np = rng.standard_normal((6, 9, 4)).astype(np.float32)
    x = tg.Tensor(x_np)
    y = x.softmax(axis=1)
    loss = (y * y).sum() + x.gelu().sum()
    loss.backward()
    xt = torch.tensor(x_np.astype(np.float64), requires_grad=True)
    yt = torch.softmax(xt, 1)
    ((yt * yt).sum() + torch.nn.functional.gelu(xt, approximate="tanh").sum()).backward()
    assert_close(x.grad, xt.grad.numpy(), RTOL_F32, "softmax(axis=1) + gelu grad")


def test_backward_seed_semantics(tg):
    x = tg.Tensor(np.array([1.0, 2.0, 3.0], np.float32))
    y = (x * x).sum()
    y.backward()
    assert np.allclose(x.grad.cpu().numpy(), [2, 4, 6])
    # explicit gradient is added to an existing grad
    x2 = tg.Tensor(np.array([1.0, 2.0], np.float32))
    z = x2 * 3.0
    z.backward(np.array([1.0, 10.0], np.float32))
    assert np.allclose(x2.grad.cpu().numpy(), [3, 30])
    # a second backward through a new graph accumulates into leaf grads
    y2 = (x * 2.0).sum()
    y2.backward()
    assert np.allclose(x.grad.cpu().numpy(), [4, 6, 8])


def test_backward_integer_seed_is_cast(tg):
    """An integer seed (Python int, int array, int tensor) is cast to the tensor's
    dtype first, as xp.asarray(gradient, dtype=self.dtype) does in the reference
    (_core.py:1447-1454): fresh grad and accumulation into an existing one."""
    for seed in (2, np.array([2, 2, 2], np.int64), torch.tensor([2, 2, 2], dtype=torch.int32)):
        x = tg.Tensor(np.array([1.0, 2.0, 3.0], np.float32))
        y = x * 3.0
        y.backward(seed)
        assert y.grad.dtype == torch.float32
        assert np.allclose(x.grad.cpu().numpy(), [6, 6, 6])
        y.backward(seed)  # existing grad: the cast seed is added
        assert np.allclose(y.grad.cpu().numpy(), [4, 4, 4])
    h = tg.Tensor(np.array([1.0, -1.0], np.float16))
    z = h * 2.0
    z.backward(np.array([1, 3], np.int64))
    assert z.grad.dtype == torch.float16
    assert np.allclose(h.grad.float().cpu().numpy(), [2, 6])


# ------------------------------------------------------------------ modules
@pytest.mark.parametrize("shape", [(4, 6, 64), (16, 1024), (3, 100)])
def test_layernorm_module(tg, shape):
    rng = np.random.default_rng(6)
    cols = shape[-1]
    ln = tg.LayerNorm(cols)
    g = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.02 * rng.standard_normal(cols)).astype(np.float32)
    ln.gamma.data = torch.as_tensor(g).cuda()
    ln.beta.data = torch.as_tensor(b).cuda()
    x_np = rng.standard_normal(shape).astype(np.float32)
    dy = rng.standard_normal(shape).astype(np.float32)
    x = tg.Tensor(x_np)
    y = ln(x)
    y.backward(dy)
    yr, xh, _, var = O.layernorm_fwd(x_np.astype(np.float64), g.astype(np.float64),
                                     b.astype(np.float64))
    dx, dg, db = O.layernorm_bwd(xh, var, g.astype(np.float64), dy.astype(np.float64))
    assert_close(y.data, yr, RTOL_F32, "ln y")
    assert_close(x.grad, dx, RTOL_F32, "ln dx")
    assert_close(ln.gamma.grad, dg, RTOL_F32, "ln dgamma")
    assert_close(ln.beta.grad, db, RTOL_F32, "ln dbeta")


@pytest.mark.parametrize("fmt", ["NCHW", "NHWC"])
@pytest.mark.parametrize("cls", ["FusedBatchNormReLU", "BatchNorm2D"])
def test_batchnorm_modules(tg, fmt, cls):
    rng = np.random.default_rng(7)
    C = 12
    shape = (4, C, 5, 6) if fmt == "NCHW" else (4, 5, 6, C)
    m = getattr(tg, cls)(C, data_format=fmt)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    m.gamma.data = torch.as_tensor(g).cuda()
    m.beta.data = torch.as_tensor(b).cuda()
    x_np = rng.standard_normal(shape).astype(np.float32)
    dy = rng.standard_normal(shape).astype(np.float32)
    x = tg.Tensor(x_np)
    y = m(x)
    y.backward(dy)
    relu = cls == "FusedBatchNormReLU"
    if fmt == "NCHW":
        yr, cache = O.batchnorm_relu_fwd(x_np.astype(np.float64), g.astype(np.float64),
                                         b.astype(np.float64), 1e-5, relu)
        dx, dg, db = O.batchnorm_relu_bwd(dy.astype(np.float64), g.astype(np.float64), cache, relu)
    else:
        yr, cache = O.batchnorm_relu_fwd_nhwc(x_np.astype(np.float64), g.astype(np.float64),
                                              b.astype(np.float64), 1e-5, relu)
        dx, dg, db = O.batchnorm_relu_bwd_nhwc(dy.astype(np.float64), g.astype(np.float64),
                                               cache, relu)
    assert_close(y.data, yr, RTOL_F32, "bn y")
    assert_close(x.grad, dx, 1e-4, "bn dx")  # mask computed from the kernel's own fp32 stats
    assert_close(m.gamma.grad, dg, 1e-4, "bn dgamma")
    assert_close(m.beta.grad, db, 1e-4, "bn dbeta")
    assert_close(m.running_mean, 0.1 * cache[5], RTOL_F32, "running mean")


def test_flash_attention_tensor_api(tg):
    rng = np.random.default_rng(8)
    for shape, causal in (((2, 3, 80, 64), True), ((2, 70, 64), False)):
        qn, kn, vn, don = (rng.standard_normal(shape).astype(np.float16) for _ in range(4))
        q, k, v = (tg.Tensor(a) for a in (qn, kn, vn))
        out = tg.flash_attention(q, k, v, is_causal=causal)
        out.backward(don)
        args = [a.astype(np.float64) for a in (qn, kn, vn)]
        oo, _ = O.flash_attention_fwd(*args, is_causal=causal)
        dq, dk, dv = O.flash_attention_bwd(*args, don.astype(np.float64), is_causal=causal)
        assert out.data.dtype == torch.float16
        assert_close(out.data, oo, RTOL_F16, "fa out")
        assert_close(q.grad, dq, RTOL_F16, "fa dq")
        assert_close(k.grad, dk, RTOL_F16, "fa dk")
        assert_close(v.grad, dv, RTOL_F16, "fa dv")


@pytest.mark.parametrize("shape,causal", [((2, 3, 80, 64), True), ((2, 70, 64), False),
                                          ((1, 2, 50, 40), False), ((3, 33, 96), True)])
def test_flash_attention_tensor_api_fp32(tg, shape, causal):
    """fp32 inputs (the reference's default dtype), 4-D (B, H, L, D) and 3-D (B, L, D),
    head dims inside and outside 64/128, at the fp32 attention bar."""
    rng = np.random.default_rng(18)
    qn, kn, vn, don = (rng.standard_normal(shape).astype(np.float32) for _ in range(4))
    q, k, v = (tg.Tensor(a) for a in (qn, kn, vn))
    out = tg.flash_attention(q, k, v, is_causal=causal)
    out.backward(don)
    args = [a.astype(np.float64) for a in (qn, kn, vn)]
    oo, _ = O.flash_attention_fwd(*args, is_causal=causal)
    dq, dk, dv = O.flash_attention_bwd(*args, don.astype(np.float64), is_causal=causal)
    assert out.data.dtype == torch.float32
    assert_close(out.data, oo, RTOL_F32_MM, "fa out")
    assert_close(q.grad, dq, RTOL_F32_MM, "fa dq")
    assert_close(k.grad, dk, RTOL_F32_MM, "fa dk")
    assert_close(v.grad, dv, RTOL_F32_MM, "fa dv")


def test_cross_entropy_ignores_upstream_grad(tg):
    # (_nn.py:1168-1180): logits.grad = (softmax - onehot)/N, out.grad never read
    rng = np.random.default_rng(9)
    x_np = (rng.standard_normal((16, 40)) * 2).astype(np.float32)
    y_np = rng.integers(0, 40, 16)
    x = tg.Tensor(x_np)
    loss = tg.CrossEntropyLoss()(x, y_np)
    scaled = loss * 1024.0
    scaled.backward()
    lo, probs = O.cross_entropy_fwd(x_np.astype(np.float64), y_np)
    assert abs(loss.item() - lo) < 1e-5 * abs(lo)
    assert_close(x.grad, O.cross_entropy_bwd(probs, y_np), RTOL_F32, "CE grad (unscaled)")


# ------------------------------------------------------------------ optimizers
@pytest.mark.parametrize("cls", ["Adam", "AdamW", "FusedAdam"])
def test_adam_family_two_steps(tg, cls):
    rng = np.random.default_rng(10)
    p_np = [rng.standard_normal(s).astype(np.float32) for s in ((7, 5), (13,), (64, 33))]
    ps = [tg.Tensor(a) for a in p_np]
    kw = {"lr": 3e-3}
    wd = {"Adam": 0.0, "AdamW": 0.01, "FusedAdam": 0.0}[cls]
    opt = getattr(tg, cls)(ps, **kw)
    ref = [(a.astype(np.float64), np.zeros(a.shape), np.zeros(a.shape)) for a in p_np]
    for t in (1, 2):
        gs = [rng.standard_normal(a.shape).astype(np.float32) for a in p_np]
        for p, g in zip(ps, gs):
            p.grad = g
        opt.step()
        ref = [O.adam_step(pp, g.astype(np.float64), m, v, t, lr=3e-3, weight_decay=wd)[:3]
               for (pp, m, v), g in zip(ref, gs)]
    for p, r in zip(ps, ref):
        assert_close(p.data, r[0], RTOL_F32, f"{cls} params")


def test_adam_zero_grad_params_still_update(tg):
    # a parameter that never received a gradient has grad 0, not None (_core.py:637)
    p = tg.Tensor(np.ones(4, np.float32))
    opt = tg.AdamW([p], lr=0.1, weight_decay=0.5)
    opt.step()
    assert np.allclose(p.data.cpu().numpy(), 1 - 0.1 * 0.5)


# ------------------------------------------------------------------ GradScaler / clipping
def test_clip_grad_norm_known_answers(tg):
    t1 = tg.Tensor(np.array([3.0, 4.0], np.float32))
    t2 = tg.Tensor(np.array([0.0, 0.0], np.float32))
    t1.grad = np.array([3.0, 4.0], np.float32)
    t2.grad = np.array([12.0, 0.0], np.float32)
    n = tg.clip_grad_norm_([t1, t2], max_norm=1.0)
    assert abs(n - 13.0) < 1e-5
    assert np.allclose(t1.grad.cpu().numpy(), [3 / 13, 4 / 13], atol=1e-5)
    assert np.allclose(t2.grad.cpu().numpy(), [12 / 13, 0], atol=1e-5)
    a = tg.Tensor(np.zeros(2, np.float32))
    b = tg.Tensor(np.zeros(2, np.float32))
    a.grad = np.array([1.0, 2.0], np.float32)
    b.grad = np.array([5.0, 3.0], np.float32)
    n = tg.clip_grad_norm_([a, b], max_norm=2.0, norm_type=float("inf"))
    assert n == 5.0
    assert abs(max(float(a.grad.abs().max()), float(b.grad.abs().max())) - 2.0) < 1e-5
    c = tg.Tensor(np.zeros(3, np.float32))
    c.grad = np.array([np.nan, 3.0, 4.0], np.float32)
    with pytest.warns(UserWarning):
        n = tg.clip_grad_norm_([c], max_norm=100.0)
    assert abs(n - 5.0) < 1e-6 and np.array_equal(c.grad.cpu().numpy(), [0.0, 3.0, 4.0])
    d = tg.Tensor(np.zeros(3, np.float32))
    d.grad = np.array([np.inf, 3.0, 4.0], np.float32)
    with pytest.raises(RuntimeError):
        tg.clip_grad_norm_([d], 1.0, error_if_nonfinite=True)
    e = tg.Tensor(np.zeros(2, np.float32), requires_grad=False)
    assert tg.clip_grad_norm_([e], 1.0) == 0.0


def test_gradscaler_overflow_and_growth(tg):
    scaler = tg.GradScaler(init_scale=65536.0, backoff_factor=0.5)
    lin = tg.Linear(2, 2)
    opt = tg.Adam(lin.parameters(), lr=0.001)
    w0 = lin.w.data.clone()
    for p in lin.parameters():
        p.grad = torch.full_like(p.data, float("inf"))
    scaler.unscale_(opt)
    assert scaler._found_inf
    assert all(float(p.grad.abs().sum()) == 0.0 for p in lin.parameters())
    scaler.step(opt)  # skipped
    assert torch.equal(lin.w.data, w0)
    scaler.update()
    assert scaler.get_scale() == 32768.0 and scaler.get_statistics()["overflow_count"] == 1
    s2 = tg.GradScaler(init_scale=1024.0, growth_interval=3, growth_factor=2.0)
    for p in lin.parameters():
        p.grad = torch.ones_like(p.data)
    for _ in range(3):
        s2.unscale_(opt)
        s2.update()
    assert s2.get_scale() == 2048.0
    s3 = tg.GradScaler(init_scale=2.0, min_scale=1.0)
    for _ in range(3):
        s3._found_inf = True
        s3.update()
    assert s3.get_scale() == 1.0


def test_gradscaler_zeroes_only_flagged_tensors(tg):
    """unscale_ with zero_nan_grads (the reference's per-parameter loop,
    _nn.py:1816-1829): a gradient holding a NaN or Inf is zeroed whole, the others are
    unscaled bit-exact; fp32 and fp64 parameters; found_inf read after the fact."""
    rng = np.random.default_rng(4)
    vals = [rng.standard_normal(n).astype(dt) * 100
            for n, dt in ((7, np.float32), (3000, np.float32), (5000, np.float32),
                          (9, np.float64), (4100, np.float64))]
    vals[1][1234] = np.inf
    vals[4][7] = np.nan
    ps = [tg.Tensor(np.zeros_like(v)) for v in vals]
    for p, v in zip(ps, vals):
        p.grad = v
    opt = tg.SGD(ps, lr=0.1)
    sc = tg.GradScaler(init_scale=4096.0)
    sc.unscale_(opt)
    for i in (0, 2, 3):
        inv = vals[i].dtype.type(1.0 / 4096.0)
        assert np.array_equal(ps[i].grad.cpu().numpy(), vals[i] * inv), i
    for i in (1, 4):
        assert not np.any(ps[i].grad.cpu().numpy()), i
    assert sc._found_inf
    sc.update()
    assert sc.get_scale() == 2048.0
    for p, v in zip(ps, vals):
        p.grad = np.nan_to_num(v, posinf=1.0, nan=1.0)
    opt._is_unscaled = False
    sc.unscale_(opt)
    assert not sc._found_inf


def test_adamw_step_planned_at_unscale(tg):
    """GradScaler.unscale_ plans the AdamW launch before clip_grad_norm_ rescales the
    gradients in place; the step must see the clipped values, and a gradient replaced
    after unscale_ must be used instead of the planned buffer.  Reference: the AdamW
    update of _nn.py:1413-1442 in float64 NumPy on the same gradients."""
    rng = np.random.default_rng(8)
    shapes = [(64, 32), (32,), (1000,)]
    w0 = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    g0 = [rng.standard_normal(s).astype(np.float32) * 50 for s in shapes]
    ps = [tg.Tensor(w.copy()) for w in w0]
    opt = tg.AdamW(ps, lr=1e-2, weight_decay=0.1)
    sc = tg.GradScaler(init_scale=4.0)
    for p, g in zip(ps, g0):
        p.grad = g * np.float32(4.0)
    sc.unscale_(opt)
    norm = tg.clip_grad_norm_(ps, 1.0)
    grads = [p.grad.double().cpu().numpy() for p in ps]  # unscaled and clipped
    assert norm > 1.0 and abs(np.sqrt(sum((g * g).sum() for g in grads)) - 1.0) < 1e-4
    replaced = rng.standard_normal(shapes[2]).astype(np.float32)
    ps[2].grad = replaced  # a new buffer after the plan
    grads[2] = replaced.astype(np.float64)
    sc.step(opt)
    sc.update()
    for w, g, p in zip(w0, grads, ps):
        w = w.astype(np.float64)
        m = 0.1 * g
        v = 0.001 * g * g
        upd = (m / 0.1) / (np.sqrt(v / 0.001) + 1e-8)
        ref = w - 1e-2 * 0.1 * w - 1e-2 * upd
        assert_close(p.data, ref, 1e-5, "AdamW planned step")


def test_adamw_plan_dropped_by_load_state_dict(tg):
    """A state loaded between unscale_ (which plans the launch) and step replaces the
    moment buffers: the step must update the loaded moments, not the planned ones.
    Reference: the AdamW recurrence of _nn.py:1413-1442 in float64 NumPy."""
    rng = np.random.default_rng(12)
    w0 = rng.standard_normal(300).astype(np.float32)
    g0 = rng.standard_normal(300).astype(np.float32)
    m0 = rng.standard_normal(300).astype(np.float32) * 0.1
    v0 = np.abs(rng.standard_normal(300)).astype(np.float32) * 0.01
    p = tg.Tensor(w0.copy())
    opt = tg.AdamW([p], lr=1e-2, weight_decay=0.1)
    sc = tg.GradScaler(init_scale=2.0)
    p.grad = g0 * np.float32(2.0)
    sc.unscale_(opt)
    opt.load_state_dict({"t": 3, "m": [m0], "v": [v0]})
    sc.step(opt)
    g, w = g0.astype(np.float64), w0.astype(np.float64)
    m = 0.9 * m0 + 0.1 * g
    v = 0.999 * v0 + 0.001 * g * g
    ref = w - 1e-2 * 0.1 * w - 1e-2 * (m / (1 - 0.9 ** 4)) / (np.sqrt(v / (1 - 0.999 ** 4)) + 1e-8)
    assert_close(p.data, ref, 1e-5, "AdamW after load_state_dict")
    assert_close(opt.m[0], m, 1e-6, "loaded first moment updated")


def test_gradscaler_unscale_bit_exact(tg):
    rng = np.random.default_rng(11)
    vals = [rng.standard_normal(n).astype(np.float32) * 100 for n in (5, 1000, 4097)]
    ps = [tg.Tensor(np.zeros_like(v)) for v in vals]
    for p, v in zip(ps, vals):
        p.grad = v
    vals[1][3] = np.nan
    ps[1].grad = vals[1]
    opt = tg.SGD(ps, lr=0.1)
    sc = tg.GradScaler(init_scale=8192.0)
    sc.unscale_(opt, zero_nan_grads=False)
    assert sc._found_inf
    inv = np.float32(1.0 / 8192.0)
    assert np.array_equal(ps[0].grad.cpu().numpy(), vals[0] * inv)
    assert np.array_equal(ps[2].grad.cpu().numpy(), vals[2] * inv)
    g1 = ps[1].grad.cpu().numpy()  # untouched (pre-existing NaN, zero_nan_grads=False)
    assert np.isnan(g1[3]) and np.array_equal(np.delete(g1, 3), np.delete(vals[1], 3))


def test_scaled_loss_backward_and_step_fp16_autocast(tg):
    """Reference semantics under autocast: activations fp16, fp32 params keep fp32
    grads, CE ignores the loss scale, so unscale_ shrinks the grads by 1/scale."""
    np.random.seed(1)
    lin = tg.Linear(32, 16)
    x = tg.Tensor(np.random.randn(8, 32).astype(np.float32), requires_grad=False)
    y = np.random.randint(0, 16, 8)
    with tg.autocast():
        logits = lin(x)
        assert logits.data.dtype == torch.float16
        loss = tg.CrossEntropyLoss()(logits, y)
    scaler = tg.GradScaler(init_scale=256.0)
    scaler.scale(loss).backward()
    assert lin.w.grad.dtype == torch.float32
    g_before = lin.w.grad.clone()
    opt = tg.AdamW(lin.parameters(), lr=1e-3, weight_decay=0.1)
    scaler.unscale_(opt)
    assert not scaler._found_inf
    assert torch.allclose(lin.w.grad, g_before / 256.0, rtol=1e-6, atol=0)
    scaler.step(opt)
    scaler.update()


def test_weight_tie_and_sync(tg):
    emb = tg.Embedding(20, 8)
    head = tg.Linear(8, 20, bias=False)
    tg.weight_tie(emb.weight, head, "w", transpose=True)
    idx = np.array([[1, 2, 2, 5]])
    h = emb(idx)
    out = head(h)
    out.sum().backward()

    class M(tg.Module):
        def __init__(self):
            super().__init__()
            self.emb, self.head = emb, head
    m = M()
    tg.sync_tied_gradients(m)
    W = emb.weight.data.double().cpu().numpy()
    # d(sum(E[idx] @ E^T))/dE = scatter of (ones @ E) rows + (E[idx]^T summed) columns
    rows = W[idx.reshape(-1)]
    want = np.zeros_like(W)
    np.add.at(want, idx.reshape(-1), np.ones((4, 20)) @ W)
    want += (np.ones((4, 20)).T @ rows)
    assert_close(emb.weight.grad, want, 1e-5, "tied embedding grad")
    assert float(head.w.grad.abs().sum()) == 0.0


def test_residual_add_grads_not_aliased(tg):
    """Same-shape adds must not share one gradient buffer between operands (a later
    accumulation into one operand's grad would leak into the other's)."""
    rng = np.random.default_rng(12)
    x_np = rng.standard_normal((8, 16)).astype(np.float32)
    w_np = rng.standard_normal((16, 16)).astype(np.float32)
    x = tg.Tensor(x_np)
    w = tg.Tensor(w_np)
    h = x @ w
    r = h + h.gelu()          # residual: h receives from the add and from gelu
    out = (r + x).sum() + (r * r).sum()
    out.backward()
    xt = torch.tensor(x_np.astype(np.float64), requires_grad=True)
    wt = torch.tensor(w_np.astype(np.float64), requires_grad=True)
    ht = xt @ wt
    rt = ht + torch.nn.functional.gelu(ht, approximate="tanh")
    ((rt + xt).sum() + (rt * rt).sum()).backward()
    assert_close(x.grad, xt.grad.numpy(), RTOL_F32_MM, "x grad")
    assert_close(w.grad, wt.grad.numpy(), RTOL_F32_MM, "w grad")


def test_view_and_add_grads_copy_on_write(tg):
    """Views and same-shape adds hand their gradient buffer on without a copy; every
    later write to either side must leave the other's values intact: a second graph
    accumulating into the same leaf, in-place edits of a read .grad, x + x."""
    rng = np.random.default_rng(21)
    x_np = rng.standard_normal((4, 6)).astype(np.float32)
    c_np = rng.standard_normal((6, 4)).astype(np.float32)
    x = tg.Tensor(x_np)
    c = tg.Tensor(c_np, requires_grad=False)

    def graph():
        y = x.reshape(6, 4)
        a = y + y * c          # y: shared from the add, then accumulated by the mul
        b = a.reshape(24)      # a: shares b's gradient
        return y, a, (b * b).sum()

    y1, a1, l1 = graph()
    l1.backward()
    xt = torch.tensor(x_np.astype(np.float64), requires_grad=True)
    yt = xt.reshape(6, 4)
    yt.retain_grad()
    at = yt + yt * torch.tensor(c_np.astype(np.float64))
    at.retain_grad()
    (at.reshape(24) ** 2).sum().backward()
    gx, gy, ga = xt.grad.numpy(), yt.grad.numpy(), at.grad.numpy()
    assert_close(x.grad, gx, RTOL_F32, "x grad")
    assert_close(y1.grad, gy, RTOL_F32, "y grad")
    assert_close(a1.grad, ga, RTOL_F32, "a grad")
    # a second graph accumulates into x.grad; the first graph's intermediates keep theirs
    y2, a2, l2 = graph()
    l2.backward()
    assert_close(x.grad, 2 * gx, RTOL_F32, "x grad after two graphs")
    assert_close(y1.grad, gy, RTOL_F32, "first graph's y grad")
    assert_close(a1.grad, ga, RTOL_F32, "first graph's a grad")
    # editing one node's grad in place leaves its sharers alone
    y2.grad.mul_(0.0)
    assert_close(a2.grad, ga, RTOL_F32, "a grad after editing y grad")
    assert_close(x.grad, 2 * gx, RTOL_F32, "x grad after editing y grad")
    # x + x: both operands are the same tensor
    z = tg.Tensor(x_np)
    (z + z).reshape(24).sum().backward()
    assert_close(z.grad, np.full((4, 6), 2.0, np.float32), 0.0, "x + x")


@pytest.mark.parametrize("autocast", [False, True])
@pytest.mark.parametrize("bias,tied", [(True, False), (False, False), (False, True)])
def test_linear_fused_bias_and_transposed_weight(tg, autocast, bias, tied):
    """Linear runs as one GEMM with the bias in its epilogue; a weight tied as the
    transpose of another parameter is used without a transposing copy.  Values and
    gradients vs float64 torch of x @ w + b (autocast: fp16 operands, 1e-2)."""
    rng = np.random.default_rng(5)
    B, T, nin, nout = 2, 96, 128, 200
    x_np = rng.standard_normal((B, T, nin)).astype(np.float32)
    lin = tg.Linear(nin, nout, bias=bias)
    if bias:
        lin.b.data = tg.Tensor(rng.standard_normal(nout).astype(np.float32),
                               requires_grad=False).data
    src = None
    if tied:
        src = tg.Tensor(rng.standard_normal((nout, nin)).astype(np.float32) * 0.1)
        tg.weight_tie(src, lin, "w", transpose=True)
    w_np = lin.w.data.double().cpu().numpy()
    x = tg.Tensor(x_np)
    if autocast:
        with tg.autocast():
            y = lin(x)
            loss = (y * y).sum()
    else:
        y = lin(x)
        loss = (y * y).sum()
    loss.backward()
    xt = torch.tensor(x_np.astype(np.float64), requires_grad=True)
    wt = torch.tensor(w_np, requires_grad=True)
    yt = xt @ wt
    if bias:
        bt = torch.tensor(lin.b.data.double().cpu().numpy(), requires_grad=True)
        yt = yt + bt
    (yt * yt).sum().backward()
    tol = RTOL_F16 if autocast else RTOL_F32_MM
    assert_close(y.data.float(), yt.detach().numpy(), tol, "y")
    assert_close(x.grad.float(), xt.grad.numpy(), tol, "x grad")
    assert_close(lin.w.grad, wt.grad.numpy(), tol, "w grad")
    if bias:
        assert_close(lin.b.grad, bt.grad.numpy(), tol, "b grad")
    if tied:
        tg.sync_tied_gradients(lin)
        assert_close(src.grad, wt.grad.numpy().T, tol, "tied source grad")


def test_host_inputs_staged_copy(tg):
    """NumPy inputs reach the device through reusable pinned buffers and a non-blocking
    copy: every copy holds its own values although slots are reused, a later change to
    the source array does not leak in, and every dtype/shape round-trips."""
    from tensor_gpu_v2 import _lib as L
    rng = np.random.default_rng(5)
    outs, srcs = [], []
    for i in range(11):  # more copies than slots
        a = rng.integers(-1000, 1000, size=(3 + i, 17)).astype(np.int64)
        outs.append(L.to_device(a))
        srcs.append(a.copy())
        a[:] = 0  # the copy was taken at call time
    for o, a in zip(outs, srcs):
        assert o.is_cuda and np.array_equal(o.cpu().numpy(), a)
    for a in (np.float32(2.5), np.arange(7, dtype=np.float64), np.zeros((0, 3), np.float32),
              rng.standard_normal((4, 5)).astype(np.float16), np.array([True, False])):
        o = L.to_device(a)
        assert o.shape == np.asarray(a).shape and np.array_equal(o.cpu().numpy(), a)
    a = rng.standard_normal((6, 6))
    t = tg.Tensor(a)  # float64 data keeps its dtype (the reference's dtype policy)
    assert t.data.dtype == torch.float64 and t.data.is_cuda
    assert np.array_equal(t.data.cpu().numpy(), a)
    t32 = tg.Tensor(a, dtype=np.float32)  # cast on the device after the copy
    assert t32.data.dtype == torch.float32
    assert np.array_equal(t32.data.cpu().numpy(), a.astype(np.float32))


def test_scalar_tensor_is_zero_dim(tg):
    """Tensor(3.0) is 0-d, as cp.asarray(3.0) is in the reference (_core.py:625-655)."""
    t = tg.Tensor(3.0)
    assert tuple(t.shape) == () and float(t.item()) == 3.0
    assert tuple(tg.Tensor(np.array(2.0)).shape) == ()
