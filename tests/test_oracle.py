"""Pin the CPU oracle (oracle/ref_ops.py) against independent references:
torch float64 autograd, central finite differences, closed forms and the
reference test-suite's known answers.  CPU only."""
import math

import numpy as np
import pytest
import torch

import oracle as O

def tt(a, grad=True):
    return torch.tensor(a, dtype=torch.float64, requires_grad=grad)


def close(a, b, tol=1e-10):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    np.testing.assert_allclose(a, b, rtol=tol, atol=tol * max(1.0, float(np.abs(b).max(initial=0))))


# ------------------------------------------------------------------ activations
@pytest.mark.parametrize("kind", ["gelu", "silu"])
def test_activation_bwd_vs_finite_differences_and_torch(kind):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4000) * 3
    dy = rng.standard_normal(4000)
    fwd = O.gelu_fwd if kind == "gelu" else O.silu_fwd
    bwd = O.gelu_bwd if kind == "gelu" else O.silu_bwd
    h = 1e-6
    fd = (fwd(x + h) - fwd(x - h)) / (2 * h) * dy
    close(bwd(x, dy), fd, 1e-7)
    xt = tt(x)
    y = torch.nn.functional.gelu(xt, approximate="tanh") if kind == "gelu" else torch.nn.functional.silu(xt)
    y.backward(torch.tensor(dy))
    close(bwd(x, dy), xt.grad.numpy(), 1e-12)
    close(fwd(x), y.detach().numpy(), 1e-12)


def test_activation_special_values():
    # gelu'(0) = 0.5, silu'(0) = 0.5; far tails: gelu' -> 1 / 0, silu' -> 1 / 0
    close(O.gelu_bwd(np.array([0.0]), np.array([1.0])), [0.5])
    close(O.silu_bwd(np.array([0.0]), np.array([1.0])), [0.5])
    close(O.gelu_bwd(np.array([30.0, -30.0]), np.ones(2)), [1.0, 0.0], 1e-12)
    close(O.silu_bwd(np.array([40.0, -40.0]), np.ones(2)), [1.0, 0.0], 1e-12)


# ------------------------------------------------------------------ softmax
def test_softmax_vs_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 129)) * 2
    dy = rng.standard_normal((37, 129))
    xt = tt(x)
    y = torch.softmax(xt, -1)
    y.backward(torch.tensor(dy))
    yo = O.softmax_fwd(x)
    close(yo, y.detach().numpy())
    close(O.softmax_bwd(yo, dy), xt.grad.numpy())
    # invariant: rows of the backward sum to zero
    close(O.softmax_bwd(yo, dy).sum(-1), np.zeros(37), 1e-12)
    assert torch.get_default_dtype() == torch.float32


# ------------------------------------------------------------------ layer norm
def test_layernorm_vs_torch():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 5, 64))
    g = 1 + 0.02 * rng.standard_normal(64)
    b = 0.02 * rng.standard_normal(64)
    dy = rng.standard_normal((3, 5, 64))
    xt, gt, bt = tt(x), tt(g), tt(b)
    y = torch.nn.functional.layer_norm(xt, (64,), gt, bt, 1e-5)
    y.backward(torch.tensor(dy))
    yo, xh, mean, var = O.layernorm_fwd(x, g, b, 1e-5)
    close(yo, y.detach().numpy())
    dx, dg, db = O.layernorm_bwd(xh, var, g, dy, 1e-5)
    close(dx, xt.grad.numpy())
    close(dg, gt.grad.numpy())
    close(db, bt.grad.numpy())


# ------------------------------------------------------------------ batch norm
@pytest.mark.parametrize("relu", [True, False])
def test_batchnorm_relu_vs_torch(relu):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 6, 5, 3))  # NCHW
    g = 1 + 0.1 * rng.standard_normal(6)
    b = 0.1 * rng.standard_normal(6)
    dy = rng.standard_normal(x.shape)
    xt, gt, bt = tt(x), tt(g), tt(b)
    y = torch.nn.functional.batch_norm(xt, None, None, gt, bt, True, 0.1, 1e-5)
    if relu:
        y = torch.relu(y)
    y.backward(torch.tensor(dy))
    yo, cache = O.batchnorm_relu_fwd(x, g, b, 1e-5, relu)
    close(yo, y.detach().numpy())
    dx, dg, db = O.batchnorm_relu_bwd(dy, g, cache, relu)
    close(dx, xt.grad.numpy(), 1e-9)
    close(dg, gt.grad.numpy())
    close(db, bt.grad.numpy())


def test_batchnorm_eval_with_batch_stats_equals_training():
    """Pins batchnorm_eval_fwd's cache: with the running statistics set to the batch's
    own mean and (population) variance, the eval-mode forward and the reference's
    backward on that cache equal the training-mode ones, which torch pins above."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4, 5, 2)) * 2 + 0.5
    g = 1 + 0.1 * rng.standard_normal(4)
    b = 0.1 * rng.standard_normal(4)
    dy = rng.standard_normal(x.shape)
    yt, ct = O.batchnorm_relu_fwd(x, g, b, 1e-5, relu=False)
    ye, ce = O.batchnorm_eval_fwd(x, g, b, x.mean(axis=(0, 2, 3)), x.var(axis=(0, 2, 3)), 1e-5)
    close(ye, yt, 1e-12)
    for a, e in zip(O.batchnorm_relu_bwd(dy, g, ce, relu=False),
                    O.batchnorm_relu_bwd(dy, g, ct, relu=False)):
        close(a, e, 1e-12)
    # with other running statistics the dvar / dmean terms no longer vanish: dx differs
    # from the plain chain rule gamma * rstd * dy of the eval forward
    _, c2 = O.batchnorm_eval_fwd(x, g, b, np.zeros(4), np.ones(4), 1e-5)
    dx2, _, _ = O.batchnorm_relu_bwd(dy, g, c2, relu=False)
    plain = dy * (g / np.sqrt(1 + 1e-5)).reshape(1, 4, 1, 1)
    assert np.abs(dx2 - plain).max() > 1e-3


def test_batchnorm_nhwc_is_transposed_nchw():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 4, 8))  # NHWC, C = 8
    g = 1 + 0.1 * rng.standard_normal(8)
    b = 0.1 * rng.standard_normal(8)
    dy = rng.standard_normal(x.shape)
    y, cache = O.batchnorm_relu_fwd_nhwc(x, g, b)
    dx, dg, db = O.batchnorm_relu_bwd_nhwc(dy, g, cache)
    xt, gt, bt = tt(x.transpose(0, 3, 1, 2).copy()), tt(g), tt(b)
    yt = torch.relu(torch.nn.functional.batch_norm(xt, None, None, gt, bt, True, 0.1, 1e-5))
    yt.backward(torch.tensor(dy.transpose(0, 3, 1, 2).copy()))
    close(y, yt.detach().numpy().transpose(0, 2, 3, 1))
    close(dx, xt.grad.numpy().transpose(0, 2, 3, 1), 1e-9)
    close(dg, gt.grad.numpy())
    close(db, bt.grad.numpy())


# ------------------------------------------------------------------ matmul / unbroadcast
# The reference's own broadcast cases (test_autograd_regressions_phase6.py:86-95).
MATMUL_CASES = [((2, 4, 5), (5, 3)), ((2, 4, 5), (1, 5, 3)), ((3, 2, 4, 5), (5, 3)),
                ((5,), (5,)), ((5,), (5, 3)), ((2, 5), (5,)), ((2, 1, 5), (5,)),
                ((5,), (2, 5, 3))]


@pytest.mark.parametrize("ash,bsh", MATMUL_CASES)
def test_matmul_bwd_vs_torch(ash, bsh):
    rng = np.random.default_rng(123)
    a = rng.standard_normal(ash)
    b = rng.standard_normal(bsh)
    at, bt = tt(a), tt(b)
    y = at @ bt
    dy = rng.standard_normal(tuple(y.shape))
    y.backward(torch.tensor(dy))
    da, db = O.matmul_bwd(a, b, dy)
    assert da.shape == ash and db.shape == bsh
    close(da, at.grad.numpy())
    close(db, bt.grad.numpy())


def test_unbroadcast_known_answer_and_errors():
    # (_core.py:1380-1424) and the reference test test_autograd_regressions_phase6.py:446-478
    r = O.unbroadcast(np.ones((2, 3, 4)), (1, 3, 1))
    assert r.shape == (1, 3, 1) and np.allclose(r, 8.0)
    with pytest.raises(ValueError):
        O.unbroadcast(np.ones((2, 3)), (2, 3, 1))
    with pytest.raises(ValueError):
        O.unbroadcast(np.ones((2, 3)), (2, 4))
    with pytest.raises(ValueError):
        O.matmul_bwd(np.float64(1.0).reshape(()), np.ones(3), np.ones(3))


# ------------------------------------------------------------------ flash attention
def naive_attention(q, k, v, causal, scale):
    s = q @ k.transpose(-1, -2) * scale
    if causal:
        L, S = s.shape[-2], s.shape[-1]
        m = torch.triu(torch.ones(L, S, dtype=torch.bool), diagonal=1)
        s = s.masked_fill(m, float("-inf"))
    return torch.softmax(s, -1) @ v


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 3, 70, 16), (2, 50, 8)])
def test_flash_attention_vs_naive_torch(causal, shape):
    rng = np.random.default_rng(5)
    q = rng.standard_normal(shape)
    k = rng.standard_normal(shape)
    v = rng.standard_normal(shape)
    do = rng.standard_normal(shape)
    scale = shape[-1] ** -0.5
    qt, kt, vt = tt(q), tt(k), tt(v)
    o = naive_attention(qt, kt, vt, causal, scale)
    o.backward(torch.tensor(do))
    oo, lse = O.flash_attention_fwd(q, k, v, causal, scale, block_size=32)
    close(oo, o.detach().numpy())
    s = torch.tensor(q) @ torch.tensor(k).transpose(-1, -2) * scale
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(shape[-2], shape[-2], dtype=torch.bool), 1),
                          float("-inf"))
    close(lse, torch.logsumexp(s, -1).numpy())
    dq, dk, dv = O.flash_attention_bwd(q, k, v, do, causal, scale, block_size=32)
    close(dq, qt.grad.numpy(), 1e-9)
    close(dk, kt.grad.numpy(), 1e-9)
    close(dv, vt.grad.numpy(), 1e-9)
    # the rowsum(dO*O) form with the exact O gives the same gradients
    dq2, dk2, dv2 = O.flash_attention_bwd(q, k, v, do, causal, scale, block_size=32, o=oo)
    close(dq2, qt.grad.numpy(), 1e-9)
    close(dk2, kt.grad.numpy(), 1e-9)
    close(dv2, vt.grad.numpy(), 1e-9)


# ------------------------------------------------------------------ Adam
def test_adam_closed_form_t1_t2():
    # t=1: m = (1-b1) g, v = (1-b2) g^2, mhat = g, vhat = g^2 -> p -= lr*g/(|g|+eps)
    g = np.array([0.5, -2.0, 1e-3])
    p0 = np.array([1.0, 2.0, 3.0])
    lr, eps = 1e-2, 1e-8
    p1, m1, v1, _ = O.adam_step(p0, g, np.zeros(3), np.zeros(3), 1, lr=lr, eps=eps)
    close(p1, p0 - lr * g / (np.abs(g) + eps), 1e-14)
    close(m1, 0.1 * g, 1e-14)
    close(v1, 0.001 * g ** 2, 1e-14)
    # t=2 with the same g: m = 0.19 g, v = 0.001999 g^2; mhat = g, vhat = g^2
    p2, m2, v2, _ = O.adam_step(p1, g, m1, v1, 2, lr=lr, eps=eps)
    close(m2, 0.19 * g, 1e-14)
    close(v2, (0.999 * 0.001 + 0.001) * g ** 2, 1e-14)
    close(p2, p1 - lr * g / (np.abs(g) + eps), 1e-12)
    # decoupled decay acts before the moments: p*(1 - lr*wd)
    p3, _, _, _ = O.adam_step(p0, np.zeros(3), np.zeros(3), np.zeros(3), 1, lr=lr,
                              weight_decay=0.1)
    close(p3, p0 * (1 - lr * 0.1), 1e-14)


# ------------------------------------------------------------------ GradScaler / clipping
def test_clip_grad_norm_known_answers():
    # test_phase4_features.py:64-101: norm sqrt(9+16+144) = 13
    gs, n = O.clip_grad_norm([np.array([3.0, 4.0]), np.array([12.0, 0.0])], 1.0)
    assert abs(n - 13.0) < 1e-12
    close(gs[0], [3 / 13.000001, 4 / 13.000001], 1e-12)
    # inf norm 5 -> max becomes 2 (test_phase4_features.py:104-129)
    gs, n = O.clip_grad_norm([np.array([1.0, 2.0]), np.array([5.0, 3.0])], 2.0, float("inf"))
    assert n == 5.0 and abs(max(np.abs(g).max() for g in gs) - 2.0) < 1e-6
    # no grads -> 0.0; NaN entries are zeroed
    assert O.clip_grad_norm([None], 1.0)[1] == 0.0
    gs, n = O.clip_grad_norm([np.array([np.nan, 3.0, np.inf, 4.0])], 100.0)
    assert n == 5.0 and np.array_equal(gs[0], [0.0, 3.0, 0.0, 4.0])


def test_gradscaler_known_answers():
    # overflow halves the scale, counts it (test_phase4_features.py:193-234)
    s = O.GradScalerRef(init_scale=65536.0)
    out = s.unscale([np.full(3, np.inf), np.ones(2)])
    assert s.found_inf and np.array_equal(out[0], np.zeros(3))
    s.update()
    assert s.scale == 32768.0 and s.overflow_count == 1
    # growth after `growth_interval` clean steps (test_phase4_features.py:261-287)
    s = O.GradScalerRef(init_scale=1024.0, growth_interval=3)
    for _ in range(3):
        s.unscale([np.ones(4)])
        s.update()
    assert s.scale == 2048.0
    # min-scale clamp (test_phase4_features.py:853-870)
    s = O.GradScalerRef(init_scale=2.0, min_scale=1.0)
    for _ in range(3):
        s.found_inf = True
        s.update()
    assert s.scale == 1.0
    # unscale multiplies by 1/scale
    s = O.GradScalerRef(init_scale=4.0)
    assert np.array_equal(s.unscale([np.array([8.0, -4.0])])[0], [2.0, -1.0])
    with pytest.raises(ValueError):
        O.GradScalerRef(init_scale=0)
    with pytest.raises(ValueError):
        O.GradScalerRef(init_scale=4.0, max_scale=2.0)


# ------------------------------------------------------------------ losses / embedding
def test_cross_entropy_vs_torch():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((9, 13)) * 3
    y = rng.integers(0, 13, 9)
    xt = tt(x)
    loss = torch.nn.functional.cross_entropy(xt, torch.tensor(y))
    loss.backward()
    lo, probs = O.cross_entropy_fwd(x, y)
    p_t = torch.softmax(torch.tensor(x), -1)[torch.arange(9), torch.tensor(y)]
    assert abs(lo - (-torch.log(p_t + 1e-10)).mean().item()) < 1e-12
    assert abs(lo - loss.item()) < 1e-4  # differs from log-softmax only by the +1e-10
    close(O.cross_entropy_bwd(probs, y), xt.grad.numpy(), 1e-9)


def test_cross_entropy_label_smoothing_vs_torch():
    """With label smoothing s the reference's target weights (1 - s + s/C at the target,
    s/C elsewhere) are torch's; the losses differ only by the +1e-10 inside the log."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((7, 11)) * 2
    y = rng.integers(0, 11, 7)
    for red in ("mean", "sum"):
        xt = tt(x)
        loss = torch.nn.functional.cross_entropy(xt, torch.tensor(y), label_smoothing=0.2,
                                                 reduction=red)
        loss.backward()
        lo, probs = O.cross_entropy_fwd(x, y, 0.2, red)
        assert abs(lo - loss.item()) < 1e-6 * 11 * 7
        close(O.cross_entropy_bwd(probs, y, 0.2, red), xt.grad.numpy(), 1e-9)
    rows, _ = O.cross_entropy_fwd(x, y, 0.0, "none")
    assert rows.shape == (7,)
    close(rows.mean(), O.cross_entropy_fwd(x, y)[0], 1e-14)


def test_embedding_bwd_repeated_indices():
    idx = np.array([[0, 2, 2], [1, 2, 0]])
    d = np.arange(6 * 4, dtype=np.float64).reshape(2, 3, 4)
    g = O.embedding_bwd(idx, d, 5)
    want = np.zeros((5, 4))
    for i, r in zip(idx.reshape(-1), d.reshape(-1, 4)):
        want[i] += r
    assert np.array_equal(g, want)


# ------------------------------------------------------------------ C1 MLP
def test_mlp_step_vs_torch():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((32, 784))
    w1 = rng.standard_normal((784, 256)) * math.sqrt(2 / 784)
    w2 = rng.standard_normal((256, 10)) * math.sqrt(2 / 256)
    b1, b2 = np.zeros(256), np.zeros(10)
    r = O.mlp_step(x, w1, b1, w2, b2)
    ts = [tt(a) for a in (w1, b1, w2, b2)]
    out = torch.nn.functional.gelu(torch.tensor(x) @ ts[0] + ts[1], approximate="tanh") @ ts[2] + ts[3]
    loss = out.mean()
    loss.backward()
    assert abs(r["loss"] - loss.item()) < 1e-12
    for name, t in zip(("dw1", "db1", "dw2", "db2"), ts):
        close(r[name], t.grad.numpy())
    opt = torch.optim.Adam(ts, lr=1e-3)
    opt.step()
    for name, t in zip(("w1", "b1", "w2", "b2"), ts):
        close(r[name], t.detach().numpy(), 1e-9)


# ------------------------------------------------------------------ other pointwise ops
_UNARY = {
    # name: (torch forward, oracle backward taking (x, y, dy), domain)
    "relu": (torch.relu, lambda x, y, dy: O.relu_bwd(y, dy), "any"),
    "leaky_relu": (lambda t: torch.nn.functional.leaky_relu(t, 0.2),
                   lambda x, y, dy: O.leaky_relu_bwd(x, dy, 0.2), "any"),
    "swish": (lambda t: t * torch.sigmoid(1.7 * t), lambda x, y, dy: O.swish_bwd(x, dy, 1.7), "any"),
    "sigmoid": (torch.sigmoid, lambda x, y, dy: O.sigmoid_bwd(y, dy), "any"),
    "tanh": (torch.tanh, lambda x, y, dy: O.tanh_bwd(y, dy), "any"),
    "exp": (torch.exp, lambda x, y, dy: O.exp_bwd(y, dy), "any"),
    "log": (torch.log, lambda x, y, dy: O.log_bwd(x, dy), "pos"),
    "pow3": (lambda t: t ** 3, lambda x, y, dy: O.pow_bwd(x, dy, 3), "any"),
    "pow-1": (lambda t: t ** -1, lambda x, y, dy: O.pow_bwd(x, dy, -1), "pos"),
    "pow0.5": (lambda t: t ** 0.5, lambda x, y, dy: O.pow_bwd(x, dy, 0.5), "pos"),
    "pow2.7": (lambda t: t ** 2.7, lambda x, y, dy: O.pow_bwd(x, dy, 2.7), "pos"),
}


@pytest.mark.parametrize("name", sorted(_UNARY))
def test_unary_bwd_vs_torch_and_finite_differences(name):
    fwd, bwd, dom = _UNARY[name]
    rng = np.random.default_rng(7)
    x = rng.standard_normal(3000) * 2
    if dom == "pos":
        x = np.abs(x) + 0.1
    x[np.abs(x) < 1e-3] = 0.5  # keep finite differences away from the kinks
    dy = rng.standard_normal(3000)
    xt = tt(x)
    y = fwd(xt)
    y.backward(torch.tensor(dy))
    got = bwd(x, y.detach().numpy(), dy)
    close(got, xt.grad.numpy(), 1e-12)
    h = 1e-6
    with torch.no_grad():
        fd = (fwd(tt(x + h, False)) - fwd(tt(x - h, False))).numpy() / (2 * h) * dy
    close(got, fd, 1e-6)


def test_unary_bwd_kinks_and_quotient():
    # relu at 0: (out > 0) is False -> 0; leaky at 0: x >= 0 -> 1 (the reference's
    # choices at the kinks, which differ from torch's leaky_relu at exactly 0)
    close(O.relu_bwd(np.array([0.0, 2.0, -1.0]), np.ones(3)), [0.0, 1.0, 0.0])
    close(O.leaky_relu_bwd(np.array([0.0, -2.0]), np.ones(2), 0.1), [1.0, 0.1])
    # a / b = a * b ** -1: d/db = -a / b^2
    b = np.array([2.0, -4.0])
    close(O.pow_bwd(b, np.array([3.0, 3.0]), -1), [-0.75, -0.1875])


@pytest.mark.parametrize("axis", [-1, 0, 1])
def test_log_softmax_vs_torch(axis):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((13, 7, 33)) * 3
    dy = rng.standard_normal((13, 7, 33))
    xt = tt(x)
    y = torch.log_softmax(xt, axis)
    y.backward(torch.tensor(dy))
    yo = O.log_softmax_fwd(x, axis)
    close(yo, y.detach().numpy())
    close(O.log_softmax_bwd(yo, dy, axis), xt.grad.numpy())


@pytest.mark.parametrize("axis,keepdims", [(None, False), (0, False), (1, True), (-1, False),
                                           ((0, 2), False)])
def test_max_bwd_vs_torch_with_ties(axis, keepdims):
    rng = np.random.default_rng(9)
    x = rng.integers(0, 4, (6, 5, 7)).astype(np.float64)  # many ties
    xt = tt(x)
    r = torch.amax(xt) if axis is None else torch.amax(xt, dim=axis, keepdim=keepdims)
    dy = rng.standard_normal(tuple(r.shape))
    r.backward(torch.tensor(dy))
    close(O.max_bwd(x, dy, axis, keepdims), xt.grad.numpy())


def test_getitem_bwd_vs_torch_repeats_and_masks():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((9, 4))
    for idx in (np.array([3, 1, 3, 3, 0]), (np.array([0, 2, 2]), np.array([1, 3, 1])),
                x > 0.3, (slice(None), np.array([2, 2, 0]))):
        xt = tt(x)
        sel = xt[tuple(torch.as_tensor(i) if isinstance(i, np.ndarray) else i
                       for i in idx) if isinstance(idx, tuple) else torch.as_tensor(idx)]
        dy = rng.standard_normal(tuple(sel.shape))
        sel.backward(torch.tensor(dy))
        close(O.getitem_bwd(x.shape, idx, dy), xt.grad.numpy())
    # add.at with a repeated index: the closed form
    close(O.getitem_bwd((3,), np.array([1, 1, 1]), np.array([1.0, 2.0, 4.0])), [0, 7, 0])
