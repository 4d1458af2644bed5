"""Pointwise, log_softmax, max and advanced-index backward on libtgbwd (tg_unary_bwd,
tg_log_softmax_bwd, tg_max_bwd, tg_index_add_sorted) against the oracle, through the
C-ABI and through the Tensor closures that call it.  GPU only.

Tolerances: fp32 rtol 1e-5 against the float64 oracle, and bit-exact against the
reference formula evaluated in float32 by NumPy where NumPy's arithmetic is exact
IEEE (products, quotients, the exp/log/tanh results taken from the forward output,
x**2 and the other exact power forms); fp16/bf16 rtol 1e-2 / 3e-2; fp64 1e-12.
The advanced-index scatter-add is bit-exact against np.add.at in the tensor's dtype
(fp32 and fp16), whose one-by-one order it reproduces."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, RTOL_F32, assert_close

pytestmark = pytest.mark.gpu

RT = {torch.float32: RTOL_F32, torch.float16: RTOL_F16, torch.bfloat16: 3e-2,
      torch.float64: 1e-12}


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def f64(t):
    return t.detach().double().cpu().numpy()


# op: (torch forward on float64, kernel operand "x"/"y", param, oracle(x, y, dy), domain)
OPS = {
    "relu": (torch.relu, "y", 0.0, lambda x, y, g: O.relu_bwd(y, g), "any"),
    "leaky_relu": (lambda t: torch.where(t >= 0, t, 0.2 * t), "x", 0.2,
                   lambda x, y, g: O.leaky_relu_bwd(x, g, 0.2), "any"),
    "swish": (lambda t: t * torch.sigmoid(1.7 * t), "x", 1.7,
              lambda x, y, g: O.swish_bwd(x, g, 1.7), "any"),
    "sigmoid": (torch.sigmoid, "y", 0.0, lambda x, y, g: O.sigmoid_bwd(y, g), "any"),
    "tanh": (torch.tanh, "y", 0.0, lambda x, y, g: O.tanh_bwd(y, g), "any"),
    "exp": (torch.exp, "y", 0.0, lambda x, y, g: O.exp_bwd(y, g), "any"),
    "log": (torch.log, "x", 0.0, lambda x, y, g: O.log_bwd(x, g), "pos"),
    "pow": (None, "x", None, None, None),  # parametrised below
}
POWERS = [2.0, 3.0, 1.5, 0.5, -1.0, -0.5, 2.7, 0.0]


def _inputs(n, dom, dt, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(n, device="cuda", generator=g, dtype=torch.float64) * 2
    if dom == "pos":
        x = x.abs() + 0.1
    dy = torch.randn(n, device="cuda", generator=g, dtype=torch.float64)
    return x.to(dt), dy.to(dt)


def _cases():
    for op in OPS:
        if op == "pow":
            for p in POWERS:
                yield ("pow", p)
        else:
            yield (op, OPS[op][2])


@pytest.mark.parametrize("op,param", list(_cases()))
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("acc", [False, True])
def test_unary_bwd_kernel_vs_oracle(cuda, op, param, dt, acc):
    # 4099 elements: vector body plus a scalar tail; the offset-1 views make every
    # operand misaligned, which takes the scalar path for the whole array
    for n, off in ((4099, 0), (1001, 1)):
        dom = "pos" if op == "log" or (op == "pow" and param != int(param)) or param < 0 else "any"
        x, dy = _inputs(n + off, dom, dt, seed=n + int(10 * param))
        x, dy = x[off:], dy[off:]
        if op == "pow":
            y = x.double() ** param
            ref_fn = lambda xx, yy, g: O.pow_bwd(xx, g, param)  # noqa: E731
        else:
            y = OPS[op][0](x.double())
            ref_fn = OPS[op][3]
        y = y.to(dt)
        a = y if OPS[op][1] == "y" else x
        base = torch.randn(n + off, device="cuda", dtype=torch.float64).to(dt)[off:]
        dx = base.clone()
        L().unary_bwd(op, a, dy, dx, acc, param)
        want = ref_fn(f64(x), f64(y), f64(dy)) + (f64(base) if acc else 0.0)
        assert_close(dx, want, RT[dt], f"{op}({param}) {dt} acc={acc} n={n}")


# exact IEEE in NumPy float32 (no pow / exp evaluated inside the backward formula)
EXACT = [("relu", 0.0), ("leaky_relu", 0.2), ("sigmoid", 0.0), ("tanh", 0.0), ("exp", 0.0),
         ("log", 0.0), ("pow", 2.0), ("pow", 3.0), ("pow", 1.5), ("pow", 0.0)]


@pytest.mark.parametrize("op,param", EXACT)
def test_unary_bwd_fp32_bit_exact(cuda, op, param):
    """fp32: the reference closure's formula evaluated by NumPy in float32 (the
    reference's CPU arithmetic) equals the kernel bit for bit."""
    dom = "pos" if op in ("log", "pow") and param == 1.5 or op == "log" else "any"
    x, dy = _inputs(5000, dom, torch.float32, 3)
    if op == "pow":
        y = x ** param
    elif op == "leaky_relu":
        y = torch.where(x >= 0, x, 0.2 * x)
    else:
        y = getattr(torch, op)(x)
    a = y if OPS[op][1] == "y" else x
    dx = torch.empty_like(x)
    L().unary_bwd(op, a, dy, dx, False, param)
    xn, yn, gn = x.cpu().numpy(), y.cpu().numpy(), dy.cpu().numpy()
    one = np.float32(1)
    want = {
        "relu": lambda: (yn > 0).astype(np.float32) * gn,
        "leaky_relu": lambda: np.where(xn >= 0, one, np.float32(0.2)) * gn,
        "sigmoid": lambda: yn * (one - yn) * gn,
        "tanh": lambda: (one - yn ** 2) * gn,
        "exp": lambda: yn * gn,
        "log": lambda: gn / xn,
        "pow": lambda: (np.float32(param) * xn ** (param - 1)) * gn,
    }[op]()
    assert want.dtype == np.float32
    assert np.array_equal(dx.cpu().numpy(), want), op


@pytest.mark.parametrize("name", ["relu", "leaky_relu", "swish", "sigmoid", "tanh", "exp", "log",
                                  "pow", "div", "rdiv"])
def test_tensor_closures_on_kernels(cuda, tg, name):
    """The Tensor ops' backward (graph, accumulation into a used-twice input) against
    the oracle in float64 for fp32 data."""
    rng = np.random.default_rng(5)
    xv = (rng.standard_normal((64, 130)) * 2).astype(np.float32)
    if name in ("log", "pow", "div", "rdiv"):
        xv = np.abs(xv) + 0.1
    bv = (np.abs(rng.standard_normal((64, 130))) + 0.5).astype(np.float32)
    dy = rng.standard_normal((64, 130)).astype(np.float32)
    x = tg.Tensor(xv)
    b = tg.Tensor(bv)
    f = {
        "relu": lambda t: t.relu(), "leaky_relu": lambda t: t.leaky_relu(0.2),
        "swish": lambda t: t.swish(1.7), "sigmoid": lambda t: t.sigmoid(),
        "tanh": lambda t: t.tanh(), "exp": lambda t: t.exp(), "log": lambda t: t.log(),
        "pow": lambda t: t ** 2.5, "div": lambda t: t / b, "rdiv": lambda t: 3.0 / t,
    }[name]
    out = f(x) + x  # x used twice: the closure's result accumulates
    out.backward(dy)
    x64, b64, g64 = xv.astype(np.float64), bv.astype(np.float64), dy.astype(np.float64)
    local = {
        "relu": lambda: O.relu_bwd(np.maximum(x64, 0), g64),
        "leaky_relu": lambda: O.leaky_relu_bwd(x64, g64, 0.2),
        "swish": lambda: O.swish_bwd(x64, g64, 1.7),
        "sigmoid": lambda: O.sigmoid_bwd(1 / (1 + np.exp(-x64)), g64),
        "tanh": lambda: O.tanh_bwd(np.tanh(x64), g64),
        "exp": lambda: O.exp_bwd(np.exp(x64), g64),
        "log": lambda: O.log_bwd(x64, g64),
        "pow": lambda: O.pow_bwd(x64, g64, 2.5),
        "div": lambda: g64 / b64,
        "rdiv": lambda: O.pow_bwd(x64, 3.0 * g64, -1),
    }[name]()
    assert_close(x.grad, local + g64, RTOL_F32, name)
    if name == "div":  # d(x / b)/db = x * d(b**-1)/db
        assert_close(b.grad, O.pow_bwd(b64, x64 * g64, -1), RTOL_F32, "div db")


@pytest.mark.parametrize("shape,axis", [((5, 1000), -1), ((37, 1001), -1), ((3, 7, 33), 1),
                                        ((4, 6), 0)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.float64])
def test_log_softmax(cuda, tg, shape, axis, dt):
    rng = np.random.default_rng(6)
    xv = rng.standard_normal(shape) * 3
    dy = rng.standard_normal(shape)
    x = tg.Tensor(torch.as_tensor(xv).to(dt).cuda())
    y = x.log_softmax(axis)
    y.backward(torch.as_tensor(dy).to(dt).cuda())
    want = O.log_softmax_bwd(f64(y.data), f64(torch.as_tensor(dy).to(dt)), axis)
    assert_close(x.grad, want, RT[dt], f"log_softmax {shape} axis {axis}")
    # kernel accumulate mode (last axis)
    if axis in (-1, len(shape) - 1):
        yy = y.data.contiguous()
        g = torch.as_tensor(dy).to(dt).cuda()
        dx = torch.ones_like(yy)
        L().log_softmax_bwd(yy, g, dx, True)
        assert_close(dx, want + 1.0, RT[dt], "accumulate")


@pytest.mark.parametrize("axis,keepdims", [(None, False), (0, False), (1, True), (-1, False),
                                           ((0, 2), False), ((1, 2), True)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_max_min_bwd_with_ties(cuda, tg, axis, keepdims, dt):
    rng = np.random.default_rng(7)
    xv = rng.integers(0, 5, (6, 50, 7)).astype(np.float32)  # many ties
    x = tg.Tensor(torch.as_tensor(xv).to(dt).cuda())
    r = x.max(axis=axis, keepdims=keepdims)
    dy = rng.standard_normal(tuple(r.data.shape))
    r.backward(torch.as_tensor(dy).to(dt).cuda())
    gd = f64(torch.as_tensor(dy).to(dt))
    assert_close(x.grad, O.max_bwd(xv.astype(np.float64), gd, axis, keepdims), RT[dt], "max")
    x2 = tg.Tensor(torch.as_tensor(xv).to(dt).cuda())
    m = x2.min(axis=axis, keepdims=keepdims)
    m.backward(torch.as_tensor(dy).to(dt).cuda())
    want = O.max_bwd(-xv.astype(np.float64), -gd, axis, keepdims) * -1
    assert_close(x2.grad, want, RT[dt], "min")


@pytest.mark.parametrize("dt,npdt", [(torch.float32, np.float32), (torch.float16, np.float16)])
def test_getitem_scatter_add_bit_exact(cuda, tg, dt, npdt):
    """Integer arrays with repeated indices, two index arrays, a boolean mask and a
    slice mixed with an array: the gradient equals zeros + np.add.at(..., g) in the
    tensor's dtype bit for bit, and adds onto an existing gradient."""
    rng = np.random.default_rng(8)
    xv = rng.standard_normal((300, 17)).astype(npdt)
    rep = rng.integers(0, 300, 5000)
    cases = [rep, (rng.integers(0, 300, 900), rng.integers(0, 17, 900)), xv > 0.5,
             (slice(10, 200), rng.integers(0, 17, 40)), np.array([7, 7, 7, 7])]
    for idx in cases:
        x = tg.Tensor(torch.as_tensor(xv).to(dt).cuda())
        sel = x[idx]
        g = rng.standard_normal(tuple(sel.data.shape)).astype(npdt)
        sel.backward(g)
        want = np.zeros(xv.shape, npdt)
        np.add.at(want, idx, g)
        got = x.grad.cpu().numpy()
        assert got.dtype == npdt
        assert np.array_equal(got, want), f"index {type(idx)}"
    # accumulation: a second selection adds onto the first gradient
    # (200 selected rows keep every fp16 sum in the backward finite)
    x = tg.Tensor(torch.as_tensor(xv).to(dt).cuda())
    (x[rep[:200]] * 2.0 + x[np.array([1, 1])].sum() * 0.0).sum().backward()
    want = np.zeros(xv.shape, np.float64)
    np.add.at(want, rep[:200], 2.0)
    assert_close(x.grad, want, RT[dt], "accumulated getitem")


def test_index_add_sorted_validates(cuda):
    g = torch.zeros(10, device="cuda")
    t = torch.zeros(2, dtype=torch.int64, device="cuda")
    with pytest.raises(ValueError, match="inconsistent"):
        L().index_add_sorted(g, t, torch.zeros(2, dtype=torch.int64, device="cuda"),
                             torch.zeros(3, dtype=torch.int64, device="cuda"),
                             torch.zeros(3, device="cuda"))
