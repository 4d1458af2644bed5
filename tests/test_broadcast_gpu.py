"""tg_broadcast_mul_sum (strided broadcast multiply with reduction) and the closures
that run on it: __mul__ backward, sum/mean backward, the general _unbroadcast, strided
gradient copies.  Checked against the oracle's unbroadcast and float64 NumPy / torch
autograd.  GPU only.

Tolerance: fp32 rtol 1e-5 (elementwise and reduction gradients); fp16/bf16 outputs
1e-2; fp64 1e-12."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, RTOL_F32, assert_close

pytestmark = pytest.mark.gpu

RT = {torch.float32: RTOL_F32, torch.float16: RTOL_F16, torch.bfloat16: RTOL_F16,
      torch.float64: 1e-12}


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def rnd(shape, dt=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64).to(dt).cuda()


def f64(t):
    return t.detach().double().cpu().numpy()


# (grad shape, target shape): leading sums, keepdims sums, mixed, rows (summed axis
# innermost), columns (kept axis innermost), one workgroup per output (many summed
# elements, few outputs), and the reference's own case
UNB = [((2, 3, 4), (1, 3, 1)), ((7, 5, 3), (3,)), ((2, 3, 4), (3, 1)), ((4, 5, 6, 7), (1, 5, 1, 7)),
       ((512, 300), (512, 1)), ((300, 512), (1, 512)), ((64, 9000), (64, 1)),
       ((3, 1, 5), (1, 1, 5)), ((6, 4), (6, 4)), ((2, 3, 4, 5, 6), (3, 1, 5, 1)),
       ((1000, 70), (1,)), ((5, 2000), (1, 1))]


@pytest.mark.parametrize("gshape,tshape", UNB)
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.float64])
def test_unbroadcast_vs_oracle(cuda, gshape, tshape, dt):
    g = rnd(gshape, dt, 1)
    out = torch.empty(tshape, dtype=dt, device="cuda")
    L().broadcast_mul_sum(out, g)
    want = O.unbroadcast(f64(g), tshape)
    assert_close(out, want, RT[dt], f"unbroadcast {gshape}->{tshape}")


@pytest.mark.parametrize("gshape,tshape", UNB[:8])
def test_mul_sum_accumulate_alpha(cuda, gshape, tshape):
    """out = 3 * out + alpha * unbroadcast(a * b) with b broadcast from a smaller shape."""
    a = rnd(gshape, torch.float32, 2)
    bshape = tuple(1 if i % 2 else s for i, s in enumerate(gshape))
    b = rnd(bshape, torch.float16, 3)
    out = rnd(tshape, torch.float32, 4)
    o0 = f64(out)
    L().broadcast_mul_sum(out, a, b, alpha=-0.5, accumulate=True)
    want = o0 + -0.5 * O.unbroadcast(f64(a) * f64(b), tshape)
    assert_close(out, want, RTOL_F32, "accumulate")


@pytest.mark.parametrize("src_dt,dst_dt", [(torch.float32, torch.float16),
                                           (torch.float16, torch.float32),
                                           (torch.float32, torch.bfloat16),
                                           (torch.float64, torch.float32),
                                           (torch.float32, torch.float64)])
def test_strided_copy_and_cast(cuda, src_dt, dst_dt):
    x = rnd((3, 70, 5, 9), src_dt, 5)
    src = x.permute(2, 0, 3, 1)  # a permuted (dense, non-contiguous) view
    dst = torch.empty(src.shape, dtype=dst_dt, device="cuda")
    L().broadcast_mul_sum(dst, src)
    assert torch.equal(dst, src.to(dst_dt))  # one rounding, exactly torch's cast
    # into a strided destination (a head-merge relayout)
    dst2 = torch.empty(5, 9, 3, 70, dtype=dst_dt, device="cuda").permute(2, 3, 0, 1)
    src2 = x.transpose(1, 2).contiguous().transpose(1, 2)  # (3, 70, 5, 9), strided
    L().broadcast_mul_sum(dst2, src2)
    assert torch.equal(dst2, x.to(dst_dt))


def test_broadcast_fill_and_empty(cuda):
    out = torch.empty(4, 6, device="cuda")
    g = torch.tensor(2.5, device="cuda")
    L().broadcast_mul_sum(out, g, alpha=0.25)
    assert torch.equal(out, torch.full((4, 6), 0.625, device="cuda"))
    # an empty summed axis writes zeros, or leaves the output with accumulate
    e = torch.empty(3, 0, device="cuda")
    z = torch.full((3, 1), 7.0, device="cuda")
    L().broadcast_mul_sum(z, e)
    assert torch.equal(z, torch.zeros(3, 1, device="cuda"))
    z.fill_(7.0)
    L().broadcast_mul_sum(z, e, accumulate=True)
    assert torch.equal(z, torch.full((3, 1), 7.0, device="cuda"))


def test_out_overlap_rejected(cuda):
    with pytest.raises(ValueError):
        L().broadcast_mul_sum(torch.zeros(1, 5, device="cuda").expand(3, 5),
                              torch.ones(3, 5, device="cuda"))


# ------------------------------------------------------------------ Tensor API
@pytest.fixture
def tg(cuda):
    import tensor_gpu_v2
    return tensor_gpu_v2


PAIRS = [((2, 4, 5), (5,)), ((2, 4, 5), (1, 5)), ((3, 1, 5), (4, 1)), ((5,), (2, 3, 5)),
         ((2, 1, 3), (2, 4, 3)), ((4, 1), (1, 6)), ((6,), (6,)), ((2, 3, 4), (2, 1, 4))]


@pytest.mark.parametrize("ash,bsh", PAIRS)
@pytest.mark.parametrize("op", ["mul", "add"])
def test_binary_backward_broadcast(tg, ash, bsh, op):
    rng = np.random.default_rng(11)
    an, bn = (rng.standard_normal(s).astype(np.float32) for s in (ash, bsh))
    a, b = tg.Tensor(an), tg.Tensor(bn)
    y = a * b if op == "mul" else a + b
    dy = rng.standard_normal(y.shape).astype(np.float32)
    y.backward(dy)
    ta, tb = (torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (an, bn))
    ((ta * tb) if op == "mul" else (ta + tb)).backward(torch.tensor(dy, dtype=torch.float64))
    assert_close(a.grad, ta.grad, RTOL_F32, f"{op} da")
    assert_close(b.grad, tb.grad, RTOL_F32, f"{op} db")


@pytest.mark.parametrize("axis,keepdims", [(None, False), (None, True), (0, False), (1, True),
                                           ((0, 2), False), (-1, False), ((1, 2), True)])
@pytest.mark.parametrize("red", ["sum", "mean"])
def test_sum_mean_backward(tg, axis, keepdims, red):
    rng = np.random.default_rng(12)
    xn = rng.standard_normal((3, 40, 7)).astype(np.float32)
    x = tg.Tensor(xn)
    y = getattr(x, red)(axis=axis, keepdims=keepdims)
    dy = rng.standard_normal(y.shape).astype(np.float32)
    y.backward(dy)
    t = torch.tensor(xn, dtype=torch.float64, requires_grad=True)
    ty = getattr(t, red)(dim=axis, keepdim=keepdims) if axis is not None else getattr(t, red)()
    if keepdims and axis is None:
        ty = ty.reshape((1,) * 3)
    ty.backward(torch.tensor(dy, dtype=torch.float64).reshape(ty.shape))
    assert_close(x.grad, t.grad, RTOL_F32, f"{red} axis={axis}")


def test_mean_of_mul_accumulates_twice(tg):
    """x appears twice (x * x, then + x): the closures accumulate into one buffer."""
    xn = np.linspace(-2, 2, 24, dtype=np.float32).reshape(4, 6)
    x = tg.Tensor(xn)
    ((x * x) + x).mean().backward()
    assert_close(x.grad, (2 * xn.astype(np.float64) + 1) / 24, RTOL_F32, "d/dx mean(x^2 + x)")


def test_getitem_slices_and_ints(tg):
    xn = np.arange(60, dtype=np.float32).reshape(3, 4, 5)
    x = tg.Tensor(xn)
    (x[1:, ::2, 3] * 2.0).sum().backward()
    (x[0, 1] * 3.0).sum().backward()
    want = np.zeros((3, 4, 5))
    want[1:, ::2, 3] += 2.0
    want[0, 1] += 3.0
    assert_close(x.grad, want, RTOL_F32, "getitem")
