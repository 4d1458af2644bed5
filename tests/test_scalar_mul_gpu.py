"""Tensor * Python scalar (the host-rounded fast path) against Tensor * a 0-d device
tensor holding the same scalar (the general broadcast path): values and gradients bit
for bit.  GPU only."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SCALARS = [0.5, 1.0 / 3.0, 1.0 / 8192, -2.5, 3, -1, 0.1, 1e-8, 70000.0, 1e40]


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("v", SCALARS)
def test_scalar_mul_equals_tensor_mul(cuda, tg, dt, v):
    g = torch.Generator().manual_seed(0)
    base = (torch.randn(37, 53, generator=g) * 3).to(dt).cuda()
    up = torch.randn(37, 53, generator=g).to(dt).cuda()

    def run(fast):
        x = tg.Tensor(base.clone())
        if fast:
            y = x * v
        else:
            s = torch.full((), float(v), dtype=torch.float64, device="cuda").to(dt)
            y = x * tg.Tensor(s, requires_grad=False)
        (y * tg.Tensor(up, requires_grad=False)).sum().backward()
        return y.data.clone(), x.grad.clone()

    y1, g1 = run(True)
    y0, g0 = run(False)
    assert y1.dtype == y0.dtype == dt
    assert torch.equal(y1.isnan(), y0.isnan())
    assert torch.equal(torch.nan_to_num(y1), torch.nan_to_num(y0))
    assert torch.equal(torch.nan_to_num(g1), torch.nan_to_num(g0))


def test_scalar_mul_variants(cuda, tg):
    """Reflected, negation and division by a scalar take the same path."""
    x = tg.Tensor(torch.arange(1, 7, dtype=torch.float32).cuda().reshape(2, 3))
    assert torch.equal((2.0 * x).data, (x * 2.0).data)
    assert torch.equal((-x).data, (x * -1.0).data)
    assert torch.equal((x / 4.0).data, (x * 0.25).data)
    m = x.mean()
    m.backward()
    assert torch.equal(x.grad, torch.full((2, 3), np.float32(1.0 / 6.0), device="cuda"))
