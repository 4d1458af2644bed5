"""The committed golden fixtures agree with the oracle and with torch float64
autograd (so a stale or corrupted fixture fails here, on the CPU)."""
import os

import numpy as np
import pytest
import torch

import oracle as O
from conftest import GOLDEN


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def chk(a, b, tol=1e-6):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape
    np.testing.assert_allclose(a, b, rtol=tol, atol=tol * max(1.0, float(np.abs(b).max())))


def test_act_fixture():
    f = load("act_bwd")
    x, dy = f["x"].astype(np.float64), f["dy"].astype(np.float64)
    chk(f["gelu"], O.gelu_bwd(x, dy))
    chk(f["silu"], O.silu_bwd(x, dy))
    xt = torch.tensor(x, requires_grad=True)
    torch.nn.functional.gelu(xt, approximate="tanh").backward(torch.tensor(dy))
    chk(f["gelu"], xt.grad.numpy())


def test_softmax_fixture():
    f = load("softmax")
    xt = torch.tensor(f["logits"].astype(np.float64), requires_grad=True)
    y = torch.softmax(xt, -1)
    chk(f["y"], y.detach().numpy())
    y32 = f["y"].astype(np.float32).astype(np.float64)
    chk(f["dx"], O.softmax_bwd(y32, f["dy"].astype(np.float64)))


def test_layernorm_fixture():
    f = load("layernorm")
    xt = torch.tensor(f["x"].astype(np.float64), requires_grad=True)
    gt = torch.tensor(f["gamma"].astype(np.float64), requires_grad=True)
    bt = torch.tensor(f["beta"].astype(np.float64), requires_grad=True)
    y = torch.nn.functional.layer_norm(xt, (1024,), gt, bt, 1e-5)
    y.backward(torch.tensor(f["dy"].astype(np.float64)))
    chk(f["y"], y.detach().numpy())
    chk(f["dx"], xt.grad.numpy(), 1e-5)
    chk(f["dgamma"], gt.grad.numpy())
    chk(f["dbeta"], bt.grad.numpy())


def test_bn_fixture():
    f = load("bn_relu_nhwc")
    x = f["x"].astype(np.float64).transpose(0, 3, 1, 2).copy()
    xt = torch.tensor(x, requires_grad=True)
    gt = torch.tensor(f["gamma"].astype(np.float64), requires_grad=True)
    bt = torch.tensor(f["beta"].astype(np.float64), requires_grad=True)
    y = torch.relu(torch.nn.functional.batch_norm(xt, None, None, gt, bt, True, 0.1, 1e-5))
    y.backward(torch.tensor(f["dy"].astype(np.float64).transpose(0, 3, 1, 2).copy()))
    chk(f["y"], y.detach().numpy().transpose(0, 2, 3, 1))
    chk(f["dx"], xt.grad.numpy().transpose(0, 2, 3, 1), 1e-5)
    chk(f["dgamma"], gt.grad.numpy())


def test_adamw_fixture():
    f = load("adamw3")
    p = torch.tensor(f["p0"].astype(np.float64), requires_grad=True)
    opt = torch.optim.AdamW([p], lr=3e-4, weight_decay=0.1)
    for g in f["g"]:
        p.grad = torch.tensor(g.astype(np.float64))
        opt.step()
    chk(f["p"], p.detach().numpy())


@pytest.mark.parametrize("tag,causal", [("full", False), ("causal", True)])
def test_flash_fixture(tag, causal):
    f = load("flash_attn")
    q, k, v, do = (torch.tensor(f[n].astype(np.float64), requires_grad=True) for n in "q k v do".split())
    s = q @ k.transpose(-1, -2) * 64 ** -0.5
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(96, 96, dtype=torch.bool), 1), float("-inf"))
    o = torch.softmax(s, -1) @ v
    o.backward(do.detach())
    chk(f[f"o_{tag}"], o.detach().numpy())
    chk(f[f"lse_{tag}"], torch.logsumexp(s, -1).detach().numpy())
    chk(f[f"dq_{tag}"], q.grad.numpy(), 1e-5)
    chk(f[f"dk_{tag}"], k.grad.numpy(), 1e-5)
    chk(f[f"dv_{tag}"], v.grad.numpy(), 1e-5)


def test_mlp_fixture_regenerates():
    f = load("mlp_c1")
    np.random.seed(0)
    x = np.random.randn(32, 784).astype(np.float32)
    w1 = np.random.randn(784, 256).astype(np.float32) * np.float32(np.sqrt(2.0 / 784))
    w2 = np.random.randn(256, 10).astype(np.float32) * np.float32(np.sqrt(2.0 / 256))
    r = O.mlp_step(x, w1, np.zeros(256, np.float32), w2, np.zeros(10, np.float32))
    assert abs(float(f["loss"]) - r["loss"]) < 1e-12
    chk(f["dw2"], r["dw2"])
    chk(f["dw1_sel"], r["dw1"].reshape(-1)[f["dw1_idx"]])
