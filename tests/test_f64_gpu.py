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
