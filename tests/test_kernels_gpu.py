"""Parity of every libtgbwd kernel with the oracle on seeded inputs, through the
C-ABI (the _lib wrappers pass raw pointers to libtgbwd.so).  GPU only."""
import os

import numpy as np
import pytest
import torch

import oracle as O
from conftest import GOLDEN, RTOL_F16, RTOL_F32, RTOL_F32_MM, assert_close

pytestmark = pytest.mark.gpu

F16S = [torch.float16, torch.bfloat16]


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def dev(a, dtype=torch.float32):
    return torch.as_tensor(np.ascontiguousarray(a)).to(device="cuda", dtype=dtype)


def f64(t):
    return t.detach().double().cpu().numpy()


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def misaligned(t):
    """Same values, contiguous, but the data pointer is 4 bytes off 16-byte alignment."""
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    v = buf[1:1 + t.numel()].view(t.shape)
    v.copy_(t)
    return v


# ------------------------------------------------------------------ activations
@pytest.mark.parametrize("kind", ["gelu", "silu"])
@pytest.mark.parametrize("n", [0, 1, 7, 4096 * 4 + 3, 1 << 20])
@pytest.mark.parametrize("acc", [False, True])
def test_act_bwd_fp32(cuda, kind, n, acc):
    rng = np.random.default_rng(n + 11)
    x = rng.standard_normal(n) * 3
    dy = rng.standard_normal(n)
    base = rng.standard_normal(n)
    xt, dyt = dev(x), dev(dy)
    dx = dev(base) if acc else torch.full((n,), float("nan"), device="cuda")
    L().act_bwd(kind, xt, dyt, dx, acc)
    ref = (O.gelu_bwd if kind == "gelu" else O.silu_bwd)(f64(xt), f64(dyt))
    if acc:
        ref = ref + f64(dev(base))
    assert_close(dx, ref, RTOL_F32, f"{kind} n={n}")


@pytest.mark.parametrize("kind", ["gelu", "silu"])
@pytest.mark.parametrize("dt", F16S)
def test_act_bwd_half(cuda, kind, dt):
    rng = np.random.default_rng(3)
    x = dev(rng.standard_normal(10007) * 3, dt)
    dy = dev(rng.standard_normal(10007), dt)
    dx = torch.empty_like(x)
    L().act_bwd(kind, x, dy, dx, False)
    ref = (O.gelu_bwd if kind == "gelu" else O.silu_bwd)(f64(x), f64(dy))
    assert_close(dx, ref, RTOL_F16, f"{kind} {dt}")


def test_act_bwd_misaligned_and_golden(cuda):
    f = golden("act_bwd")
    x, dy = misaligned(dev(f["x"])), misaligned(dev(f["dy"]))
    for kind in ("gelu", "silu"):
        dx = misaligned(torch.zeros(x.numel(), device="cuda"))
        L().act_bwd(kind, x, dy, dx, False)
        assert_close(dx, f[kind], RTOL_F32, f"golden {kind}")


@pytest.mark.parametrize("kind", ["gelu", "silu"])
def test_act_fwd(cuda, kind):
    x = dev(np.random.default_rng(0).standard_normal(5003) * 4)
    y = L().act_fwd(kind, x)
    ref = (O.gelu_fwd if kind == "gelu" else O.silu_fwd)(f64(x))
    assert_close(y, ref, RTOL_F32, kind)


# ------------------------------------------------------------------ softmax
SOFTMAX_SHAPES = [(1, 1), (3, 10), (64, 4096), (7, 1000), (5, 12288), (2, 40000), (130, 64)]


@pytest.mark.parametrize("shape", SOFTMAX_SHAPES)
@pytest.mark.parametrize("acc", [False, True])
def test_softmax_fp32(cuda, shape, acc):
    rng = np.random.default_rng(sum(shape))
    lg = dev(rng.standard_normal(shape) * 2)
    y = L().softmax_fwd(lg)
    assert_close(y, O.softmax_fwd(f64(lg)), RTOL_F32, f"softmax fwd {shape}")
    dy = dev(rng.standard_normal(shape))
    base = dev(rng.standard_normal(shape))
    dx = base.clone() if acc else torch.empty_like(y)
    L().softmax_bwd(y, dy, dx, acc)
    ref = O.softmax_bwd(f64(y), f64(dy)) + (f64(base) if acc else 0)
    assert_close(dx, ref, RTOL_F32, f"softmax bwd {shape}")


@pytest.mark.parametrize("dt", F16S)
def test_softmax_half(cuda, dt):
    rng = np.random.default_rng(9)
    lg = dev(rng.standard_normal((33, 2048)) * 2, dt)
    y = L().softmax_fwd(lg)
    assert_close(y, O.softmax_fwd(f64(lg)), RTOL_F16, "softmax fwd half")
    dy = dev(rng.standard_normal((33, 2048)), dt)
    dx = torch.empty_like(y)
    L().softmax_bwd(y, dy, dx, False)
    assert_close(dx, O.softmax_bwd(f64(y), f64(dy)), RTOL_F16, "softmax bwd half")


def test_softmax_golden(cuda):
    f = golden("softmax")
    y = L().softmax_fwd(dev(f["logits"]))
    assert_close(y, f["y"], RTOL_F32, "golden softmax fwd")
    dx = torch.empty_like(y)
    L().softmax_bwd(dev(f["y"]), dev(f["dy"]), dx, False)
    assert_close(dx, f["dx"], RTOL_F32, "golden softmax bwd")


# ------------------------------------------------------------------ layer norm
LN_SHAPES = [(1, 8), (37, 1024), (8, 4096), (3, 100), (2, 20000), (300, 256), (5, 8192),
             # several rows per block (one block per CU): odd and even iteration counts,
             # a partial last round, both prefetch depths
             (773, 4096), (2309, 512), (2048, 1024)]


def ln_ref(x, g, b, dy, eps=1e-5):
    y, xh, mean, var = O.layernorm_fwd(x, g, b, eps)
    dx, dg, db = O.layernorm_bwd(xh, var, g, dy, eps)
    return y, dx, dg, db


@pytest.mark.parametrize("shape", LN_SHAPES)
@pytest.mark.parametrize("acc", [False, True])
def test_layernorm_fp32(cuda, shape, acc):
    rows, cols = shape
    rng = np.random.default_rng(rows * 7 + cols)
    x = dev(rng.standard_normal(shape))
    g = dev(1 + 0.02 * rng.standard_normal(cols))
    b = dev(0.02 * rng.standard_normal(cols))
    dy = dev(rng.standard_normal(shape))
    y, mean, rstd = L().layernorm_fwd(x, g, b, 1e-5)
    yr, dxr, dgr, dbr = ln_ref(f64(x), f64(g), f64(b), f64(dy))
    assert_close(y, yr, RTOL_F32, f"ln fwd {shape}")
    bx, bg, bb = dev(rng.standard_normal(shape)), dev(rng.standard_normal(cols)), dev(rng.standard_normal(cols))
    dx = bx.clone() if acc else torch.empty_like(x)
    dg = bg.clone() if acc else torch.empty_like(g)
    db = bb.clone() if acc else torch.empty_like(b)
    L().layernorm_bwd(x, mean, rstd, g, dy, dx, dg, db, acc, acc)
    a = 1.0 if acc else 0.0
    assert_close(dx, dxr + a * f64(bx), RTOL_F32, f"ln dx {shape}")
    assert_close(dg, dgr + a * f64(bg), RTOL_F32, f"ln dgamma {shape}")
    assert_close(db, dbr + a * f64(bb), RTOL_F32, f"ln dbeta {shape}")


@pytest.mark.parametrize("dt", F16S)
@pytest.mark.parametrize("rows,cols,acc", [(64, 1024, False), (2309, 1024, True), (8192, 1024, True),
                                           (1029, 4096, True), (600, 8192, False)])
def test_layernorm_half(cuda, dt, rows, cols, acc):
    rng = np.random.default_rng(4 + rows)
    x = dev(rng.standard_normal((rows, cols)), dt)
    g = dev(1 + 0.02 * rng.standard_normal(cols))
    b = dev(0.02 * rng.standard_normal(cols))
    dy = dev(rng.standard_normal((rows, cols)), dt)
    y, mean, rstd = L().layernorm_fwd(x, g, b, 1e-5)
    yr, dxr, dgr, dbr = ln_ref(f64(x), f64(g), f64(b), f64(dy))
    assert_close(y, yr, RTOL_F16, "ln fwd half")
    bx = dev(rng.standard_normal((rows, cols)), dt)
    dx = bx.clone() if acc else torch.empty_like(x)
    dg, db = torch.empty_like(g), torch.empty_like(b)
    L().layernorm_bwd(x, mean, rstd, g, dy, dx, dg, db, acc, False)
    a = 1.0 if acc else 0.0
    assert_close(dx, dxr + a * f64(bx), RTOL_F16, "ln dx half")
    assert_close(dg, dgr, RTOL_F16, "ln dgamma half")
    assert_close(db, dbr, RTOL_F16, "ln dbeta half")


def test_layernorm_golden(cuda):
    f = golden("layernorm")
    x, g, b, dy = (dev(f[k]) for k in ("x", "gamma", "beta", "dy"))
    y, mean, rstd = L().layernorm_fwd(x, g, b, 1e-5)
    assert_close(y, f["y"], RTOL_F32, "golden ln y")
    assert_close(mean, f["mean"], RTOL_F32, "golden ln mean")
    assert_close(rstd, f["rstd"], RTOL_F32, "golden ln rstd")
    dx, dg, db = torch.empty_like(x), torch.empty_like(g), torch.empty_like(b)
    L().layernorm_bwd(x, mean, rstd, g, dy, dx, dg, db, False, False)
    assert_close(dx, f["dx"], RTOL_F32, "golden ln dx")
    assert_close(dg, f["dgamma"], RTOL_F32, "golden ln dgamma")
    assert_close(db, f["dbeta"], RTOL_F32, "golden ln dbeta")


# ------------------------------------------------------------------ batch norm
BN_CASES = [("NHWC", (4, 7, 9, 64)), ("NHWC", (2, 5, 5, 6)), ("NHWC", (3, 4, 4, 300)),
            ("NCHW", (4, 64, 7, 9)), ("NCHW", (3, 5, 4, 4)), ("NCHW", (2, 8, 3, 5))]


def bn_inputs(layout, shape, seed):
    rng = np.random.default_rng(seed)
    C = shape[3] if layout == "NHWC" else shape[1]
    x = dev(rng.standard_normal(shape))
    g = dev(1 + 0.1 * rng.standard_normal(C))
    b = dev(0.1 * rng.standard_normal(C))
    dy = dev(rng.standard_normal(shape))
    return x, g, b, dy, C


@pytest.mark.parametrize("layout,shape", BN_CASES)
@pytest.mark.parametrize("relu", [True, False])
def test_batchnorm(cuda, layout, shape, relu):
    x, g, b, dy, C = bn_inputs(layout, shape, sum(shape))
    lay = L().NHWC if layout == "NHWC" else L().NCHW
    rm, rv = torch.zeros(C, device="cuda"), torch.ones(C, device="cuda")
    y, mean, rstd, var = L().batchnorm_fwd_train(x, g, b, 1e-5, 0.1, rm, rv, relu, lay)
    if layout == "NHWC":
        yr, cache = O.batchnorm_relu_fwd_nhwc(f64(x), f64(g), f64(b), 1e-5, relu)
    else:
        yr, cache = O.batchnorm_relu_fwd(f64(x), f64(g), f64(b), 1e-5, relu)
    assert_close(y, yr, RTOL_F32, "bn y")
    assert_close(mean, cache[5], RTOL_F32, "bn mean")
    assert_close(var, cache[6], RTOL_F32, "bn var")
    assert_close(rm, 0.1 * cache[5], RTOL_F32, "running mean")
    assert_close(rv, 0.9 + 0.1 * cache[6], RTOL_F32, "running var")
    # backward with the oracle's own statistics (float32) so both sides apply the
    # same ReLU mask; the reference mask is out > 0 on the fp32 forward output
    mean32 = dev(cache[5])
    rstd32 = dev(1.0 / np.sqrt(cache[6] + 1e-5))
    dx, dg, db = torch.empty_like(x), torch.empty_like(g), torch.empty_like(b)
    L().batchnorm_bwd(x, mean32, rstd32, g, b, dy, dx, dg, db, relu, False, False, lay)
    if layout == "NHWC":
        dxr, dgr, dbr = O.batchnorm_relu_bwd_nhwc(f64(dy), f64(g), cache, relu)
    else:
        dxr, dgr, dbr = O.batchnorm_relu_bwd(f64(dy), f64(g), cache, relu)
    assert_close(dx, dxr, RTOL_F32, "bn dx")
    assert_close(dg, dgr, RTOL_F32, "bn dgamma")
    assert_close(db, dbr, RTOL_F32, "bn dbeta")


def test_batchnorm_accumulate_and_golden(cuda):
    f = golden("bn_relu_nhwc")
    x, g, b, dy = (dev(f[k]) for k in ("x", "gamma", "beta", "dy"))
    rm, rv = torch.zeros(36, device="cuda"), torch.ones(36, device="cuda")
    y, mean, rstd, _ = L().batchnorm_fwd_train(x, g, b, 1e-5, 0.1, rm, rv, True, L().NHWC)
    assert_close(y, f["y"], RTOL_F32, "golden bn y")
    dx, dg, db = torch.ones_like(x), torch.ones_like(g), torch.ones_like(b)
    L().batchnorm_bwd(x, mean, rstd, g, b, dy, dx, dg, db, True, True, True, L().NHWC)
    assert_close(dx, f["dx"] + 1.0, RTOL_F32, "golden bn dx (+1)")
    assert_close(dg, f["dgamma"] + 1.0, RTOL_F32, "golden bn dgamma (+1)")
    assert_close(db, f["dbeta"] + 1.0, RTOL_F32, "golden bn dbeta (+1)")


# ------------------------------------------------------------------ column sums
@pytest.mark.parametrize("rows,cols", [(1, 1), (32, 10), (8192, 1024), (1000, 4097), (3, 40000),
                                       (64, 8192), (8, 4098), (65, 4096), (8192, 4096),
                                       (777, 1000), (40, 24)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_reduce_rows(cuda, rows, cols, dt):
    rng = np.random.default_rng(rows + cols)
    g = dev(rng.standard_normal((rows, cols)), dt)
    out = dev(rng.standard_normal(cols))
    base = f64(out)
    L().reduce_rows(g, out, True)
    tol = RTOL_F32 if dt == torch.float32 else 1e-4
    assert_close(out, base + f64(g).sum(0), tol, "reduce_rows acc")
    L().reduce_rows(g, out, False)
    assert_close(out, f64(g).sum(0), tol, "reduce_rows")


# ------------------------------------------------------------------ GEMM
GEMM_SHAPES = [(256, 256, 256), (100, 70, 50), (32, 256, 784), (130, 10, 256), (1, 1, 1),
               (257, 129, 33), (64, 64, 0), (384, 640, 96), (1000, 136, 48), (512, 128, 1024),
               # DMA-staged path (K % 64 == 0) with partial 128-row/column tiles
               (200, 136, 128), (72, 520, 192), (1000, 1000, 64), (136, 64, 256)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_gemm(cuda, M, N, K, ta, tb, dt):
    rng = np.random.default_rng(M * 3 + N * 5 + K)
    a = dev(rng.standard_normal((K, M) if ta else (M, K)), dt)
    b = dev(rng.standard_normal((N, K) if tb else (K, N)), dt)
    c0 = dev(rng.standard_normal((M, N)))
    c = c0.clone()
    L().gemm(a, b, c, ta, tb, 0.5, 2.0, M, N, K, a.shape[1], b.shape[1], N)
    A = f64(a).T if ta else f64(a)
    B = f64(b).T if tb else f64(b)
    ref = 0.5 * (A @ B) + 2.0 * f64(c0)
    # products of dt-rounded inputs are exact in fp32 accumulation up to the sum order
    assert_close(c, ref, RTOL_F32_MM, f"gemm {dt} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_large_tiles(cuda, ta, tb):
    """Shape with >= one 256x128 tile per CU (the 8-wave block) and partial edge tiles;
    reference: torch float64 matmul of the same fp16 inputs."""
    M, N, K = 4104, 2056, 128
    g = torch.Generator(device="cuda").manual_seed(7)
    a = torch.randn((K, M) if ta else (M, K), device="cuda", generator=g).half()
    b = torch.randn((N, K) if tb else (K, N), device="cuda", generator=g).half()
    c = torch.empty(M, N, device="cuda")
    L().gemm(a, b, c, ta, tb, 1.0, 0.0, M, N, K, a.shape[1], b.shape[1], N)
    ref = (a.double().T if ta else a.double()) @ (b.double().T if tb else b.double())
    err = float((c.double() - ref).abs().max())
    assert err <= RTOL_F32_MM * float(ref.abs().max()), f"max error {err}"


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("odt,beta", [(torch.float32, 0.0), (torch.float16, 0.0),
                                      (torch.float32, 1.0), (torch.float16, 1.0)])
def test_gemm_huge_tiles(cuda, ta, tb, odt, beta):
    """Enough 256x256 tiles for the one-wave-per-SIMD block, with partial edge tiles
    (per-element epilogue) and full interior tiles (LDS-staged epilogue, beta read);
    reference: torch float64 matmul of the same fp16 inputs."""
    M, N, K = 4104, 4104, 192
    g = torch.Generator(device="cuda").manual_seed(11)
    a = torch.randn((K, M) if ta else (M, K), device="cuda", generator=g).half()
    b = torch.randn((N, K) if tb else (K, N), device="cuda", generator=g).half()
    c0 = torch.randn(M, N, device="cuda", generator=g).to(odt)
    c = c0.clone()
    L().gemm(a, b, c, ta, tb, 1.0, beta, M, N, K, a.shape[1], b.shape[1], N)
    ref = (a.double().T if ta else a.double()) @ (b.double().T if tb else b.double())
    ref = ref + beta * c0.double()
    tol = RTOL_F32_MM if odt == torch.float32 else 2.0 ** -10
    err = float((c.double() - ref).abs().max())
    assert err <= tol * float(ref.abs().max()), f"max error {err}"


@pytest.mark.parametrize("M,N,K,tb", [(8, 24, 40, False), (200, 136, 72, True),
                                      (1000, 1000, 64, False), (4104, 2056, 128, True),
                                      (4104, 4104, 128, False)])
@pytest.mark.parametrize("dt,odt", [(torch.float16, torch.float16), (torch.float16, torch.float32),
                                    (torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32)])
def test_gemm_bias(cuda, M, N, K, tb, dt, odt):
    """tg_gemm_bias = A @ op(B) + bias[n] with the bias added before the output
    rounding, on every kernel path (scalar, register-staged, DMA-staged 128/256 with
    edge tiles); reference: float64 of the same rounded inputs."""
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    a = torch.randn(M, K, device="cuda", generator=g).to(dt)
    b = torch.randn((N, K) if tb else (K, N), device="cuda", generator=g).to(dt)
    bias = torch.randn(N, device="cuda", generator=g)
    out = torch.empty(M, N, device="cuda", dtype=odt)
    L().gemm_bias(a, b, bias, out, trans_b=tb)
    ref = a.double() @ (b.double().T if tb else b.double()) + bias.double()
    tol = RTOL_F32_MM if odt == torch.float32 else (2.0 ** -10 if odt == torch.float16 else 2.0 ** -7)
    err = float((out.double() - ref).abs().max())
    assert err <= tol * float(ref.abs().max()), f"max error {err}"


def test_gemm_batched_broadcast_and_half_out(cuda):
    rng = np.random.default_rng(1)
    a = dev(rng.standard_normal((3, 40, 24)), torch.float16)
    b = dev(rng.standard_normal((24, 56)), torch.float16)
    c = torch.empty(3, 40, 56, dtype=torch.float16, device="cuda")
    L().gemm(a, b, c, False, False, 1.0, 0.0, 40, 56, 24, 24, 56, 56, 40 * 24, 0, 40 * 56, 3)
    assert_close(c, f64(a) @ f64(b), RTOL_F16, "batched gemm, B broadcast")


# ------------------------------------------------------------------ Adam / AdamW
@pytest.mark.parametrize("amsgrad", [False, True])
def test_adam_multi_tensor(cuda, amsgrad):
    rng = np.random.default_rng(2)
    sizes = [1, 3, 4096, 10007, 0, 65, 25 * 4096]
    ps = [dev(rng.standard_normal(n)) for n in sizes]
    ms = [torch.zeros_like(p) for p in ps]
    vs = [torch.zeros_like(p) for p in ps]
    vms = [torch.zeros_like(p) for p in ps] if amsgrad else None
    ref = [(f64(p), np.zeros(p.numel()), np.zeros(p.numel()), np.zeros(p.numel())) for p in ps]
    for t in range(1, 4):
        gs = [dev(rng.standard_normal(n) * 1e-2) for n in sizes]
        L().adam_step(ps, gs, ms, vs, vms, 3e-4, 0.9, 0.999, 1e-8, 0.1, 1 - 0.9 ** t, 1 - 0.999 ** t)
        ref = [O.adam_step(p, f64(g), m, v, t, lr=3e-4, weight_decay=0.1, amsgrad=amsgrad,
                           v_max=vm)
               for (p, m, v, vm), g in zip(ref, gs)]
    for p, m, v, r in zip(ps, ms, vs, ref):
        assert_close(p, r[0], RTOL_F32, "adam p")
        assert_close(m, r[1], RTOL_F32, "adam m")
        assert_close(v, r[2], RTOL_F32, "adam v")


def test_adamw_golden(cuda):
    f = golden("adamw3")
    p = dev(f["p0"])
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    for t, g in enumerate(f["g"], start=1):
        L().adam_step([p], [dev(g)], [m], [v], None, 3e-4, 0.9, 0.999, 1e-8, 0.1,
                      1 - 0.9 ** t, 1 - 0.999 ** t)
    assert_close(p, f["p"], RTOL_F32, "golden adamw p")
    assert_close(m, f["m"], RTOL_F32, "golden adamw m")


# ------------------------------------------------------------------ GradScaler kernels
def test_unscale_check_bit_exact(cuda):
    rng = np.random.default_rng(5)
    host = [rng.standard_normal(n).astype(np.float32) * 1e3 for n in (1000, 5000, 7, 40000)]
    host[1][17] = np.inf
    host[3][39999] = np.nan
    gs = [dev(h) for h in host]
    inv = np.float32(1.0 / 65536.0)
    flags = L().unscale_check(gs, float(inv))
    assert flags == [0, 3, 0, 3]
    for g, h in zip(gs, host):
        want = h * inv  # fp32 multiply, as the kernel
        got = g.cpu().numpy()
        fin = np.isfinite(want)
        assert np.array_equal(got[fin], want[fin])
        assert np.array_equal(np.isnan(got), np.isnan(want))
    # overflow after scaling (mul > 1) sets bit 1 only
    big = [dev(np.array([3e38, 1.0], np.float32))]
    assert L().unscale_check(big, 4.0) == [2]
    # fp16 grads: finite input that overflows fp16 after scaling
    h16 = [dev(np.array([60000.0, 1.0]), torch.float16)]
    assert L().unscale_check(h16, 2.0) == [2]


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_grad_norm(cuda, kind):
    rng = np.random.default_rng(6)
    host = [rng.standard_normal(n).astype(np.float32) for n in (10, 4096, 70000, 1)]
    host[2][5] = np.nan
    gs = [dev(h) for h in host]
    val, flags = L().grad_norm(gs, kind, 3.0)
    fin = [np.where(np.isfinite(h), h, 0).astype(np.float64) for h in host]
    if kind == 0:
        want = sum((f ** 2).sum() for f in fin)
    elif kind == 1:
        want = max(np.abs(f).max() for f in fin)
    else:
        want = sum((np.abs(f) ** 3).sum() for f in fin)
    assert abs(val - want) <= 1e-9 * abs(want)
    assert flags == [0, 0, 1, 0]
    L().zero_nonfinite(gs)
    assert np.array_equal(gs[2].cpu().numpy(), fin[2].astype(np.float32))


def test_multi_tensor_many_and_misaligned(cuda):
    """More tensors than one launch holds, mixed sizes (full chunks, tails, 16-byte
    misaligned views) through Adam, unscale, grad norm and zero_nonfinite."""
    rng = np.random.default_rng(11)
    sizes = [(4096 * (i % 5) + 37 * i + 1) for i in range(45)]

    def make(n, i, dt=torch.float32):
        t = dev(rng.standard_normal(n), dt)
        return misaligned(t) if i % 7 == 3 else t
    ps = [make(n, i) for i, n in enumerate(sizes)]
    gs = [make(n, i) * 1e-2 for i, n in enumerate(sizes)]
    ms = [torch.zeros_like(p) for p in ps]
    vs = [torch.zeros_like(p) for p in ps]
    ref = [(f64(p), np.zeros(p.numel()), np.zeros(p.numel())) for p in ps]
    L().adam_step(ps, gs, ms, vs, None, 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.1, 0.001)
    for (p0, m0, v0), p, m, v, g in zip(ref, ps, ms, vs, gs):
        rp, rm, rv = O.adam_step(p0, f64(g), m0, v0, 1, lr=1e-3, weight_decay=0.01)[:3]
        assert_close(p, rp, RTOL_F32, "adam p")
        assert_close(m, rm, RTOL_F32, "adam m")
        assert_close(v, rv, RTOL_F32, "adam v")
    for dt in (torch.float32, torch.float16):
        hs = [make(n, i, dt) for i, n in enumerate(sizes)]
        bad = {5: 0, 17: sizes[17] - 1, 40: sizes[40] // 2}
        for i, pos in bad.items():
            hs[i][pos] = float("inf") if i != 17 else float("nan")
        host = [f64(h) for h in hs]
        val, flags = L().grad_norm(hs, 0)
        fin = [np.where(np.isfinite(h), h, 0.0) for h in host]
        want = sum((f.astype(np.float64) ** 2).sum() for f in fin)
        assert abs(val - want) <= 1e-9 * want
        assert flags == [1 if i in bad else 0 for i in range(len(sizes))]
        flags = L().unscale_check(hs, 0.5)
        assert flags == [3 if i in bad else 0 for i in range(len(sizes))]
        npdt = np.float16 if dt == torch.float16 else np.float32
        half = [(x * 0.5).astype(npdt).astype(np.float64) for x in host]  # rounded as stored
        for h, exp in zip(hs, half):
            got = f64(h)
            ok = np.isfinite(exp)
            assert np.array_equal(got[ok], exp[ok])
        L().zero_nonfinite(hs)
        for h, exp in zip(hs, half):
            assert np.array_equal(f64(h), np.where(np.isfinite(exp), exp, 0.0))


@pytest.mark.parametrize("n", [1, 7, 8, 4099, 1 << 20])
@pytest.mark.parametrize("dx,dy", [(torch.float16, torch.float16), (torch.float16, torch.float32),
                                   (torch.float32, torch.float16), (torch.bfloat16, torch.float32),
                                   (torch.float32, torch.float32)])
@pytest.mark.parametrize("mis", [False, True])
def test_axpby(cuda, n, dx, dy, mis):
    """y = alpha*x + beta*y (fp32 arithmetic, one rounding to y's dtype); beta = 0 must
    not read y (NaN-filled y stays out of the result)."""
    rng = np.random.default_rng(n)
    x = dev(rng.standard_normal(n), dx)
    y0 = dev(rng.standard_normal(n), dy)
    if mis:
        x, y0 = misaligned(x), misaligned(y0)
    y = y0.clone() if not mis else misaligned(y0.clone())
    L().axpby(x, y, 0.5, -2.0)
    want = (0.5 * x.float() + -2.0 * y0.float()).to(dy)
    assert torch.equal(y, want)
    y.fill_(float("nan"))
    L().axpby(x, y, 3.0, 0.0)
    assert torch.equal(y, (3.0 * x.float()).to(dy))


@pytest.mark.parametrize("M,N,K,beta", [(1024, 4096, 8192, 0.0), (1024, 1024, 8192, 1.0), (512, 256, 32000, 1.0),
                                        (256, 512, 4096, 0.0)])
def test_matmul2d_k_split(cuda, M, N, K, beta):
    """Weight-gradient shapes (op(A) = X^T over a long token axis) that run as a K-split
    batched GEMM plus the deterministic partial sum; fp16 operands, fp32 output,
    overwrite and accumulate, against a float64 product (rtol 1e-4)."""
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    x = torch.randn(K, M, device="cuda", generator=g).half()
    y = torch.randn(K, N, device="cuda", generator=g).half()
    out = torch.randn(M, N, device="cuda", generator=g)
    want = x.double().t() @ y.double() + (out.double() if beta else 0.0)
    L().matmul2d(x, y, out, trans_a=True, beta=beta)
    assert_close(out, want.cpu().numpy(), RTOL_F32_MM, "k-split matmul")


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("rows,cols", [(512, 1024), (300, 1000), (65, 7)])
def test_layernorm_bwd_add_matches_in_place(cuda, dt, rows, cols):
    """tg_layernorm_bwd_add (dx = LayerNorm dx + dx_add from another buffer) is
    bit-identical to accumulating in place into a copy of dx_add, on the register
    kernels (cols 1024, 1000) and the generic ones (7), and leaves dx_add untouched."""
    g = torch.Generator(device="cuda").manual_seed(rows + cols)
    x = torch.randn(rows, cols, device="cuda", generator=g).to(dt)
    dy = torch.randn(rows, cols, device="cuda", generator=g).to(dt)
    gam = torch.randn(cols, device="cuda", generator=g)
    bet = torch.randn(cols, device="cuda", generator=g)
    _, mean, rstd = L().layernorm_fwd(x, gam, bet, 1e-5)
    add = torch.randn(rows, cols, device="cuda", generator=g).to(dt)
    add0 = add.clone()
    ref = add.clone()
    dg1, db1 = torch.zeros(cols, device="cuda"), torch.zeros(cols, device="cuda")
    dg2, db2 = torch.zeros(cols, device="cuda"), torch.zeros(cols, device="cuda")
    L().layernorm_bwd(x, mean, rstd, gam, dy, ref, dg1, db1, True, False)
    out = torch.full_like(add, float("nan"))
    L().layernorm_bwd(x, mean, rstd, gam, dy, out, dg2, db2, True, False, dx_add=add)
    assert torch.equal(out, ref)
    assert torch.equal(add, add0)
    assert torch.equal(dg1, dg2) and torch.equal(db1, db2)


@pytest.mark.parametrize("M,N,K", [(300, 200, 128), (129, 257, 64), (64, 72, 40), (520, 136, 192)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_gemm_padded_leading_dims(cuda, M, N, K, ta, tb, dt):
    """A, B and C as sub-blocks of wider buffers (leading dimensions larger than the
    logical width, kept 16-byte multiples so the DMA-staged path stays eligible): the
    product equals the one of the compact copies, and C's padding is left untouched."""
    pa, pb, pc = 64, 8, 16
    rng = np.random.default_rng(M + 7 * N + 13 * K)
    ra, ca = (K, M) if ta else (M, K)
    rb, cb = (N, K) if tb else (K, N)
    A = dev(rng.standard_normal((ra, ca + pa)), dt)
    B = dev(rng.standard_normal((rb, cb + pb)), dt)
    C = dev(rng.standard_normal((M, N + pc)))
    C0 = C.clone()
    L().gemm(A, B, C, ta, tb, 1.5, 0.5, M, N, K, ca + pa, cb + pb, N + pc)
    a, b = f64(A[:, :ca]), f64(B[:, :cb])
    ref = 1.5 * ((a.T if ta else a) @ (b.T if tb else b)) + 0.5 * f64(C0[:, :N])
    assert_close(C[:, :N], ref, RTOL_F32_MM, f"gemm padded {dt} {M}x{N}x{K} ta={ta} tb={tb}")
    assert torch.equal(C[:, N:], C0[:, N:])
