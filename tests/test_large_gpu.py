"""Operands past 2^31 elements: the streaming and row kernels index with 64-bit offsets,
so windows at the start, across the 2^31 boundary and at the end of one large call must
match the oracle and the same kernel run on that window alone.  Misaligned operands at
a few million elements take the scalar loop spread over the whole grid and must equal
the aligned vector path bit for bit.  GPU only; about 16 GiB of device memory."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, RTOL_F32, assert_close

pytestmark = pytest.mark.gpu

BIG = (1 << 31) + 4099  # not a multiple of the 8-element vector: exercises the tail too
WIN = 1 << 16


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def f64(t):
    return t.detach().double().cpu().numpy()


def windows(n, w):
    """Starts of windows at the beginning, across 2^31 and covering the last element."""
    return [0, (1 << 31) - w // 2, n - w]


@pytest.fixture
def free_after():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("kind", ["gelu", "silu"])
def test_act_past_2e31(cuda, free_after, kind):
    gen = torch.Generator(device="cuda").manual_seed(17)
    x = torch.randn(BIG, dtype=torch.float16, device="cuda", generator=gen) * 3
    dy = torch.randn(BIG, dtype=torch.float16, device="cuda", generator=gen)
    dx = torch.empty_like(x)
    L().act_bwd(kind, x, dy, dx, False)
    y = L().act_fwd(kind, x)
    fwd = O.gelu_fwd if kind == "gelu" else O.silu_fwd
    bwd = O.gelu_bwd if kind == "gelu" else O.silu_bwd
    for s in windows(BIG, WIN):
        xs, ds = x[s:s + WIN].clone(), dy[s:s + WIN].clone()
        got_b, got_f = dx[s:s + WIN], y[s:s + WIN]
        assert_close(got_b, bwd(f64(xs), f64(ds)), RTOL_F16, f"{kind} bwd window {s}")
        assert_close(got_f, fwd(f64(xs)), RTOL_F16, f"{kind} fwd window {s}")
        small = torch.empty_like(xs)
        L().act_bwd(kind, xs, ds, small, False)
        assert torch.equal(small, got_b), f"{kind} bwd window {s} differs from a small call"
        assert torch.equal(L().act_fwd(kind, xs), got_f), f"{kind} fwd window {s}"
    # accumulate into the same buffer: dx += dy * act'(x), checked on the last window
    s = BIG - WIN
    before = dx[s:].float().clone()
    L().act_bwd(kind, x, dy, dx, True)
    ref = bwd(f64(x[s:]), f64(dy[s:])) + before.double().cpu().numpy()
    assert_close(dx[s:], ref, RTOL_F16, f"{kind} accumulate tail")


def test_axpby_past_2e31(cuda, free_after):
    gen = torch.Generator(device="cuda").manual_seed(18)
    x = torch.randn(BIG, dtype=torch.float16, device="cuda", generator=gen)
    y = torch.randn(BIG, dtype=torch.float16, device="cuda", generator=gen)
    y0 = {s: y[s:s + WIN].clone() for s in windows(BIG, WIN)}
    L().axpby(x, y, 0.5, -2.0)
    for s, ys in y0.items():
        want = 0.5 * f64(x[s:s + WIN]) - 2.0 * f64(ys)
        assert_close(y[s:s + WIN], want, RTOL_F16, f"axpby window {s}")
        small = ys.clone()
        L().axpby(x[s:s + WIN].clone(), small, 0.5, -2.0)
        assert torch.equal(small, y[s:s + WIN]), f"axpby window {s} differs from a small call"


def test_layernorm_past_2e31(cuda, free_after):
    """rows * cols > 2^31 (fp16): per-row outputs on row windows against the oracle, and
    dgamma / dbeta (sums over every row) against an fp32 sum in row chunks."""
    cols = 1024
    rows = (1 << 21) + 5
    gen = torch.Generator(device="cuda").manual_seed(19)
    x = torch.randn(rows, cols, dtype=torch.float16, device="cuda", generator=gen)
    dy = torch.randn(rows, cols, dtype=torch.float16, device="cuda", generator=gen)
    rng = np.random.default_rng(19)
    g = torch.as_tensor(1 + 0.02 * rng.standard_normal(cols), dtype=torch.float32).cuda()
    b = torch.as_tensor(0.02 * rng.standard_normal(cols), dtype=torch.float32).cuda()
    y, mean, rstd = L().layernorm_fwd(x, g, b, 1e-5)
    dx = torch.empty_like(x)
    dg, db = torch.empty_like(g), torch.empty_like(b)
    L().layernorm_bwd(x, mean, rstd, g, dy, dx, dg, db, False, False)
    w = 64
    for r in windows(rows, w):
        yr, xh, _, var = O.layernorm_fwd(f64(x[r:r + w]), f64(g), f64(b), 1e-5)
        dxr, _, _ = O.layernorm_bwd(xh, var, f64(g), f64(dy[r:r + w]), 1e-5)
        assert_close(y[r:r + w], yr, RTOL_F16, f"ln y rows {r}")
        assert_close(dx[r:r + w], dxr, RTOL_F16, f"ln dx rows {r}")
    sg = torch.zeros(cols, dtype=torch.float64, device="cuda")
    sb = torch.zeros(cols, dtype=torch.float64, device="cuda")
    step = 1 << 16
    for r in range(0, rows, step):
        xc = x[r:r + step].float()
        xh = (xc - mean[r:r + step, None]) * rstd[r:r + step, None]
        dc = dy[r:r + step].float()
        sg += (dc * xh).sum(0, dtype=torch.float64)
        sb += dc.sum(0, dtype=torch.float64)
    assert_close(dg, sg.cpu().numpy(), RTOL_F32 * 10, "ln dgamma")
    assert_close(db, sb.cpu().numpy(), RTOL_F32 * 10, "ln dbeta")


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("kind", ["gelu", "silu"])
def test_act_misaligned_large_equals_aligned(cuda, dt, kind):
    """Every operand 2 or 4 bytes off 16-byte alignment runs the scalar loop over a grid
    of many blocks; its results equal the vector path's bit for bit."""
    n = 3_000_017
    gen = torch.Generator(device="cuda").manual_seed(20)
    x = (torch.randn(n, device="cuda", generator=gen) * 3).to(dt)
    dy = torch.randn(n, device="cuda", generator=gen).to(dt)
    base = torch.randn(n, device="cuda", generator=gen).to(dt)

    def off(t):
        buf = torch.empty(n + 8, dtype=dt, device="cuda")
        v = buf[1:1 + n]
        v.copy_(t)
        return v

    for acc in (False, True):
        want = base.clone()
        L().act_bwd(kind, x, dy, want, acc)
        got = off(base)
        L().act_bwd(kind, off(x), off(dy), got, acc)
        assert torch.equal(got, want), f"{kind} bwd acc={acc}"
    want = L().act_fwd(kind, x)
    got = off(torch.zeros_like(x))
    L().act_fwd(kind, off(x), got)
    assert torch.equal(got, want), f"{kind} fwd"


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.float64])
@pytest.mark.parametrize("op,param", [("relu", 0.0), ("leaky_relu", 0.01), ("sigmoid", 0.0),
                                      ("tanh", 0.0), ("exp", 0.0), ("log", 0.0), ("swish", 1.0),
                                      ("pow", 3.0)])
def test_unary_misaligned_large_equals_aligned(cuda, dt, op, param):
    """tg_unary_bwd with every operand off 16-byte alignment (the scalar loop over a grid
    of many blocks) equals the aligned vector path bit for bit, plain and accumulating."""
    n = 1_500_007
    gen = torch.Generator(device="cuda").manual_seed(21)
    a = torch.rand(n, device="cuda", generator=gen).to(dt) + 0.5  # log and pow need a > 0
    dy = torch.randn(n, device="cuda", generator=gen).to(dt)
    base = torch.randn(n, device="cuda", generator=gen).to(dt)

    def off(t):
        buf = torch.empty(n + 8, dtype=dt, device="cuda")
        v = buf[1:1 + n]
        v.copy_(t)
        return v

    for acc in (False, True):
        want = base.clone()
        L().unary_bwd(op, a, dy, want, acc, param)
        got = off(base)
        L().unary_bwd(op, off(a), off(dy), got, acc, param)
        assert torch.equal(got, want), f"{op} {dt} acc={acc}"


@pytest.mark.parametrize("dx_,dy_", [(torch.float32, torch.float16), (torch.float16, torch.float16),
                                     (torch.float32, torch.bfloat16), (torch.float16, torch.float32)])
@pytest.mark.parametrize("beta", [0.0, 0.75])
def test_axpby_paths_round_alike(cuda, dx_, dy_, beta):
    """tg_axpbyz: the 8-wide vector body, its scalar tail and the misaligned kernel give
    the same bits for the same elements."""
    n = 1_000_003  # 3 tail elements
    gen = torch.Generator(device="cuda").manual_seed(22)
    x = torch.randn(n, device="cuda", generator=gen).to(dx_)
    y = torch.randn(n, device="cuda", generator=gen).to(dy_)
    want = L().axpbyz(x, y, 1.3, beta)

    def off(t):
        buf = torch.empty(n + 8, dtype=t.dtype, device="cuda")
        v = buf[1:1 + n]
        v.copy_(t)
        return v

    got = L().axpbyz(off(x), off(y), 1.3, beta, out=off(torch.zeros_like(y)))
    assert torch.equal(got, want)
    # the last 16 elements (3 of them the aligned call's scalar tail) as a call of their
    # own, where all 16 run through the vector body
    k = n - 16
    part = L().axpbyz(x[k:].clone(), y[k:].clone(), 1.3, beta)
    assert torch.equal(part, want[k:])


@pytest.mark.parametrize("trans_b", [False, True])
def test_gemm_row_major_operand_past_2gib(cuda, free_after, trans_b):
    """An fp16 A of 1,050,000 x 1024 (2.15 GB, past the 2 GiB a buffer window covers)
    still runs on the DMA-staged kernel: each block's window starts at its own rows.
    Row windows at the start, across byte 2^31 and at the end against float64, and bit
    for bit against the same rows computed as a small call."""
    import time
    M, K, N = 1_050_000, 1024, 256
    gen = torch.Generator(device="cuda").manual_seed(23)
    a = torch.randn(M, K, dtype=torch.float16, device="cuda", generator=gen)
    b = torch.randn((N, K) if trans_b else (K, N), dtype=torch.float16, device="cuda",
                    generator=gen) * 0.05
    c = L().matmul2d(a, b, trans_b=trans_b)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    L().matmul2d(a, b, out=c, trans_b=trans_b)
    torch.cuda.synchronize()
    print(f"[{M}x{N}x{K}] {2 * M * N * K / (time.perf_counter() - t0) / 1e12:.0f} TFLOP/s",
          flush=True)
    bd = b.double().t() if trans_b else b.double()
    w = 256
    for r in [0, (1 << 20) - w // 2, M - w]:  # row 2^20 starts at byte 2^31
        assert_close(c[r:r + w], (a[r:r + w].double() @ bd).cpu().numpy(), RTOL_F16,
                     f"rows {r}")
        small = L().matmul2d(a[r:r + w].clone(), b, trans_b=trans_b)
        assert torch.equal(small, c[r:r + w]), f"rows {r} differ from a small call"


def test_flash_attention_past_2e31(cuda, free_after):
    """B*H*S*D = 2^31 + 3*2048 (fp16, 2^21 + 3 heads of 16 x 64; ~34 GB for Q, K, V, O,
    dO, dQ, dK, dV): batches at the start, across element 2^31 and at the end against
    the float64 oracle and bit for bit against the same batches as a small call, causal
    and not."""
    B, H, S, D = (1 << 20) + 3, 2, 16, 64
    gen = torch.Generator(device="cuda").manual_seed(24)
    q, k, v, do = (torch.randn(B, H, S, D, dtype=torch.float16, device="cuda",
                               generator=gen) for _ in range(4))
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    for causal in (False, True):
        o, lse = L().flash_attn_fwd(q, k, v, D ** -0.5, causal)
        L().flash_attn_bwd(q, k, v, o, do, lse, dq, dk, dv, D ** -0.5, causal, False)
        for b in [0, 1 << 20, B - 1]:  # batch 2^20 starts at element 2^31
            sl = slice(b, b + 1)
            qs, ks, vs, ds = (t[sl].clone() for t in (q, k, v, do))
            os_, ls = L().flash_attn_fwd(qs, ks, vs, D ** -0.5, causal)
            assert torch.equal(os_, o[sl]) and torch.equal(ls, lse[sl]), f"fwd batch {b}"
            g = [torch.empty_like(qs) for _ in range(3)]
            L().flash_attn_bwd(qs, ks, vs, os_, ds, ls, *g, D ** -0.5, causal, False)
            for got, big, n in zip(g, (dq, dk, dv), ("dq", "dk", "dv")):
                assert torch.equal(got, big[sl]), f"{n} batch {b} causal={causal}"
            oo, _ = O.flash_attention_fwd(f64(qs), f64(ks), f64(vs), causal)
            assert_close(o[sl], oo, RTOL_F16, f"O batch {b}")
            rq, rk, rv = O.flash_attention_bwd(f64(qs), f64(ks), f64(vs), f64(ds), causal)
            for got, want, n in ((dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
                assert_close(got[sl], want, RTOL_F16, f"{n} batch {b} causal={causal}")
