"""Weight + bias gradient entry point (tg_gemm_wgrad) against float64 torch sums of the
same inputs, through the C-ABI: dW (+)= X^T G and db (+)= G.sum(0) — the matmul node's
dB = A^T @ dC (reference _core.py:1064-1068) and the bias add's unbroadcast sum
(_core.py:1380-1424) of a Linear layer.  Covers the fp16/bf16 path that sums G's columns
inside the GEMM (K split into fp32 partials, or not split), ragged edge tiles, the fp32
and fp64 paths (GEMM then row reduction), unaligned operands, accumulation into
existing gradients, no bias, and the empty extents.  GPU only."""
import pytest
import torch

from conftest import RTOL_F16, RTOL_F32, RTOL_F32_MM, assert_close

pytestmark = pytest.mark.gpu


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def _case(M, N, K, dt, wdt, bdt, acc, seed, bias=True, offset=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    xb = torch.randn(K * M + offset, device="cuda", generator=g).to(dt)
    gb = torch.randn(K * N + offset, device="cuda", generator=g).to(dt)
    x = xb[offset:].view(K, M)
    gr = gb[offset:].view(K, N)
    w0 = torch.randn(M, N, device="cuda", generator=g).to(wdt)
    b0 = torch.randn(N, device="cuda", generator=g).to(bdt)
    dw, db = w0.clone(), b0.clone()
    L().wgrad(x, gr, dw, acc, db if bias else None, acc)
    ref_w = x.double().T @ gr.double() + (w0.double() if acc else 0.0)
    ref_b = gr.double().sum(0) + (b0.double() if acc else 0.0)
    return dw, db, b0, ref_w, ref_b


def _tol(dt):
    return RTOL_F16 if dt in (torch.float16, torch.bfloat16) else RTOL_F32_MM


@pytest.mark.parametrize("M,N,K", [
    (1024, 1024, 8192),   # eight K splits (projection weights over 8192 tokens)
    (1024, 4096, 8192),   # two K splits (FC weight)
    (136, 200, 2048),     # ragged edge tiles, two K splits
    (512, 384, 1024),     # short K: one pass, dW written by the GEMM itself
    (2048, 4096, 4096),   # enough tiles: no split, 256x256 blocks
])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("acc", [False, True])
def test_wgrad_fused(cuda, M, N, K, dt, acc):
    dw, db, _, ref_w, ref_b = _case(M, N, K, dt, torch.float32, torch.float32, acc, M + N + K)
    what = f"{dt} {M}x{N}x{K} acc={acc}"
    assert_close(dw, ref_w, RTOL_F32_MM, "dW " + what)
    assert_close(db, ref_b, RTOL_F32, "db " + what)


@pytest.mark.parametrize("split", [False, True])
def test_wgrad_lowp_outputs(cuda, split):
    """dW and db in the operands' own 16-bit dtype (rounded once from fp32 sums)."""
    M, N, K = (256, 256, 4096) if split else (512, 384, 1024)
    for dt in (torch.float16, torch.bfloat16):
        dw, db, _, ref_w, ref_b = _case(M, N, K, dt, dt, dt, True, 5)
        assert_close(dw, ref_w, _tol(dt), f"dW {dt}")
        assert_close(db, ref_b, _tol(dt), f"db {dt}")


@pytest.mark.parametrize("M,N,K,dt", [
    (256, 260, 4096, torch.float32),   # fp32 operands, K split, bias by row reduction
    (96, 130, 3000, torch.float32),    # N % 4 != 0: no split
    (40, 24, 300, torch.float64),      # fp64 matrix cores, fp64 sums
    (128, 100, 2048, torch.float16),   # N % 8 != 0: 16-bit operands off the fused path
])
def test_wgrad_unfused(cuda, M, N, K, dt):
    wdt = torch.float64 if dt == torch.float64 else torch.float32
    for acc in (False, True):
        dw, db, _, ref_w, ref_b = _case(M, N, K, dt, wdt, wdt, acc, 9)
        rtol = 1e-12 if dt == torch.float64 else RTOL_F32_MM
        assert_close(dw, ref_w, rtol, f"dW {dt} {M}x{N}x{K} acc={acc}")
        assert_close(db, ref_b, 1e-12 if dt == torch.float64 else RTOL_F32, f"db {dt} acc={acc}")


def test_wgrad_unaligned(cuda):
    """Operands 2 bytes off 16-byte alignment take the GEMM + reduction path."""
    dw, db, _, ref_w, ref_b = _case(256, 256, 4096, torch.float16, torch.float32, torch.float32,
                                    True, 13, offset=1)
    assert_close(dw, ref_w, RTOL_F32_MM, "dW unaligned")
    assert_close(db, ref_b, RTOL_F32, "db unaligned")


def test_wgrad_no_bias(cuda):
    dw, db, b0, ref_w, _ = _case(1024, 1024, 8192, torch.float16, torch.float32, torch.float32,
                                 False, 17, bias=False)
    assert_close(dw, ref_w, RTOL_F32_MM, "dW without bias")
    assert torch.equal(db, b0)


def test_wgrad_empty(cuda):
    g = torch.randn(64, 32, device="cuda").half()
    # M = 0: only the bias gradient
    db = torch.ones(32, device="cuda")
    L().wgrad(torch.empty(64, 0, device="cuda").half(), g, torch.empty(0, 32, device="cuda"),
              False, db, True)
    assert_close(db, 1.0 + g.double().sum(0), RTOL_F32, "db with M = 0")
    # K = 0: gradients are zero (overwrite) or unchanged (accumulate)
    x0 = torch.empty(0, 16, device="cuda").half()
    g0 = torch.empty(0, 32, device="cuda").half()
    dw = torch.full((16, 32), 3.0, device="cuda")
    db = torch.full((32,), 2.0, device="cuda")
    L().wgrad(x0, g0, dw, True, db, True)
    assert torch.all(dw == 3.0) and torch.all(db == 2.0)
    L().wgrad(x0, g0, dw, False, db, False)
    assert torch.all(dw == 0.0) and torch.all(db == 0.0)


def test_linear_autocast_accumulated(cuda):
    """tg.Linear under fp16 autocast (the fused path, K split over 4096 tokens), two
    backward passes accumulating into the fp32 gradients, against float64 torch."""
    import numpy as np
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(21)
    nin, nout = 256, 384
    x_np = rng.standard_normal((8, 512, nin)).astype(np.float32)
    lin = tg.Linear(nin, nout)
    lin.b.data = tg.Tensor(rng.standard_normal(nout).astype(np.float32) * 0.1,
                           requires_grad=False).data
    x = tg.Tensor(x_np)
    for _ in range(2):
        with tg.autocast():
            y = lin(x)
            loss = (y * y).sum()
        loss.backward()
    # reference: the fp16-rounded operands of the autocast GEMMs, in float64
    xs = torch.tensor(x_np).half().double().reshape(-1, nin)
    ws = lin.w.data.half().double().cpu()
    bs = lin.b.data.double().cpu()
    yh = (xs @ ws + bs).half().double()  # the fp16 forward output
    gy = 2.0 * yh                        # d(sum y^2)/dy, formed in fp16 by the engine
    assert_close(lin.w.grad, 2 * (xs.T @ gy).numpy(), RTOL_F16, "Linear dW")
    assert_close(lin.b.grad, 2 * gy.sum(0).numpy(), RTOL_F16, "Linear db")
