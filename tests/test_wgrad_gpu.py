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


# ---------------------------------------------------------------- grouped members
def _group_case(n, M, N, K, dt, wdt, bdt, seed, bias=(), acc=()):
    """n members with their own operands; N: one width or a list of n; bias / acc:
    member indices with a bias gradient / accumulating into existing gradients."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    Ns = list(N) if isinstance(N, (list, tuple)) else [N] * n
    xs = [torch.randn(K, M, device="cuda", generator=g).to(dt) for _ in range(n)]
    gs = [torch.randn(K, Ns[i], device="cuda", generator=g).to(dt) for i in range(n)]
    w0 = [torch.randn(M, Ns[i], device="cuda", generator=g).to(wdt) for i in range(n)]
    b0 = [torch.randn(Ns[i], device="cuda", generator=g).to(bdt) for i in range(n)]
    dws = [w.clone() for w in w0]
    dbs = [b.clone() if i in bias else None for i, b in enumerate(b0)]
    accs = [i in acc for i in range(n)]
    L().wgrad_group(xs, gs, dws, accs, dbs if bias else None, accs if bias else None)
    for i in range(n):
        ref_w = xs[i].double().T @ gs[i].double() + (w0[i].double() if accs[i] else 0.0)
        rtol = RTOL_F32_MM if wdt == torch.float32 else _tol(wdt)
        assert_close(dws[i], ref_w, rtol, f"dW member {i} of {n} ({M}x{N}x{K} {dt})")
        if i in bias:
            ref_b = gs[i].double().sum(0) + (b0[i].double() if accs[i] else 0.0)
            assert_close(dbs[i], ref_b, RTOL_F32 if bdt == torch.float32 else _tol(bdt),
                         f"db member {i}")


@pytest.mark.parametrize("n,M,N,K", [
    (16, 1024, 1024, 8192),  # q/k/v/o projections of four blocks: 256x256 whole-K tiles
    (4, 1024, 4096, 8192),   # FC weights of four blocks
    (6, 1024, 1024, 2048),   # 256x128 tiles
    (3, 256, 256, 1024),     # too few tiles: one by one (K split)
])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_wgrad_group(cuda, n, M, N, K, dt):
    _group_case(n, M, N, K, dt, torch.float32, torch.float32, n + M + K,
                bias=set(range(n)), acc={i for i in range(n) if i % 2})


def test_wgrad_group_mixed_bias_lowp_outputs(cuda):
    """Members without a bias beside members with one; gradients in the operands'
    16-bit dtype."""
    for dt in (torch.float16, torch.bfloat16):
        _group_case(8, 1024, 1024, 4096, dt, dt, dt, 3, bias={0, 3, 5}, acc={1, 3, 4})


def test_wgrad_group_chunks(cuda):
    """40 members: a first launch of 32, the remaining 8 (too few tiles) one by one;
    and a group without any bias."""
    _group_case(40, 512, 512, 256, torch.float16, torch.float32, torch.float32, 7,
                bias=set(range(0, 40, 3)), acc=set(range(0, 40, 2)))
    _group_case(5, 1024, 2048, 1024, torch.bfloat16, torch.float32, torch.float32, 8)


def test_wgrad_group_ragged_and_rejects(cuda):
    """Ragged edge tiles (M, N not multiples of the tile) and the checks of the
    wrapper: duplicate gradient buffers and unequal shapes."""
    _group_case(12, 1000, 776, 2048, torch.float16, torch.float32, torch.float32, 11,
                bias=set(range(12)), acc={2})
    x = torch.randn(64, 64, device="cuda").half()
    dw = torch.empty(64, 64, device="cuda")
    with pytest.raises(ValueError):
        L().wgrad_group([x, x], [x, x], [dw, dw], [False, False])
    with pytest.raises(ValueError):
        L().wgrad_group([x, x[:32]], [x, x[:32]], [dw, torch.empty_like(dw)], [False, False])


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_wgrad_group_mixed_widths(cuda, dt):
    """Members of one input shape with different output widths in one launch: the
    packed Q/K/V (N = 3d) and output (N = d) projections of four blocks; and a mix in
    which unaligned or small members run one by one beside the grouped ones."""
    _group_case(8, 1024, [3072] * 4 + [1024] * 4, 8192, dt, torch.float32, torch.float32, 21,
                bias=set(range(8)), acc={1, 6})
    _group_case(6, 512, [1536, 100, 512, 776, 2048, 64], 2048, dt, torch.float32,
                torch.float32, 22, bias={0, 1, 3}, acc={3, 4})


def _mlp_grads(defer, seed=4):
    """Gradients of a stack of equal Linear layers (one applied twice) under fp16
    autocast over two backward passes; defer False turns the queue off by setting its
    byte limit to zero."""
    import numpy as np
    import tensor_gpu_v2 as tg
    from tensor_gpu_v2 import _core
    rng = np.random.default_rng(seed)
    d = 1024
    # ten layers over 8192 tokens: the sweep queues nine products (layer 1's second
    # use to layer 2; grouped) until layer 1's first use flushes them, then two (one by one)
    layers = [tg.Linear(d, d) for _ in range(10)]
    for lin in layers:
        lin.w.data = tg.Tensor(rng.standard_normal((d, d)).astype(np.float32) * 0.04).data
        lin.b.data = tg.Tensor(rng.standard_normal(d).astype(np.float32) * 0.1).data
    xs = [rng.standard_normal((8, 1024, d)).astype(np.float32) for _ in range(2)]
    saved = _core._WG_MAX_BYTES
    _core._WG_MAX_BYTES = saved if defer else -1
    try:
        for x_np in xs:
            h = tg.Tensor(x_np)
            with tg.autocast():
                for lin in layers + [layers[1]]:  # layer 1 twice: its gradient accumulates
                    h = lin(h).relu()
                loss = (h * h).mean()
            loss.backward()
            assert not _core._WG_QUEUE and not _core._WG_TARGETS
    finally:
        _core._WG_MAX_BYTES = saved
    return [(lin.w.grad.clone(), lin.b.grad.clone()) for lin in layers]


def test_linear_deferred_weight_gradients(cuda):
    """The engine's queued, grouped weight gradients against the same network with
    every product run at once (queue limit zero): same tolerance as one GEMM against
    another (the products sum K in a different order)."""
    a = _mlp_grads(True)
    b = _mlp_grads(False)
    for i, ((wa, ba), (wb, bb)) in enumerate(zip(a, b)):
        assert_close(wa, wb.double(), RTOL_F16, f"layer {i} dW")
        assert_close(ba, bb.double(), RTOL_F16, f"layer {i} db")


def test_deferred_weight_gradients_flushed_when_backward_raises(cuda):
    """A node that raises during the sweep: the weight gradients queued before it are
    still computed (backward's finally), the queue and its bookkeeping are empty, and
    a later backward runs normally."""
    import numpy as np
    import tensor_gpu_v2 as tg
    from tensor_gpu_v2 import _core
    rng = np.random.default_rng(41)
    l1, l2 = tg.Linear(256, 256), tg.Linear(256, 256)
    x = tg.Tensor(rng.standard_normal((512, 256)).astype(np.float32))
    with tg.autocast():
        h = l1(x)
        y = l2(h.relu())
        loss = (y * y).mean()

    def boom():
        raise RuntimeError("injected")
    h._backward = boom  # l2's weight gradient is queued before h's node runs
    with pytest.raises(RuntimeError, match="injected"):
        loss.backward()
    assert not _core._WG_QUEUE and not _core._WG_TARGETS and _core._WG_STATE == [0, 0]
    g2 = l2.w.grad.double()
    assert torch.isfinite(g2).all() and float(g2.abs().sum()) > 0
    for p in (l1.w, l1.b, l2.w, l2.b):
        p.zero_grad()
    with tg.autocast():
        loss2 = (l2(l1(x).relu()) ** 2).mean()
    loss2.backward()
    assert torch.isfinite(l1.w.grad).all() and float(l1.w.grad.abs().sum()) > 0
