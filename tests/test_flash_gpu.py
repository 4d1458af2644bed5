"""FlashAttention forward/backward kernels vs the oracle (float64 on the same
fp16/bf16-rounded inputs).  GPU only.

Tolerance: fp16 rtol 1e-2 (the autocast bar); bf16 rtol 3e-2, because P and dS
enter the second GEMMs rounded to bf16's 8-bit mantissa."""
import os

import numpy as np
import pytest
import torch

import oracle as O
from conftest import GOLDEN, RTOL_F16, RTOL_F32_MM, assert_close

pytestmark = pytest.mark.gpu
RTOL = {torch.float16: RTOL_F16, torch.bfloat16: 3e-2}


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def rnd(shape, dt, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dt).cuda()


def f64(t):
    return t.detach().double().cpu().numpy()


def run(q, k, v, do, causal):
    scale = q.shape[-1] ** -0.5
    o, lse = L().flash_attn_fwd(q, k, v, scale, causal)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    L().flash_attn_bwd(q, k, v, o, do, lse, dq, dk, dv, scale, causal, False)
    return o, lse, dq, dk, dv


CASES = [(1, 2, 96, 96, 64), (2, 3, 128, 128, 64), (1, 2, 200, 200, 128), (1, 1, 33, 33, 64),
         (1, 2, 100, 150, 64), (1, 1, 150, 70, 128), (2, 1, 256, 256, 128),
         # several staged tiles on both sides (double-buffer stages alternate), 1 x 1
         (1, 2, 257, 513, 64), (1, 1, 640, 384, 128), (1, 1, 3, 5, 64)]


@pytest.mark.parametrize("B,H,Sq,Sk,D", CASES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_flash_vs_oracle(cuda, B, H, Sq, Sk, D, causal, dt):
    q = rnd((B, H, Sq, D), dt, 1)
    k = rnd((B, H, Sk, D), dt, 2)
    v = rnd((B, H, Sk, D), dt, 3)
    do = rnd((B, H, Sq, D), dt, 4)
    o, lse, dq, dk, dv = run(q, k, v, do, causal)
    oo, ll = O.flash_attention_fwd(f64(q), f64(k), f64(v), causal)
    rt = RTOL[dt]
    assert_close(o, oo, rt, "O")
    assert_close(lse, ll, 1e-5, "lse")
    # fp16: the reference formula, row term rowsum(P*dP).  bf16: the row term from the
    # kernel's stored O (rowsum(dO*O)), since bf16's 8-bit O rounding can dominate
    # dP - rowsum where that difference cancels (rows that see few keys).
    ro = f64(o) if dt == torch.bfloat16 else None
    rq, rk, rv = O.flash_attention_bwd(f64(q), f64(k), f64(v), f64(do), causal, o=ro)
    assert_close(dq, rq, rt, "dQ")
    assert_close(dk, rk, rt, "dK")
    assert_close(dv, rv, rt, "dV")


@pytest.mark.parametrize("D", [64, 128])
def test_flash_single_key(cuda, D):
    """One key: softmax is exactly 1, so dS = P*(dP - D) is exactly 0 and dQ = dK = 0;
    the kernel's dP (MFMA sums) and D (row sums of dO*O) round differently, so the
    check is absolute, scaled by |dO||V|.  dV = sum of dO over the queries."""
    q, k, v, do = (rnd((1, 2, 7, D), torch.float16, s) for s in (1, 2, 3, 4))
    k, v = k[:, :, :1].contiguous(), v[:, :, :1].contiguous()
    _, _, dq, dk, dv = run(q, k, v, do, False)
    bound = 1e-4 * float(do.float().abs().max() * v.float().abs().max()) * D
    assert float(dq.float().abs().max()) <= bound
    assert float(dk.float().abs().max()) <= bound
    assert_close(dv, f64(do).sum(axis=2, keepdims=True), RTOL_F16, "dV")


def test_flash_golden(cuda):
    f = np.load(os.path.join(GOLDEN, "flash_attn.npz"), allow_pickle=False)
    q, k, v, do = (torch.as_tensor(f[n]).cuda() for n in ("q", "k", "v", "do"))
    for tag, causal in (("full", False), ("causal", True)):
        o, lse, dq, dk, dv = run(q, k, v, do, causal)
        assert_close(o, f[f"o_{tag}"], RTOL_F16, f"golden O {tag}")
        assert_close(lse, f[f"lse_{tag}"], 1e-5, f"golden lse {tag}")
        assert_close(dq, f[f"dq_{tag}"], RTOL_F16, f"golden dQ {tag}")
        assert_close(dk, f[f"dk_{tag}"], RTOL_F16, f"golden dK {tag}")
        assert_close(dv, f[f"dv_{tag}"], RTOL_F16, f"golden dV {tag}")


def test_flash_accumulate(cuda):
    q, k, v, do = (rnd((1, 2, 64, 64), torch.float16, s) for s in range(4))
    scale = 0.125
    o, lse = L().flash_attn_fwd(q, k, v, scale, True)
    d1 = [torch.empty_like(q) for _ in range(3)]
    L().flash_attn_bwd(q, k, v, o, do, lse, *d1, scale, True, False)
    d2 = [t.clone() for t in d1]
    L().flash_attn_bwd(q, k, v, o, do, lse, *d2, scale, True, True)
    for a, b in zip(d1, d2):
        assert_close(b, 2 * f64(a), RTOL_F16, "accumulate doubles")


def assert_close_rows(actual, expected, rtol, what):
    """assert_close with the absolute term taken from the larger of the tensor's rms
    and the element's own row's rms (a row = one query or key of one head).  Each
    gradient row is its own reduction over up to S products whose fp16 roundings (dS
    and P enter the products as fp16, as in every fp16 FlashAttention backward) scale
    with that row's terms: under causal masking the first keys collect ~S large terms
    that cancel to a small result, so their error budget is the row's magnitude, not
    the head's average.  Never stricter than assert_close, looser only on rows whose
    own rms exceeds the tensor's."""
    a = actual.detach().double()
    e = expected.detach().double().to(a.device)
    assert a.shape == e.shape, what
    assert bool(torch.isfinite(a).all()), f"{what}: non-finite values"
    scale = torch.maximum(e.pow(2).mean().sqrt(), e.pow(2).mean(-1, keepdim=True).sqrt())
    err = (a - e).abs()
    lim = rtol * e.abs() + rtol * scale
    bad = err > lim
    if bool(bad.any()):
        i = tuple(int(v) for v in torch.nonzero((err - lim) == (err - lim).max())[0])
        raise AssertionError(f"{what}: {int(bad.sum())}/{a.numel()} elements outside "
                             f"rtol={rtol} (worst at {i}: got {float(a[i])!r}, want "
                             f"{float(e[i])!r}, bound {float(lim[i]):.3e})")


def _head_invariants(q, k, v, o, do, dq, dk, dv):
    """Per-head identities of attention's gradients, in float64 on the device, for
    every (b, h) at once.  With P's rows summing to 1 and dS = P*(dP - rowsum):
      sum_keys dV = sum_queries dO                 (dV = P^T dO)
      sum_keys dK = 0                              (each row of dS sums to 0)
      <dQ, Q> = <dK, K>                            (both are sum(dS * Q K^T))
      <dV, V> = <dO, O>                            (O = P V)
    Each returns the worst ratio |lhs - rhs| / sqrt(sum of squared terms), i.e. the
    error against the size the identity's terms would have if it failed; fp16
    rounding gives ~1e-3, a gradient taken from the wrong head or row gives ~1."""
    d = lambda t: t.double()  # noqa: E731
    q, k, v, o, do, dq, dk, dv = map(d, (q, k, v, o, do, dq, dk, dv))
    out = {}
    lhs, rhs = dv.sum(2), do.sum(2)
    out["sum dV = sum dO"] = ((lhs - rhs).abs() / (dv.pow(2).sum(2).sqrt() + 1e-30)).max()
    out["sum dK = 0"] = (dk.sum(2).abs() / (dk.pow(2).sum(2).sqrt() + 1e-30)).max()
    a, b = (dq * q).sum((2, 3)), (dk * k).sum((2, 3))
    sc = ((dq * q).pow(2).sum((2, 3)) + (dk * k).pow(2).sum((2, 3))).sqrt()
    out["<dQ,Q> = <dK,K>"] = ((a - b).abs() / sc).max()
    a, b = (dv * v).sum((2, 3)), (do * o).sum((2, 3))
    sc = ((dv * v).pow(2).sum((2, 3)) + (do * o).pow(2).sum((2, 3))).sqrt()
    out["<dV,V> = <dO,O>"] = ((a - b).abs() / sc).max()
    return {n: float(x) for n, x in out.items()}


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_full_size_all_heads(cuda, D, causal):
    """C4 shape B=8, H=16, S=2048.  All 128 (b, h) heads are checked element by
    element against float64 torch autograd of softmax(Q K^T s + mask) V (run on the
    device, one batch of 16 heads at a time; rtol 1e-2 with the row-scaled absolute
    term of assert_close_rows) and through the per-head identities at the fp16 bar;
    six heads spread over the dispatch's head groups (groups of 8 heads per XCD range:
    first, last of group 0, first of group 1, both sides of the middle, last) are also
    checked against the NumPy oracle."""
    B, H, S = 8, 16, 2048
    print(f"C4 full size D={D} causal={causal}", flush=True)
    q, k, v, do = (rnd((B, H, S, D), torch.float16, 10 + s) for s in range(4))
    o, lse, dq, dk, dv = run(q, k, v, do, causal)
    inv = _head_invariants(q, k, v, o, do, dq, dk, dv)
    print("identity errors:", {n: f"{x:.2e}" for n, x in inv.items()}, flush=True)
    for n, x in inv.items():
        assert x < RTOL_F16, f"{n}: {x:.3e}"
    scale = D ** -0.5
    for b in range(B):
        qd, kd, vd = (t[b].double().requires_grad_() for t in (q, k, v))
        sc = qd @ kd.transpose(-1, -2) * scale
        if causal:
            sc = sc.masked_fill(torch.ones(S, S, dtype=torch.bool, device=sc.device).triu(1),
                                float("-inf"))
        od = torch.softmax(sc, -1) @ vd
        od.backward(do[b].double())
        assert_close_rows(o[b], od.detach(), RTOL_F16, f"O batch {b}")
        assert_close_rows(dq[b], qd.grad, RTOL_F16, f"dQ batch {b}")
        assert_close_rows(dk[b], kd.grad, RTOL_F16, f"dK batch {b}")
        assert_close_rows(dv[b], vd.grad, RTOL_F16, f"dV batch {b}")
        del qd, kd, vd, sc, od
    for flat in (0, 7, 8, 63, 64, 127):
        b, hh = divmod(flat, H)
        sl = (slice(b, b + 1), slice(hh, hh + 1))
        oo, ll = O.flash_attention_fwd(f64(q[sl]), f64(k[sl]), f64(v[sl]), causal)
        assert_close(o[sl], oo, RTOL_F16, f"O head {flat}")
        assert_close(lse[sl], ll, 1e-5, f"lse head {flat}")
        rq, rk, rv = O.flash_attention_bwd(f64(q[sl]), f64(k[sl]), f64(v[sl]), f64(do[sl]),
                                           causal)
        assert_close(dq[sl], rq, RTOL_F16, f"dQ head {flat}")
        assert_close(dk[sl], rk, RTOL_F16, f"dK head {flat}")
        assert_close(dv[sl], rv, RTOL_F16, f"dV head {flat}")


def test_flash_rejects_bad_shapes(cuda):
    q = rnd((1, 1, 16, 264), torch.float16, 0)
    with pytest.raises(RuntimeError, match="head dim"):
        L().flash_attn_fwd(q, q, q, 0.1, False)


# fp32 (the reference's default dtype) and head dims the fp16/bf16 tuned kernels do not
# cover run on the generic kernels (fp32 matrix cores): fp32 at the 1e-4 attention bar
GEN_CASES = [(1, 2, 96, 96, 64), (2, 1, 70, 70, 8), (1, 2, 33, 100, 40), (1, 1, 130, 65, 80),
             (2, 2, 64, 64, 96), (1, 1, 100, 100, 128), (1, 1, 77, 140, 160),
             (1, 1, 64, 96, 256), (1, 3, 1, 7, 32), (1, 1, 200, 50, 200)]


@pytest.mark.parametrize("B,H,Sq,Sk,D", GEN_CASES)
@pytest.mark.parametrize("causal", [False, True])
def test_flash_fp32_vs_oracle(cuda, B, H, Sq, Sk, D, causal):
    q = rnd((B, H, Sq, D), torch.float32, 1)
    k = rnd((B, H, Sk, D), torch.float32, 2)
    v = rnd((B, H, Sk, D), torch.float32, 3)
    do = rnd((B, H, Sq, D), torch.float32, 4)
    o, lse, dq, dk, dv = run(q, k, v, do, causal)
    oo, ll = O.flash_attention_fwd(f64(q), f64(k), f64(v), causal)
    assert_close(o, oo, RTOL_F32_MM, "O")
    assert_close(lse, ll, 1e-5, "lse")
    rq, rk, rv = O.flash_attention_bwd(f64(q), f64(k), f64(v), f64(do), causal)
    for got, want, n in ((dq, rq, "dQ"), (dk, rk, "dK"), (dv, rv, "dV")):
        if not np.any(want):
            # one visible key per query (causal, Sq = 1): dS = P*(dP - D) is 0 exactly,
            # the kernel's dP and D round differently: an absolute bound
            assert float(got.abs().max()) < 1e-5, n
        else:
            assert_close(got, want, RTOL_F32_MM, n)


@pytest.mark.parametrize("D", [32, 48, 96, 256])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_flash_generic_head_dims_half(cuda, D, dt):
    q, k, v, do = (rnd((1, 2, 150, D), dt, s) for s in range(4))
    o, lse, dq, dk, dv = run(q, k, v, do, True)
    oo, _ = O.flash_attention_fwd(f64(q), f64(k), f64(v), True)
    assert_close(o, oo, RTOL[dt], "O")
    rq, rk, rv = O.flash_attention_bwd(f64(q), f64(k), f64(v), f64(do), True, o=f64(o))
    assert_close(dq, rq, RTOL[dt], "dQ")
    assert_close(dk, rk, RTOL[dt], "dK")
    assert_close(dv, rv, RTOL[dt], "dV")


@pytest.mark.parametrize("D", [40, 64])
def test_flash_fp32_bshd_layout_and_accumulate(cuda, D):
    """The generic kernels read and write the (B, S, H, D) head split in place, and
    accumulate adds to existing gradients."""
    B, H, S = 2, 3, 90
    g = torch.Generator(device="cuda").manual_seed(D)
    mk = lambda: torch.randn(B, S, H, D, device="cuda", generator=g)  # noqa: E731
    qs, ks, vs, dos = mk(), mk(), mk(), mk()
    q1, k1, v1, do1 = (t.permute(0, 2, 1, 3) for t in (qs, ks, vs, dos))
    q0, k0, v0, do0 = (t.contiguous() for t in (q1, k1, v1, do1))
    sc = D ** -0.5
    o0, l0 = L().flash_attn_fwd(q0, k0, v0, sc, True, 0)
    o1, l1 = L().flash_attn_fwd(q1, k1, v1, sc, True, 1)
    assert torch.equal(o0, o1) and torch.equal(l0, l1)
    outs = []
    for lay, (q, k, v, o, do) in ((0, (q0, k0, v0, o0, do0)), (1, (q1, k1, v1, o1, do1))):
        d = [L().fa_empty(B, H, S, D, q.dtype, q.device, lay) for _ in range(3)]
        for t in d:
            t.fill_(0.5)
        L().flash_attn_bwd(q, k, v, o, do, l0, *d, sc, True, True, lay)
        outs.append(d)
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    rq, rk, rv = O.flash_attention_bwd(f64(q0), f64(k0), f64(v0), f64(do0), True)
    for got, want, n in zip(outs[0], (rq, rk, rv), ("dq", "dk", "dv")):
        assert_close(got, want + 0.5, RTOL_F32_MM, n)


def test_flash_many_heads_chunked(cuda):
    """B*H above the 65535 limit of one launch's grid: the batches are split over
    several launches."""
    B, H, S, D = 33000, 2, 3, 8
    q, k, v, do = (rnd((B, H, S, D), torch.float32, s) for s in range(4))
    o, lse, dq, dk, dv = run(q, k, v, do, False)
    for b in (0, 32767, 32768, B - 1):
        sl = slice(b, b + 1)
        oo, ll = O.flash_attention_fwd(f64(q[sl]), f64(k[sl]), f64(v[sl]), False)
        assert_close(o[sl], oo, RTOL_F32_MM, f"O b={b}")
        rq, rk, rv = O.flash_attention_bwd(f64(q[sl]), f64(k[sl]), f64(v[sl]), f64(do[sl]), False)
        assert_close(dq[sl], rq, RTOL_F32_MM, f"dQ b={b}")
        assert_close(dk[sl], rk, RTOL_F32_MM, f"dK b={b}")
        assert_close(dv[sl], rv, RTOL_F32_MM, f"dV b={b}")


@pytest.mark.parametrize("B,H,Sq,Sk,D", [(2, 3, 257, 513, 64), (1, 4, 192, 192, 128),
                                         (2, 2, 1, 5, 64), (1, 1, 130, 70, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_bshd_layout_matches_contiguous(cuda, B, H, Sq, Sk, D, causal):
    """(B,S,H,D) memory read and written in place (layout 1) gives bit-identical O,
    LSE, dQ, dK, dV to the same values in contiguous (B,H,S,D) (layout 0): only the
    addressing differs."""
    g = torch.Generator(device="cuda").manual_seed(B * 7 + Sq + Sk)
    mk = lambda S: torch.randn(B, S, H, D, device="cuda", generator=g).half()  # noqa: E731
    qs, ks, vs, dos = mk(Sq), mk(Sk), mk(Sk), mk(Sq)
    q1, k1, v1, do1 = (t.permute(0, 2, 1, 3) for t in (qs, ks, vs, dos))
    q0, k0, v0, do0 = (t.contiguous() for t in (q1, k1, v1, do1))
    s = D ** -0.5
    o0, l0 = L().flash_attn_fwd(q0, k0, v0, s, causal, 0)
    o1, l1 = L().flash_attn_fwd(q1, k1, v1, s, causal, 1)
    assert L()._fa_in(o1, 1)
    assert torch.equal(o0, o1) and torch.equal(l0, l1)
    outs = []
    for lay, (q, k, v, o, do) in ((0, (q0, k0, v0, o0, do0)), (1, (q1, k1, v1, o1, do1))):
        dq = L().fa_empty(B, H, Sq, D, q.dtype, q.device, lay)
        dk = L().fa_empty(B, H, Sk, D, q.dtype, q.device, lay)
        dv = L().fa_empty(B, H, Sk, D, q.dtype, q.device, lay)
        L().flash_attn_bwd(q, k, v, o, do, l0, dq, dk, dv, s, causal, False, lay)
        outs.append((dq, dk, dv))
    for a, b, n in zip(outs[0], outs[1], ("dq", "dk", "dv")):
        assert torch.equal(a, b), n
