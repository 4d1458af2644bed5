"""FlashAttention on one packed Q/K/V projection (tg_flash_attn_fwd_qkv / _bwd_qkv and
the flash_attention_qkv op).  GPU only.

The packed entry points run the same kernels as the separate-tensor (B, S, H, D)
layout with other row strides, so their results must equal, bit for bit, the layout-1
calls on the three column blocks copied out; one case per dtype is also checked
against the float64 oracle at the dtype's bar (fp16 1e-2, bf16 3e-2, fp32 1e-4)."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, assert_close

pytestmark = pytest.mark.gpu
RTOL = {torch.float16: RTOL_F16, torch.bfloat16: 3e-2, torch.float32: 1e-4}


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def rnd(shape, dt, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dt).cuda()


def split(qkv, H):
    """The three (B, H, S, D) views (layout 1 memory) of copies of the column blocks."""
    B, S, C3 = qkv.shape
    C = C3 // 3
    return [qkv[:, :, i * C:(i + 1) * C].contiguous().view(B, S, H, C // H).permute(0, 2, 1, 3)
            for i in range(3)]


def separate(qkv, do, H, causal, acc=None):
    """o (B, S, HD) and dqkv from the layout-1 entry points on copies (dqkv added to
    copies of acc's column blocks when acc is given)."""
    B, S, C3 = qkv.shape
    D = C3 // 3 // H
    q, k, v = split(qkv, H)
    scale = D ** -0.5
    o, lse = L().flash_attn_fwd(q, k, v, scale, causal, 1)
    d4 = do.view(B, S, H, D).permute(0, 2, 1, 3)
    if acc is None:
        dq, dk, dv = (L().fa_empty(B, H, S, D, qkv.dtype, qkv.device, 1) for _ in range(3))
    else:
        dq, dk, dv = split(acc, H)
    L().flash_attn_bwd(q, k, v, o, d4, lse, dq, dk, dv, scale, causal, acc is not None, 1)
    merge = [t.permute(0, 2, 1, 3).reshape(B, S, H * D) for t in (o, dq, dk, dv)]
    return merge[0], lse, torch.cat(merge[1:], dim=-1)


CASES = [(2, 3, 128, 64), (1, 2, 200, 128), (1, 4, 257, 64), (2, 1, 33, 128), (1, 2, 96, 48),
         (1, 3, 70, 80)]


@pytest.mark.parametrize("B,H,S,D", CASES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_packed_equals_separate(cuda, B, H, S, D, causal, dt):
    qkv = rnd((B, S, 3 * H * D), dt, 1)
    do = rnd((B, S, H * D), dt, 2)
    scale = D ** -0.5
    o, lse = L().flash_attn_fwd_qkv(qkv, H, scale, causal)
    dqkv = torch.full_like(qkv, float("nan"))  # every element must be written
    L().flash_attn_bwd_qkv(qkv, o, do, lse, dqkv, H, scale, causal, False)
    o_ref, lse_ref, dqkv_ref = separate(qkv, do, H, causal)
    assert torch.equal(o, o_ref)
    assert torch.equal(lse, lse_ref)
    assert torch.equal(dqkv, dqkv_ref)
    # accumulate adds (in fp32, rounded once) into every column block
    acc = rnd(qkv.shape, dt, 3)
    want = separate(qkv, do, H, causal, acc)[2]
    L().flash_attn_bwd_qkv(qkv, o, do, lse, acc, H, scale, causal, True)
    assert torch.equal(acc, want)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_packed_vs_oracle(cuda, dt):
    B, H, S, D = 1, 2, 160, 64
    qkv = rnd((B, S, 3 * H * D), dt, 4)
    do = rnd((B, S, H * D), dt, 5)
    scale = D ** -0.5
    o, lse = L().flash_attn_fwd_qkv(qkv, H, scale, True)
    dqkv = torch.empty_like(qkv)
    L().flash_attn_bwd_qkv(qkv, o, do, lse, dqkv, H, scale, True, False)
    q, k, v = (t.double().cpu().numpy() for t in split(qkv, H))
    d4 = do.view(B, S, H, D).permute(0, 2, 1, 3).double().cpu().numpy()
    oo, ll = O.flash_attention_fwd(q, k, v, True)
    # bf16: the row term from the kernel's stored O (as in the separate-tensor tests)
    ro = o.view(B, S, H, D).permute(0, 2, 1, 3).double().cpu().numpy()
    gq, gk, gv = O.flash_attention_bwd(q, k, v, d4, True,
                                       o=ro if dt == torch.bfloat16 else None)
    rt = RTOL[dt]
    assert_close(o.view(B, S, H, D).permute(0, 2, 1, 3), oo, rt, "O")
    for i, (g, name) in enumerate(((gq, "dq"), (gk, "dk"), (gv, "dv"))):
        got = dqkv[:, :, i * H * D:(i + 1) * H * D].reshape(B, S, H, D).permute(0, 2, 1, 3)
        assert_close(got, g, rt, name)


def test_packed_batch_chunks(cuda):
    """More than 65535 heads: launches over batch chunks, whose offsets in the packed
    buffer are three times those of a separate tensor."""
    B, H, S, D = 33000, 2, 3, 64
    qkv = rnd((B, S, 3 * H * D), torch.float16, 6)
    do = rnd((B, S, H * D), torch.float16, 7)
    scale = D ** -0.5
    o, lse = L().flash_attn_fwd_qkv(qkv, H, scale, True)
    dqkv = torch.empty_like(qkv)
    L().flash_attn_bwd_qkv(qkv, o, do, lse, dqkv, H, scale, True, False)
    o_ref, lse_ref, dqkv_ref = separate(qkv, do, H, True)
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref) and torch.equal(dqkv, dqkv_ref)


def test_packed_rejects_bad_input(cuda):
    qkv = rnd((1, 8, 3 * 2 * 64), torch.float16, 8)
    with pytest.raises(ValueError):
        L().flash_attn_fwd_qkv(qkv[:, :, :300], 2, 0.125, False)  # not 3*H*D wide
    with pytest.raises(ValueError):
        L().flash_attn_fwd_qkv(rnd((2, 8, 384), torch.float16, 8).transpose(0, 1), 2, 0.125,
                               False)
    with pytest.raises(TypeError):
        L().flash_attn_fwd_qkv(qkv.double(), 2, 0.125, False)
    lib = L().load()
    q = rnd((1, 2, 8, 64), torch.float16, 9)
    lse = torch.empty(1, 2, 8, device="cuda")
    # the layout entry points accept only layouts 0 and 1
    st = lib.tg_flash_attn_fwd_layout(L().dtype_code(q), L().ptr(q), L().ptr(q), L().ptr(q),
                                      L().ptr(torch.empty_like(q)), L().ptr(lse), 1, 2, 8, 8,
                                      64, 0.125, 0, 2, L().stream_handle())
    assert st != 0


@pytest.mark.parametrize("dt", [torch.float16, torch.float32, torch.float64])
def test_flash_attention_qkv_op(cuda, tg, dt):
    """The Tensor op: output and qkv gradient equal flash_attention on the head splits
    (with the merge-heads transpose), accumulated into an existing gradient: bit for bit
    in fp32, within 2e-3 in fp16 (one rounding fewer), 1e-12 in float64 (the fp64 path
    runs on copies of the splits)."""
    B, S, H, D = 2, 96, 2, 64
    C = H * D
    g = np.random.default_rng(0)
    xv = g.standard_normal((B, S, 3 * C))
    gv = g.standard_normal((B, S, C))
    npdt = {torch.float16: np.float16, torch.float32: np.float32, torch.float64: np.float64}[dt]

    def run(packed):
        x = tg.Tensor(xv.astype(npdt))
        y = x * 1.0
        if packed:
            out = tg.flash_attention_qkv(y, H, is_causal=True)
        else:
            def heads(t):
                return t.reshape(B, S, H, D).transpose(0, 2, 1, 3)
            o = tg.flash_attention(heads(y[:, :, :C]), heads(y[:, :, C:2 * C]),
                                   heads(y[:, :, 2 * C:]), is_causal=True)
            out = o.transpose(0, 2, 1, 3).reshape(B, S, C)
        loss = (out * tg.Tensor(gv.astype(npdt), requires_grad=False)).sum() + (y * y).sum()
        loss.backward()
        return out.data.double().cpu(), x.grad.double().cpu()

    o1, g1 = run(True)
    o0, g0 = run(False)
    if dt == torch.float64:
        assert torch.allclose(o1, o0, rtol=1e-12, atol=1e-12)
        assert torch.allclose(g1, g0, rtol=1e-12, atol=1e-12)
    elif dt == torch.float32:
        assert torch.equal(o1, o0)
        assert torch.equal(g1, g0)
    else:
        # the packed backward adds its fp32 result to the existing fp16 gradient with one
        # rounding; the separate path rounds dq/dk/dv to fp16 first, then adds
        assert torch.equal(o1, o0)
        assert_close(g1, g0, 2e-3, "qkv grad")
