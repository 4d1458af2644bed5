"""Embedding backward (deterministic sorted scatter-add) and the tied-weight transfer
(tg_transpose_add) vs the oracle / closed forms.  GPU only.

fp32 embedding gradients are compared bit-exactly with np.add.at (the kernel sums
each index's rows in their original order, as np.add.at does)."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import RTOL_F16, RTOL_F32, assert_close

pytestmark = pytest.mark.gpu


def L():
    from tensor_gpu_v2 import _lib
    return _lib


# includes many-token, few-row and few-token, many-row cases; 32-bit sort keys (index
# and position bits fit 32) and 64-bit ones (the last case), one sorted chunk and
# several merged ones (n > 8192); up to 8192 tokens the band kernel (no sort) runs,
# also with thousands of tokens on one row
@pytest.mark.parametrize("n,V,dim", [(1, 1, 1), (24, 5, 7), (8192, 32000, 64), (300, 50, 1000),
                                     (16384, 3, 12), (20000, 64, 8), (500, 70000, 4),
                                     (9000, 1 << 20, 4), (8192, 3, 1024), (4097, 129, 130),
                                     (8192, 64, 256)])
def test_embedding_bwd_bit_exact_fp32(cuda, n, V, dim):
    rng = np.random.default_rng(n + V)
    idx = rng.integers(0, V, n)
    idx[: n // 3] = idx[0]  # many repeats of one index
    d = rng.standard_normal((n, dim)).astype(np.float32)
    want = O.embedding_bwd(idx, d, V)
    grad = torch.empty(V, dim, device="cuda")
    L().embedding_bwd(torch.tensor(d, device="cuda"), torch.tensor(idx, device="cuda"), grad,
                      False)
    assert np.array_equal(grad.cpu().numpy(), want)


@pytest.mark.parametrize("n,V", [(200, 40), (17000, 40)])
def test_embedding_bwd_half_accumulate_and_bounds(cuda, n, V):
    rng = np.random.default_rng(9)
    dim = 33
    idx = rng.integers(0, V, n)
    idx[5], idx[6] = -V - 1, V  # out of range: skipped
    idx[7], idx[8] = -1, -V  # count from the end (rows V-1 and 0)
    d = rng.standard_normal((n, dim)).astype(np.float16)
    base = rng.standard_normal((V, dim)).astype(np.float32)
    grad = torch.tensor(base, device="cuda")
    L().embedding_bwd(torch.tensor(d, device="cuda"), torch.tensor(idx, device="cuda"), grad, True)
    ok = (idx >= -V) & (idx < V)
    want = base.astype(np.float64) + O.embedding_bwd(idx[ok] % V, d[ok].astype(np.float64), V)
    assert_close(grad, want, RTOL_F32, "accumulated fp16 rows")


def test_embedding_module(cuda):
    import tensor_gpu_v2 as tg
    rng = np.random.default_rng(2)
    emb = tg.Embedding(10, 4)
    ids = np.array([[1, 2, 2], [-1, 0, 9]])
    out = emb(ids)
    w = emb.weight.data.cpu().numpy()
    assert np.array_equal(out.data.cpu().numpy(), w[ids % 10])
    g = rng.standard_normal((2, 3, 4)).astype(np.float32)
    (out * tg.Tensor(g, requires_grad=False)).sum().backward()
    assert np.array_equal(emb.weight.grad.cpu().numpy(), O.embedding_bwd(ids % 10, g, 10))
    with pytest.raises(IndexError):
        emb(np.array([10]))


@pytest.mark.parametrize("acc", [False, True])
def test_embedding_bwd_out_of_range_power_of_two_rows(cuda, acc):
    """Indices -V-1 and V with V a power of two share their low bits with the valid keys
    V-1 and 0; they must still be skipped, and rows V-1 and 0 summed exactly once (-1
    counts from the end: row V-1, in token order with the other 63s)."""
    V, dim = 64, 24
    rng = np.random.default_rng(21)
    idx = np.array([63, -65, 0, 64, 63, -1, 0, 64, 5] * 7)
    d = rng.standard_normal((idx.size, dim)).astype(np.float32)
    base = rng.standard_normal((V, dim)).astype(np.float32)
    grad = torch.tensor(base, device="cuda")
    L().embedding_bwd(torch.tensor(d, device="cuda"), torch.tensor(idx, device="cuda"), grad, acc)
    ok = (idx >= -V) & (idx < V)
    want = O.embedding_bwd(idx[ok] % V, d[ok], V)
    if acc:
        want = base + want.astype(np.float32)
    assert np.array_equal(grad.cpu().numpy(), want.astype(np.float32))


@pytest.mark.parametrize("R,C", [(1, 1), (100, 70), (130, 1000), (64, 128), (320, 192)])
@pytest.mark.parametrize("ds,dd", [(torch.float32, torch.float32), (torch.float16, torch.float32)])
def test_transpose_add(cuda, R, C, ds, dd):
    g = torch.Generator(device="cuda").manual_seed(R * C)
    src = torch.randn(R, C, device="cuda", generator=g).to(ds)
    dst = torch.randn(C, R, device="cuda", generator=g).to(dd)
    want = dst.double() + 0.5 * src.double().t()
    L().transpose_add(src, dst, 0.5)
    assert_close(dst, want.cpu().numpy(), RTOL_F32 if ds == torch.float32 else RTOL_F16, "dst")


def test_sync_tied_gradients(cuda):
    """source.grad += target.grad.T and the target's grad is reset
    (_training.py:264-284), for a source with and without a gradient yet."""
    import tensor_gpu_v2 as tg
    emb = tg.Embedding(6, 3)
    head = tg.Linear(3, 6, bias=False)
    tg.weight_tie(emb.weight, head, "w", transpose=True)
    model = tg.Module()
    model.emb, model.head = emb, head
    rng = np.random.default_rng(1)
    ht = rng.standard_normal((3, 6)).astype(np.float32)
    head.w.grad = ht
    emb.weight.zero_grad()
    tg.sync_tied_gradients(model)
    assert np.array_equal(emb.weight.grad.cpu().numpy(), ht.T)
    assert not head.w.grad.cpu().numpy().any()
    head.w.grad = ht
    tg.sync_tied_gradients(model)
    assert_close(emb.weight.grad, 2.0 * ht.T.astype(np.float64), RTOL_F32, "accumulated")


@pytest.mark.parametrize("dim,odt", [(1024, torch.float16), (64, torch.float32), (13, torch.bfloat16)])
def test_embedding_fwd_gather(cuda, dim, odt):
    """tg_embedding_fwd = weight[idx] cast to the output dtype, bit-exact with torch's
    gather + cast; negative indices wrap, indices outside [-V, V) give zero rows."""
    from tensor_gpu_v2 import _lib as L
    V = 300
    g = torch.Generator(device="cuda").manual_seed(dim)
    w = torch.randn(V, dim, device="cuda", generator=g)
    idx = torch.randint(-V, V, (5, 37), device="cuda", generator=g)
    out = L.embedding_fwd(w, idx, odt)
    want = w[torch.where(idx < 0, idx + V, idx)].to(odt)
    assert out.shape == (5, 37, dim) and torch.equal(out, want)
    bad = torch.tensor([V, -V - 1, 3], device="cuda")
    o2 = L.embedding_fwd(w, bad, odt)
    assert float(o2[:2].abs().sum()) == 0.0 and torch.equal(o2[2], w[3].to(odt))
