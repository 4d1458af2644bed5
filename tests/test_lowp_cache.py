"""The autocast weight-cast cache: a leaf parameter's fp16/bf16 copy is reused
between forwards while the parameter is unchanged, rebuilt after an in-place torch
write (version counter), rewritten by the Adam pass (tg_adam_step_lowp), and every
other cached view of an updated storage is dropped.  The CPU tests exercise the
cache logic on host tensors; the GPU tests check the fused copy against a plain cast
and that autocast training with the cache gives bit-identical results to training
that recasts every forward (the reference's behaviour, _core.py:185-191)."""
import numpy as np
import pytest
import torch


def lowp():
    from tensor_gpu_v2 import _lowp
    _lowp.clear()
    return _lowp


def test_cast_reused_until_inplace_write():
    c = lowp()
    w = torch.randn(8, 4)
    a = c.cast(w, torch.float16)
    assert c.cast(w, torch.float16) is a
    assert torch.equal(a, w.half())
    w.mul_(2.0)  # advances torch's version counter
    b = c.cast(w, torch.float16)
    assert b is not a and torch.equal(b, w.half())
    # a different dtype is its own entry
    assert c.cast(w, torch.bfloat16).dtype == torch.bfloat16


def test_freed_source_never_validates():
    c = lowp()
    w = torch.randn(16)
    c.cast(w, torch.float16)
    sk = c._storage_key(w)
    (vk, e), = c._CACHE[sk].items()
    del w
    assert not c._valid(e)


def test_refresh_targets_keeps_exact_view_and_drops_others():
    c = lowp()
    w = torch.randn(6, 4)
    other = torch.randn(5)
    full = c.cast(w, torch.float16)
    c.cast(w[2:4], torch.float16)  # another (contiguous) view of the same storage
    c.cast(other, torch.float16)
    t = c.refresh_targets([w, torch.randn(3)])
    assert t[0] is full and t[1] is None
    views = c._CACHE[c._storage_key(w)]
    assert list(views) == [c._view_key(w, torch.float16)]
    assert c._storage_key(other) in c._CACHE  # untouched storage keeps its entry


def test_refresh_targets_one_dtype_and_stale_dropped():
    c = lowp()
    w1, w2, w3 = torch.randn(4), torch.randn(4), torch.randn(4)
    c.cast(w1, torch.float16)
    c.cast(w2, torch.bfloat16)
    c.cast(w3, torch.float16)
    w3.add_(1.0)  # stale entry
    t = c.refresh_targets([w1, w2, w3])
    assert t[0] is not None and t[0].dtype == torch.float16
    assert t[1] is None and not c._CACHE[c._storage_key(w2)]  # other dtype dropped
    assert t[2] is None and not c._CACHE[c._storage_key(w3)]  # stale dropped


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_adam_lowp_copy_matches_cast(cuda, dt):
    from tensor_gpu_v2 import _lib as L
    g = torch.Generator(device="cuda").manual_seed(3)
    sizes = [1000, 4096 * 3 + 5, 1, 70000]
    mk = lambda: [torch.randn(n, device="cuda", generator=g) for n in sizes]
    p0, gr, m0, v0 = mk(), mk(), mk(), [x.abs() for x in mk()]
    pa, ma, va = [x.clone() for x in p0], [x.clone() for x in m0], [x.clone() for x in v0]
    pb, mb, vb = [x.clone() for x in p0], [x.clone() for x in m0], [x.clone() for x in v0]
    cp = [torch.empty(n, device="cuda", dtype=dt) for n in sizes]
    cp[2] = None  # a param without a copy
    args = (3e-4, 0.9, 0.999, 1e-8, 0.1, 0.1, 0.001)
    L.adam_step(pa, gr, ma, va, None, *args)
    L.adam_step(pb, gr, mb, vb, None, *args, lowp=cp)
    for i in range(len(sizes)):
        assert torch.equal(pa[i], pb[i]) and torch.equal(ma[i], mb[i]) and torch.equal(va[i], vb[i])
        if cp[i] is not None:
            assert torch.equal(cp[i], pb[i].to(dt)), f"copy {i}"


@pytest.mark.gpu
def test_autocast_training_identical_with_and_without_cache(cuda):
    import tensor_gpu_v2 as tg
    from tensor_gpu_v2 import _lowp

    def run(use_cache, poke):
        _lowp.clear()
        rng = np.random.default_rng(0)
        l1, l2 = tg.Linear(64, 128), tg.Linear(128, 32)
        for lin in (l1, l2):
            lin.w.data = tg.Tensor((rng.standard_normal(lin.w.shape) * 0.1).astype(np.float32),
                                   requires_grad=False).data
        opt = tg.AdamW([l1.w, l1.b, l2.w, l2.b], lr=1e-2)
        x = tg.Tensor(rng.standard_normal((16, 64)).astype(np.float32), requires_grad=False)
        losses = []
        for step in range(4):
            if not use_cache:
                _lowp.clear()
            opt.zero_grad()
            with tg.autocast():
                loss = (l2(l1(x).gelu()) * 0.5).mean()
            loss.backward()
            opt.step()
            if poke and step == 1:
                l1.w.data.mul_(0.5)  # in-place torch write between steps
            losses.append(float(loss.item()))
        return losses, [t.data.clone() for t in (l1.w, l1.b, l2.w, l2.b)]

    for poke in (False, True):
        la, pa = run(True, poke)
        lb, pb = run(False, poke)
        assert la == lb, (poke, la, lb)
        for a, b in zip(pa, pb):
            assert torch.equal(a, b)


@pytest.mark.gpu
def test_autocast_tied_head_identical_with_and_without_cache(cuda):
    """Tied transposed head (the GPT configuration): the cached copy belongs to the
    embedding weight, which the optimizer updates."""
    import tensor_gpu_v2 as tg
    from tensor_gpu_v2 import _lowp

    def run(use_cache):
        _lowp.clear()
        rng = np.random.default_rng(1)
        V, d = 96, 32
        emb = tg.Embedding(V, d)
        emb.weight.data = tg.Tensor((rng.standard_normal((V, d)) * 0.1).astype(np.float32),
                                    requires_grad=False).data
        head = tg.Linear(d, V, bias=False)
        tg.weight_tie(emb.weight, head, "w", transpose=True)
        opt = tg.AdamW([emb.weight], lr=1e-2)
        ids = rng.integers(0, V, size=(4, 8))
        tgt = rng.integers(0, V, size=32)
        lossf = tg.CrossEntropyLoss()
        losses = []
        for _ in range(4):
            if not use_cache:
                _lowp.clear()
            opt.zero_grad()
            head.w.zero_grad()
            with tg.autocast():
                logits = head(emb(ids)).reshape(32, V)
                loss = lossf(logits, tgt)
            loss.backward()
            tg.sync_tied_gradients(_Holder(emb, head))
            opt.step()
            losses.append(float(loss.item()))
        return losses, emb.weight.data.clone()

    class _Holder(tg.Module):
        def __init__(self, emb, head):
            super().__init__()
            self.emb, self.head = emb, head

    la, wa = run(True)
    lb, wb = run(False)
    assert la == lb, (la, lb)
    assert torch.equal(wa, wb)


def test_cross_entropy_strict_chain_rule_needs_scalar_loss():
    import tensor_gpu_v2 as tg
    with pytest.raises(ValueError, match="strict_chain_rule"):
        tg.CrossEntropyLoss(reduction="none", strict_chain_rule=True)
    assert tg.CrossEntropyLoss(strict_chain_rule=True).strict_chain_rule
    assert not tg.CrossEntropyLoss().strict_chain_rule


def test_scalar_like_int_out_of_range_raises():
    """A Python int outside an integer tensor's dtype raises OverflowError, as NumPy 2's
    weak-scalar rule does, instead of wrapping (checked before any device work)."""
    import torch
    from tensor_gpu_v2._core import _scalar_like
    ref = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(OverflowError, match="out of bounds"):
        _scalar_like(2 ** 40, ref)
    with pytest.raises(OverflowError, match="out of bounds"):
        _scalar_like(-(2 ** 31) - 1, ref)
    with pytest.raises(OverflowError):
        _scalar_like(300, torch.zeros(2, dtype=torch.uint8))
