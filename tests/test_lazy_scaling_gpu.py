"""GradScaler.unscale_ and clip_grad_norm_ with their scalings left pending on the
gradients (applied by AdamW as it reads them), against the same steps with every
gradient rewritten in place (the reference's order: unscale _nn.py:1795-1833, clip
_nn.py:1563-1626, AdamW _nn.py:1413-1442).  The two must agree bit for bit: the norm,
the flags, every gradient value read back, and the parameters after the step.  GPU only."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture
def tg(cuda):
    import tensor_gpu_v2
    return tensor_gpu_v2


def L():
    from tensor_gpu_v2 import _lib
    return _lib


def _grads(dt, seed, n_small=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    sizes = [7, 3000, 5000, 4096 * 33 + 5, 1, 1 << 20] + [17 + 3 * i for i in range(n_small)]
    ts = [(torch.randn(n, device="cuda", generator=g) * 300).to(dt) for n in sizes]
    ts[2][1234] = float("inf")
    return ts


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n_small", [0, 130])  # 130 more tensors: several launches
def test_unscale_norm_matches_unscale_then_norm(cuda, dt, n_small):
    """tg_unscale_norm: the flags and the squared norm of the unscaled, flag-zeroed
    gradients, bit-exact against tg_unscale_check(write) + tg_zero_flagged +
    tg_grad_norm; the gradients themselves keep their scaled values except the zeroed
    ones."""
    inv = 1.0 / 1000.0  # not a power of two: the rounding of g * inv matters
    a = _grads(dt, 3, n_small)
    b = [t.clone() for t in a]
    raw = [t.clone() for t in a]
    flags_e = L().unscale_deferred(a, inv)()
    val_e, _ = L().grad_norm(a, 0)
    flags_l, val_l = L().unscale_norm_deferred(b, inv)()
    assert flags_l == flags_e and flags_l[2] != 0 and sum(f != 0 for f in flags_l) == 1
    assert val_l == val_e
    for i, (x, r) in enumerate(zip(b, raw)):
        if flags_l[i]:
            assert not torch.any(x != 0), i
        else:
            assert torch.equal(x, r), i
    L().scale_(b, inv)
    for i, (x, y) in enumerate(zip(b, a)):
        assert torch.equal(x, y), i


@pytest.mark.parametrize("lowp", [False, True])
def test_adam_scaled_matches_scaled_gradients(cuda, lowp):
    """tg_adam_step_scaled(m1, m2) on loss-scaled gradients = tg_adam_step(_lowp) after
    scaling the gradients in place by m1, then by m2: bit-exact parameters, moments and
    autocast copies."""
    g = torch.Generator(device="cuda").manual_seed(5)
    sizes = [64 * 32, 32, 1000, 4097]
    ps = [torch.randn(n, device="cuda", generator=g) for n in sizes]
    gs = [torch.randn(n, device="cuda", generator=g) * 4096 for n in sizes]
    ms = [torch.randn(n, device="cuda", generator=g) * 0.01 for n in sizes]
    vs = [torch.rand(n, device="cuda", generator=g) * 0.01 for n in sizes]
    m1, m2 = 1.0 / 4096, 0.37
    runs = []
    for scaled in (False, True):
        p2, g2, m2_, v2 = ([t.clone() for t in ts] for ts in (ps, gs, ms, vs))
        lp = [torch.empty(n, device="cuda", dtype=torch.float16) for n in sizes] if lowp else None
        launch = L().adam_prepare(p2, g2, m2_, v2, None, lowp=lp)
        if scaled:
            launch(1e-3, 0.9, 0.999, 1e-8, 0.1, 0.1, 0.001, gmul=(m1, m2))
        else:
            L().scale_(g2, m1)
            L().scale_(g2, m2)
            launch(1e-3, 0.9, 0.999, 1e-8, 0.1, 0.1, 0.001)
        runs.append((p2, m2_, v2, lp or []))
    for a, b in zip(*runs):
        for x, y in zip(a, b):
            assert torch.equal(x, y)


def _mlp(tg, seed):
    rng = np.random.default_rng(seed)
    l1, l2 = tg.Linear(64, 128), tg.Linear(128, 16)
    for lin in (l1, l2):
        lin.w.data = tg.Tensor(rng.standard_normal(lin.w.shape).astype(np.float32) * 0.2).data
    x = tg.Tensor(rng.standard_normal((256, 64)).astype(np.float32))
    return [l1.w, l1.b, l2.w, l2.b], lambda: (l2(l1(x).gelu()) ** 2).mean()


def _train(tg, mode, init_scale, max_norm, steps=3):
    """mode 'lazy': the plain recipe; 'eager': every gradient read right after unscale_
    (the read applies the pending unscale, so clip computes and rescales in place);
    'read': the lazy recipe with the gradients read after the clip.  Returns the
    parameters after each step, the clip norms, and the gradients read ('read' and
    'eager' modes, after the clip)."""
    params, loss_fn = _mlp(tg, 11)
    opt = tg.AdamW(params, lr=1e-2, weight_decay=0.1)
    sc = tg.GradScaler(init_scale=init_scale)
    out, norms, seen = [], [], []
    for _ in range(steps):
        for p in params:
            p.zero_grad()
        with tg.autocast():
            loss = loss_fn()
        sc.scale(loss).backward()
        sc.unscale_(opt)
        if mode == "eager":
            for p in params:
                p.grad
        norms.append(tg.clip_grad_norm_(params, max_norm))
        if mode in ("eager", "read"):
            seen.append([p.grad.clone() for p in params])
        sc.step(opt)
        sc.update()
        out.append([p.data.clone() for p in params])
    return out, norms, seen


@pytest.mark.parametrize("init_scale", [2.0 ** 12, 1000.0])
@pytest.mark.parametrize("max_norm", [1e-3, 1e3])  # clip active / inactive
def test_lazy_unscale_clip_step_matches_in_place(tg, init_scale, max_norm):
    lazy = _train(tg, "lazy", init_scale, max_norm)
    eager = _train(tg, "eager", init_scale, max_norm)
    read = _train(tg, "read", init_scale, max_norm)
    assert lazy[1] == eager[1] == read[1]  # clip norms
    if max_norm < 1:
        assert all(n > max_norm for n in lazy[1])
    for a, b, c in zip(lazy[0], eager[0], read[0]):
        for x, y, z in zip(a, b, c):
            assert torch.equal(x, y) and torch.equal(x, z)
    for a, b in zip(eager[2], read[2]):
        for x, y in zip(a, b):
            assert torch.equal(x, y)


def test_lazy_unscale_found_inf(tg):
    """A non-finite gradient: found_inf, the step skipped, the flagged gradient reads as
    zeros and the others as unscaled values; the next step (finite) runs."""
    params, loss_fn = _mlp(tg, 12)
    opt = tg.AdamW(params, lr=1e-2)
    sc = tg.GradScaler(init_scale=2.0 ** 10)
    with tg.autocast():
        loss = loss_fn()
    sc.scale(loss).backward()
    params[1].grad[3] = float("nan")
    raw = [p.grad.clone() for p in params]
    w0 = [p.data.clone() for p in params]
    sc.unscale_(opt)
    tg.clip_grad_norm_(params, 1e9)  # no clipping: the gradients are only unscaled
    sc.step(opt)
    sc.update()
    assert sc.get_scale() == 2.0 ** 9
    for p, w in zip(params, w0):
        assert torch.equal(p.data, w)
    assert not torch.any(params[1].grad != 0)
    for i in (0, 2, 3):
        assert torch.equal(params[i].grad, raw[i] * (1.0 / 2 ** 10)), i
    for p in params:
        p.zero_grad()
    with tg.autocast():
        loss = loss_fn()
    sc.scale(loss).backward()
    sc.unscale_(opt)
    tg.clip_grad_norm_(params, 1.0)
    sc.step(opt)
    assert any(not torch.equal(p.data, w) for p, w in zip(params, w0))


def test_clip_on_other_parameters_falls_back(tg):
    """clip_grad_norm_ over a different parameter list than unscale_'s: the in-place
    path, with the pending unscale applied first."""
    params, loss_fn = _mlp(tg, 13)
    opt = tg.AdamW(params, lr=1e-2)
    sc = tg.GradScaler(init_scale=2.0 ** 8)
    with tg.autocast():
        loss = loss_fn()
    sc.scale(loss).backward()
    raw = [p.grad.clone() for p in params]
    sc.unscale_(opt)
    n = tg.clip_grad_norm_(params[:2], 1e9)
    ref = sum(float((r.double() / 2 ** 8).pow(2).sum()) for r in raw[:2]) ** 0.5
    assert abs(n - ref) <= 1e-6 * ref
    for p, r in zip(params, raw):
        assert torch.equal(p.grad, r * (1.0 / 2 ** 8))


def test_pending_scalings_dropped_by_zero_grad_and_replacement(tg):
    """zero_grad() discards a gradient's pending factors (nothing is computed for a
    buffer being cleared), a replaced gradient (p.grad = ...) reads as given, and an
    untouched one reads as scaled."""
    from tensor_gpu_v2 import _core
    params, loss_fn = _mlp(tg, 14)
    opt = tg.AdamW(params, lr=1e-2)
    sc = tg.GradScaler(init_scale=2.0 ** 6)
    with tg.autocast():
        loss = loss_fn()
    sc.scale(loss).backward()
    raw = [p.grad.clone() for p in params]
    sc.unscale_(opt)
    assert all(_core._grad_factors(p) == (2.0 ** -6,) for p in params)
    params[0].zero_grad()
    assert id(params[0]) not in _core._GSCALE
    assert not torch.any(params[0].grad != 0)
    new = torch.full_like(raw[1], 3.0)
    params[1].grad = new
    assert id(params[1]) not in _core._GSCALE and torch.equal(params[1].grad, new)
    assert torch.equal(params[2].grad, raw[2] * (2.0 ** -6))
    assert id(params[2]) not in _core._GSCALE  # applied by the read
    assert _core._grad_factors(params[3]) == (2.0 ** -6,)
    for p in params:
        p.zero_grad()
    assert not any(id(p) in _core._GSCALE for p in params)


def test_pending_scaling_entry_leaves_with_its_tensor(tg):
    """A parameter dropped while a scaling is pending takes its entry with it."""
    import gc
    from tensor_gpu_v2 import _core
    p = tg.Tensor(np.ones(10, np.float32))
    p.grad = np.ones(10, np.float32)
    _core._grad_scale_pending(p, 0.5)
    k = id(p)
    assert k in _core._GSCALE
    del p
    gc.collect()
    assert k not in _core._GSCALE
