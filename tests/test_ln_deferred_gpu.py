"""LayerNorm parameter gradients finished together at the end of backward()
(tg_layernorm_bwd_partials + tg_sum_partials2_group) against the immediate per-layer
finish (tg_layernorm_bwd with dgamma/dbeta), bit for bit.  GPU only."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _grads(tg, deferred, dt, twice, seed=0, shared=False):
    from tensor_gpu_v2 import _lib as L
    rng = np.random.default_rng(seed)
    orig = L.layernorm_bwd_partials
    if not deferred:
        L.layernorm_bwd_partials = lambda *a, **k: None
    try:
        d = 256
        lns = [tg.LayerNorm(d) for _ in range(3)]
        # shared: the first module is applied again as the third (one gamma, two nodes)
        uses = [lns[0], lns[1], lns[0]] if shared else lns
        for ln in lns:
            ln.gamma.data = torch.as_tensor(1 + 0.1 * rng.standard_normal(d).astype(np.float32)).cuda()
            ln.beta.data = torch.as_tensor(0.1 * rng.standard_normal(d).astype(np.float32)).cuda()
        x = tg.Tensor(rng.standard_normal((64, 32, d)).astype(np.float32))
        for _ in range(2 if twice else 1):
            with tg.autocast(enabled=dt != torch.float32, dtype=dt):
                h = x * 1.0
                # the residual stream's gradient is shared with each LayerNorm input
                for ln in uses:
                    h = h + ln(h) * 0.5
                loss = (h * h).mean()
            loss.backward()
        out = [p.grad.clone() for ln in dict.fromkeys(uses) for p in (ln.gamma, ln.beta)]
        out.append(x.grad.clone())
    finally:
        L.layernorm_bwd_partials = orig
    return out


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("twice", [False, True])
def test_deferred_ln_param_grads_equal_immediate(cuda, tg, dt, twice):
    a = _grads(tg, True, dt, twice)
    b = _grads(tg, False, dt, twice)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_deferred_ln_shared_module(cuda, tg, dt):
    """A LayerNorm applied twice in one graph: the second node to run finds its gamma's
    finish queued, which runs first, so the two contributions add in the immediate
    order."""
    a = _grads(tg, True, dt, False, shared=True)
    b = _grads(tg, False, dt, False, shared=True)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_sum_partials2_group_matches_single(cuda):
    """Members of different K and widths in one launch, with and without accumulation,
    equal each finished on its own (tg_sum_partials2 through layernorm_bwd)."""
    from tensor_gpu_v2 import _lib as L
    g = torch.Generator(device="cuda").manual_seed(3)
    parts = [torch.randn(2, K, c, device="cuda", generator=g) for K, c in
             ((256, 1024), (7, 300), (2048, 64), (100, 4096))]
    dgs = [torch.randn(p.shape[2], device="cuda", generator=g) for p in parts]
    dbs = [torch.randn(p.shape[2], device="cuda", generator=g) for p in parts]
    accs = [True, False, True, False]
    want_g = [(d if a else 0) + p[0].sum(0) for p, d, a in zip(parts, dgs, accs)]
    got_g, got_b = [d.clone() for d in dgs], [b.clone() for b in dbs]
    L.sum_partials2_group(parts, got_g, got_b, accs)
    for w, gg in zip(want_g, got_g):
        torch.testing.assert_close(gg, w, rtol=1e-5, atol=1e-4)
    for p, b0, bb, a in zip(parts, dbs, got_b, accs):
        torch.testing.assert_close(bb, (b0 if a else 0) + p[1].sum(0), rtol=1e-5, atol=1e-4)
