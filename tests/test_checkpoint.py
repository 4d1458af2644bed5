"""Checkpoint file format (reference _training.py:19-166): the pickled dict layout, the
round trip of model / optimizer / scaler / scheduler state, and the restricted loader.
The CPU tests use stand-in objects with state_dict()/load_state_dict(); the GPU test
round-trips real modules."""
import os
import pickle

import numpy as np
import pytest


def tr():
    from tensor_gpu_v2 import _training
    return _training


class _Obj:
    def __init__(self, state):
        self.state = state
        self.loaded = None

    def state_dict(self):
        return self.state

    def load_state_dict(self, st):
        self.loaded = st


class _Sched:
    last_epoch, base_lr = 7, 0.01


def test_layout_and_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    model = _Obj({"param_0": rng.standard_normal((3, 4)).astype(np.float32),
                  "param_1": np.zeros(4, np.float32)})
    opt = _Obj({"lr": 1e-3, "betas": (0.9, 0.999), "t": 5,
                "m": [np.ones(3, np.float32)], "v": [np.full(3, 2.0, np.float32)]})
    scaler = _Obj({"scale": 65536.0, "growth_tracker": 3})
    path = os.path.join(tmp_path, "sub", "ck.pkl")
    tr().save_checkpoint(path, model, opt, scaler, _Sched(), epoch=2, global_step=40,
                         extra_state={"note": "x"})
    with open(path, "rb") as f:
        raw = pickle.load(f)   # a file this test wrote itself
    assert raw["version"] == "1.0" and raw["epoch"] == 2 and raw["global_step"] == 40
    assert set(raw["model_state_dict"]) == {"param_0", "param_1"}
    assert raw["scheduler_state_dict"] == {"last_epoch": 7, "base_lr": 0.01}
    m2, o2, s2, sch = _Obj({}), _Obj({}), _Obj({}), _Sched()
    sch.last_epoch = -1
    info = tr().load_checkpoint(path, m2, o2, s2, sch)
    assert info == {"epoch": 2, "global_step": 40, "extra_state": {"note": "x"}}
    np.testing.assert_array_equal(m2.loaded["param_0"], model.state["param_0"])
    assert o2.loaded["betas"] == (0.9, 0.999) and o2.loaded["t"] == 5
    np.testing.assert_array_equal(o2.loaded["v"][0], opt.state["v"][0])
    assert s2.loaded == scaler.state and sch.last_epoch == 7


def test_loader_refuses_other_globals(tmp_path):
    class Evil:
        def __reduce__(self):
            return (os.getcwd, ())
    path = os.path.join(tmp_path, "evil.pkl")
    with open(path, "wb") as f:
        pickle.dump({"version": "1.0", "model_state_dict": Evil()}, f)
    with pytest.raises(pickle.UnpicklingError):
        tr().load_checkpoint(path, _Obj({}))


def test_version_mismatch_warns(tmp_path):
    path = os.path.join(tmp_path, "old.pkl")
    with open(path, "wb") as f:
        pickle.dump({"version": "0.9", "model_state_dict": {}}, f)
    with pytest.warns(UserWarning):
        tr().load_checkpoint(path, _Obj({}))


@pytest.mark.gpu
def test_real_modules_round_trip(cuda, tmp_path):
    import tensor_gpu_v2 as tg
    np.random.seed(3)
    lin = tg.Linear(16, 8)
    opt = tg.AdamW(lin.parameters(), lr=1e-2)
    scaler = tg.GradScaler(init_scale=1024.0)
    x = tg.Tensor(np.random.randn(4, 16).astype(np.float32), requires_grad=False)
    (lin(x) * lin(x)).sum().backward()
    opt.step()
    path = os.path.join(tmp_path, "real.pkl")
    tg.save_checkpoint(path, lin, opt, scaler, epoch=1, global_step=9)
    lin2 = tg.Linear(16, 8)
    opt2 = tg.AdamW(lin2.parameters(), lr=1e-3)
    scaler2 = tg.GradScaler()
    info = tg.load_checkpoint(path, lin2, opt2, scaler2)
    assert info["global_step"] == 9
    for a, b in zip(lin.parameters(), lin2.parameters()):
        assert np.array_equal(a.numpy(), b.numpy())
    assert opt2.t == opt.t and opt2.lr == opt.lr
    for a, b in zip(opt.m + opt.v, opt2.m + opt2.v):
        assert bool((a == b).all())
    assert scaler2.get_scale() == 1024.0
