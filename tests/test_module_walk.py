"""Module.named_parameters (reference _nn.py:71-94) walks dir(self): public names in
sorted order, Tensors that require grad, child Modules recursively, first name wins
for a shared Tensor.  The walk skips names that are plain methods on the class; these
CPU tests check that the result equals the plain dir() walk, names and order, on
modules with nested children, lists, properties, class-level tensors, shared and
frozen parameters.  Tensors are built without device storage (no GPU here)."""
import pytest


def _fake_tensor(requires_grad=True):
    from tensor_gpu_v2 import Tensor
    t = Tensor.__new__(Tensor)
    t._requires_grad = requires_grad
    return t


def _dir_walk(mod):
    """The plain dir()-based walk the reference performs."""
    from tensor_gpu_v2 import Tensor
    from tensor_gpu_v2._nn import Module
    params, seen = [], set()
    for name in dir(mod):
        if name.startswith("_"):
            continue
        try:
            attr = getattr(mod, name)
        except AttributeError:
            continue
        if isinstance(attr, Tensor) and attr._requires_grad:
            if id(attr) not in seen:
                params.append((name, attr))
                seen.add(id(attr))
        elif isinstance(attr, Module) and attr is not mod:
            for cn, cp in _dir_walk(attr):
                if id(cp) not in seen:
                    params.append((f"{name}.{cn}", cp))
                    seen.add(id(cp))
        elif isinstance(attr, (list, tuple)):
            for i, item in enumerate(attr):
                if isinstance(item, Module):
                    for cn, cp in _dir_walk(item):
                        if id(cp) not in seen:
                            params.append((f"{name}.{i}.{cn}", cp))
                            seen.add(id(cp))
    return params


def _make():
    from tensor_gpu_v2._nn import Module

    class Leaf(Module):
        cls_param = _fake_tensor()  # class-level tensor: listed by dir(), kept

        def __init__(self):
            super().__init__()
            self.w = _fake_tensor()
            self.b = _fake_tensor()
            self.frozen = _fake_tensor(requires_grad=False)

        @property
        def alias(self):  # a property is evaluated like any attribute
            return self.w

        @property
        def broken(self):
            raise AttributeError("not available")

        def forward(self, x):
            return x

    class Root(Module):
        def __init__(self):
            super().__init__()
            self.z_first = Leaf()
            self.blocks = [Leaf(), Leaf()]
            self.a_shared = self.z_first.w  # shared: first name in sorted order wins
            self.forward = _fake_tensor()  # instance attribute shadowing a method name

        def helper(self):
            return 1

    return Root()


def test_walk_matches_dir_walk():
    root = _make()
    got = root.named_parameters()
    want = _dir_walk(root)
    assert [n for n, _ in got] == [n for n, _ in want]
    assert all(a is b for (_, a), (_, b) in zip(got, want))
    names = [n for n, _ in got]
    assert "a_shared" in names and "forward" in names
    assert not any(n.endswith("frozen") for n in names)
    assert any(n.endswith("cls_param") for n in names)
    assert root.parameters() == [p for _, p in want]


def test_walk_sees_attributes_added_later():
    root = _make()
    before = len(root.named_parameters())
    root.zz_late = _fake_tensor()
    got = root.named_parameters()
    assert len(got) == before + 1 and got[-1][0] == "zz_late"
    assert [n for n, _ in got] == [n for n, _ in _dir_walk(root)]
