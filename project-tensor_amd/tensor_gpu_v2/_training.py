"""Training utilities on the gradient path (reference: tensor_gpu_v2/_training.py):
FusedAdam, weight tying and the checkpoint file format."""
import importlib
import os
import pickle

import numpy as np
import torch

from . import _lib as L
from ._core import Tensor
from ._nn import Adam


class FusedAdam(Adam):
    """Adam whose step is one fused kernel pass over every fp32 parameter
    (_training.py:2223-2305; kernel _training.py:2198-2220).  step() takes no clip
    argument, like the reference."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        super().__init__(params, lr, betas, eps, weight_decay)

    def step(self):
        self._apply(self.lr, self.weight_decay)

    def state_dict(self):
        st = super().state_dict()
        st.pop("amsgrad", None)
        return st


class TiedWeight:
    """View of a source tensor (optionally transposed) (_training.py:171-201)."""

    def __init__(self, source, transpose=False):
        self.source = source
        self.transpose = transpose

    @property
    def data(self):
        return self.source.data.t() if self.transpose else self.source.data

    @property
    def grad(self):
        return None

    @property
    def shape(self):
        return tuple(self.data.shape)


def weight_tie(source, target_module, target_attr, transpose=False):
    """Make target_module.<target_attr> share source's storage, transposed if asked
    (_training.py:204-261).  Gradients reaching the target are folded into the
    source by sync_tied_gradients()."""
    target = getattr(target_module, target_attr)
    ss, ts = tuple(source.shape), tuple(target.shape)
    if transpose:
        exp = ss[::-1] if len(ss) == 2 else ss
        if ts != exp:
            raise ValueError(
                f"Shape mismatch for weight tying with transpose=True: source.T shape {exp} != "
                f"target shape {ts}. Source has shape {ss}.")
    elif ss != ts:
        raise ValueError(
            f"Shape mismatch for weight tying: source shape {ss} != target shape {ts}. "
            "Use transpose=True if shapes should be transposed.")
    target._tied_source = source
    target._tied_transpose = transpose
    target.data = source.data.t() if transpose else source.data


def sync_tied_gradients(model):
    """source.grad += target.grad (transposed when tied transposed), then reset the
    target's grad (_training.py:264-284)."""
    for p in model.parameters():
        try:
            src = p._tied_source
        except AttributeError:
            src = None
        if src is None or not p._has_grad():
            continue
        if src._has_grad():
            g = p.grad
            if p._tied_transpose and g.dim() == 2 and g.is_contiguous():
                buf, acc = src._grad_target()
                if not acc:
                    L.fill(buf, 0.0)
                L.transpose_add(g, buf)
            else:
                src._accumulate(g.t() if p._tied_transpose else g)
            p.zero_grad()


# ---------------------------------------------------------------- checkpoints
CHECKPOINT_VERSION = "1.0"


def _to_host(obj):
    """Device tensors -> NumPy arrays, recursively through dicts, lists and tuples, so a
    checkpoint holds only NumPy arrays and Python builtins (as the reference's does)."""
    if isinstance(obj, torch.Tensor):
        return obj.detach().cpu().numpy()
    if isinstance(obj, Tensor):
        return obj.numpy()
    if isinstance(obj, dict):
        return {k: _to_host(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return type(obj)(_to_host(v) for v in obj)
    return obj


def save_checkpoint(path, model, optimizer=None, scaler=None, scheduler=None, epoch=0,
                    global_step=0, extra_state=None):
    """Write a training checkpoint in the reference's layout (_training.py:19-64): one
    pickled dict with 'version', 'epoch', 'global_step', 'model_state_dict' (the
    model's `param_{i}` arrays) and, when given, 'optimizer_state_dict',
    'scaler_state_dict', 'scheduler_state_dict' {'last_epoch', 'base_lr'} and
    'extra_state'.  Arrays are stored as NumPy arrays, so files move between this
    engine and the reference in both directions."""
    ckpt = {"version": CHECKPOINT_VERSION, "epoch": epoch, "global_step": global_step,
            "model_state_dict": _to_host(model.state_dict())}
    if optimizer is not None and hasattr(optimizer, "state_dict"):
        ckpt["optimizer_state_dict"] = _to_host(optimizer.state_dict())
    if scaler is not None and hasattr(scaler, "state_dict"):
        ckpt["scaler_state_dict"] = _to_host(scaler.state_dict())
    if scheduler is not None:
        ckpt["scheduler_state_dict"] = {"last_epoch": scheduler.last_epoch,
                                        "base_lr": scheduler.base_lr}
    if extra_state:
        ckpt["extra_state"] = extra_state
    d = os.path.dirname(os.path.abspath(path))
    if d:
        os.makedirs(d, exist_ok=True)
    with open(path, "wb") as f:
        pickle.dump(ckpt, f)


_NP_ALLOWED = {
    ("numpy", "ndarray"), ("numpy", "dtype"),
    ("numpy.core.multiarray", "_reconstruct"), ("numpy._core.multiarray", "_reconstruct"),
    ("numpy.core.multiarray", "scalar"), ("numpy._core.multiarray", "scalar"),
    ("numpy.core.numeric", "_frombuffer"), ("numpy._core.numeric", "_frombuffer"),
}
_BUILTINS_ALLOWED = {"dict", "list", "set", "frozenset", "tuple", "int", "float", "complex",
                     "str", "bytes", "bool"}


class _CheckpointUnpickler(pickle.Unpickler):
    """Resolves only NumPy array reconstruction and builtin containers/scalars (the
    reference's SafeUnpickler, _training.py:67-88, admits the same plus CuPy, which is
    not used here); any other global is refused."""

    def find_class(self, module, name):
        if (module, name) in _NP_ALLOWED:
            mod = module.replace("numpy.core", "numpy._core") if hasattr(np, "_core") else module
            try:
                return getattr(importlib.import_module(mod), name)
            except (ImportError, AttributeError):
                return getattr(importlib.import_module(module), name)
        if module == "builtins" and name in _BUILTINS_ALLOWED:
            return getattr(importlib.import_module("builtins"), name)
        raise pickle.UnpicklingError(f"Global '{module}.{name}' is forbidden")


def load_checkpoint(path, model, optimizer=None, scaler=None, scheduler=None, strict=True):
    """Read a checkpoint written by save_checkpoint or by the reference
    (_training.py:91-134), restore the given objects and return {'epoch',
    'global_step', 'extra_state'}.  A version other than '1.0' warns, as the
    reference does."""
    with open(path, "rb") as f:
        ckpt = _CheckpointUnpickler(f).load()
    version = ckpt.get("version", "0.0")
    if version != CHECKPOINT_VERSION:
        import warnings
        warnings.warn(f"Checkpoint version {version} differs from current {CHECKPOINT_VERSION}")
    model.load_state_dict(ckpt["model_state_dict"])
    if optimizer is not None and "optimizer_state_dict" in ckpt:
        optimizer.load_state_dict(ckpt["optimizer_state_dict"])
    if scaler is not None and "scaler_state_dict" in ckpt:
        scaler.load_state_dict(ckpt["scaler_state_dict"])
    if scheduler is not None and "scheduler_state_dict" in ckpt:
        scheduler.last_epoch = ckpt["scheduler_state_dict"].get("last_epoch", -1)
    return {"epoch": ckpt.get("epoch", 0), "global_step": ckpt.get("global_step", 0),
            "extra_state": ckpt.get("extra_state", {})}
