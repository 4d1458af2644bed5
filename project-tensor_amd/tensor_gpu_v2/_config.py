"""Global configuration: device, default dtype, grad mode and the autocast policy.

Mirrors the module globals and context managers of the reference
(tensor_gpu_v2/_core.py:116-398).  Tensors live on the GPU only: the reference's
NumPy 'cpu' device is its CPU path, which this engine does not reimplement
(device='cpu' raises).
"""
import functools

import numpy as np
import torch

_device = "cuda"
_default_dtype = np.dtype(np.float32)
_mixed_precision = False
_grad_enabled = True
_active_autocast_dtype = None  # numpy/torch dtype while autocast is active
# A GELU output consumed by exactly one Linear layer: the Linear's backward applies the
# GELU derivative in its input-gradient GEMM and the GELU output's own gradient is not
# formed (reading .grad of that intermediate then gives zeros).  False keeps the
# reference's materialised intermediate gradient (two kernels, same values).
fuse_gelu_backward = True

_NP_TO_TORCH = {
    np.dtype(np.float32): torch.float32,
    np.dtype(np.float16): torch.float16,
    np.dtype(np.float64): torch.float64,
    np.dtype(np.int64): torch.int64,
    np.dtype(np.int32): torch.int32,
    np.dtype(np.int16): torch.int16,
    np.dtype(np.int8): torch.int8,
    np.dtype(np.uint8): torch.uint8,
    np.dtype(np.bool_): torch.bool,
}
_TORCH_TO_NP = {v: k for k, v in _NP_TO_TORCH.items()}


def _canonicalize_device(device):
    """'cuda', 'gpu', 'cuda:N' -> 'cuda' (_core.py:131-142).  'cpu' is not served
    by this engine."""
    if device is None:
        return _device
    if not isinstance(device, str):
        raise TypeError(f"device must be a string, got {type(device).__name__}")
    d = device.strip().lower()
    if d == "cuda" or d.startswith("cuda:") or d == "gpu":
        return "cuda"
    if d == "cpu":
        raise NotImplementedError(
            "tensor_gpu_v2 (MI355X engine) runs on the GPU only; the reference's NumPy "
            "'cpu' device is not provided")
    raise ValueError(f"Unknown device: {device}")


def to_torch_dtype(dtype):
    """Accept numpy dtypes, dtype strings ('float16', 'bfloat16', ...) and torch dtypes."""
    if dtype is None:
        return None
    if isinstance(dtype, torch.dtype):
        return dtype
    if isinstance(dtype, str) and dtype.strip().lower() in ("bfloat16", "bf16"):
        return torch.bfloat16
    try:
        nd = np.dtype(dtype)
    except (TypeError, ValueError) as exc:
        raise TypeError(f"Invalid dtype: {dtype!r}") from exc
    if nd == np.dtype(np.object_):
        raise TypeError("object dtype is not supported")
    if nd not in _NP_TO_TORCH:
        raise TypeError(f"dtype {nd} is not supported on the device")
    return _NP_TO_TORCH[nd]


def to_numpy_dtype(tdtype):
    """numpy dtype for a torch dtype (bfloat16 has none: the torch dtype is returned)."""
    return _TORCH_TO_NP.get(tdtype, tdtype)


def resolve_dtype(inferred, explicit=None):
    """Target dtype of a new device tensor (_core.py:173-193): explicit dtype wins;
    inside autocast every floating tensor takes the autocast dtype; with the global
    mixed-precision flag floats wider than 2 bytes become float16."""
    if explicit is not None:
        return to_torch_dtype(explicit)
    if inferred is None:
        inferred = to_torch_dtype(_default_dtype)
    if _active_autocast_dtype is not None and inferred.is_floating_point:
        return to_torch_dtype(_active_autocast_dtype)
    if _mixed_precision and inferred.is_floating_point and inferred.itemsize > 2:
        return torch.float16
    return inferred


def set_device(device):
    global _device
    _device = _canonicalize_device(device)


def get_device():
    return _device


def enable_mixed_precision(enable=True):
    global _mixed_precision
    _mixed_precision = enable


def is_mixed_precision():
    return _mixed_precision


def get_default_dtype():
    return _default_dtype


def set_default_dtype(dtype):
    global _default_dtype
    _default_dtype = np.dtype(dtype)


def is_grad_enabled():
    return _grad_enabled


def set_grad_enabled(mode):
    global _grad_enabled
    _grad_enabled = bool(mode)


class _GradMode:
    _mode = True

    def __enter__(self):
        global _grad_enabled
        self._prev = _grad_enabled
        _grad_enabled = self._mode
        return self

    def __exit__(self, *args):
        global _grad_enabled
        _grad_enabled = self._prev

    def __call__(self, fn):
        mode_cls = type(self)

        @functools.wraps(fn)
        def wrapper(*a, **k):
            with mode_cls():
                return fn(*a, **k)
        return wrapper


class no_grad(_GradMode):
    """Disable graph recording in a block or decorated function (_core.py:233-268)."""
    _mode = False


class enable_grad(_GradMode):
    """Re-enable graph recording inside no_grad (_core.py:271-302)."""
    _mode = True


class autocast:
    """Mixed precision: inside the block every new floating device tensor takes
    `dtype` (default float16) (_core.py:328-398)."""

    def __init__(self, enabled=True, dtype=None):
        self.enabled = enabled
        if dtype is None:
            dtype = np.float16
        try:
            self._dtype = to_torch_dtype(dtype)
        except TypeError:
            self._dtype = torch.float16

    def __enter__(self):
        global _mixed_precision, _active_autocast_dtype
        self._prev_mp, self._prev_dtype = _mixed_precision, _active_autocast_dtype
        if self.enabled:
            _mixed_precision = True
            _active_autocast_dtype = self._dtype
        return self

    def __exit__(self, *args):
        global _mixed_precision, _active_autocast_dtype
        _mixed_precision, _active_autocast_dtype = self._prev_mp, self._prev_dtype

    def __call__(self, fn):
        enabled, dtype = self.enabled, self._dtype

        @functools.wraps(fn)
        def wrapper(*a, **k):
            with autocast(enabled=enabled, dtype=dtype):
                return fn(*a, **k)
        return wrapper


def autocast_dtype():
    return _active_autocast_dtype
