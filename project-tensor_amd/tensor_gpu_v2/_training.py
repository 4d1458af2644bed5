"""Training utilities on the gradient path (reference: tensor_gpu_v2/_training.py):
FusedAdam and weight tying."""
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
