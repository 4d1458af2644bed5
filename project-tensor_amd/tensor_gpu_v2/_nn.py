"""Modules, losses, optimizers and gradient tools (reference: tensor_gpu_v2/_nn.py).

The modules on the backward hot path — Linear (matmul + bias reduction),
LayerNorm, BatchNorm2D / FusedBatchNormReLU, Adam/AdamW, clip_grad_norm_,
GradScaler — run their gradient math in libtgbwd's HIP kernels.
"""
import math
import operator
import types
import warnings
import weakref

import numpy as np
import torch

from . import _config as cfg
from . import _lib as L
from . import _core, _lowp
from ._core import Tensor, _as, _linear, _linear_gelu, _linear_residual


def _targets(tensors):
    """Grad buffers for kernels that write several gradients with one accumulate
    flag: returns (buffers, accumulate); a tensor without grad yields None."""
    live = [t for t in tensors if t is not None and t._has_grad()]
    if live and all(t._gz for t in live):
        return [t._grad_target()[0] if (t is not None and t._has_grad()) else None
                for t in tensors], False
    bufs = []
    for t in tensors:
        bufs.append(t.grad if (t is not None and t._has_grad()) else None)
    return bufs, True


# ============================================================================ Module
_CLASS_NAMES = {}


def _walk_names(obj):
    """The public names ``dir(obj)`` lists, in its sorted order, minus those that are
    plain functions (or static/class methods) on the class and not shadowed by an
    instance attribute: those yield bound methods, never a Tensor, Module or list.
    Properties and class-level data are kept and evaluated by the caller."""
    cls = type(obj)
    names = _CLASS_NAMES.get(cls)
    if names is None:
        names = set()
        for name in dir(cls):
            if name.startswith("_"):
                continue
            for k in cls.__mro__:
                if name in k.__dict__:
                    if not isinstance(k.__dict__[name],
                                      (types.FunctionType, staticmethod, classmethod)):
                        names.add(name)
                    break
        names = frozenset(names)
        _CLASS_NAMES[cls] = names
    inst = getattr(obj, "__dict__", None)
    if inst:
        return sorted(names.union(n for n in inst if not n.startswith("_")))
    return sorted(names)


class Module:
    """Module base (_nn.py:24-255): parameter discovery over public attributes."""

    def __init__(self):
        self._device = cfg.get_device()
        self._training = True

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def zero_grad(self):
        for p in self.parameters():
            if p._has_grad():
                p.zero_grad()

    def named_parameters(self):
        params, seen = [], set()
        for name in _walk_names(self):
            try:
                attr = getattr(self, name)
            except AttributeError:
                continue
            if isinstance(attr, Tensor) and attr._requires_grad:
                if id(attr) not in seen:
                    params.append((name, attr))
                    seen.add(id(attr))
            elif isinstance(attr, Module) and attr is not self:
                for cn, cp in attr.named_parameters():
                    if id(cp) not in seen:
                        params.append((f"{name}.{cn}", cp))
                        seen.add(id(cp))
            elif isinstance(attr, (list, tuple)):
                for i, item in enumerate(attr):
                    if isinstance(item, Module):
                        for cn, cp in item.named_parameters():
                            if id(cp) not in seen:
                                params.append((f"{name}.{i}.{cn}", cp))
                                seen.add(id(cp))
        return params

    def parameters(self):
        return [p for _, p in self.named_parameters()]

    def named_modules(self, memo=None, prefix=""):
        if memo is None:
            memo = set()
        if id(self) in memo:
            return
        memo.add(id(self))
        yield prefix, self
        for name in dir(self):
            if name.startswith("_"):
                continue
            try:
                attr = getattr(self, name)
            except AttributeError:
                continue
            if isinstance(attr, Module) and attr is not self:
                yield from attr.named_modules(memo, prefix + ("." if prefix else "") + name)

    def _children(self):
        for name in dir(self):
            if name.startswith("_"):
                continue
            try:
                attr = getattr(self, name)
            except AttributeError:
                continue
            if isinstance(attr, Module) and attr is not self:
                yield attr
            elif isinstance(attr, (list, tuple)):
                for it in attr:
                    if isinstance(it, Module):
                        yield it

    def train(self):
        self._training = True
        for c in self._children():
            c.train()
        return self

    def eval(self):
        self._training = False
        for c in self._children():
            c.eval()
        return self

    def to(self, device):
        cfg._canonicalize_device(device)
        return self

    def cuda(self):
        return self

    def num_parameters(self):
        return sum(p.size for p in self.parameters())

    def state_dict(self):
        """`param_{i}` keys in parameters() order (_nn.py:180-185)."""
        return {f"param_{i}": p.numpy() for i, p in enumerate(self.parameters())}

    def load_state_dict(self, state):
        for i, p in enumerate(self.parameters()):
            k = f"param_{i}"
            if k in state:
                p.data = torch.as_tensor(np.asarray(state[k]), device="cuda").to(p.data.dtype)

    def __repr__(self):
        return f"{self.__class__.__name__}()"


# ============================================================================ Linear
class Linear(Module):
    """y = x @ w + b with w [nin, nout] (_nn.py:258-285).  Initialisation draws
    w ~ N(0,1)*sqrt(2/nin) from NumPy's global RNG (the reference draws from the
    array module's RNG), b = 0."""

    def __init__(self, nin, nout, bias=True):
        super().__init__()
        scale = np.float32(np.sqrt(2.0 / nin))
        self.w = Tensor(np.random.randn(nin, nout).astype(np.float32) * scale, dtype=np.float32)
        self.use_bias = bias
        self.b = Tensor(np.zeros(nout, dtype=np.float32), dtype=np.float32) if bias else None

    def __call__(self, x, *, activation=None, residual=None):
        """x @ w + b as one GEMM with the bias in its epilogue (same values and
        gradients as x @ w followed by + b).  Keyword options, not in the reference
        (which composes the ops): activation="gelu" returns gelu(x @ w + b) and
        residual=r returns r + (x @ w + b), each with the extra op applied in the same
        GEMM's epilogue where the fused kernel serves the shape (fp16 / bf16), values
        and graph identical to the separate ops."""
        b = self.b if self.use_bias else None
        if activation is not None and residual is not None:
            raise ValueError("Linear: activation and residual cannot be combined")
        if activation is not None:
            if activation != "gelu":
                raise ValueError(f"Linear: unsupported activation {activation!r}")
            return _linear_gelu(x, self.w, b)
        if residual is not None:
            return _linear_residual(x, self.w, b, residual)
        return _linear(x, self.w, b)

    def parameters(self):
        return [self.w, self.b] if self.use_bias else [self.w]

    def __repr__(self):
        nin, nout = self.w.shape
        return f"Linear(in_features={nin}, out_features={nout}, bias={self.use_bias})"


# ============================================================================ norms
class LayerNorm(Module):
    """LayerNorm over the trailing `normalized_shape` (_nn.py:885-951); forward saves
    mean/rstd per row, backward runs tg_layernorm_bwd (dx, dgamma, dbeta in one pass
    plus a partial-sum reduction)."""

    def __init__(self, normalized_shape, eps=1e-5):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        size = int(np.prod(self.normalized_shape))
        self.gamma = Tensor(np.ones(size, dtype=np.float32), dtype=np.float32)
        self.beta = Tensor(np.zeros(size, dtype=np.float32), dtype=np.float32)

    def __call__(self, x):
        nd = len(self.normalized_shape)
        if tuple(x.shape[-nd:]) != self.normalized_shape:
            raise ValueError(f"LayerNorm expects trailing shape {self.normalized_shape}, "
                             f"got {x.shape}")
        xd = x.data.contiguous()
        if xd.dtype not in L._TORCH_TO_CODE:
            raise TypeError(f"LayerNorm: unsupported dtype {xd.dtype}")
        g32 = self.gamma.data.float().contiguous()
        b32 = self.beta.data.float().contiguous()
        y, mean, rstd = L.layernorm_fwd(xd, g32, b32, self.eps)
        out = Tensor._wrap(y, (x, self.gamma, self.beta), "LayerNorm")
        self._cache = (mean, rstd)
        gamma, beta = self.gamma, self.beta

        if out._requires_grad:
            def _backward():
                dy = out._grad_out()
                if dy.dtype != xd.dtype or not dy.is_contiguous():
                    dy = dy.to(xd.dtype).contiguous()
                (dg, db), accp = _targets([gamma, beta])
                if dg is not None and dg.dtype != torch.float32 or db is not None and db.dtype != torch.float32:
                    raise TypeError("LayerNorm parameters must be float32")
                if x._has_grad():
                    dx, src = x._grad_target_add()
                    acc_dx = src is not None
                    add = src if src is not None and src is not dx else None
                else:
                    dx, acc_dx, add = torch.empty_like(xd), False, None
                # inside backward(), the parameter gradients' finishing sums are queued
                # and run with the other layers' in one launch when the sweep ends
                part = None
                if _core._WG_STATE[0] > 0 and (dg is not None or db is not None):
                    part = L.layernorm_bwd_partials(xd, mean, rstd, g32, dy, dx, acc_dx,
                                                    dx_add=add)
                if part is not None:
                    _core._ln_defer(part[0], gamma, dg, beta, db, accp)
                elif add is not None:  # x's gradient is shared: the sum goes to x's own buffer
                    L.layernorm_bwd(xd, mean, rstd, g32, dy, dx, dg, db, True, accp, dx_add=add)
                else:
                    L.layernorm_bwd(xd, mean, rstd, g32, dy, dx, dg, db, acc_dx, accp)
            out._backward = _backward
        return out

    def parameters(self):
        return [self.gamma, self.beta]

    def __repr__(self):
        return f"LayerNorm({self.normalized_shape}, eps={self.eps})"


class _BatchNormBase(Module):
    _relu = False

    def __init__(self, num_features, eps=1e-5, momentum=0.1, data_format="NCHW"):
        super().__init__()
        if data_format not in ("NCHW", "NHWC"):
            raise ValueError("data_format must be 'NCHW' or 'NHWC'")
        self.num_features = num_features
        self.eps = eps
        self.momentum = momentum
        self.data_format = data_format
        self.gamma = Tensor(np.ones(num_features, dtype=np.float32), dtype=np.float32)
        self.beta = Tensor(np.zeros(num_features, dtype=np.float32), dtype=np.float32)
        self.running_mean = torch.zeros(num_features, dtype=torch.float32, device="cuda")
        self.running_var = torch.ones(num_features, dtype=torch.float32, device="cuda")

    def _layout(self):
        return L.NHWC if self.data_format == "NHWC" else L.NCHW

    def __call__(self, x):
        if x.ndim != 4:
            raise ValueError(f"{type(self).__name__} expects a 4-D input, got {x.shape}")
        xd = x.data.contiguous()
        fp64 = xd.dtype == torch.float64
        if not fp64 and xd.dtype != torch.float32:
            xd = xd.float()
        C = xd.shape[3] if self.data_format == "NHWC" else xd.shape[1]
        if C != self.num_features:
            raise ValueError(f"expected {self.num_features} channels, got {C}")
        gamma, beta = self.gamma, self.beta
        g32 = gamma.data.float().contiguous()
        b32 = beta.data.float().contiguous()
        if not self._training:
            return self._eval_forward(x, xd, g32, b32)
        relu, layout = self._relu, self._layout()
        if fp64:
            # float64 data is computed in double (_nn.py:794-833 on float64 arrays); the
            # reference's running-stat update promotes its float32 buffers to float64
            self.running_mean = self.running_mean.to(torch.float64).contiguous()
            self.running_var = self.running_var.to(torch.float64).contiguous()
            y, mean, rstd, var = L.batchnorm_fwd_train_f64(
                xd, g32, b32, self.eps, self.momentum, self.running_mean, self.running_var,
                relu, layout)
        else:
            rm, rv = self.running_mean, self.running_var
            wide = rm.dtype != torch.float32  # float64 after an earlier float64 batch
            if wide:
                rm, rv = rm.float(), rv.float()
            y, mean, rstd, var = L.batchnorm_fwd_train(xd, g32, b32, self.eps, self.momentum,
                                                       rm, rv, relu, layout)
            if wide:
                self.running_mean.copy_(rm)
                self.running_var.copy_(rv)
        out = Tensor._wrap(y, (x, gamma, beta), type(self).__name__)
        self._cache = (mean, rstd)

        if out._requires_grad:
            def _backward():
                dy = out._grad_out()
                if dy.dtype != xd.dtype or not dy.is_contiguous():
                    dy = dy.to(xd.dtype).contiguous()
                (dg, db), accp = _targets([gamma, beta])
                direct = x._has_grad() and x.data.dtype == xd.dtype
                if direct:
                    dx, accx = x._grad_target()
                else:
                    dx, accx = torch.empty_like(xd), False
                if fp64:
                    L.batchnorm_bwd_stats(xd, mean, rstd, g32, b32, dy, dx, dg, db, relu, accx,
                                          accp, layout)
                else:
                    L.batchnorm_bwd(xd, mean, rstd, g32, b32, dy, dx, dg, db, relu, accx, accp,
                                    layout)
                if x._has_grad() and not direct:
                    x._accumulate(dx, True)
            out._backward = _backward
        return out

    def _eval_forward(self, x, xd, g32, b32):
        shp = (1, 1, 1, -1) if self.data_format == "NHWC" else (1, -1, 1, 1)
        rm, rv = self.running_mean, self.running_var
        if self._relu:
            # FusedBatchNormReLU inference (_nn.py:780-787, :857-862): fp32 scale and shift
            # folded from the running statistics, no graph
            inv = 1.0 / torch.sqrt(rv + self.eps)
            scale = (g32 * inv).to(torch.float32)
            shift = (b32 - g32 * rm * inv).to(torch.float32)
            y = torch.clamp_min(xd * scale.reshape(shp) + shift.reshape(shp), 0)
            return Tensor(y, requires_grad=False)
        # BatchNorm2D in eval mode (_nn.py:706-745) normalises with the running statistics
        # and keeps its backward, the training formula applied to those statistics
        inv = 1.0 / torch.sqrt(rv + self.eps)
        y = g32.to(xd.dtype).reshape(shp) * ((xd - rm.reshape(shp)) * inv.reshape(shp)) \
            + b32.to(xd.dtype).reshape(shp)
        y = y.to(torch.promote_types(xd.dtype, rm.dtype))
        gamma, beta = self.gamma, self.beta
        out = Tensor._wrap(y, (x, gamma, beta), type(self).__name__)
        if out._requires_grad:
            # std_inv in the running statistics' own dtype, as the reference forms it
            mean64 = rm.to(torch.float64).contiguous()
            rstd64 = inv.to(torch.float64).contiguous()
            layout = self._layout()

            def _backward():
                dy = out._grad_out()
                if dy.dtype != xd.dtype or not dy.is_contiguous():
                    dy = dy.to(xd.dtype).contiguous()
                (dg, db), accp = _targets([gamma, beta])
                direct = x._has_grad() and x.data.dtype == xd.dtype
                if direct:
                    dx, accx = x._grad_target()
                else:
                    dx, accx = torch.empty_like(xd), False
                L.batchnorm_bwd_stats(xd, mean64, rstd64, g32, b32, dy, dx, dg, db, False, accx,
                                      accp, layout)
                if x._has_grad() and not direct:
                    x._accumulate(dx, True)
            out._backward = _backward
        return out

    def parameters(self):
        return [self.gamma, self.beta]

    def __repr__(self):
        return (f"{type(self).__name__}({self.num_features}, eps={self.eps}, "
                f"momentum={self.momentum})")


class BatchNorm2D(_BatchNormBase):
    """BatchNorm over (N,H,W) per channel (_nn.py:681-747); data_format 'NCHW'
    (the reference layout) or 'NHWC'."""
    _relu = False


class FusedBatchNormReLU(_BatchNormBase):
    """Training-mode BatchNorm + ReLU (_nn.py:750-882) with the backward of
    _nn.py:812-833 fused into two HBM passes (tg_batchnorm_bwd).  data_format
    'NCHW' matches the reference; 'NHWC' is the channel-last layout."""
    _relu = True


# ============================================================================ misc modules
class Dropout(Module):
    """(_nn.py:1027-1058)"""

    def __init__(self, p=0.5):
        super().__init__()
        self.p = p

    def __call__(self, x):
        if not self._training or self.p == 0:
            return x
        if self.p >= 1.0:
            return Tensor._wrap(torch.zeros_like(x.data), (x,), "Dropout")
        mask = (torch.rand(x.data.shape, device="cuda") > self.p).to(x.data.dtype)
        scale = 1.0 / (1.0 - self.p)
        out = Tensor._wrap(x.data * mask * scale, (x,), "Dropout")
        if out._requires_grad:
            def _backward():
                if x._has_grad():
                    x._accumulate(out._grad_out() * mask * scale, True)
            out._backward = _backward
        return out


class Embedding(Module):
    """Lookup table (_nn.py:1061-1092): forward gathers rows, backward scatter-adds
    the output gradient rows into weight.grad (repeated indices accumulate)."""

    def __init__(self, num_embeddings, embedding_dim):
        super().__init__()
        self.weight = Tensor(np.random.randn(num_embeddings, embedding_dim).astype(np.float32)
                             * np.float32(0.01), dtype=np.float32)
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim

    def __call__(self, indices):
        V = self.num_embeddings
        if isinstance(indices, Tensor):
            idx = indices.data
        elif isinstance(indices, torch.Tensor):
            idx = indices
        else:
            host = np.asarray(indices)
            # checked here: an out-of-range gather on the device would assert in-kernel
            if host.size and (host.min() < -V or host.max() >= V):
                raise IndexError(f"Embedding: index outside [-{V}, {V})")
            idx = L.to_device(host.astype(np.int64, copy=False), self.weight.data.device)
        idx = idx.to(device=self.weight.data.device, dtype=torch.int64).contiguous()
        weight = self.weight
        # gather and the dtype policy's cast in one kernel; negative indices wrap
        w = weight.data if weight.data.is_contiguous() else weight.data.contiguous()
        rows = L.embedding_fwd(w, idx, cfg.resolve_dtype(w.dtype))
        out = Tensor._wrap(rows, (weight,), "Embedding")
        dim = self.embedding_dim
        flat = idx.reshape(-1)  # negative indices wrap in the backward kernels too
        if out._requires_grad:
            def _backward():
                if not weight._has_grad():
                    return
                g = out._grad_out().reshape(-1, dim).contiguous()
                buf, acc = weight._grad_target()
                L.embedding_bwd(g, flat, buf, acc)
            out._backward = _backward
        return out

    def parameters(self):
        return [self.weight]


# ============================================================================ losses
class MSELoss(Module):
    def __init__(self, reduction="mean"):
        super().__init__()
        self.reduction = reduction

    def __call__(self, y_pred, y_true):
        if not isinstance(y_true, Tensor):
            y_true = Tensor(y_true, requires_grad=False)
        sq = (y_pred - y_true) ** 2
        if self.reduction == "mean":
            return sq.mean()
        if self.reduction == "sum":
            return sq.sum()
        return sq


class CrossEntropyLoss(Module):
    """Cross-entropy over logits [N, C] (_nn.py:1128-1185).  As in the reference,
    the backward writes (softmax - onehot)/N (mean) into logits.grad without
    multiplying by the loss's upstream gradient (_nn.py:1168-1180), so a GradScaler
    loss scale never reaches the gradients.

    strict_chain_rule=True (not in the reference; default off) multiplies by the
    upstream gradient as the chain rule asks, so scaled fp16 gradients stay in fp16's
    normal range.  It needs a scalar loss (reduction 'mean' or 'sum'), keeps the loss
    in fp32 also under autocast (an fp16 loss times a 2^16 scale overflows fp16's
    65504, and so would its upstream gradient) and reads the upstream gradient back to
    the host once per backward."""

    def __init__(self, reduction="mean", label_smoothing=0.0, strict_chain_rule=False,
                 grad_in_forward=True):
        super().__init__()
        if strict_chain_rule and reduction not in ("mean", "sum"):
            raise ValueError("strict_chain_rule needs reduction 'mean' or 'sum'")
        self.reduction = reduction
        self.label_smoothing = label_smoothing
        self.strict_chain_rule = bool(strict_chain_rule)
        # One-pass mode (default): when grad mode is on and the logits require grad, the
        # forward also writes the logits' gradient (one more logits-sized write, and a
        # logits-sized buffer held by the loss graph until its backward runs or the
        # graph is dropped: 512 MiB at [8192, 32000] fp16).  False keeps the
        # reference's order: the gradient is formed only inside backward.
        self.grad_in_forward = bool(grad_in_forward)

    def __call__(self, logits, targets):
        ld = logits.data
        if ld.dim() != 2:
            raise ValueError(f"CrossEntropyLoss expects logits [N, C], got {tuple(ld.shape)}")
        N, C = ld.shape
        on_device = isinstance(targets, (Tensor, torch.Tensor))
        if on_device:
            tg = targets.data if isinstance(targets, Tensor) else targets
            tg = tg.to(device=ld.device, dtype=torch.int64).reshape(-1).contiguous()
            # negative targets wrap as in the reference (in the kernels); targets
            # outside [-C, C) are not checked on the device (that would need a
            # device-to-host read): their loss is NaN
        else:
            host = np.asarray(targets).astype(np.int64, copy=False).reshape(-1)
            # the reference indexes probs[arange(N), targets] (NumPy / CuPy indexing):
            # targets in [-C, 0) wrap, anything outside [-C, C) raises
            if host.size and (host.min() < -C or host.max() >= C):
                raise IndexError(f"CrossEntropyLoss: target outside [-{C}, {C})")
            tg = L.to_device(host, ld.device)  # negative targets wrap in the kernels
        if tg.numel() != N:
            raise ValueError(f"CrossEntropyLoss: {tg.numel()} targets for {N} rows")
        ldc = ld.contiguous()
        strict = self.strict_chain_rule
        scale = 1.0 / N if self.reduction == "mean" else 1.0
        smoothing = self.label_smoothing
        # The gradient does not depend on the upstream one (the reference's rule): when
        # a backward may follow, it is formed here, from the same read of the logits.
        pre = (self.grad_in_forward and not strict and smoothing == 0 and cfg._grad_enabled
               and logits._requires_grad and L.cross_entropy_fwd_grad_ok(ldc))
        grad = None
        if pre:
            lse, loss, grad = L.cross_entropy_fwd_grad(ldc, tg, scale)
        else:
            lse, loss = L.cross_entropy_fwd(ldc, tg, self.label_smoothing)
        if self.reduction == "mean":
            lv = loss.mean()
        elif self.reduction == "sum":
            lv = loss.sum()
        else:
            lv = loss
        out = Tensor._wrap(lv.to(ld.dtype), (logits,), "CrossEntropy")
        if strict:
            out.data = lv  # fp32, past the autocast cast of _wrap
        if out._requires_grad:
            def _backward():
                if not logits._has_grad():
                    return
                if grad is not None:
                    # formed by the forward: adopted as the logits' gradient buffer
                    # when it has none yet, else added
                    logits._accumulate(grad.reshape(ld.shape), owned=True)
                    return
                sc = scale * float(out._grad_out().reshape(-1)[0]) if strict else scale
                buf, acc = logits._grad_target()
                if buf.is_contiguous() and buf.shape == ldc.shape:
                    L.cross_entropy_bwd(ldc, tg, lse, buf, sc, acc, smoothing)
                else:
                    g = torch.empty_like(ldc)
                    L.cross_entropy_bwd(ldc, tg, lse, g, sc, False, smoothing)
                    logits._accumulate(g, True)
            out._backward = _backward
        return out


# ============================================================================ optimizers
class SGD:
    """(_nn.py:1316-1374)"""

    def __init__(self, params, lr=0.01, momentum=0.0, weight_decay=0.0, nesterov=False):
        self.params = list(params)
        self.lr, self.momentum, self.weight_decay, self.nesterov = lr, momentum, weight_decay, nesterov
        self._device = "cuda"
        self.velocities = [torch.zeros_like(p.data) for p in self.params]

    def step(self):
        for i, p in enumerate(self.params):
            if not p._has_grad():
                continue
            g = p.grad
            if self.weight_decay > 0:
                g = g + self.weight_decay * p.data
            if self.momentum > 0:
                self.velocities[i] = self.momentum * self.velocities[i] + g
                upd = g + self.momentum * self.velocities[i] if self.nesterov else self.velocities[i]
            else:
                upd = g
            p.data -= self.lr * upd

    def zero_grad(self):
        for p in self.params:
            if p._has_grad():
                p.zero_grad()

    def state_dict(self):
        """Hyper-parameters and momentum velocities, the reference's keys
        (_nn.py:1356-1364)."""
        return {"lr": self.lr, "momentum": self.momentum, "weight_decay": self.weight_decay,
                "nesterov": self.nesterov, "velocities": [v.cpu().numpy() for v in self.velocities]}

    def load_state_dict(self, state):
        """(_nn.py:1366-1374): missing keys keep the current values; velocities load as
        fp32."""
        self.lr = state.get("lr", self.lr)
        self.momentum = state.get("momentum", self.momentum)
        self.weight_decay = state.get("weight_decay", self.weight_decay)
        self.nesterov = state.get("nesterov", self.nesterov)
        if "velocities" in state:
            self.velocities = [torch.as_tensor(np.asarray(v, dtype=np.float32), device="cuda")
                               for v in state["velocities"]]


class Adam:
    """Adam with decoupled weight decay (_nn.py:1377-1480).  The step for every
    fp32 parameter is one multi-tensor launch of tg_adam_step (28 B/param)."""

    def __init__(self, params, lr=0.001, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                 amsgrad=False):
        self.params = list(params)
        self.lr = lr
        self.beta1, self.beta2 = betas
        self.eps = eps
        self.weight_decay = weight_decay
        self.amsgrad = amsgrad
        self._device = "cuda"
        self.m = [torch.zeros(p.data.shape, dtype=p.data.dtype, device="cuda") for p in self.params]
        self.v = [torch.zeros(p.data.shape, dtype=p.data.dtype, device="cuda") for p in self.params]
        if amsgrad:
            self.v_max = [torch.zeros_like(m) for m in self.m]
        self.t = 0

    def clip_grad_norm(self, max_norm=1.0):
        """Global L2 clip without NaN handling (_nn.py:1396-1411)."""
        grads = [p.grad for p in self.params if p._has_grad()]
        if not grads:
            return 0.0
        sq, _ = L.grad_norm(grads, 0)
        total = math.sqrt(sq)
        if total > max_norm:
            L.scale_(grads, max_norm / (total + 1e-6))
        return total

    def _plan(self):
        """Launchers of the step for the current gradient buffers: one multi-tensor
        launch per parameter dtype, fp32 (with the autocast copies) and fp64
        (parameters made from float64 arrays, updated in double), with every check and
        pointer array done here.  Returns (gradient buffers, lowp generation,
        launchers), or gradient buffers None when a gradient was converted to its
        parameter's dtype (the launcher then holds a copy that an in-place change of
        the gradient would not reach, so the plan is only good for an immediate
        launch); a plan is reused while its buffers and generation are unchanged."""
        groups = {}
        gbufs = []
        copied = False
        for i, p in enumerate(self.params):
            if not p._has_grad():
                gbufs.append(None)
                continue
            dt = p.data.dtype
            if dt not in (torch.float32, torch.float64) or not p.data.is_contiguous():
                raise TypeError("Adam: parameters must be contiguous float32 or float64 "
                                "device tensors")
            # a gradient with scalings pending is read as it is stored (the launch
            # applies them), unless it needs converting
            if _core._grad_factors(p) and p._g.dtype == dt:
                g = p._g
            else:
                g = p.grad
            gbufs.append(p._g)
            if g.dtype != dt:
                g = _as(g, dt)
                copied = True
            ps, gs, ms, vs, vms = groups.setdefault(dt, ([], [], [], [], []))
            ps.append(p.data)
            gs.append(g)
            ms.append(self.m[i])
            vs.append(self.v[i])
            if self.amsgrad:
                vms.append(self.v_max[i])
        launchers = [
            (dt, L.adam_prepare(ps, gs, ms, vs, vms if self.amsgrad else None,
                                lowp=_lowp.refresh_targets(ps) if dt == torch.float32 else None))
            for dt, (ps, gs, ms, vs, vms) in groups.items()]
        return (None if copied else gbufs), _lowp._GEN[0], launchers

    def _prepare(self):
        """Plan the next step now (GradScaler.unscale_ calls this while the device is
        still busy with the backward), so the step after the last read-back only
        launches."""
        self._planned = self._plan()

    def _apply(self, lr, wd):
        self.t += 1
        bc1 = 1 - self.beta1 ** self.t
        bc2 = 1 - self.beta2 ** self.t
        plan = getattr(self, "_planned", None)
        self._planned = None
        params = self.params
        live = [p for p in params if p._gz or p._g is not None]
        if plan is not None:
            gbufs, gen, _ = plan
            if (gbufs is None or gen != _lowp._GEN[0] or len(gbufs) != len(params)
                    or not all(map(operator.is_, gbufs,
                                   [p._g if (p._gz or p._g is not None) else None
                                    for p in params]))):
                plan = None
        if plan is None:
            plan = self._plan()
        # Scalings pending on the gradients (unscale, clip) go into the launch when every
        # fp32 gradient carries the same one or two; otherwise they are applied first.
        get = _core._GSCALE.get
        ents = [get(id(p)) for p in live]
        f32 = [p.data.dtype == torch.float32 for p in live]
        fac = {(e[1] if e is not None else ()) for e, is32 in zip(ents, f32) if is32}
        gmul = (1.0, 1.0)
        if len(fac) == 1 and 0 < len(next(iter(fac))) <= 2:
            f = next(iter(fac))
            gmul = (f[0], f[1] if len(f) > 1 else 1.0)
        else:
            fac = set()
        for p, e, is32 in zip(live, ents, f32):
            if e is not None and not (fac and is32):
                _core._settle(p)  # in place: the planned pointers stay valid
        for dt, launch in plan[2]:
            launch(lr, self.beta1, self.beta2, self.eps, wd, bc1, bc2,
                   gmul=gmul if dt == torch.float32 else (1.0, 1.0))

    def step(self, clip_grad_norm=None):
        if clip_grad_norm is not None:
            self.clip_grad_norm(clip_grad_norm)
        self._apply(self.lr, self.weight_decay)

    def zero_grad(self):
        for p in self.params:
            if p._has_grad():
                p.zero_grad()

    def state_dict(self):
        st = {"lr": self.lr, "betas": (self.beta1, self.beta2), "eps": self.eps,
              "weight_decay": self.weight_decay, "amsgrad": self.amsgrad, "t": self.t,
              "m": [m.cpu().numpy() for m in self.m], "v": [v.cpu().numpy() for v in self.v]}
        if self.amsgrad:
            st["v_max"] = [vm.cpu().numpy() for vm in self.v_max]
        return st

    def load_state_dict(self, state):
        self._planned = None  # a planned launch holds the moment buffers replaced below
        self.lr = state.get("lr", self.lr)
        self.t = state.get("t", self.t)
        if "betas" in state:
            self.beta1, self.beta2 = state["betas"]
        self.eps = state.get("eps", self.eps)
        self.weight_decay = state.get("weight_decay", self.weight_decay)
        # moments take their parameter's dtype (fp32, or fp64 for float64 parameters)
        def _load(vals):
            return [torch.as_tensor(np.asarray(v), device="cuda").to(p.data.dtype)
                    for v, p in zip(vals, self.params)]
        if "m" in state:
            self.m = _load(state["m"])
        if "v" in state:
            self.v = _load(state["v"])
        if self.amsgrad and "v_max" in state:
            self.v_max = _load(state["v_max"])


class AdamW(Adam):
    """Adam with decoupled weight decay, default 0.01 (_nn.py:1483-1487)."""

    def __init__(self, params, lr=0.001, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01):
        super().__init__(params, lr, betas, eps, weight_decay)


# ============================================================================ clipping
class _UnscaledNorm:
    """The squared L2 norm GradScaler.unscale_ formed for `params` while leaving the
    unscale pending; good for clip_grad_norm_ as long as every one of those gradients
    still holds the same buffer with only that scaling pending (any other access
    applies the scaling and ends the match)."""

    def __init__(self, params, inv, resolve):
        # weak: the cache must not keep a discarded model or a cleared gradient alive
        self.params = [weakref.ref(p) for p in params]
        self.bufs = [weakref.ref(p._g) for p in params]
        self.factors = (float(inv),)
        self.resolve = resolve

    def matches(self, params):
        if len(params) != len(self.params):
            return False
        for p, q, b in zip(params, self.params, self.bufs):
            if p is not q() or p._g is not b() or _core._grad_factors(p) != self.factors:
                return False
        return True


_NORM_CACHE = [None]


def clip_grad_norm_(parameters, max_norm, norm_type=2.0, error_if_nonfinite=False):
    """Global-norm clip (_nn.py:1563-1626): non-finite entries are zeroed (warning)
    or raise; the norm is one multi-tensor reduction; grads are rescaled by
    max_norm/(norm+1e-6) when that is < 1.  Returns the pre-clip norm.  Right after
    GradScaler.unscale_ over the same parameters, the norm that unscale_ formed is used
    and the rescale is left pending on the gradients like the unscale (the optimizer
    applies both as it reads them)."""
    params = [p for p in parameters if p._has_grad()]
    if not params:
        return 0.0
    cache, _NORM_CACHE[0] = _NORM_CACHE[0], None
    if norm_type == 2.0 and cache is not None and cache.matches(params):
        # flagged gradients were zeroed by unscale_: nothing non-finite is left
        value = cache.resolve()[1]
        total = value ** (1.0 / 2.0)
        if total == 0.0:
            return 0.0
        coef = max_norm / (total + 1e-6)
        if coef < 1.0:
            _core._grad_scale_pending_many(params, coef)
        return total
    grads = [p.grad for p in params]
    if norm_type == float("inf"):
        kind, pw = 1, 1.0
    elif norm_type == 2.0:
        kind, pw = 0, 2.0
    else:
        kind, pw = 2, float(norm_type)
    value, flags = L.grad_norm(grads, kind, pw)
    bad = [g for g, f in zip(grads, flags) if f & 1]
    if bad:
        if error_if_nonfinite:
            raise RuntimeError("Gradient contains NaN or Inf values")
        L.zero_nonfinite(bad)
        warnings.warn("clip_grad_norm_: Found NaN/Inf in gradients, zeroed them. "
                      "Consider reducing learning rate or checking loss computation.")
    total = value if kind == 1 else value ** (1.0 / pw)
    if total == 0.0:
        return 0.0
    coef = max_norm / (total + 1e-6)
    if coef < 1.0:
        L.scale_(grads, coef)
    return total


def clip_grad_value_(parameters, clip_value):
    """(_nn.py:1629-1640)"""
    for p in parameters:
        if p._has_grad():
            p.grad.clamp_(-clip_value, clip_value)


# ============================================================================ GradScaler
class GradScaler:
    """Dynamic loss scaling (_nn.py:1713-1912).  unscale_ is one multi-tensor
    kernel pass (scale + non-finite flags) instead of the reference's per-parameter
    host checks; with zero_nan_grads the flagged gradients are zeroed on the device and
    the flags are read back only when found_inf is first needed (step, update), which
    after clip_grad_norm_'s own read-back costs no further synchronisation.  The scale
    state machine is unchanged."""

    def __init__(self, init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5,
                 growth_interval=2000, min_scale=1.0, max_scale=2 ** 24, enabled=True):
        if init_scale <= 0:
            raise ValueError(f"init_scale must be positive, got {init_scale}")
        if min_scale <= 0:
            raise ValueError(f"min_scale must be positive, got {min_scale}")
        if max_scale < init_scale:
            raise ValueError(f"max_scale ({max_scale}) must be >= init_scale ({init_scale})")
        self._scale = init_scale
        self.growth_factor = growth_factor
        self.backoff_factor = backoff_factor
        self.growth_interval = growth_interval
        self.min_scale = min_scale
        self.max_scale = max_scale
        self.enabled = enabled
        self._growth_tracker = 0
        self._pending = None
        self._found_inf = False
        self._overflow_count = 0
        self._step_count = 0
        self._consecutive_successes = 0

    @property
    def _found_inf(self):
        if self._pending is not None:
            resolve, self._pending = self._pending, None
            self._found_inf_v = any(f != 0 for f in resolve())
        return self._found_inf_v

    @_found_inf.setter
    def _found_inf(self, value):
        self._pending = None
        self._found_inf_v = bool(value)

    def scale(self, loss):
        if not self.enabled:
            return loss
        return loss * self._scale

    def unscale_(self, optimizer, zero_nan_grads=True):
        if not self.enabled:
            return
        if getattr(optimizer, "_is_unscaled", False):
            return
        inv = 1.0 / self._scale
        self._found_inf = False
        params = [p for p in optimizer.params if p._has_grad()]
        grads = [p.grad for p in params]
        if grads and zero_nan_grads and all(
                g.dtype in (torch.float32, torch.float16, torch.bfloat16) for g in grads):
            # One read-only pass: flags, the zeroing of flagged gradients, and the norm
            # clip_grad_norm_ would compute next.  The unscale itself stays pending on
            # the gradients (applied by the optimizer as it reads them, or by any other
            # access first); found_inf is read lazily.
            resolve = L.unscale_norm_deferred(grads, inv)
            for p in params:
                _core._grad_scale_pending(p, inv)
            _NORM_CACHE[0] = _UnscaledNorm(params, inv, resolve)
            self._pending = lambda: resolve()[0]
            prep = getattr(optimizer, "_prepare", None)
            if prep is not None:
                prep()
        elif grads and zero_nan_grads:
            # flagged gradients are zeroed on the device; found_inf is read lazily
            self._pending = L.unscale_deferred(grads, inv)
            prep = getattr(optimizer, "_prepare", None)
            if prep is not None:
                prep()
        elif grads:
            # pre-existing non-finite gradients are left as they are (not unscaled)
            pre = L.unscale_check(grads, 1.0, write=False)
            clean = [g for g, f in zip(grads, pre) if not (f & 1)]
            post = L.unscale_check(clean, inv, write=True) if clean else []
            if any(f & 1 for f in pre) or any(post):
                self._found_inf = True
        optimizer._is_unscaled = True

    def step(self, optimizer, clip_grad_norm=None):
        if not self.enabled:
            optimizer.step(clip_grad_norm=clip_grad_norm)
            return
        if not getattr(optimizer, "_is_unscaled", False):
            self.unscale_(optimizer)
        if self._found_inf:
            optimizer._is_unscaled = False
            return
        optimizer.step(clip_grad_norm=clip_grad_norm)
        optimizer._is_unscaled = False

    def update(self):
        if not self.enabled:
            return
        self._step_count += 1
        if self._found_inf:
            self._overflow_count += 1
            self._consecutive_successes = 0
            self._scale = max(self._scale * self.backoff_factor, self.min_scale)
            self._growth_tracker = 0
        else:
            self._consecutive_successes += 1
            self._growth_tracker += 1
            if self._growth_tracker >= self.growth_interval:
                self._scale = min(self._scale * self.growth_factor, self.max_scale)
                self._growth_tracker = 0

    @property
    def scale_factor(self):
        return self._scale

    def get_scale(self):
        return self._scale

    def state_dict(self):
        return {"scale": self._scale, "growth_tracker": self._growth_tracker,
                "overflow_count": self._overflow_count, "step_count": self._step_count,
                "consecutive_successes": self._consecutive_successes}

    def load_state_dict(self, state):
        s = state.get("scale", self._scale)
        if s <= 0:
            raise ValueError(f"Checkpoint contains invalid scale ({s}), must be positive")
        self._scale = s
        self._growth_tracker = state.get("growth_tracker", 0)
        self._overflow_count = state.get("overflow_count", 0)
        self._step_count = state.get("step_count", 0)
        self._consecutive_successes = state.get("consecutive_successes", 0)

    def get_statistics(self):
        return {"current_scale": self._scale, "total_steps": self._step_count,
                "overflow_count": self._overflow_count,
                "overflow_rate": self._overflow_count / max(1, self._step_count),
                "consecutive_successes": self._consecutive_successes}
