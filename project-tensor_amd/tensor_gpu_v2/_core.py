"""Autograd Tensor with the reference's API (tensor_gpu_v2/_core.py:609-1467).

Storage is a torch device tensor (torch serves as allocator and stream
provider).  Every gradient on the backward hot path — activation, softmax,
matmul, broadcast reductions, attention, normalisation — runs in libtgbwd's
HIP kernels through _lib; view/reshape bookkeeping and the elementwise
arithmetic of ops outside the hot path use device tensor ops, the role CuPy
plays for the reference.

Gradient buffers are allocated lazily: a tensor that records gradients starts
with an implicit zero gradient (the reference allocates zeros eagerly,
_core.py:637).  The first contribution is written straight into a fresh buffer
(kernel `accumulate` = 0), later ones accumulate (`accumulate` = 1), which is
the reference's `parent.grad += local` with one read pass fewer.  Reading
`.grad` materialises the zeros, so observable behaviour matches.
"""

import weakref

import numpy as np
import torch

from . import _config as cfg
from . import _lib as L
from . import _lowp


def _noop():
    return None


# ------------------------------------------------------- deferred weight gradients
# During Tensor.backward() a 16-bit Linear layer's weight (and bias) gradient is queued
# instead of computed at once; the queue is flushed before backward() returns, with the
# equal-shaped products of all layers run as one grouped launch (L.wgrad_group).  Each
# queued parameter leaf has already claimed its gradient buffer; any other access to
# that gradient first flushes the queue, so the order of accumulation is unchanged.
_WG_QUEUE = []       # (A2, G2, wbuf, wacc, bbuf, bacc) in sweep order
_LN_QUEUE = []       # LayerNorm parameter gradients: (partials, dgamma buf, dbeta buf, acc)
_WG_TARGETS = {}     # id -> Tensor whose gradient a queued record writes
_WG_STATE = [0, 0]   # [backward nesting depth, bytes of operands the queue keeps alive]
_WG_MAX_BYTES = 4 << 30  # flush early once the queue keeps this much alive


# ------------------------------------------------------- pending gradient scalings
# GradScaler.unscale_ and clip_grad_norm_ may leave their factor pending on a parameter's
# gradient instead of rewriting it: _GSCALE[id(t)] = (t, (f1, f2, ...)) means the
# gradient is its buffer scaled in place by f1, then by f2, ... (one fp32 rounding each).
# The optimizer applies the factors as it reads the buffers; any other access to the
# gradient applies them first (_settle), so every value read is the rewritten one.  The
# tensor is held weakly: an entry leaves with its tensor (no model is kept alive by it,
# and a later object reusing the id never inherits its factors).
_GSCALE = {}


def _grad_scale_pending(t, factor):
    """Record one more pending in-place scaling of t's gradient buffer by factor."""
    k = id(t)
    e = _GSCALE.get(k)
    if e is not None:
        _GSCALE[k] = (e[0], e[1] + (float(factor),))
        return

    def _gone(ref, k=k):
        cur = _GSCALE.get(k)
        if cur is not None and cur[0] is ref:
            del _GSCALE[k]
    _GSCALE[k] = (weakref.ref(t, _gone), (float(factor),))


def _grad_scale_pending_many(ts, factor):
    """_grad_scale_pending for each of ts with one factor (the common case, tensors that
    already carry an entry, handled inline)."""
    f = (float(factor),)
    get = _GSCALE.get
    for t in ts:
        k = id(t)
        e = get(k)
        if e is not None:
            _GSCALE[k] = (e[0], e[1] + f)
        else:
            _grad_scale_pending(t, f[0])


def _grad_factors(t):
    """Pending scaling factors of t's gradient (empty tuple: none)."""
    e = _GSCALE.get(id(t))
    return e[1] if e is not None else ()


def _settle(t, drop=False):
    """Before an access to t's gradient: run the queued weight-gradient products if
    one writes it, then apply its pending scalings (drop: discard them, the buffer is
    being replaced or cleared)."""
    if _WG_TARGETS and id(t) in _WG_TARGETS:
        _wgrad_flush()
    e = _GSCALE.pop(id(t), None)
    if e is not None and not drop and t._g is not None:
        for f in e[1]:
            L.scale_([t._g], f)


def _wgrad_defer(A2, G2, w, wbuf, wacc, b=None, bbuf=None, bacc=False):
    _WG_QUEUE.append((A2, G2, wbuf, wacc, bbuf, bacc))
    _WG_TARGETS[id(w)] = w
    if b is not None:
        _WG_TARGETS[id(b)] = b
    _WG_STATE[1] += A2.numel() * A2.element_size() + G2.numel() * G2.element_size()
    if _WG_STATE[1] > _WG_MAX_BYTES:
        _wgrad_flush()


def _ln_defer(partials, gamma, dg, beta, db, acc):
    """Queue the finish of a LayerNorm's parameter gradients (dg/db: the claimed
    gradient buffers, either may be None) from its partial sums."""
    _LN_QUEUE.append((partials, dg, db, acc))
    for p, b in ((gamma, dg), (beta, db)):
        if b is not None:
            _WG_TARGETS[id(p)] = p
    _WG_STATE[1] += partials.numel() * 4
    if _WG_STATE[1] > _WG_MAX_BYTES:
        _wgrad_flush()


def _wgrad_flush():
    """Run the queued weight-gradient products: records of one input shape [K, M] and
    dtype set (any output width N) as one grouped call, in the order their groups first
    appear; and the queued LayerNorm parameter-gradient finishes, all in one launch."""
    if not _WG_QUEUE and not _LN_QUEUE:
        return
    recs = list(_WG_QUEUE)
    lns = list(_LN_QUEUE)
    _WG_QUEUE.clear()
    _LN_QUEUE.clear()
    _WG_TARGETS.clear()
    _WG_STATE[1] = 0
    if lns:
        L.sum_partials2_group([r[0] for r in lns], [r[1] for r in lns], [r[2] for r in lns],
                              [r[3] for r in lns])
    groups = {}
    for r in recs:
        A2, G2, wbuf, _, bbuf, _ = r
        key = (tuple(A2.shape), A2.dtype, wbuf.dtype, None if bbuf is None else bbuf.dtype)
        groups.setdefault(key, []).append(r)
    for (a_shape, _, _, _), rs in groups.items():
        K = a_shape[1]
        if len(rs) == 1:
            A2, G2, wbuf, wacc, bbuf, bacc = rs[0]
            N = G2.shape[1]
            L.wgrad(A2, G2, wbuf.view(K, N), wacc, None if bbuf is None else bbuf.view(N), bacc)
        else:
            has_b = rs[0][4] is not None
            L.wgrad_group([r[0] for r in rs], [r[1] for r in rs],
                          [r[2].view(K, r[1].shape[1]) for r in rs], [r[3] for r in rs],
                          [r[4].view(r[1].shape[1]) for r in rs] if has_b else None,
                          [r[5] for r in rs] if has_b else None)


def _to_device_tensor(data, dtype):
    """Convert array-likes / torch tensors to a device tensor of `dtype` (or the
    inferred dtype when None).  Returns (tensor, inferred_dtype)."""
    if isinstance(data, Tensor):
        data = data.data
    if isinstance(data, torch.Tensor):
        t = data
        inferred = t.dtype
    else:
        arr = np.asarray(data)
        if arr.dtype == np.object_:
            raise TypeError("object dtype is not supported")
        inferred = cfg.to_torch_dtype(arr.dtype) if arr.dtype.kind != "U" else None
        if inferred is None:
            raise TypeError(f"unsupported data of dtype {arr.dtype}")
        # (np.ascontiguousarray would turn a 0-d array into shape (1,))
        t = torch.from_numpy(arr if arr.flags.c_contiguous else np.ascontiguousarray(arr))
    return t, inferred


class Tensor:
    """Autograd tensor on the MI355X (reference: _core.py:609-1467)."""

    __slots__ = ("data", "_g", "_gz", "_gsh", "_backward", "_prev", "_op", "label", "_device",
                 "_requires_grad", "_is_view", "_base", "_grad_fn", "__weakref__",
                 "_tied_source", "_tied_transpose", "_nuse", "_act")

    def __init__(self, data, _children=(), _op="", label="", device=None, requires_grad=True,
                 dtype=None):
        device = cfg._canonicalize_device(device or cfg._device)
        t, inferred = _to_device_tensor(data, dtype)
        target = cfg.resolve_dtype(inferred, dtype)
        if t.device.type != "cuda":
            try:  # pinned staging, non-blocking copy; the dtype cast runs on the device
                t = L.to_device(t.numpy())
            except (TypeError, RuntimeError):
                t = t.to(device="cuda")
        if t.dtype != target:
            t = t.to(target)
        self.data = t
        rg = bool(requires_grad) and cfg._grad_enabled
        self._g = None
        self._gz = rg  # implicit zero gradient
        self._gsh = False  # _g may alias another node's gradient (copy-on-write)
        self._backward = _noop
        self._prev = _unique(_children)
        self._nuse = 0  # graph nodes recorded with this tensor as an operand
        self._act = None  # GELU output: (input tensor, its contiguous data)
        for c in self._prev:
            c._nuse += 1
        self._op = _op
        self.label = label
        self._device = device
        self._requires_grad = rg
        self._is_view = False
        self._base = None
        self._grad_fn = None

    # ------------------------------------------------------------ construction
    @staticmethod
    def _wrap(t, children=(), op="", requires_grad=True):
        """Fast constructor for op outputs already on the device; applies the dtype
        policy (autocast) like Tensor.__init__."""
        out = object.__new__(Tensor)
        target = cfg.resolve_dtype(t.dtype)
        out.data = t if t.dtype == target else t.to(target)
        rg = requires_grad and cfg._grad_enabled
        out._g = None
        out._gz = rg
        out._gsh = False
        out._backward = _noop
        out._prev = _unique(children) if rg else ()
        out._nuse = 0
        out._act = None
        for c in out._prev:
            c._nuse += 1
        out._op = op
        out.label = ""
        out._device = "cuda"
        out._requires_grad = rg
        out._is_view = False
        out._base = None
        out._grad_fn = None
        return out

    @staticmethod
    def _create_view_fast(data, device="cuda", requires_grad=False):
        """(_core.py:763-778)"""
        out = Tensor._wrap(data, (), "", requires_grad)
        out.data = data
        out._is_view = True
        return out

    @staticmethod
    def randn(*shape, device=None, requires_grad=True, dtype=None):
        """Standard-normal tensor drawn from NumPy's global RNG (so np.random.seed
        makes it reproducible), then moved to the device."""
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        return Tensor(np.random.randn(*shape).astype(np.float32), device=device,
                      requires_grad=requires_grad, dtype=dtype)

    @staticmethod
    def zeros(*shape, device=None, requires_grad=True, dtype=None):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        return Tensor(np.zeros(shape, dtype=np.float32), device=device,
                      requires_grad=requires_grad, dtype=dtype)

    @staticmethod
    def ones(*shape, device=None, requires_grad=True, dtype=None):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        return Tensor(np.ones(shape, dtype=np.float32), device=device,
                      requires_grad=requires_grad, dtype=dtype)

    # ------------------------------------------------------------ grad storage
    def _new_buf(self, fill=None):
        d = self.data
        buf = torch.empty(d.shape, dtype=d.dtype, device=d.device)
        if fill is not None:
            _fill(buf, fill)
        return buf

    @property
    def grad(self):
        if _WG_TARGETS or _GSCALE:
            _settle(self)
        if self._gz:
            self._g = self._new_buf(0)
            self._gz = False
        elif self._gsh or (self._g is not None and not self._g.is_contiguous()):
            self._privatize()
        return self._g

    @grad.setter
    def grad(self, value):
        if _WG_TARGETS or _GSCALE:
            _settle(self, drop=True)
        self._gz = False
        self._gsh = False
        if value is None:
            self._g = None
            return
        if isinstance(value, Tensor):
            value = value.data
        if not isinstance(value, torch.Tensor):
            value = torch.as_tensor(np.asarray(value))
        if value.device.type != "cuda":
            value = value.to("cuda")
        if not value.is_contiguous():
            value = value.contiguous()
        self._g = value

    def _has_grad(self):
        return self._gz or self._g is not None

    def _grad_out(self):
        """Gradient flowing into this node's closure (zeros if nothing arrived).
        Read-only: it may be shared with other nodes."""
        if _WG_TARGETS or _GSCALE:
            _settle(self)
        if self._gz:
            return self._new_buf(0)
        return self._g

    def _privatize(self):
        """Give this node its own contiguous copy of a gradient buffer it shares (or
        holds with strides)."""
        if _WG_TARGETS or _GSCALE:
            _settle(self)
        buf = self._new_buf()
        _copy_into(buf, self._g)
        self._g = buf
        self._gsh = False

    def _grad_target(self):
        """(buffer, accumulate) for a kernel that adds this tensor's gradient."""
        if _WG_TARGETS or _GSCALE:
            _settle(self)
        if self._gz:
            self._g = self._new_buf()
            self._gz = False
            return self._g, False
        if self._gsh or not self._g.is_contiguous():
            self._privatize()
        return self._g, True

    def _grad_target_add(self):
        """(buffer, source) for a kernel that writes buffer = its result + source:
        source None means no prior gradient (overwrite).  A gradient shared with
        another node is not copied first: the kernel reads it as the source and writes
        this tensor's own new buffer; otherwise source is the buffer itself."""
        if _WG_TARGETS or _GSCALE:
            _settle(self)
        if (not self._gz and self._gsh and self._g.is_contiguous()
                and self._g.dtype == self.data.dtype and self._g.shape == self.data.shape):
            src = self._g
            self._g = self._new_buf()
            self._gsh = False
            return self._g, src
        buf, acc = self._grad_target()
        return buf, (buf if acc else None)

    def _share_grad(self, donor, g):
        """First gradient of this node is `g`, a read-only view of donor's gradient
        buffer (the reshape/view/transpose/add pass-through).  Adopted without a copy,
        also when it is a permuted view of a dense buffer (a transpose's gradient);
        both nodes are marked shared, so the first in-place write to either one
        copies (out of place for an accumulation, which moves no more bytes than the
        in-place one would)."""
        if _WG_TARGETS or _GSCALE:
            _settle(self)
        if not self._gz or g.dtype != self.data.dtype or not (g.is_contiguous() or _dense(g)):
            self._accumulate(g)
            return
        if g.shape != self.data.shape:
            if not g.is_contiguous():  # a strided buffer is only adopted in its own shape
                self._accumulate(g)
                return
            g = g.reshape(self.data.shape)
        self._g = g
        self._gz = False
        self._gsh = True
        donor._gsh = True

    def _accumulate_unb(self, g, donor=None):
        """self.grad += unbroadcast(g).  The reduced tensor is fresh (owned) unless no
        reduction was needed, in which case it is `g` itself: another node's gradient,
        adopted as a shared buffer when the donor is known, else copied."""
        u = _unbroadcast_dev(g, self.data.shape, self.data.dtype)
        if u is g and donor is not None:
            self._share_grad(donor, g)
        else:
            self._accumulate(u, owned=u is not g)

    def _accumulate(self, g, owned=False):
        """self.grad += g (g: torch tensor broadcast-compatible in shape, any float dtype)."""
        if _WG_TARGETS or _GSCALE:
            _settle(self)
        if not self._has_grad():
            return
        if g.shape != self.data.shape:
            g = g.reshape(self.data.shape)
        if self._gz:
            self._gz = False
            if owned and g.dtype == self.data.dtype and (g.is_contiguous() or _dense(g)):
                # an owned strided buffer (e.g. a head-split attention gradient) is kept
                # as is; the first write or read through .grad makes it contiguous
                self._g = g
            else:
                buf = self._new_buf()
                _copy_into(buf, g)
                self._g = buf
            return
        if (g.is_contiguous() and self._g.is_contiguous() and g.dtype in L._TORCH_TO_CODE
                and self._g.dtype in L._TORCH_TO_CODE):
            if self._gsh:
                self._g = L.axpbyz(g, self._g, 1.0, 1.0)
                self._gsh = False
            else:
                L.axpby(g, self._g, 1.0, 1.0)
        else:
            if self._gsh or not self._g.is_contiguous():
                self._privatize()
            L.broadcast_mul_sum(self._g, g, accumulate=True)

    # ------------------------------------------------------------ properties
    @property
    def xp(self):
        return torch

    @property
    def shape(self):
        return tuple(self.data.shape)

    @property
    def ndim(self):
        return self.data.dim()

    @property
    def dtype(self):
        return cfg.to_numpy_dtype(self.data.dtype)

    @property
    def size(self):
        return self.data.numel()

    @property
    def T(self):
        return self.transpose()

    @property
    def requires_grad(self):
        return self._requires_grad

    def to(self, device):
        cfg._canonicalize_device(device)
        return self

    def cuda(self):
        return self

    def cpu(self):
        return self.to("cpu")

    def numpy(self):
        t = self.data
        if t.dtype == torch.bfloat16:
            t = t.float()
        return t.detach().cpu().numpy()

    def item(self):
        return float(self.data.reshape(-1)[0]) if self.data.numel() == 1 else float(self.data)

    def clone(self):
        return Tensor(self.data.clone(), requires_grad=self._requires_grad)

    def detach(self):
        return Tensor(self.data.clone(), requires_grad=False)

    def contiguous(self):
        if self.data.is_contiguous():
            return self
        return Tensor(self.data.contiguous(), requires_grad=self._requires_grad)

    def half(self):
        return Tensor(self.data.to(torch.float16), requires_grad=self._requires_grad,
                      dtype=np.float16)

    def float(self):
        return Tensor(self.data.to(torch.float32), requires_grad=self._requires_grad,
                      dtype=np.float32)

    def zero_grad(self):
        if _WG_TARGETS or _GSCALE:
            _settle(self, drop=True)
        if self._has_grad():
            self._g = None
            self._gz = True
            self._gsh = False

    def __repr__(self):
        rg = f", requires_grad={self._requires_grad}" if self._requires_grad else ""
        op = f", op='{self._op}'" if self._op else ""
        return f"Tensor({list(self.data.shape)}, dtype={self.dtype}, device='cuda'{op}{rg})"

    def __len__(self):
        return self.data.shape[0]

    # ------------------------------------------------------------ helpers
    def _other(self, other):
        return other if isinstance(other, Tensor) else Tensor(
            _scalar_like(other, self.data), requires_grad=False)

    def _out(self, t, children, op):
        return Tensor._wrap(t, children, op)

    # ------------------------------------------------------------ arithmetic
    def __add__(self, other):
        other = self._other(other)
        return self._add_node(other, self.data + other.data)

    def _add_node(self, other, data):
        """The node of self + other with its sum already computed (data)."""
        out = self._out(data, (self, other), "+")
        if out._requires_grad:
            def _backward():
                g = out._grad_out()
                if self._has_grad():
                    self._accumulate_unb(g, out)
                if other._has_grad():
                    other._accumulate_unb(g, out)
            out._backward = _backward
        return out

    def __radd__(self, other):
        return self + other

    def __mul__(self, other):
        if (type(other) is float or (type(other) is int and -(1 << 53) <= other <= 1 << 53)) \
                and self.data.is_floating_point():
            return self._scalar_mul(other)
        other = self._other(other)
        out = self._out(self.data * other.data, (self, other), "*")
        if out._requires_grad:
            def _backward():
                g = out._grad_out()
                # t.grad (+)= unbroadcast(u * g): one strided multiply-and-sum kernel
                for t, u in ((self, other), (other, self)):
                    if t._has_grad():
                        _check_unbroadcast(tuple(g.shape), tuple(t.data.shape))
                        buf, acc = t._grad_target()
                        L.broadcast_mul_sum(buf, g, u.data, accumulate=acc)
            out._backward = _backward
        return out

    def _scalar_mul(self, v):
        """self * v for a Python scalar v and a floating tensor: v rounded to the
        tensor's dtype (the NumPy 2 weak-scalar rule, as the device scalar of the
        general path is), one multiply, and g * v in the backward; the same values as
        the general path, with no scalar tensor made on the device."""
        vr = _round_scalar(v, self.data.dtype)
        out = self._out(self.data * vr, (self,), "*")
        if out._requires_grad:
            def _backward():
                if self._has_grad():
                    g = out._grad_out()
                    buf, acc = self._grad_target()
                    L.broadcast_mul_sum(buf, g, alpha=vr, accumulate=acc)
            out._backward = _backward
        return out

    def __rmul__(self, other):
        return self * other

    def __pow__(self, other):
        assert isinstance(other, (int, float)), "only supporting int/float powers"
        out = self._out(self.data ** other, (self,), f"**{other}")
        if out._requires_grad:
            # (other * x ** (other - 1)) * g (_core.py:973-981) on tg_unary_bwd; a / b
            # reaches here as a * b ** -1 (_core.py:993-995)
            out._backward = _unary_backward(self, out, "pow", False, float(other))
        return out

    def __neg__(self):
        return self * -1

    def __sub__(self, other):
        return self + (-other)

    def __rsub__(self, other):
        return other + (-self)

    def __truediv__(self, other):
        return self * (other ** -1)

    def __rtruediv__(self, other):
        return other * (self ** -1)

    def __matmul__(self, other):
        other = self._other(other)
        return _matmul(self, other)

    # ------------------------------------------------------------ reductions
    def sum(self, axis=None, keepdims=False):
        if axis is None:
            r = self.data.sum()
            if keepdims:
                r = r.reshape((1,) * self.data.dim())
        else:
            r = self.data.sum(dim=axis, keepdim=keepdims)
        out = self._out(r, (self,), "sum")
        if out._requires_grad:
            def _backward():
                if not self._has_grad():
                    return
                g = out._grad_out()
                if not keepdims and axis is not None:
                    axes = (axis,) if isinstance(axis, int) else tuple(axis)
                    for ax in sorted(a % self.data.dim() for a in axes):
                        g = g.unsqueeze(ax)
                elif not keepdims:
                    g = g.reshape((1,) * self.data.dim())
                buf, acc = self._grad_target()  # a broadcast fill of the upstream grad
                L.broadcast_mul_sum(buf, g, accumulate=acc)
            out._backward = _backward
        return out

    def mean(self, axis=None, keepdims=False):
        s = self.sum(axis=axis, keepdims=keepdims)
        if axis is None:
            n = self.data.numel()
        else:
            axes = (axis,) if isinstance(axis, int) else axis
            n = int(np.prod([self.data.shape[i] for i in axes]))
        return s * (1.0 / float(n))

    def var(self, axis=None, keepdims=False, correction=0):
        m = self.mean(axis=axis, keepdims=True)
        d = self - m
        sq = d ** 2
        if axis is None:
            n = self.data.numel()
        else:
            axes = (axis,) if isinstance(axis, int) else axis
            n = int(np.prod([self.data.shape[i] for i in axes]))
        return sq.sum(axis=axis, keepdims=keepdims) * (1.0 / float(n - correction))

    def std(self, axis=None, keepdims=False, correction=0):
        return (self.var(axis=axis, keepdims=keepdims, correction=correction) + 1e-8) ** 0.5

    def max(self, axis=None, keepdims=False):
        if axis is None:
            r = self.data.max()
        else:
            r = self.data.amax(dim=axis, keepdim=keepdims)
        out = self._out(r, (self,), "max")
        if out._requires_grad:
            def _backward():
                # mask * g / count(mask) over the reduced axes (_core.py:1115-1132) on
                # tg_max_bwd: x is viewed as [kept, reduced] (the reduced axes moved
                # last by the strided copy kernel when they are not already last)
                if not self._has_grad():
                    return
                dt = self.data.dtype
                shape = tuple(self.data.shape)
                nd = len(shape)
                if axis is None:
                    red = tuple(range(nd))
                else:
                    red = tuple(sorted(a % nd for a in ((axis,) if isinstance(axis, int)
                                                        else axis)))
                perm = [d for d in range(nd) if d not in red] + list(red)
                outer = int(np.prod([shape[d] for d in perm[:nd - len(red)]]))
                nred = int(np.prod([shape[d] for d in red]))
                ident = perm == list(range(nd))
                x2 = _as(self.data if ident else self.data.permute(perm), dt).reshape(outer, nred)
                r2 = _as(r, dt).reshape(outer)
                g2 = _as(out._grad_out(), dt).reshape(outer)
                if ident:
                    buf, acc = self._grad_target()
                    L.max_bwd(x2, r2, g2, buf.reshape(outer, nred), acc)
                else:
                    dx2 = L.max_bwd(x2, r2, g2, torch.empty_like(x2), False)
                    inv = [perm.index(d) for d in range(nd)]
                    self._accumulate(dx2.reshape([shape[d] for d in perm]).permute(inv), True)
            out._backward = _backward
        return out

    def min(self, axis=None, keepdims=False):
        return (-self).max(axis=axis, keepdims=keepdims) * -1

    def argmax(self, axis=None):
        return self.data.argmax() if axis is None else self.data.argmax(dim=axis)

    def argmin(self, axis=None):
        return self.data.argmin() if axis is None else self.data.argmin(dim=axis)

    # ------------------------------------------------------------ activations
    def gelu(self):
        """tanh-approx GELU; forward and backward on libtgbwd (_core.py:1172-1209)."""
        return _activation(self, "gelu")

    def silu(self):
        """SiLU; forward and backward on libtgbwd (_core.py:1211-1246)."""
        return _activation(self, "silu")

    def relu(self):
        out = self._out(torch.clamp_min(self.data, 0), (self,), "ReLU")
        if out._requires_grad:  # (y > 0) * g (_core.py:1149-1157)
            out._backward = _unary_backward(self, out, "relu", True)
        return out

    def leaky_relu(self, negative_slope=0.01):
        out = self._out(torch.where(self.data >= 0, self.data, negative_slope * self.data),
                        (self,), "LeakyReLU")
        if out._requires_grad:  # where(x >= 0, 1, slope) * g (_core.py:1159-1170)
            out._backward = _unary_backward(self, out, "leaky_relu", False, float(negative_slope))
        return out

    def swish(self, beta=1.0):
        if beta == 1.0:
            return self.silu()
        s = torch.sigmoid(beta * self.data)
        out = self._out(self.data * s, (self,), "Swish")
        if out._requires_grad:  # (s + beta*x*s*(1 - s)) * g (_core.py:1248-1260)
            out._backward = _unary_backward(self, out, "swish", False, float(beta))
        return out

    def sigmoid(self):
        out = self._out(torch.sigmoid(self.data), (self,), "sigmoid")
        if out._requires_grad:  # y * (1 - y) * g (_core.py:1262-1272)
            out._backward = _unary_backward(self, out, "sigmoid", True)
        return out

    def tanh(self):
        out = self._out(torch.tanh(self.data), (self,), "tanh")
        if out._requires_grad:  # (1 - y**2) * g (_core.py:1274-1282)
            out._backward = _unary_backward(self, out, "tanh", True)
        return out

    def exp(self):
        out = self._out(torch.exp(self.data), (self,), "exp")
        if out._requires_grad:  # y * g
            out._backward = _unary_backward(self, out, "exp", True)
        return out

    def log(self):
        out = self._out(torch.log(self.data), (self,), "log")
        if out._requires_grad:  # g / x
            out._backward = _unary_backward(self, out, "log", False)
        return out

    def softmax(self, axis=-1):
        """Softmax; forward and backward on libtgbwd along the last axis
        (_core.py:1286-1299); other axes are moved last around the kernel."""
        nd = self.data.dim()
        ax = axis % nd if nd else 0
        moved = nd > 0 and ax != nd - 1
        x = self.data.movedim(ax, -1).contiguous() if moved else self.data.contiguous()
        if x.dtype not in L._TORCH_TO_CODE:
            raise TypeError(f"softmax: unsupported dtype {x.dtype}")
        y = L.softmax_fwd(x)
        out = self._out(y.movedim(-1, ax) if moved else y, (self,), "softmax")
        if out._requires_grad:
            def _backward():
                if not self._has_grad():
                    return
                dt = self.data.dtype
                yy = _as(out.data.movedim(ax, -1) if moved else out.data, dt)
                g = out._grad_out()
                g = _as(g.movedim(ax, -1) if moved else g, dt)
                if moved:
                    dx = L.softmax_bwd(yy, g, torch.empty_like(yy), False)
                    self._accumulate(dx.movedim(-1, ax), True)
                else:
                    buf, acc = self._grad_target()
                    L.softmax_bwd(yy, g, buf, acc)
            out._backward = _backward
        return out

    def log_softmax(self, axis=-1):
        r = torch.log_softmax(self.data.float(), dim=axis).to(self.data.dtype)
        out = self._out(r, (self,), "log_softmax")
        if out._requires_grad:
            nd = self.data.dim()
            ax = axis % nd if nd else 0
            moved = nd > 0 and ax != nd - 1

            def _backward():
                # g - exp(y) * sum(g, axis) (_core.py:1301-1314) on tg_log_softmax_bwd;
                # other axes are moved last around the kernel
                if not self._has_grad():
                    return
                dt = self.data.dtype
                yy = out.data.movedim(ax, -1) if moved else out.data
                g = out._grad_out()
                yy = _as(yy, dt)
                g = _as(g.movedim(ax, -1) if moved else g, dt)
                if moved:
                    dx = L.log_softmax_bwd(yy, g, torch.empty_like(yy), False)
                    self._accumulate(dx.movedim(-1, ax), True)
                else:
                    buf, acc = self._grad_target()
                    L.log_softmax_bwd(yy, g, buf, acc)
            out._backward = _backward
        return out

    # ------------------------------------------------------------ shapes / views
    def _view_out(self, t, op, back):
        if not self._requires_grad or not cfg._grad_enabled:
            return Tensor._create_view_fast(t, self._device, False)
        out = Tensor._wrap(t, (self,), op)
        out.data = t
        out._is_view = True

        def _backward():
            if self._has_grad() and out._has_grad():
                self._share_grad(out, back(out._grad_out()))
        out._backward = _backward
        return out

    def reshape(self, *shape):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        orig = self.data.shape
        return self._view_out(self.data.reshape(shape), "reshape", lambda g: g.reshape(orig))

    def view(self, *shape):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        orig = self.data.shape
        return self._view_out(self.data.reshape(shape), "view", lambda g: g.reshape(orig))

    def flatten(self, start_dim=0, end_dim=-1):
        if end_dim < 0:
            end_dim = self.ndim + end_dim
        shape = list(self.shape[:start_dim]) + [-1] + list(self.shape[end_dim + 1:])
        return self.reshape(tuple(shape))

    def transpose(self, *axes):
        if not axes:
            axes = tuple(range(self.ndim - 1, -1, -1))
        elif len(axes) == 1 and isinstance(axes[0], (tuple, list)):
            axes = tuple(axes[0])
        inv = [0] * len(axes)
        for i, a in enumerate(axes):
            inv[a] = i
        out = self._out(self.data.permute(*axes), (self,), "transpose")
        if out._requires_grad:
            def _backward():
                if self._has_grad():
                    self._share_grad(out, out._grad_out().permute(*inv))
            out._backward = _backward
        return out

    def permute(self, *dims):
        return self.transpose(*dims)

    def squeeze(self, dim=None):
        orig = self.data.shape
        t = self.data.squeeze() if dim is None else self.data.squeeze(dim)
        out = self._out(t, (self,), "squeeze")
        if out._requires_grad:
            def _backward():
                if self._has_grad():
                    self._share_grad(out, out._grad_out().reshape(orig))
            out._backward = _backward
        return out

    def unsqueeze(self, dim):
        out = self._out(self.data.unsqueeze(dim), (self,), "unsqueeze")
        if out._requires_grad:
            def _backward():
                if self._has_grad():
                    self._share_grad(out, out._grad_out().squeeze(dim))
            out._backward = _backward
        return out

    def expand(self, *sizes):
        if len(sizes) == 1 and isinstance(sizes[0], (tuple, list)):
            sizes = tuple(sizes[0])
        out = self._out(self.data.expand(*sizes), (self,), "expand")
        if out._requires_grad:
            def _backward():
                if self._has_grad():
                    self._accumulate_unb(out._grad_out())
            out._backward = _backward
        return out

    def __getitem__(self, idx):
        idx_t = _index_to_torch(idx)
        out = self._out(self.data[idx_t], (self,), "getitem")
        if out._requires_grad:
            basic = _basic_index(idx_t)
            if not basic:
                # integer-array / mask indexing: the flat source index of every selected
                # element, stably sorted, with the segment of each distinct target; the
                # backward's scatter-add then needs no index arithmetic
                seg = _scatter_segments(self.data, idx_t)

            def _backward():
                if not self._has_grad():
                    return
                g = out._grad_out()
                buf, acc = self._grad_target()
                if not acc:
                    _fill(buf, 0.0)
                if basic:
                    # a view of the gradient buffer: one strided add into it
                    L.broadcast_mul_sum(buf[idx_t], g, accumulate=True)
                else:
                    # grad += add.at(zeros, idx, g) (_core.py:918-929) in add.at's order
                    L.index_add_sorted(buf, *seg, _as(g, buf.dtype).reshape(-1))
            out._backward = _backward
        return out

    def __setitem__(self, idx, value):
        v = value.data if isinstance(value, Tensor) else value
        self.data[_index_to_torch(idx)] = v if not isinstance(v, np.ndarray) else torch.as_tensor(
            v, device="cuda", dtype=self.data.dtype)

    # ------------------------------------------------------------ backward
    @staticmethod
    def _unbroadcast(grad, shape):
        """Reference-compatible validation wrapper (_core.py:1380-1424)."""
        if shape is None or not isinstance(shape, (tuple, list)):
            raise TypeError(f"shape must be tuple/list of ints, got {shape!r}")
        try:
            target = tuple(int(d) for d in shape)
        except Exception as exc:
            raise TypeError(f"shape must contain integer dimensions, got {shape!r}") from exc
        if any(d < 0 for d in target):
            raise ValueError(f"shape dimensions must be non-negative, got {target}")
        if grad is None:
            raise ValueError("grad cannot be None")
        if not isinstance(grad, torch.Tensor):
            grad = torch.as_tensor(np.asarray(grad))
        return _unbroadcast_dev(grad, target, grad.dtype)

    def backward(self, gradient=None):
        """Reverse-mode sweep (_core.py:1426-1461): topological order over the
        recorded graph (iterative DFS), seed with `gradient` (added to any existing
        grad) or ones when the grad is absent or all zero, then run each closure once
        in reverse order and drop it.  Weight gradients of 16-bit Linear layers queued
        during the sweep are computed, grouped by shape, before it returns."""
        topo = []
        visited = set()
        stack = [(self, False)]
        while stack:
            v, expanded = stack.pop()
            if expanded:
                topo.append(v)
                continue
            if id(v) in visited:
                continue
            visited.add(id(v))
            stack.append((v, True))
            for c in reversed(v._prev):
                if id(c) not in visited:
                    stack.append((c, False))
        if gradient is not None:
            g = gradient.data if isinstance(gradient, Tensor) else gradient
            if not isinstance(g, torch.Tensor):
                g = torch.as_tensor(np.asarray(g))
            if g.device.type != "cuda":
                g = g.to(device="cuda")
            # the reference takes xp.asarray(gradient, dtype=self.dtype): an integer or
            # differently-typed seed is cast to the tensor's dtype first
            if g.dtype != self.data.dtype:
                g = g.to(dtype=self.data.dtype)
            if not self._has_grad():
                self._g = self._new_buf()
                _copy_into(self._g, g)
                self._gz = False
                self._gsh = False
            else:
                if self._gz:
                    self._g = self._new_buf()
                    _copy_into(self._g, g)
                    self._gz = False
                else:
                    if self._gsh or not self._g.is_contiguous():
                        self._privatize()
                    L.broadcast_mul_sum(self._g, g, accumulate=True)
        elif self._gz or self._g is None or not bool(torch.any(self._g != 0)):
            self._g = self._new_buf(1)
            self._gz = False
            self._gsh = False
        _WG_STATE[0] += 1
        try:
            for v in reversed(topo):
                v._backward()
                v._backward = _noop
        finally:
            _WG_STATE[0] -= 1
            if _WG_STATE[0] == 0:
                _wgrad_flush()


# ====================================================================== helpers
def _dense(t):
    """True if t covers its storage span without gaps or overlaps (a permutation of a
    contiguous tensor)."""
    n = 1
    for size, stride in sorted(zip(t.shape, t.stride()), key=lambda x: x[1]):
        if size == 1:
            continue
        if stride != n:
            return False
        n *= size
    return True


def _unique(children):
    seen = set()
    out = []
    for c in children:
        if id(c) not in seen:
            seen.add(id(c))
            out.append(c)
    return tuple(out)


_ROUNDED = {}


def _round_scalar(v, dt):
    """The Python number v as a value of floating dtype dt (a Python float): through
    float64, with the conversion a device cast from float64 applies (for the 16-bit
    types through float32, as torch's casts do; out of range: inf)."""
    if dt == torch.float64:
        return float(v)
    if dt == torch.float32:
        with np.errstate(over="ignore"):
            return float(np.float32(float(v)))
    key = (float(v), dt)
    r = _ROUNDED.get(key)
    if r is None:
        if len(_ROUNDED) > 4096:
            _ROUNDED.clear()
        r = _ROUNDED[key] = torch.tensor(float(v), dtype=torch.float64).to(dt).item()
    return r


def _scalar_like(v, ref):
    """Python scalars / arrays as device tensors.  Float scalars adopt the reference
    tensor's dtype (NumPy 2 weak-scalar promotion keeps fp32 op fp32).  A scalar is
    made on the device by a fill kernel and an array goes through the pinned staging
    copy: a pageable host-to-device copy (torch.tensor(v, device=...)) would block the
    host until the device queue drains, e.g. in every GradScaler.scale(loss)."""
    if isinstance(v, torch.Tensor):
        return v
    if isinstance(v, (bool, int, float)):
        dt = ref.dtype if ref.is_floating_point() or isinstance(v, int) else torch.float32
        if isinstance(v, float) and not ref.is_floating_point():
            dt = torch.float32
        # made in a wide dtype, then cast: a float outside dt's range becomes inf as the
        # weak-scalar cast does (65536.0 as fp16 is inf), where a fill in dt itself
        # would raise; an out-of-range int raises (checked below)
        wide = torch.float64 if dt.is_floating_point else torch.int64
        if dt == torch.bool:
            wide = torch.bool
        elif isinstance(v, int) and not isinstance(v, bool) and not dt.is_floating_point:
            # NumPy 2's weak-scalar rule: a Python int outside the integer dtype's range
            # raises instead of wrapping
            info = torch.iinfo(dt)
            if v < info.min or v > info.max:
                raise OverflowError(f"Python integer {v} out of bounds for {dt}")
        return torch.full((), v, dtype=wide, device="cuda").to(dt)
    return L.to_device(np.asarray(v))


def _basic_index(idx):
    items = idx if isinstance(idx, tuple) else (idx,)
    return all(i is None or i is Ellipsis or isinstance(i, (int, slice)) for i in items)


def _index_to_torch(idx):
    if isinstance(idx, tuple):
        return tuple(_index_to_torch(i) for i in idx)
    if isinstance(idx, Tensor):
        return idx.data.long() if not idx.data.dtype == torch.bool else idx.data
    if isinstance(idx, np.ndarray):
        return L.to_device(idx)
    if isinstance(idx, list):
        return L.to_device(np.asarray(idx))
    return idx


def _unbroadcast_dev(grad, shape, dtype):
    """Sum `grad` down to `shape` with the reference's rules (_core.py:1380-1424).
    Leading-axis sums onto a contiguous suffix shape (the bias-gradient case) run in
    tg_reduce_rows; other patterns are summed by device tensor ops.  Result has `dtype`."""
    shape = tuple(shape)
    if tuple(grad.shape) == shape:
        return grad if grad.dtype == dtype else grad.to(dtype)
    if grad.dim() < len(shape):
        raise ValueError(
            f"cannot unbroadcast grad with shape {tuple(grad.shape)} to higher-rank shape {shape}")
    lead = grad.dim() - len(shape)
    tail = tuple(grad.shape[lead:])
    if tail == shape and grad.is_cuda and grad.is_contiguous() and grad.dtype in L._TORCH_TO_CODE \
            and dtype in L._TORCH_TO_CODE and len(shape) > 0:
        out = torch.empty(shape, dtype=dtype, device=grad.device)
        L.reduce_rows(grad, out, False)
        return out
    _check_unbroadcast(tuple(grad.shape), shape)
    out = torch.empty(shape, dtype=dtype, device=grad.device)
    return L.broadcast_mul_sum(out, grad)


def _check_unbroadcast(gshape, shape):
    """The reference's unbroadcast rules (_core.py:1402-1422): the target has no more
    axes than the gradient, and each target axis equals the gradient's or is 1."""
    if len(gshape) < len(shape):
        raise ValueError(
            f"cannot unbroadcast grad with shape {gshape} to higher-rank shape {shape}")
    tail = gshape[len(gshape) - len(shape):]
    for ax, (gd, sd) in enumerate(zip(tail, shape)):
        if sd != 1 and gd != sd:
            raise ValueError(
                f"incompatible unbroadcast axis {ax}: grad dim {gd} cannot map to target dim {sd}")


def _as(t, dtype):
    """t as a contiguous tensor of `dtype`: t itself when it already is one, else a new
    buffer written by the strided copy kernel (which also materialises broadcasts)."""
    if t.dtype == dtype and t.is_contiguous():
        return t
    out = torch.empty(t.shape, dtype=dtype, device=t.device)
    _copy_into(out, t)
    return out


def _unary_backward(x, out, op, use_y, param=0.0):
    """Closure for out = op(x): x.grad (+)= op'(.) * out.grad on tg_unary_bwd, with
    the op's input (use_y False) or output (True) as the kernel's operand."""
    def _backward():
        if not x._has_grad():
            return
        dt = x.data.dtype
        a = _as(out.data if use_y else x.data, dt)
        g = _as(out._grad_out(), dt)
        buf, acc = x._grad_target()
        L.unary_bwd(op, a, g, buf, acc, param)
    return _backward


def _scatter_segments(data, idx_t):
    """(targets, starts, order) of an advanced index into `data`: the flat indices the
    selected elements come from, grouped by target in a stable sort (so each group
    keeps the selection order NumPy's add.at adds in)."""
    lin = torch.arange(data.numel(), device=data.device).reshape(data.shape)[idx_t].reshape(-1)
    srt, order = torch.sort(lin, stable=True)
    targets, counts = torch.unique_consecutive(srt, return_counts=True)
    starts = torch.zeros(targets.numel() + 1, dtype=torch.int64, device=data.device)
    torch.cumsum(counts, 0, out=starts[1:])
    return targets.contiguous(), starts, order.contiguous()


def _fill(buf, value):
    if buf.dtype in L._TORCH_TO_CODE and buf.is_contiguous():
        L.fill(buf, value)
    else:
        buf.fill_(value)


def _copy_into(dst, src):
    """dst = src (broadcast to dst's shape), any strides and float dtypes, on the kernels."""
    if (dst.is_contiguous() and src.is_contiguous() and src.shape == dst.shape
            and src.dtype in L._TORCH_TO_CODE and dst.dtype in L._TORCH_TO_CODE):
        L.axpby(src, dst, 1.0, 0.0)
    else:
        L.broadcast_mul_sum(dst, src)


def _activation(x, kind):
    xd = x.data
    if xd.dtype not in L._TORCH_TO_CODE:
        raise TypeError(f"{kind}: unsupported dtype {xd.dtype}")
    xc = xd.contiguous()
    return _activation_node(x, kind, xc, L.act_fwd(kind, xc))


def _activation_node(x, kind, xc, y):
    """The graph node of y = act(x) (xc: x's contiguous data): its closure adds
    dy * act'(x) to x's gradient.  A GELU output also records (x, xc), so a Linear
    layer that is its only consumer can apply the derivative in its own backward."""
    out = Tensor._wrap(y, (x,), "GELU" if kind == "gelu" else "SiLU")
    if kind == "gelu" and out._requires_grad:
        out._act = (x, xc)
    if out._requires_grad:
        def _backward():
            if not x._has_grad():
                return
            g = out._grad_out()
            g = _as(g, xc.dtype)
            buf, acc = x._grad_target()
            L.act_bwd(kind, xc, g, buf, acc)
        out._backward = _backward
    return out


# ====================================================================== matmul
_GEMM_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float64)


def _compute_dtype(a, b):
    """Operand dtype of the GEMM: the autocast dtype inside autocast, else the
    promoted dtype (CuPy promotion, then the Tensor policy)."""
    ac = cfg.autocast_dtype()
    if ac is not None and ac in (torch.float16, torch.bfloat16):
        return ac
    return torch.promote_types(a.dtype, b.dtype)


def _operand(t, cdt):
    """A GEMM operand in compute dtype cdt, contiguous: float data through the copy
    kernel, integer data (the reference's integer @ float promotes it) through torch."""
    if t.dtype in L._TORCH_TO_CODE:
        return _as(t, cdt)
    return t.to(cdt).contiguous()


def _wide(cdt):
    """Accumulation (output) dtype of a GEMM computing in cdt: fp64 for fp64, else fp32."""
    return torch.float64 if cdt == torch.float64 else torch.float32


def _direct_out(buf_dtype, cdt):
    """Whether a gradient buffer of buf_dtype can be the GEMM's output: the compute dtype
    itself, or fp32 for a 16-bit compute dtype."""
    return buf_dtype == cdt or (buf_dtype == torch.float32 and cdt != torch.float64)


def _matmul(self, other):
    a, b = self.data, other.data
    if a.dim() == 0 or b.dim() == 0:
        raise ValueError("matmul requires operands with ndim >= 1")
    cdt = _compute_dtype(a, b)
    if cdt not in _GEMM_DTYPES:
        raise TypeError(f"matmul: dtype {cdt} is not supported by the MFMA GEMM "
                        "(float32, float16, bfloat16, float64)")
    ac = _operand(a, cdt)
    bc = _operand(b, cdt)
    out_t = _matmul_fwd(ac, bc)
    out = Tensor._wrap(out_t, (self, other), "@")
    if out._requires_grad:
        def _backward():
            _matmul_bwd(self, other, ac, bc, out)
        out._backward = _backward
    return out


def _weight_operand(w, wd, wt, cdt):
    """The GEMM operand for weight `w` in compute dtype `cdt`: wd ([K, N]), or its
    contiguous transpose ([N, K]) when `wt`.  A leaf parameter cast to a lower precision
    (autocast) comes from the cast cache, owned by the tensor whose storage it is (the
    source of a tied weight), so the optimizer can refresh it in its update pass."""
    src = wd.t() if wt else wd
    if cdt == torch.float64:
        return _as(src, cdt)  # promoted: the copy kernel casts (no cast cache for fp64)
    if src.dtype == cdt or w._prev or not src.is_contiguous():
        return src.to(cdt).contiguous()
    tied = getattr(w, "_tied_source", None)
    if tied is not None:
        sd = tied.data
        if (sd.data_ptr() == src.data_ptr() and tuple(sd.shape) == tuple(src.shape)
                and sd.is_contiguous()):
            src = sd  # the persistent tensor the optimizer updates
    return _lowp.cast(src, cdt)


def _linear_operands(x, w):
    """(A2 [rows, K] in the compute dtype, B operand, wt, cdt, K, N, lead) of
    x @ w for a 2-D weight, or None when x @ w is not a plain 2-D-weight product."""
    a, wd = x.data, w.data
    if a.dim() < 2 or wd.dim() != 2 or a.shape[-1] != wd.shape[0]:
        return None
    cdt = _compute_dtype(a, wd)
    if cdt not in _GEMM_DTYPES:
        raise TypeError(f"matmul: dtype {cdt} is not supported by the MFMA GEMM "
                        "(float32, float16, bfloat16, float64)")
    K, N = wd.shape
    lead = tuple(a.shape[:-1])
    if a.dtype == cdt and a.is_contiguous():
        A2 = a.view(-1, K)
    else:
        A2 = (_as(a, cdt) if cdt == torch.float64 else a.to(cdt).contiguous()).reshape(-1, K)
    wt = not wd.is_contiguous() and wd.t().is_contiguous()
    bc = _weight_operand(w, wd, wt, cdt)  # [N, K] if wt
    return A2, bc, wt, cdt, K, N, lead


def _linear(x, w, b):
    """y = x @ w + b for a 2-D weight as one GEMM with the bias added in its epilogue
    (Linear.__call__, _nn.py:258-285, which builds a matmul node and a broadcast-add
    node; the gradients are those of the pair: dx = g @ w^T, dw = x^T @ g, db = g
    summed over the leading axes).  A weight that is the transpose of a contiguous
    tensor (a tied head) is cast without transposing and used through op(B) = B^T."""
    ops = _linear_operands(x, w)
    if ops is None:
        out = x @ w
        return out + b if b is not None else out
    A2, bc, wt, cdt, K, N, lead = ops
    a = x.data
    if b is not None and cdt == torch.float64:
        # fp64: the product, then the bias added by the broadcast kernel (in fp64)
        y = L.matmul2d(A2, bc, trans_b=wt)
        L.broadcast_mul_sum(y, b.data.reshape(1, N), accumulate=True)
    elif b is not None:
        bd = b.data
        odt = cfg.resolve_dtype(torch.promote_types(cdt, bd.dtype))
        if odt in (torch.float32, cdt) and bd.dtype == torch.float32 and bd.dim() == 1 \
                and bd.numel() == N and bd.is_contiguous():
            # the operands are built here (contiguous, checked shapes): launch directly
            L.ensure_device(A2.get_device())
            y = torch.empty(A2.shape[0], N, dtype=odt, device=a.device)
            L._gemm_bias_launch(A2, bc, bd, y, wt)
            return _linear_node(x, w, b, A2, bc, wt, cdt, K, N, y.reshape(*lead, N))
        bias = bd.to(torch.float32).contiguous().reshape(N)
        if odt in (torch.float32, cdt):
            y = torch.empty(A2.shape[0], N, dtype=odt, device=a.device)
            L.gemm_bias(A2, bc, bias, y, trans_b=wt)
        else:
            y = torch.empty(A2.shape[0], N, dtype=torch.float32, device=a.device)
            L.gemm_bias(A2, bc, bias, y, trans_b=wt)
            y = y.to(odt)
    else:
        y = L.matmul2d(A2, bc, trans_b=wt)
    return _linear_node(x, w, b, A2, bc, wt, cdt, K, N, y.reshape(*lead, N))


def _fused_out_dtype(cdt, b):
    """The output dtype of a fused-epilogue Linear: cdt when the plain path would also
    produce cdt (16-bit operands whose bias promotion resolves back to cdt), else None."""
    if cdt not in (torch.float16, torch.bfloat16):
        return None
    if b is None:
        return cdt
    return cdt if cfg.resolve_dtype(torch.promote_types(cdt, b.data.dtype)) == cdt else None


def _linear_gelu(x, w, b):
    """gelu(x @ w + b) with the GELU applied in the GEMM's epilogue (tg_gemm_epilogue,
    both the pre-activation and the activation written; bit-identical to the Linear
    then gelu nodes, which it builds).  Falls back to the two kernels where the fused
    kernel does not serve the shape."""
    ops = _linear_operands(x, w)
    if ops is not None:
        A2, bc, wt, cdt, K, N, lead = ops
        if not wt and _fused_out_dtype(cdt, b) is not None:
            h = torch.empty(A2.shape[0], N, dtype=cdt, device=A2.device)
            act = torch.empty_like(h)
            bias = None if b is None else b.data.to(torch.float32).contiguous().reshape(N)
            if L.gemm_epilogue("gelu_fwd", A2, bc, act, h, bias):
                hn = _linear_node(x, w, b, A2, bc, wt, cdt, K, N, h.reshape(*lead, N))
                return _activation_node(hn, "gelu", h.reshape(*lead, N), act.reshape(*lead, N))
    return _linear(x, w, b).gelu()


def _linear_residual(x, w, b, r):
    """r + (x @ w + b) with the residual added in the GEMM's epilogue
    (tg_gemm_epilogue; bit-identical to the Linear then add nodes, which it builds:
    the Linear node keeps the sum's buffer as its data, which its backward never
    reads).  Falls back to the two kernels where the fused kernel does not serve the
    shape or r does not match the output."""
    ops = _linear_operands(x, w)
    if ops is not None and isinstance(r, Tensor):
        A2, bc, wt, cdt, K, N, lead = ops
        rd = r.data
        if (not wt and _fused_out_dtype(cdt, b) is not None and rd.dtype == cdt
                and tuple(rd.shape) == lead + (N,) and rd.is_contiguous()):
            out = torch.empty(A2.shape[0], N, dtype=cdt, device=A2.device)
            bias = None if b is None else b.data.to(torch.float32).contiguous().reshape(N)
            if L.gemm_epilogue("residual", A2, bc, rd.reshape(-1, N), out, bias):
                o = out.reshape(*lead, N)
                y = _linear_node(x, w, b, A2, bc, wt, cdt, K, N, o)
                return r._add_node(y, o)
    return r + _linear(x, w, b)


def _linear_node(x, w, b, A2, bc, wt, cdt, K, N, y):
    """The graph node of y = x @ w + b (A2, bc: the GEMM operands the forward used)."""
    children = (x, w) if b is None else (x, w, b)
    out = Tensor._wrap(y, children, "linear")
    if out._requires_grad:
        def _backward():
            g = out._grad_out()
            G2 = _as(g, cdt).reshape(-1, N)
            if x._has_grad():
                if not _gelu_input_grad(x, G2, bc, wt, cdt):
                    buf, acc = x._grad_target()
                    if _direct_out(buf.dtype, cdt):
                        L.matmul2d(G2, bc, out=buf.view(-1, K), trans_b=not wt,
                                   beta=1.0 if acc else 0.0)
                    else:
                        da = L.matmul2d(G2, bc, trans_b=not wt, out_dtype=_wide(cdt))
                        if acc:
                            x._accumulate(da.reshape(buf.shape), True)
                        else:
                            _copy_into(buf, da.reshape(buf.shape))
            fuse = (w._has_grad() and b is not None and b._has_grad() and g.dtype == cdt
                    and b.data.numel() == N and b.data.shape[-1] == N)
            # 16-bit products into leaf parameters wait for the end of the sweep
            defer = (_WG_STATE[0] > 0 and cdt in (torch.float16, torch.bfloat16)
                     and not w._prev and (b is None or not b._prev))
            if fuse:
                # dW and db from one pass over the output gradient
                wbuf, wacc = w._grad_target()
                bbuf, bacc = b._grad_target()
                if _direct_out(wbuf.dtype, cdt) and _direct_out(bbuf.dtype, cdt):
                    if defer:
                        _wgrad_defer(A2, G2, w, wbuf, wacc, b, bbuf, bacc)
                    elif A2.is_contiguous() and G2.is_contiguous():
                        # operands built by this node: launch without re-checking
                        L._wgrad_launch(A2, G2, wbuf.view(K, N), wacc, bbuf.view(N), bacc)
                    else:
                        L.wgrad(A2, G2, wbuf.view(K, N), wacc, bbuf.view(N), bacc)
                else:
                    _wgrad_into(G2, wbuf, wacc)
                    L.reduce_rows(G2, bbuf.view(N), bacc)
                return
            if w._has_grad():
                wbuf, wacc = w._grad_target()
                if defer and _direct_out(wbuf.dtype, cdt):
                    _wgrad_defer(A2, G2, w, wbuf, wacc)
                else:
                    _wgrad_into(G2, wbuf, wacc)
            if b is not None and b._has_grad():
                b._accumulate_unb(g)

        def _wgrad_into(G2, buf, acc):
            """w's gradient buffer (+)= A2^T @ G2."""
            if _direct_out(buf.dtype, cdt):
                L.matmul2d(A2, G2, out=buf.view(K, N), trans_a=True, beta=1.0 if acc else 0.0)
            else:
                dw = L.matmul2d(A2, G2, trans_a=True, out_dtype=_wide(cdt))
                if acc:
                    w._accumulate(dw, True)
                else:
                    _copy_into(buf, dw)
        out._backward = _backward
    return out


def _gelu_input_grad(x, G2, bc, wt, cdt):
    """When x is a GELU output whose only consumer is this Linear layer, x's gradient is
    exactly G2 @ w^T: the GELU's input gradient is formed from it in the GEMM's
    epilogue (tg_gemm_epilogue "gelu_bwd", bit-identical to the two kernels) and the
    GELU node's own closure is retired, so x's gradient buffer is never formed.
    Returns False (nothing done) when the pattern or the fused kernel does not apply."""
    act = x._act
    if act is None or x._nuse != 1 or wt or not cfg.fuse_gelu_backward:
        return False
    src, xc = act
    if xc.dtype != cdt or not x._gz:  # x must not hold a gradient from elsewhere
        return False
    if not src._has_grad():
        x._backward = _noop
        return True
    if src.data.dtype != cdt or cdt not in (torch.float16, torch.bfloat16):
        return False
    buf, acc = src._grad_target()
    M = G2.shape[0]
    x2, b2 = xc.reshape(M, -1), buf.view(M, -1)
    if not L.gemm_epilogue("gelu_bwd", G2, bc, x2, b2, beta=1.0 if acc else 0.0):
        # the fused kernel does not serve this shape: the same two kernels the separate
        # closures would run (the GELU input's buffer is already claimed)
        L.act_bwd("gelu", x2, L.matmul2d(G2, bc, trans_b=True), b2, acc)
    x._backward = _noop
    return True


def _batch_view(x, batch_shape, m, n):
    """Broadcast x [..., m, n] to batch_shape + [m, n]; return (tensor3d, stride) with
    stride 0 when x has no batch extent to broadcast."""
    bsz = int(np.prod(batch_shape)) if batch_shape else 1
    if x.dim() == 2:
        return x, 0, bsz
    xb = tuple(x.shape[:-2])
    if xb == tuple(batch_shape):
        return x.reshape(bsz, m, n), m * n, bsz
    xe = _as(x.expand(*batch_shape, m, n), x.dtype)
    return xe.reshape(bsz, m, n), m * n, bsz


def _matmul_fwd(a, b):
    av, bv = a.dim() == 1, b.dim() == 1
    A = a.unsqueeze(0) if av else a
    Bm = b.unsqueeze(1) if bv else b
    M, K = A.shape[-2], A.shape[-1]
    N = Bm.shape[-1]
    if Bm.shape[-2] != K:
        raise ValueError(f"matmul: shapes {tuple(a.shape)} and {tuple(b.shape)} not aligned")
    if Bm.dim() == 2:
        # fold all leading dims of A into M: one GEMM
        lead = tuple(A.shape[:-2])
        res = L.matmul2d(A.reshape(-1, K), Bm)
        res = res.reshape(*lead, M, N)
    else:
        batch_shape = torch.broadcast_shapes(tuple(A.shape[:-2]), tuple(Bm.shape[:-2]))
        A3, sa, bsz = _batch_view(A, batch_shape, M, K)
        B3, sb, _ = _batch_view(Bm, batch_shape, K, N)
        res = torch.empty(bsz, M, N, dtype=a.dtype, device=a.device)
        L.gemm(A3, B3, res, False, False, 1.0, 0.0, M, N, K, K, N, N, sa, sb, M * N, bsz)
        res = res.reshape(*batch_shape, M, N)
    if av:
        res = res.squeeze(-2)
    if bv:
        res = res.squeeze(-1)
    return res


def _matmul_bwd(self, other, ac, bc, out):
    """dA = dC @ B^T, dB = A^T @ dC on the MFMA GEMM, with the reference's vector
    promotion, validation and unbroadcast (_core.py:1003-1068)."""
    lhs, rhs = self.data, other.data
    if lhs.dim() == 0 or rhs.dim() == 0:
        raise ValueError(
            f"matmul backward requires operands with ndim >= 1, got {lhs.dim()} and {rhs.dim()}")
    g = out._grad_out()
    exp = tuple(out.data.shape)
    if exp == ():
        if g.numel() != 1:
            raise ValueError(f"matmul backward expected scalar grad_out, got shape {tuple(g.shape)}")
        g = g.reshape(())
    elif tuple(g.shape) != exp:
        raise ValueError(
            f"matmul backward grad_out shape mismatch: expected {exp}, got {tuple(g.shape)}")
    if self._has_grad() and not lhs.is_floating_point():
        raise TypeError(f"matmul backward requires floating/complex lhs, got {lhs.dtype}")
    if other._has_grad() and not rhs.is_floating_point():
        raise TypeError(f"matmul backward requires floating/complex rhs, got {rhs.dtype}")
    cdt = ac.dtype
    av, bv = ac.dim() == 1, bc.dim() == 1
    A = ac.unsqueeze(0) if av else ac
    Bm = bc.unsqueeze(1) if bv else bc
    if av and bv:
        G = g.reshape(1, 1)
    elif av:
        G = g.unsqueeze(-2)
    elif bv:
        G = g.unsqueeze(-1)
    else:
        G = g
    G = _as(G, cdt)
    M, K = A.shape[-2], A.shape[-1]
    N = Bm.shape[-1]
    if Bm.dim() == 2:
        lead = tuple(A.shape[:-2])
        G2 = G.reshape(-1, N)
        A2 = A.reshape(-1, K)
        if self._has_grad():
            # dA[.., m, k] = G @ B^T
            buf, acc = self._grad_target()
            if _direct_out(buf.dtype, cdt):
                L.matmul2d(G2, Bm, out=buf.view(A2.shape[0], K), trans_b=True,
                           beta=1.0 if acc else 0.0)
            else:
                da = L.matmul2d(G2, Bm, trans_b=True, out_dtype=_wide(cdt))
                L.broadcast_mul_sum(buf, da.reshape(buf.shape), accumulate=acc)
        if other._has_grad():
            # dB[k, n] = sum over all leading rows of A^T @ G: one TN GEMM with K' = rows
            buf, acc = other._grad_target()
            if _direct_out(buf.dtype, cdt):
                L.matmul2d(A2, G2, out=buf.view(K, N), trans_a=True, beta=1.0 if acc else 0.0)
            else:
                db = L.matmul2d(A2, G2, trans_a=True, out_dtype=_wide(cdt))
                L.broadcast_mul_sum(buf, db.reshape(buf.shape), accumulate=acc)
        return
    # batched operands
    batch_shape = torch.broadcast_shapes(tuple(A.shape[:-2]), tuple(Bm.shape[:-2]))
    bsz = int(np.prod(batch_shape))
    G3 = _as(G.expand(*batch_shape, M, N), cdt).reshape(bsz, M, N)
    if self._has_grad():
        B3, sb, _ = _batch_view(Bm, batch_shape, K, N)
        da = torch.empty(bsz, M, K, dtype=_wide(cdt), device=A.device)
        L.gemm(G3, B3, da, False, True, 1.0, 0.0, M, K, N, N, N, K, M * N, sb, M * K, bsz)
        da = da.reshape(*batch_shape, M, K)
        if av:
            da = da.squeeze(-2)
        self._accumulate(_unbroadcast_dev(da, tuple(lhs.shape), lhs.dtype), True)
    if other._has_grad():
        A3, sa, _ = _batch_view(A, batch_shape, M, K)
        db = torch.empty(bsz, K, N, dtype=_wide(cdt), device=A.device)
        L.gemm(A3, G3, db, True, False, 1.0, 0.0, K, N, M, K, N, N, sa, M * N, K * N, bsz)
        db = db.reshape(*batch_shape, K, N)
        if bv:
            db = db.squeeze(-1)
        other._accumulate(_unbroadcast_dev(db, tuple(rhs.shape), rhs.dtype), True)


# ====================================================================== attention
def flash_attention(query, key, value, block_size=64, is_causal=False, scale=None,
                    dropout_p=0.0):
    """FlashAttention forward/backward on libtgbwd (_core.py:1686-1870).
    query/key/value: (B, H, L, D) or (B, L, D).  The forward saves the row
    log-sum-exp; the backward recomputes P from it (no S x S matrix is stored)."""
    q, k, v = query.data, key.data, value.data
    three = q.dim() == 3
    if three:
        B, Lq, D = q.shape
        q4 = q.reshape(B, 1, Lq, D)
        k4 = k.reshape(B, 1, k.shape[1], D)
        v4 = v.reshape(B, 1, v.shape[1], D)
    else:
        q4, k4, v4 = q, k, v
    D = q4.shape[-1]
    scale = scale or D ** -0.5
    dt = q4.dtype
    if dt not in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        raise TypeError(f"flash_attention: unsupported dtype {dt}")
    q4c, k4c, v4c = q4, k4.to(dt), v4.to(dt)
    # (B, S, H, D) memory (the head split of a projection, viewed as (B, H, S, D)) is read
    # and written in place; any other strides are made contiguous.
    lay = 1 if all(L._fa_in(t, 1) for t in (q4c, k4c, v4c)) else 0
    if lay == 0:
        q4c, k4c, v4c = q4c.contiguous(), k4c.contiguous(), v4c.contiguous()
    o, lse = L.flash_attn_fwd(q4c, k4c, v4c, scale, is_causal, lay)
    if dropout_p > 0 and cfg._grad_enabled:
        keep = (torch.rand(o.shape, device=o.device) > dropout_p).to(o.dtype)
        o_out = o * keep / (1 - dropout_p)
    else:
        o_out = o
    out = Tensor._wrap(o_out.reshape(q.shape) if three else o_out, (query, key, value),
                       "FlashAttention")
    if out._requires_grad:
        def _backward():
            g = out._grad_out().reshape(q4c.shape)
            B_, H_, Sq_, D_ = q4c.shape
            if g.dtype != dt or not L._fa_in(g, lay):
                gl = L.fa_empty(B_, H_, Sq_, D_, dt, q4c.device, lay)
                _copy_into(gl, g)
                g = gl
            Sk_ = k4c.shape[2]
            dq = L.fa_empty(B_, H_, Sq_, D_, dt, q4c.device, lay)
            dk = L.fa_empty(B_, H_, Sk_, D_, dt, q4c.device, lay)
            dv = L.fa_empty(B_, H_, Sk_, D_, dt, q4c.device, lay)
            L.flash_attn_bwd(q4c, k4c, v4c, o, g, lse, dq, dk, dv, scale, is_causal, False, lay)
            if query._has_grad():
                query._accumulate(dq.reshape(query.data.shape), True)
            if key._has_grad():
                key._accumulate(dk.reshape(key.data.shape), True)
            if value._has_grad():
                value._accumulate(dv.reshape(value.data.shape), True)
        out._backward = _backward
    return out


def flash_attention_qkv(qkv, num_heads, is_causal=False, scale=None):
    """Self-attention on one packed projection: qkv (B, S, 3*H*D) holds the query heads in
    columns [0, HD), the keys in [HD, 2HD) and the values in [2HD, 3HD) (the output of
    one Linear(d, 3d) in place of the reference module's three projections w_q, w_k,
    w_v, _training.py:1885-1904).  Returns the merged heads (B, S, H*D): the values of
    flash_attention on the head splits of the three column blocks followed by the
    merge-heads transpose (_training.py:1894-1913), from the same kernels reading q, k
    and v in place, with no split or merge copy.  The backward writes dq, dk and dv
    straight into qkv's gradient columns.  fp16, bf16 and fp32; float64 runs through
    flash_attention on copies of the head splits."""
    x = qkv.data
    if x.dim() != 3 or x.shape[2] % (3 * num_heads):
        raise ValueError(f"flash_attention_qkv: qkv must be (B, S, 3*H*D) with H = "
                         f"{num_heads}, got {tuple(x.shape)}")
    B, S, C3 = x.shape
    C = C3 // 3
    D = C // num_heads
    scale = scale or D ** -0.5
    if x.dtype == torch.float64:
        def heads(t):
            return t.reshape(B, S, num_heads, D).transpose(0, 2, 1, 3)
        q, k, v = (heads(qkv[:, :, i * C:(i + 1) * C]) for i in range(3))
        o = flash_attention(q, k, v, is_causal=is_causal, scale=scale)
        return o.transpose(0, 2, 1, 3).reshape(B, S, C)
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"flash_attention_qkv: unsupported dtype {x.dtype}")
    dt = x.dtype
    xc = x.contiguous()
    o, lse = L.flash_attn_fwd_qkv(xc, num_heads, scale, is_causal)
    out = Tensor._wrap(o, (qkv,), "FlashAttention")
    if out._requires_grad:
        def _backward():
            if not qkv._has_grad():
                return
            g = out._grad_out()
            if g.dtype != dt or not g.is_contiguous():
                gl = torch.empty(B, S, C, dtype=dt, device=xc.device)
                _copy_into(gl, g)
                g = gl
            buf, acc = qkv._grad_target()
            if buf.dtype == dt:
                L.flash_attn_bwd_qkv(xc, o, g, lse, buf, num_heads, scale, is_causal, acc)
            else:
                d = torch.empty_like(xc)
                L.flash_attn_bwd_qkv(xc, o, g, lse, d, num_heads, scale, is_causal, False)
                L.broadcast_mul_sum(buf, d, accumulate=acc)
        out._backward = _backward
    return out


def scaled_dot_product_attention(query, key, value, attn_mask=None, dropout_p=0.0,
                                 is_causal=False, scale=None, use_flash=False, block_size=64):
    """Materialised attention (_core.py:1606-1683): scores = q k^T * scale, causal fill
    -1e9, softmax, @ v — each step an autograd op (GEMM and softmax kernels)."""
    if use_flash and query.shape[-2] > block_size:
        return flash_attention(query, key, value, block_size=block_size, is_causal=is_causal,
                               scale=scale, dropout_p=dropout_p)
    squeeze = query.ndim == 3
    if squeeze:
        query, key, value = query.unsqueeze(1), key.unsqueeze(1), value.unsqueeze(1)
    B, H, Lq, D = query.shape
    S = key.shape[2]
    scale = scale or D ** -0.5
    scores = (query @ key.transpose(0, 1, 3, 2)) * scale
    if is_causal:
        m = torch.triu(torch.ones(Lq, S, dtype=torch.bool, device="cuda"), diagonal=1)
        scores.data = torch.where(m, torch.full((), -1e9, dtype=scores.data.dtype,
                                                device="cuda"), scores.data)
    if attn_mask is not None:
        am = attn_mask.data if isinstance(attn_mask, Tensor) else L.to_device(
            np.asarray(attn_mask))
        scores.data = scores.data + am.to(scores.data.dtype)
    attn = scores.softmax(axis=-1)
    if dropout_p > 0 and cfg._grad_enabled:
        keep = (torch.rand(attn.shape, device="cuda") > dropout_p).float() / (1 - dropout_p)
        attn = attn * Tensor(keep, requires_grad=False)
    o = attn @ value
    return o.squeeze(1) if squeeze else o


def multi_head_attention(query, key, value, embed_dim, num_heads, q_proj, k_proj, v_proj,
                         out_proj, attn_mask=None, dropout_p=0.0, is_causal=False):
    """(_core.py:1873-1913)"""
    B, Lq, _ = query.shape
    S = key.shape[1]
    hd = embed_dim // num_heads
    q = q_proj(query).reshape(B, Lq, num_heads, hd).transpose(0, 2, 1, 3)
    k = k_proj(key).reshape(B, S, num_heads, hd).transpose(0, 2, 1, 3)
    v = v_proj(value).reshape(B, S, num_heads, hd).transpose(0, 2, 1, 3)
    o = scaled_dot_product_attention(q, k, v, attn_mask, dropout_p, is_causal)
    return out_proj(o.transpose(0, 2, 1, 3).reshape(B, Lq, embed_dim))


def sync():
    torch.cuda.synchronize()


def memory_info():
    used = torch.cuda.memory_allocated()
    total = torch.cuda.memory_reserved()
    return {"used_bytes": used, "total_bytes": total, "used_mb": used / 2 ** 20,
            "total_mb": total / 2 ** 20, "n_free_blocks": 0}
