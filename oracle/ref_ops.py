"""NumPy restatement of the reference backward path (test infrastructure only).

Each function states the reference lines it follows.  Inputs are NumPy arrays;
the arithmetic runs in the inputs' dtype.
"""

import numpy as np

__all__ = [
    "gelu_fwd", "gelu_bwd", "silu_fwd", "silu_bwd", "softmax_fwd", "softmax_bwd",
    "layernorm_fwd", "layernorm_bwd", "batchnorm_relu_fwd", "batchnorm_relu_bwd",
    "batchnorm_eval_fwd", "batchnorm_relu_fwd_nhwc", "batchnorm_relu_bwd_nhwc", "unbroadcast",
    "matmul_bwd",
    "flash_attention_fwd", "flash_attention_bwd", "adam_step", "GradScalerRef",
    "clip_grad_norm", "cross_entropy_fwd", "cross_entropy_bwd", "embedding_bwd",
    "mlp_step", "relu_bwd", "leaky_relu_bwd", "swish_bwd", "sigmoid_bwd", "tanh_bwd",
    "exp_bwd", "log_bwd", "pow_bwd", "log_softmax_fwd", "log_softmax_bwd", "max_bwd",
    "getitem_bwd",
]

_C0 = 0.7978845608028654  # sqrt(2/pi)
_C1 = 0.044715


# ---------------------------------------------------------------- activations
def gelu_fwd(x):
    """tanh-approx GELU (_core.py:1194-1197)."""
    t = np.tanh(_C0 * (x + _C1 * x ** 3))
    return x * (0.5 * (1 + t))


def gelu_bwd(x, dy):
    """dx = dy * gelu'(x) (_core.py:493-507 kernel, _core.py:1199-1206 xp path)."""
    inner = _C0 * (x + _C1 * x ** 3)
    t = np.tanh(inner)
    sech2 = 1 - t ** 2
    dinner = _C0 * (1 + 3 * _C1 * x ** 2)
    return dy * (0.5 * (1 + t) + 0.5 * x * sech2 * dinner)


def silu_fwd(x):
    """x * sigmoid(x) (_core.py:1233-1234)."""
    return x * (1 / (1 + np.exp(-x)))


def silu_bwd(x, dy):
    """dx = dy * s * (1 + x*(1-s)), s = sigmoid(x) (_core.py:522-533, :1237-1243)."""
    s = 1 / (1 + np.exp(-x))
    return dy * (s * (1 + x * (1 - s)))


# ---------------------------------------------------------------- other pointwise ops
def relu_bwd(y, dy):
    """(out > 0) * g with y = relu(x) (_core.py:1149-1157)."""
    return (y > 0) * dy


def leaky_relu_bwd(x, dy, slope=0.01):
    """where(x >= 0, 1, slope) * g (_core.py:1159-1170)."""
    return np.where(x >= 0, 1.0, slope) * dy


def swish_bwd(x, dy, beta=1.0):
    """(s + beta*x*s*(1 - s)) * g, s = 1/(1 + exp(-beta*x)) (_core.py:1248-1260)."""
    s = 1 / (1 + np.exp(-beta * x))
    return (s + beta * x * s * (1 - s)) * dy


def sigmoid_bwd(y, dy):
    """out * (1 - out) * g (_core.py:1262-1272)."""
    return y * (1 - y) * dy


def tanh_bwd(y, dy):
    """(1 - out**2) * g (_core.py:1274-1282)."""
    return (1 - y ** 2) * dy


def exp_bwd(y, dy):
    """out * g: d/dx exp(x) = exp(x)."""
    return y * dy


def log_bwd(x, dy):
    """g / x: d/dx log(x) = 1/x."""
    return dy / x


def pow_bwd(x, dy, p):
    """(p * x**(p - 1)) * g (_core.py:973-981); a / b is a * b**-1 (_core.py:993-995)."""
    return (p * x ** (p - 1)) * dy


def log_softmax_fwd(x, axis=-1):
    """shifted - log(sum(exp(shifted))) (_core.py:1301-1307)."""
    sh = x - x.max(axis=axis, keepdims=True)
    return sh - np.log(np.exp(sh).sum(axis=axis, keepdims=True))


def log_softmax_bwd(y, dy, axis=-1):
    """g - exp(out) * sum(g) (_core.py:1309-1312)."""
    return dy - np.exp(y) * dy.sum(axis=axis, keepdims=True)


def max_bwd(x, dy, axis=None, keepdims=False):
    """mask * broadcast(g) / count(mask) over the reduced axes (_core.py:1115-1132)."""
    r = x.max(axis=axis, keepdims=keepdims)
    if axis is None:
        mask = x == r
    else:
        mask = x == (r if keepdims else np.expand_dims(r, axis))
    count = mask.sum(axis=axis, keepdims=True)
    g = np.expand_dims(dy, axis) if (not keepdims and axis is not None) else dy
    return mask * np.broadcast_to(g, x.shape) / count


def getitem_bwd(shape, idx, dy, dtype=np.float64):
    """zeros; add.at(zeros, idx, g) (_core.py:918-929; the CPU path's _scatter_add is
    np.add.at, :890-916): repeated indices accumulate in index order."""
    grad = np.zeros(shape, dtype=dtype)
    np.add.at(grad, idx, dy)
    return grad


# ---------------------------------------------------------------- softmax
def softmax_fwd(x, axis=-1):
    """Max-shifted softmax (_core.py:1286-1291)."""
    e = np.exp(x - x.max(axis=axis, keepdims=True))
    return e / e.sum(axis=axis, keepdims=True)


def softmax_bwd(y, dy, axis=-1):
    """dx = y * (dy - sum(dy*y)) (_core.py:1294-1297)."""
    return y * (dy - (dy * y).sum(axis=axis, keepdims=True))


# ---------------------------------------------------------------- layer norm
def layernorm_fwd(x, gamma, beta, eps=1e-5):
    """LayerNorm over the last axis (_nn.py:900-919): population variance,
    xhat = (x - mean)/sqrt(var + eps), y = gamma*xhat + beta.
    Returns y, xhat, mean, var (the module cache)."""
    mean = x.mean(axis=-1, keepdims=True)
    var = x.var(axis=-1, keepdims=True)
    xhat = (x - mean) / np.sqrt(var + eps)
    return gamma * xhat + beta, xhat, mean, var


def layernorm_bwd(xhat, var, gamma, dy, eps=1e-5):
    """(_nn.py:921-942): dgamma = sum dy*xhat, dbeta = sum dy over leading axes;
    dx = g*rstd - mean(g)*rstd - xhat*mean(g*xhat)*rstd, g = dy*gamma."""
    lead = tuple(range(dy.ndim - 1))
    dgamma = (dy * xhat).sum(axis=lead)
    dbeta = dy.sum(axis=lead)
    g = dy * gamma
    rstd = 1.0 / np.sqrt(var + eps)
    dx = g * rstd
    dx = dx - g.mean(axis=-1, keepdims=True) * rstd
    dx = dx - xhat * (g * xhat).mean(axis=-1, keepdims=True) * rstd
    return dx, dgamma, dbeta


# ---------------------------------------------------------------- batch norm + relu
def batchnorm_relu_fwd(x, gamma, beta, eps=1e-5, relu=True):
    """Training forward of FusedBatchNormReLU on NCHW (_nn.py:794-810).
    Returns out, cache = (x_norm, x_centered, std_inv, m, out, mean, var)."""
    N, C, H, W = x.shape
    m = N * H * W
    mean = x.mean(axis=(0, 2, 3))
    var = x.var(axis=(0, 2, 3))
    std_inv = 1.0 / np.sqrt(var.reshape(1, C, 1, 1) + eps)
    xc = x - mean.reshape(1, C, 1, 1)
    xn = xc * std_inv
    out = gamma.reshape(1, C, 1, 1) * xn + beta.reshape(1, C, 1, 1)
    if relu:
        out = np.maximum(0, out)
    return out, (xn, xc, std_inv, m, out, mean, var)


def batchnorm_relu_bwd(dy, gamma, cache, relu=True):
    """FusedBatchNormReLU backward (_nn.py:812-833), the reference's dvar/dmean
    chain.  Returns dx, dgamma, dbeta."""
    xn, xc, std_inv, m, out, _, _ = cache
    C = gamma.shape[0]
    d = dy * (out > 0).astype(dy.dtype) if relu else dy
    dgamma = (d * xn).sum(axis=(0, 2, 3))
    dbeta = d.sum(axis=(0, 2, 3))
    dxn = d * gamma.reshape(1, C, 1, 1)
    dvar = (dxn * xc * (-0.5) * std_inv ** 3).sum(axis=(0, 2, 3), keepdims=True)
    dmean = (dxn * (-std_inv)).sum(axis=(0, 2, 3), keepdims=True)
    dmean = dmean + dvar * (-2.0 / m) * xc.sum(axis=(0, 2, 3), keepdims=True)
    dx = dxn * std_inv + dvar * (2.0 / m) * xc + dmean / m
    return dx, dgamma, dbeta


def batchnorm_eval_fwd(x, gamma, beta, running_mean, running_var, eps=1e-5):
    """BatchNorm2D forward in eval mode on NCHW (_nn.py:706-718): the running statistics
    take the place of the batch ones.  The reference keeps the backward of
    _nn.py:720-736, so the returned cache feeds batchnorm_relu_bwd(..., relu=False)
    unchanged (with m = N*H*W and sum(xc) no longer zero)."""
    N, C, H, W = x.shape
    std_inv = 1.0 / np.sqrt(running_var.reshape(1, C, 1, 1) + eps)
    xc = x - running_mean.reshape(1, C, 1, 1)
    xn = xc * std_inv
    out = gamma.reshape(1, C, 1, 1) * xn + beta.reshape(1, C, 1, 1)
    return out, (xn, xc, std_inv, N * H * W, out, running_mean, running_var)


def batchnorm_relu_fwd_nhwc(x, gamma, beta, eps=1e-5, relu=True):
    """NHWC input: the reference module is NCHW-only (_nn.py:791), so the NHWC
    result is the reference math on x.transpose(0,3,1,2), transposed back."""
    out, cache = batchnorm_relu_fwd(x.transpose(0, 3, 1, 2), gamma, beta, eps, relu)
    return out.transpose(0, 2, 3, 1), cache


def batchnorm_relu_bwd_nhwc(dy, gamma, cache, relu=True):
    dx, dg, db = batchnorm_relu_bwd(dy.transpose(0, 3, 1, 2), gamma, cache, relu)
    return dx.transpose(0, 2, 3, 1), dg, db


# ---------------------------------------------------------------- matmul
def unbroadcast(grad, shape):
    """Tensor._unbroadcast (_core.py:1380-1424): sum leading axes, then keepdims-sum
    size-1 axes; ValueError for a higher-rank target or an incompatible axis."""
    shape = tuple(int(d) for d in shape)
    if grad.shape == shape:
        return grad
    if grad.ndim < len(shape):
        raise ValueError(f"cannot unbroadcast {grad.shape} to higher-rank {shape}")
    while grad.ndim > len(shape):
        grad = grad.sum(axis=0)
    for ax, (g, s) in enumerate(zip(grad.shape, shape)):
        if s == 1:
            if g != 1:
                grad = grad.sum(axis=ax, keepdims=True)
        elif g != s:
            raise ValueError(f"incompatible unbroadcast axis {ax}: {g} vs {s}")
    return grad


def matmul_bwd(a, b, dc):
    """Gradients of c = a @ b (_core.py:999-1068): vector operands are promoted to
    matrices, dA = dC @ B^T, dB = A^T @ dC, then unbroadcast to the operand shapes."""
    if a.ndim == 0 or b.ndim == 0:
        raise ValueError("matmul backward requires operands with ndim >= 1")
    av, bv = a.ndim == 1, b.ndim == 1
    am = a[None, :] if av else a
    bm = b[:, None] if bv else b
    if av and bv:
        g = np.asarray(dc).reshape(1, 1)
    elif av:
        g = np.expand_dims(dc, -2)
    elif bv:
        g = np.expand_dims(dc, -1)
    else:
        g = dc
    da = np.matmul(g, np.swapaxes(bm, -1, -2))
    if av:
        da = da.squeeze(-2)
    db = np.matmul(np.swapaxes(am, -1, -2), g)
    if bv:
        db = db.squeeze(-1)
    return unbroadcast(da, a.shape), unbroadcast(db, b.shape)


# ---------------------------------------------------------------- flash attention
def _as4(t):
    return (t[:, None], True) if t.ndim == 3 else (t, False)


def flash_attention_fwd(q, k, v, is_causal=False, scale=None, block_size=64):
    """Query-blocked attention forward (_core.py:1686-1786), returning (o, lse).
    Each block sees all keys, so the online update reduces to an exact softmax;
    lse (natural log-sum-exp of the scaled, masked scores) is what the HIP forward
    saves for its backward."""
    q4, sq = _as4(q)
    k4, _ = _as4(k)
    v4, _ = _as4(v)
    B, H, L, D = q4.shape
    S = k4.shape[2]
    scale = scale or D ** -0.5
    o = np.zeros((B, H, L, D), dtype=q4.dtype)
    lse = np.zeros((B, H, L), dtype=q4.dtype)
    for i in range(0, L, block_size):
        j = min(i + block_size, L)
        s = np.einsum("bhid,bhjd->bhij", q4[:, :, i:j], k4) * scale
        if is_causal:
            mask = np.arange(S)[None, None, None, :] > np.arange(i, j)[None, None, :, None]
            s = np.where(mask, -1e9, s)
        mx = s.max(-1, keepdims=True)
        e = np.exp(s - mx)
        den = e.sum(-1, keepdims=True)
        o[:, :, i:j] = np.einsum("bhij,bhjd->bhid", e, v4) / den
        lse[:, :, i:j] = (mx + np.log(den))[..., 0]
    if sq:
        return o[:, 0], lse[:, 0]
    return o, lse


def flash_attention_bwd(q, k, v, do, is_causal=False, scale=None, block_size=64, o=None):
    """FlashAttention backward (_core.py:1799-1867): per query block recompute
    P = softmax(QK^T s [masked -1e9]); dV += P^T dO; dP = dO V^T;
    dS = P*(dP - rowsum(P*dP))*s (masked -> 0); dQ = dS K; dK += dS^T Q.

    With `o` (the forward output as stored), the row term is rowsum(dO*O) instead, the
    identity rowsum(P*dP) = rowsum(dO*O) that holds for exact O: this isolates a
    kernel's arithmetic from the rounding of its stored O."""
    q4, sq = _as4(q)
    k4, _ = _as4(k)
    v4, _ = _as4(v)
    do4, _ = _as4(do)
    B, H, L, D = q4.shape
    S = k4.shape[2]
    scale = scale or D ** -0.5
    dq = np.zeros_like(q4)
    dk = np.zeros_like(k4)
    dv = np.zeros_like(v4)
    for i in range(0, L, block_size):
        j = min(i + block_size, L)
        qi, doi = q4[:, :, i:j], do4[:, :, i:j]
        s = np.einsum("bhid,bhjd->bhij", qi, k4) * scale
        mask = None
        if is_causal:
            mask = np.arange(S)[None, None, None, :] > np.arange(i, j)[None, None, :, None]
            s = np.where(mask, -1e9, s)
        e = np.exp(s - s.max(-1, keepdims=True))
        p = e / e.sum(-1, keepdims=True)
        dv += np.einsum("bhij,bhid->bhjd", p, doi)
        dp = np.einsum("bhid,bhjd->bhij", doi, v4)
        if o is None:
            row = (p * dp).sum(-1, keepdims=True)
        else:
            row = (doi * _as4(o)[0][:, :, i:j]).sum(-1, keepdims=True)
        ds = p * (dp - row) * scale
        if mask is not None:
            ds = np.where(mask, 0.0, ds)
        dq[:, :, i:j] += np.einsum("bhij,bhjd->bhid", ds, k4)
        dk += np.einsum("bhij,bhid->bhjd", ds, qi)
    if sq:
        return dq[:, 0], dk[:, 0], dv[:, 0]
    return dq, dk, dv


# ---------------------------------------------------------------- optimizers
def adam_step(p, g, m, v, t, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
              amsgrad=False, v_max=None):
    """One Adam/AdamW step for step count t (already incremented), returning new
    (p, m, v, v_max) (_nn.py:1413-1442; FusedAdam _training.py:2198-2220):
    decoupled decay first, then moments, bias corrections and the update."""
    b1, b2 = betas
    p = p.copy()
    if weight_decay > 0:
        p = p - lr * weight_decay * p
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g ** 2
    mh = m / (1 - b1 ** t)
    vh = v / (1 - b2 ** t)
    if amsgrad:
        v_max = np.maximum(v_max, vh)
        den = np.sqrt(v_max) + eps
    else:
        den = np.sqrt(vh) + eps
    p = p - lr * mh / den
    return p, m, v, v_max


class GradScalerRef:
    """Dynamic loss-scale state machine of GradScaler (_nn.py:1713-1912) over NumPy
    grads held in a list of dicts {'grad': array}.  Restated for the oracle."""

    def __init__(self, init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5,
                 growth_interval=2000, min_scale=1.0, max_scale=2.0 ** 24, enabled=True):
        if init_scale <= 0:
            raise ValueError("init_scale must be positive")
        if min_scale <= 0:
            raise ValueError("min_scale must be positive")
        if max_scale < init_scale:
            raise ValueError("max_scale must be >= init_scale")
        self.scale = init_scale
        self.growth_factor, self.backoff_factor = growth_factor, backoff_factor
        self.growth_interval, self.min_scale, self.max_scale = growth_interval, min_scale, max_scale
        self.enabled = enabled
        self.tracker = 0
        self.found_inf = False
        self.overflow_count = 0
        self.step_count = 0
        self.successes = 0

    def unscale(self, grads, zero_nan_grads=True):
        """Per grad: non-finite before -> found, zero; else multiply by 1/scale and
        check again (_nn.py:1810-1831).  Returns the new grad list."""
        inv = 1.0 / self.scale
        self.found_inf = False
        out = []
        for g in grads:
            if g is None:
                out.append(None)
                continue
            if not np.all(np.isfinite(g)):
                self.found_inf = True
                out.append(np.zeros_like(g) if zero_nan_grads else g)
                continue
            gs = g * np.asarray(inv, dtype=g.dtype)
            if not np.all(np.isfinite(gs)):
                self.found_inf = True
                gs = np.zeros_like(gs) if zero_nan_grads else gs
            out.append(gs)
        return out

    def update(self):
        """(_nn.py:1851-1868)."""
        self.step_count += 1
        if self.found_inf:
            self.overflow_count += 1
            self.successes = 0
            self.scale = max(self.scale * self.backoff_factor, self.min_scale)
            self.tracker = 0
        else:
            self.successes += 1
            self.tracker += 1
            if self.tracker >= self.growth_interval:
                self.scale = min(self.scale * self.growth_factor, self.max_scale)
                self.tracker = 0


def clip_grad_norm(grads, max_norm, norm_type=2.0):
    """clip_grad_norm_ (_nn.py:1563-1626) without the warning: zero non-finite
    entries, total norm (Python float accumulation), rescale when
    max_norm/(norm+1e-6) < 1.  Returns (new_grads, total_norm)."""
    grads = [None if g is None else np.where(np.isfinite(g), g, 0).astype(g.dtype)
             for g in grads]
    live = [g for g in grads if g is not None]
    if not live:
        return grads, 0.0
    if norm_type == float("inf"):
        total = max(float(np.abs(g).max()) for g in live)
    else:
        total = sum(float((np.abs(g) ** norm_type).sum()) for g in live) ** (1.0 / norm_type)
    if total == 0.0:
        return grads, 0.0
    coef = max_norm / (total + 1e-6)
    if coef < 1.0:
        grads = [None if g is None else g * np.asarray(coef, dtype=g.dtype) for g in grads]
    return grads, total


# ---------------------------------------------------------------- losses / embedding
def _ce_weights(n, c, targets, label_smoothing):
    w = np.full((n, c), label_smoothing / c)
    w[np.arange(n), targets] += 1.0 - label_smoothing
    return w


def cross_entropy_fwd(logits, targets, label_smoothing=0.0, reduction="mean"):
    """Cross-entropy with logits (_nn.py:1136-1164): probs by max shift;
    loss_i = -log(p_target + 1e-10), or with label smoothing s
    loss_i = -sum_c w_c log(p_c + 1e-10), w = s/C + (1-s) onehot (_nn.py:1152-1156);
    reduced by mean / sum / none.  Returns (loss, probs)."""
    sh = logits - logits.max(axis=1, keepdims=True)
    e = np.exp(sh)
    probs = e / e.sum(axis=1, keepdims=True)
    n, c = logits.shape
    if label_smoothing > 0:
        w = _ce_weights(n, c, targets, label_smoothing)
        rows = -(w * np.log(probs + 1e-10)).sum(axis=1)
    else:
        rows = -np.log(probs[np.arange(n), targets] + 1e-10)
    if reduction == "mean":
        return rows.mean(), probs
    if reduction == "sum":
        return rows.sum(), probs
    return rows, probs


def cross_entropy_bwd(probs, targets, label_smoothing=0.0, reduction="mean"):
    """(_nn.py:1168-1180): logits.grad += (probs - w)/N for the mean (w the target
    distribution), unscaled for sum / none.  The upstream gradient of the loss is NOT
    applied (the reference closure never reads out.grad)."""
    n, c = probs.shape
    g = probs - _ce_weights(n, c, targets, label_smoothing)
    return g / n if reduction == "mean" else g


def embedding_bwd(idx, dout, num_embeddings):
    """Embedding backward (_nn.py:1083-1089): scatter-add of dout rows by index."""
    dim = dout.shape[-1]
    g = np.zeros((num_embeddings, dim), dtype=dout.dtype)
    np.add.at(g, idx.reshape(-1), dout.reshape(-1, dim))
    return g


# ---------------------------------------------------------------- C1 MLP step
def mlp_step(x, w1, b1, w2, b2, lr=1e-3, dtype=np.float64):
    """README MLP (config 1): h = gelu(x@w1 + b1); out = h@w2 + b2; loss = out.mean();
    backward (mean -> add -> matmul -> gelu -> add -> matmul); one Adam step
    (t = 1, betas 0.9/0.999, eps 1e-8, no decay).  Returns dict of loss, grads and
    updated params."""
    x, w1, b1, w2, b2 = (np.asarray(a, dtype=dtype) for a in (x, w1, b1, w2, b2))
    z1 = x @ w1 + b1
    h = gelu_fwd(z1)
    out = h @ w2 + b2
    loss = out.mean()
    dout = np.full(out.shape, 1.0 / out.size, dtype=dtype)
    db2 = unbroadcast(dout, b2.shape)
    dh, dw2 = matmul_bwd(h, w2, dout)
    dz1 = gelu_bwd(z1, dh)
    db1 = unbroadcast(dz1, b1.shape)
    _, dw1 = matmul_bwd(x, w1, dz1)
    res = {"loss": loss, "dw1": dw1, "db1": db1, "dw2": dw2, "db2": db2}
    for name, p, g in (("w1", w1, dw1), ("b1", b1, db1), ("w2", w2, dw2), ("b2", b2, db2)):
        z = np.zeros_like(p)
        res[name], _, _, _ = adam_step(p, g, z, z, 1, lr=lr)
    return res
