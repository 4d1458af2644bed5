"""ctypes binding of libtgbwd.so (the gfx950 kernels) and thin typed wrappers.

Every wrapper takes torch device tensors (torch is used only as the device
allocator and stream provider), checks shapes/dtypes on the host, passes raw
pointers and sizes across the C-ABI declared in include/tgbwd.h, and raises
RuntimeError with the library's message on a non-zero status.

There is no fallback: if the shared library is missing or cannot be loaded,
every wrapper raises.  Build it with ``python project-tensor_amd/build_lib.py``.
"""
import ctypes
import os
import threading

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("TG_HIP_LIB", os.path.join(_HERE, "libtgbwd.so"))

F32, F16, BF16, F64 = 0, 1, 2, 3
NHWC, NCHW = 0, 1

_TORCH_TO_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
                  torch.float64: F64}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_sz = ctypes.c_size_t

# name -> (restype, argtypes).  Mirrors include/tgbwd.h one to one.
SIGNATURES = {
    "tg_init": (_i32, [_i32]),
    "tg_last_error": (ctypes.c_char_p, []),
    "tg_version": (_i32, []),
    "tg_stream_sync": (_i32, [_vp]),
    "tg_gelu_bwd": (_i32, [_i32, _vp, _vp, _vp, _i64, _i32, _vp]),
    "tg_silu_bwd": (_i32, [_i32, _vp, _vp, _vp, _i64, _i32, _vp]),
    "tg_gelu_fwd": (_i32, [_i32, _vp, _vp, _i64, _vp]),
    "tg_unary_bwd": (_i32, [_i32, _i32, _vp, _vp, _vp, _i64, _f64, _i32, _vp]),
    "tg_log_softmax_bwd": (_i32, [_i32, _vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "tg_index_add_sorted": (_i32, [_i32, _vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    "tg_max_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "tg_gemm_epilogue": (_i32, [_i32, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp,
                                _i64, _f32, _vp, _i64, _vp]),
    "tg_silu_fwd": (_i32, [_i32, _vp, _vp, _i64, _vp]),
    "tg_axpby": (_i32, [_i32, _vp, _i32, _vp, _i64, _f32, _f32, _vp]),
    "tg_axpbyz": (_i32, [_i32, _vp, _i32, _vp, _vp, _i64, _f32, _f32, _vp]),
    "tg_axpbyz64": (_i32, [_i32, _vp, _i32, _vp, _vp, _i64, _f64, _f64, _vp]),
    "tg_fill": (_i32, [_i32, _vp, _i64, _f32, _vp]),
    "tg_softmax_fwd": (_i32, [_i32, _vp, _vp, _i64, _i64, _vp]),
    "tg_softmax_bwd": (_i32, [_i32, _vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "tg_layernorm_fwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _vp]),
    "tg_layernorm_bwd_workspace": (_sz, [_i32, _i64, _i64]),
    "tg_layernorm_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                _i32, _i32, _vp, _sz, _vp]),
    "tg_layernorm_bwd_add": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                    _i64, _i32, _vp, _sz, _vp]),
    "tg_layernorm_bwd_noalloc_max_scratch": (_sz, []),
    "tg_layernorm_bwd_noalloc": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                        _i64, _i32, _i32, _vp]),
    "tg_broadcast_mul_sum": (_i32, [_i32, _vp, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _vp,
                                    _f64, _i32, _vp]),
    "tg_reduce_rows_workspace": (_sz, [_i64, _i64]),
    "tg_reduce_rows": (_i32, [_i32, _vp, _i32, _vp, _i64, _i64, _i32, _vp, _sz, _vp]),
    "tg_batchnorm_workspace": (_sz, [_i32, _i64, _i64, _i64]),
    "tg_batchnorm_fwd_train": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f32,
                                      _i64, _i64, _i64, _f32, _i32, _vp, _sz, _vp]),
    "tg_batchnorm_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                _i64, _i32, _i32, _i32, _vp, _sz, _vp]),
    "tg_adam_step": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _f64, _f64, _f64, _f64, _f64,
                            _f64, _f64, _vp]),
    "tg_cross_entropy_fwd_f64": (_i32, [_vp, _vp, _i64, _i64, _f64, _vp, _vp, _vp]),
    "tg_cross_entropy_bwd_f64": (_i32, [_vp, _vp, _vp, _i64, _i64, _f64, _f64, _vp, _i32,
                                        _vp]),
    "tg_adam_step_f64": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _f64, _f64, _f64, _f64,
                                _f64, _f64, _f64, _vp]),
    "tg_adam_step_lowp": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _f64, _f64, _f64, _f64,
                                 _f64, _f64, _f64, _i32, _vp, _vp]),
    "tg_adam_step_scaled": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _f64, _f64, _f64, _f64,
                                   _f64, _f64, _f64, _f32, _f32, _i32, _vp, _vp]),
    "tg_unscale_check": (_i32, [_i32, _i32, _vp, _vp, _f32, _i32, _vp, _vp]),
    "tg_unscale_norm_workspace": (_sz, [_i32, _vp]),
    "tg_unscale_norm": (_i32, [_i32, _i32, _vp, _vp, _f32, _vp, _vp, _vp, _sz, _vp]),
    "tg_grad_norm_workspace": (_sz, [_i32, _vp]),
    "tg_grad_norm": (_i32, [_i32, _i32, _vp, _vp, _i32, _f32, _vp, _vp, _vp, _sz, _vp]),
    "tg_zero_nonfinite": (_i32, [_i32, _i32, _vp, _vp, _vp]),
    "tg_zero_flagged": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp]),
    "tg_gemm": (_i32, [_i32, _i32, _i32, _i32, _i64, _i64, _i64, _f32, _vp, _i64, _i64, _vp,
                       _i64, _i64, _f32, _vp, _i64, _i64, _i64, _vp]),
    "tg_gemm_bias": (_i32, [_i32, _i32, _i32, _i32, _i64, _i64, _i64, _f32, _vp, _i64, _vp, _i64,
                            _vp, _vp, _i64, _vp]),
    "tg_gemm_wgrad_workspace": (_sz, [_i32, _i64, _i64, _i64, _i32]),
    "tg_gemm_wgrad": (_i32, [_i32, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i32, _vp, _i64, _i32,
                             _i32, _vp, _i32, _vp, _sz, _vp]),
    "tg_gemm_wgrad_group_workspace": (_sz, [_i32, _i32, _i64, _i64, _i64, _i32]),
    "tg_gemm_wgrad_group_n_workspace": (_sz, [_i32, _i32, _i64, _vp, _i64, _i32]),
    "tg_gemm_wgrad_group_n": (_i32, [_i32, _i32, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i32,
                                     _vp, _vp, _vp, _i32, _vp, _vp, _vp, _sz, _vp]),
    "tg_gemm_wgrad_group": (_i32, [_i32, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i32,
                                   _vp, _i64, _vp, _i32, _vp, _vp, _vp, _sz, _vp]),
    "tg_flash_attn_fwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                 _f32, _i32, _vp]),
    "tg_flash_attn_fwd_layout": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                        _i64, _f32, _i32, _i32, _vp]),
    "tg_flash_attn_bwd_layout": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                        _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i32, _vp, _sz,
                                        _vp]),
    "tg_flash_attn_fwd_qkv": (_i32, [_i32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _i32,
                                     _vp]),
    "tg_flash_attn_bwd_qkv": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32,
                                     _i32, _i32, _vp, _sz, _vp]),
    "tg_flash_attn_bwd_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "tg_flash_attn_f64_workspace": (_sz, [_i64, _i64, _i64, _i64]),
    "tg_flash_attn_fwd_f64": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f64,
                                     _i32, _i32, _vp, _sz, _vp]),
    "tg_flash_attn_bwd_f64": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                     _i64, _i64, _i64, _f64, _i32, _i32, _i32, _vp, _sz, _vp]),
    "tg_batchnorm_stats_workspace": (_sz, [_i64]),
    "tg_batchnorm_fwd_train_f64": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _f64, _i64, _i64, _i64, _f64, _i32, _vp]),
    "tg_batchnorm_bwd_stats": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _i64, _i64, _i64, _i32, _i32, _i32, _vp, _sz, _vp]),
    "tg_flash_attn_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                 _i64, _i64, _i64, _f32, _i32, _i32, _vp, _sz, _vp]),
    "tg_cross_entropy_fwd": (_i32, [_i32, _vp, _vp, _i64, _i64, _f32, _vp, _vp, _vp]),
    "tg_cross_entropy_fwd_grad_max_classes": (_i32, [_i32]),
    "tg_cross_entropy_fwd_grad": (_i32, [_i32, _vp, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _vp]),
    "tg_embedding_bwd_workspace": (_sz, [_i64, _i64]),
    "tg_layernorm_bwd_partials": (_i64, [_i32, _vp, _vp, _vp, _vp, _i64, _i64]),
    "tg_sum_partials2_group": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tg_embedding_fwd": (_i32, [_i32, _vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp]),
    "tg_embedding_bwd": (_i32, [_i32, _vp, _vp, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _sz, _vp]),
    "tg_transpose_add": (_i32, [_i32, _vp, _i64, _i64, _i32, _vp, _f32, _vp]),
    "tg_cross_entropy_bwd": (_i32, [_i32, _vp, _vp, _vp, _i64, _i64, _f32, _f32, _i32, _vp, _i32,
                                    _vp]),
}

_lib = None
_lib_lock = threading.Lock()
_inited = set()


def load():
    """Load libtgbwd.so and bind every exported function (no GPU needed)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libtgbwd.so not found at {LIB_PATH}; build it with "
                "`python project-tensor_amd/build_lib.py` (no fallback path exists)")
        lib = ctypes.CDLL(LIB_PATH)
        missing = []
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError:
                missing.append(name)
                continue
            fn.restype = res
            fn.argtypes = args
        if missing:
            raise RuntimeError(f"{LIB_PATH} lacks exported symbols {missing}; rebuild it")
        _lib = lib
    return _lib


def last_error():
    return load().tg_last_error().decode(errors="replace")


def _check(name, status):
    if status != 0:
        raise RuntimeError(f"{name} failed (status {status}): {last_error()}")


def ensure_device(device_index=None):
    """tg_init once per device (checks the part is gfx950)."""
    if device_index is None:
        device_index = torch.cuda.current_device()
    if device_index not in _inited:
        _check("tg_init", load().tg_init(int(device_index)))
        _inited.add(device_index)


if hasattr(torch._C, "_cuda_getCurrentRawStream") and hasattr(torch._C, "_cuda_getDevice"):
    _raw_stream = torch._C._cuda_getCurrentRawStream
    _cur_dev = torch._C._cuda_getDevice

    def stream_handle():
        """The current HIP stream of the current device (torch's current stream), as
        the integer handle a c_void_p argument takes."""
        return _raw_stream(_cur_dev())
else:
    def stream_handle():
        return torch.cuda.current_stream().cuda_stream


# Host-to-device copies of NumPy inputs (token ids, targets, data batches) go through a
# small ring of reusable pinned buffers with a non-blocking copy on the current stream:
# a pageable copy would block the host until the device queue drains, so the host could
# never run ahead of the GPU.  A slot is reused only after the event recorded behind
# its previous copy has completed.
_STAGE_SLOTS = 4
_STAGE_MAX = 64 << 20
_stage = [[None, None] for _ in range(_STAGE_SLOTS)]
_stage_next = [0]


def to_device(arr, device=None):
    """A contiguous device copy of the NumPy array `arr` (same dtype and shape)."""
    a = np.asarray(arr)
    if not a.flags.c_contiguous:
        a = np.ascontiguousarray(a)  # (only for ndim >= 1: it would make a 0-d array 1-d)
    dev = torch.device("cuda") if device is None else torch.device(device)
    if a.nbytes == 0 or a.nbytes > _STAGE_MAX or a.dtype.hasobject:
        return torch.as_tensor(a, device=dev)
    src_t = torch.from_numpy(a)
    slot = _stage[_stage_next[0] % _STAGE_SLOTS]
    _stage_next[0] += 1
    if slot[1] is not None:
        slot[1].synchronize()
    if slot[0] is None or slot[0].numel() < a.nbytes:
        slot[0] = torch.empty(max(a.nbytes, 1 << 20), dtype=torch.uint8, pin_memory=True)
    pinned = slot[0][: a.nbytes].view(src_t.dtype).view(src_t.shape)
    pinned.copy_(src_t)
    out = torch.empty(src_t.shape, dtype=src_t.dtype, device=dev)
    out.copy_(pinned, non_blocking=True)
    ev = torch.cuda.Event()
    ev.record()
    slot[1] = ev
    return out


def dtype_code(t):
    try:
        return _TORCH_TO_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype} for the HIP kernels "
                        "(float32, float16, bfloat16, float64 are supported)") from None


def ptr(t):
    # a c_void_p argument takes the integer address (None: NULL)
    return t.data_ptr() if t is not None else None


def _dev(t, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a torch device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def workspace(nbytes, device):
    """Caller-owned scratch from torch's caching allocator."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _same(name, *ts):
    shape, dt = ts[0].shape, ts[0].dtype
    for t in ts[1:]:
        if t.shape != shape or t.dtype != dt:
            raise ValueError(f"{name}: operands must share shape and dtype, got "
                             f"{[tuple(x.shape) for x in ts]} / {[x.dtype for x in ts]}")


# ---------------------------------------------------------------- elementwise
def act_bwd(kind, x, dy, dx, accumulate):
    """dx (+)= dy * act'(x) for kind in {'gelu', 'silu'}."""
    for n, t in (("x", x), ("dy", dy), ("dx", dx)):
        _dev(t, n)
    _same(f"{kind}_bwd", x, dy, dx)
    ensure_device(x.device.index)
    fn = load().tg_gelu_bwd if kind == "gelu" else load().tg_silu_bwd
    _check(f"tg_{kind}_bwd", fn(dtype_code(x), ptr(x), ptr(dy), ptr(dx), x.numel(),
                                int(bool(accumulate)), stream_handle()))
    return dx


UNARY_OPS = {"relu": 0, "leaky_relu": 1, "sigmoid": 2, "tanh": 3, "exp": 4, "log": 5,
             "pow": 6, "swish": 7}


def unary_bwd(op, a, dy, dx, accumulate, param=0.0):
    """dx (+)= f'(a) * dy (tg_unary_bwd); a is the op's input x or output y as
    include/tgbwd.h lists per op; param is the LeakyReLU slope or the exponent."""
    for n, t in (("a", a), ("dy", dy), ("dx", dx)):
        _dev(t, n)
    _same(f"{op}_bwd", a, dy, dx)
    ensure_device(a.device.index)
    _check("tg_unary_bwd", load().tg_unary_bwd(dtype_code(a), UNARY_OPS[op], ptr(a), ptr(dy),
                                               ptr(dx), a.numel(), float(param),
                                               int(bool(accumulate)), stream_handle()))
    return dx


def log_softmax_bwd(y, dy, dx, accumulate):
    """dx (+)= dy - exp(y) * sum_row(dy) over the last axis (tg_log_softmax_bwd)."""
    for n, t in (("y", y), ("dy", dy), ("dx", dx)):
        _dev(t, n)
    _same("log_softmax_bwd", y, dy, dx)
    rows, cols = _rows_cols(y)
    ensure_device(y.device.index)
    _check("tg_log_softmax_bwd",
           load().tg_log_softmax_bwd(dtype_code(y), ptr(y), ptr(dy), ptr(dx), rows, cols,
                                     int(bool(accumulate)), stream_handle()))
    return dx


GEMM_EPI = {"gelu_bwd": 1, "gelu_fwd": 2, "residual": 3}


def gemm_epilogue(epi, a, b, x, out, bias=None, beta=0.0):
    """A Linear layer's GEMM with a fused epilogue (tg_gemm_epilogue): "gelu_bwd"
    out (+)= (a @ b.T) * gelu'(x); "gelu_fwd" out = a @ b + bias and x = gelu(out);
    "residual" out = a @ b + bias + x.  a [M, K]; b [N, K] for gelu_bwd, else [K, N];
    x and out [M, N]; all fp16 or all bf16, contiguous.  Returns False (nothing run)
    when the fused kernel does not serve the shape or layout."""
    for n, t in (("a", a), ("b", b), ("x", x), ("out", out)):
        _dev(t, n)
    dt = a.dtype
    if dt not in (torch.float16, torch.bfloat16) or any(t.dtype != dt for t in (b, x, out)):
        return False
    M, K = a.shape
    N = b.shape[0] if epi == "gelu_bwd" else b.shape[1]
    if (b.shape[1] if epi == "gelu_bwd" else b.shape[0]) != K or tuple(x.shape) != (M, N) \
            or tuple(out.shape) != (M, N):
        raise ValueError(f"gemm_epilogue: shapes {tuple(a.shape)} {tuple(b.shape)} "
                         f"{tuple(x.shape)} {tuple(out.shape)}")
    if bias is not None:
        _dev(bias, "bias")
        if bias.dtype != torch.float32 or bias.numel() != N:
            raise ValueError("gemm_epilogue: bias must be fp32 [N]")
    if _split_k(M, N, K, a.device) > 1:
        # the plain product would run K-split (another summation order): not fused, so
        # a fused result always equals the separate kernels' bit for bit
        return False
    ensure_device(a.device.index)
    st = load().tg_gemm_epilogue(dtype_code(a), GEMM_EPI[epi], M, N, K, ptr(a), K, ptr(b),
                                 b.shape[1], ptr(bias), ptr(x), N, float(beta), ptr(out), N,
                                 stream_handle())
    if st == -3:
        return False
    _check("tg_gemm_epilogue", st)
    return True


def max_bwd(x, r, g, dx, accumulate):
    """dx (+)= (x == r) * g / count per row of x [rows, cols] (tg_max_bwd); r and g
    hold one value per row."""
    for n, t in (("x", x), ("r", r), ("g", g), ("dx", dx)):
        _dev(t, n)
    _same("max_bwd", x, dx)
    _same("max_bwd", r, g)
    rows, cols = _rows_cols(x)
    if r.numel() != rows or r.dtype != x.dtype:
        raise ValueError("max_bwd: one maximum per row of x's dtype expected")
    ensure_device(x.device.index)
    _check("tg_max_bwd", load().tg_max_bwd(dtype_code(x), ptr(x), ptr(r), ptr(g), ptr(dx), rows,
                                           cols, int(bool(accumulate)), stream_handle()))
    return dx


def index_add_sorted(grad, target, start, order, src):
    """grad.flat[target[s]] += in-order sum of src.flat[order[start[s]:start[s+1]]]
    (tg_index_add_sorted): the scatter-add of an advanced-index __getitem__."""
    _dev(grad, "grad")
    _dev(src, "src")
    for n, t in (("target", target), ("start", start), ("order", order)):
        _dev(t, n)
        if t.dtype != torch.int64:
            raise TypeError(f"index_add_sorted: {n} must be int64")
    if src.dtype != grad.dtype:
        raise ValueError("index_add_sorted: src and grad dtypes differ")
    nseg = target.numel()
    if start.numel() != nseg + 1 or order.numel() != src.numel():
        raise ValueError("index_add_sorted: inconsistent segment arrays")
    ensure_device(grad.device.index)
    _check("tg_index_add_sorted",
           load().tg_index_add_sorted(dtype_code(grad), ptr(grad), nseg, ptr(target),
                                      ptr(start), ptr(order), ptr(src), stream_handle()))
    return grad


def act_fwd(kind, x, y=None):
    _dev(x, "x")
    if y is None:
        y = torch.empty_like(x)
    _same(f"{kind}_fwd", x, y)
    ensure_device(x.device.index)
    fn = load().tg_gelu_fwd if kind == "gelu" else load().tg_silu_fwd
    _check(f"tg_{kind}_fwd", fn(dtype_code(x), ptr(x), ptr(y), x.numel(), stream_handle()))
    return y


def axpby(x, y, alpha=1.0, beta=1.0):
    """y = alpha*x + beta*y in place (x, y contiguous, same numel; dtypes may differ)."""
    _dev(x, "x")
    _dev(y, "y")
    if x.numel() != y.numel():
        raise ValueError(f"axpby: numel mismatch {x.numel()} vs {y.numel()}")
    ensure_device(y.device.index)
    if torch.float64 in (x.dtype, y.dtype):  # double scalars for fp64 arithmetic
        _check("tg_axpbyz64", load().tg_axpbyz64(dtype_code(x), ptr(x), dtype_code(y), ptr(y),
                                                 ptr(y), y.numel(), float(alpha), float(beta),
                                                 stream_handle()))
        return y
    _check("tg_axpby", load().tg_axpby(dtype_code(x), ptr(x), dtype_code(y), ptr(y), y.numel(),
                                       float(alpha), float(beta), stream_handle()))
    return y


def axpbyz(x, y, alpha=1.0, beta=1.0, out=None):
    """out = alpha*x + beta*y (contiguous, same numel; out has y's dtype)."""
    _dev(x, "x")
    _dev(y, "y")
    if x.numel() != y.numel():
        raise ValueError(f"axpbyz: numel mismatch {x.numel()} vs {y.numel()}")
    if out is None:
        out = torch.empty(y.shape, dtype=y.dtype, device=y.device)
    elif out.dtype != y.dtype or out.numel() != y.numel() or not out.is_contiguous():
        raise ValueError("axpbyz: out must be contiguous with y's dtype and numel")
    ensure_device(y.device.index)
    fn = load().tg_axpbyz64 if torch.float64 in (x.dtype, y.dtype) else load().tg_axpbyz
    _check("tg_axpbyz", fn(dtype_code(x), ptr(x), dtype_code(y), ptr(y), ptr(out), y.numel(),
                           float(alpha), float(beta), stream_handle()))
    return out


def fill(y, value):
    _dev(y, "y")
    ensure_device(y.device.index)
    _check("tg_fill", load().tg_fill(dtype_code(y), ptr(y), y.numel(), float(value),
                                     stream_handle()))
    return y


_BCAST_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float64: 3}


def _i64_array(vals):
    return (ctypes.c_int64 * max(len(vals), 1))(*vals)


def _bcast_space(shapes):
    """NumPy broadcast of the shapes (right-aligned), as torch.broadcast_shapes."""
    nd = max(len(sh) for sh in shapes)
    space = [1] * nd
    for sh in shapes:
        off = nd - len(sh)
        for i, n in enumerate(sh):
            cur = space[off + i]
            if n != cur:
                if cur == 1:
                    space[off + i] = n
                elif n != 1:
                    raise RuntimeError(f"shapes {shapes} are not broadcastable")
    return tuple(space)


def _bcast_strides(t, space):
    """Strides of t viewed expanded to space (0 on broadcast axes), as
    t.expand(space).stride()."""
    off = len(space) - t.dim()
    st = [0] * len(space)
    for i, (n, s_) in enumerate(zip(t.shape, t.stride())):
        st[off + i] = s_ if n == space[off + i] else 0
    return st


_BCAST_PLANS = {}


def _bcast_plan(out, a, b):
    """(nd, space, strides of a, b, out) as ctypes int64 arrays for broadcast_mul_sum,
    cached by the operands' shapes and strides (training loops repeat them)."""
    key = (a.shape, a.stride(), out.shape, out.stride(),
           None if b is None else (b.shape, b.stride()))
    plan = _BCAST_PLANS.get(key)
    if plan is not None:
        return plan
    shapes = [tuple(a.shape), tuple(out.shape)] + ([tuple(b.shape)] if b is not None else [])
    space = _bcast_space(shapes)
    if len(out.shape) > len(space):
        raise ValueError(f"broadcast_mul_sum: out {tuple(out.shape)} has more axes than {space}")
    for size, stride in zip(out.shape, out.stride()):
        if size > 1 and stride == 0:
            raise ValueError("broadcast_mul_sum: out overlaps itself (a zero stride)")
    nd = len(space)
    plan = (nd, _i64_array(space), _i64_array(_bcast_strides(a, space)),
            _i64_array(_bcast_strides(b, space)) if (b is not None and nd) else None,
            _i64_array(_bcast_strides(out, space)))
    if len(_BCAST_PLANS) > 4096:
        _BCAST_PLANS.clear()
    _BCAST_PLANS[key] = plan
    return plan


def broadcast_mul_sum(out, a, b=None, alpha=1.0, accumulate=False):
    """out (+)= alpha * a * b, with a and b broadcast (NumPy rules) to the index space
    broadcast(a, b, out) and the result summed over every axis where out has extent 1
    (or that out lacks, counted from the right).  Any strides and any mix of fp32 /
    fp16 / bf16 / fp64; b may be None.  Returns out."""
    for n, t in (("out", out), ("a", a), ("b", b)):
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise TypeError(f"broadcast_mul_sum: {n} must be a torch device tensor")
        if t.dtype not in _BCAST_CODE:
            raise TypeError(f"broadcast_mul_sum: unsupported dtype {t.dtype} for {n}")
    nd, space, sa, sb, so = _bcast_plan(out, a, b)
    ensure_device(out.get_device())
    _check("tg_broadcast_mul_sum", (_lib or load()).tg_broadcast_mul_sum(
        nd, space, _BCAST_CODE[a.dtype], a.data_ptr(), sa,
        _BCAST_CODE[b.dtype] if b is not None else 0, b.data_ptr() if b is not None else None,
        sb, _BCAST_CODE[out.dtype], out.data_ptr(), so, float(alpha), int(bool(accumulate)),
        stream_handle()))
    return out


# ---------------------------------------------------------------- row-wise
def _rows_cols(t):
    cols = t.shape[-1] if t.dim() > 0 else 1
    rows = t.numel() // cols if cols else 0
    return rows, cols


def softmax_fwd(x, y=None):
    _dev(x, "x")
    if y is None:
        y = torch.empty_like(x)
    _same("softmax_fwd", x, y)
    rows, cols = _rows_cols(x)
    ensure_device(x.device.index)
    _check("tg_softmax_fwd", load().tg_softmax_fwd(dtype_code(x), ptr(x), ptr(y), rows, cols,
                                                   stream_handle()))
    return y


def softmax_bwd(y, dy, dx, accumulate):
    for n, t in (("y", y), ("dy", dy), ("dx", dx)):
        _dev(t, n)
    _same("softmax_bwd", y, dy, dx)
    rows, cols = _rows_cols(y)
    ensure_device(y.device.index)
    _check("tg_softmax_bwd", load().tg_softmax_bwd(dtype_code(y), ptr(y), ptr(dy), ptr(dx), rows,
                                                   cols, int(bool(accumulate)), stream_handle()))
    return dx


def layernorm_fwd(x, gamma, beta, eps, y=None, mean=None, rstd=None):
    _dev(x, "x")
    cols = gamma.numel()
    rows = x.numel() // cols
    if y is None:
        y = torch.empty_like(x)
    # row statistics in fp32, or fp64 for fp64 input; the parameters are fp32
    sdt = torch.float64 if x.dtype == torch.float64 else torch.float32
    if mean is None:
        mean = torch.empty(rows, dtype=sdt, device=x.device)
    if rstd is None:
        rstd = torch.empty(rows, dtype=sdt, device=x.device)
    for n, t, want in (("gamma", gamma, torch.float32), ("beta", beta, torch.float32),
                       ("mean", mean, sdt), ("rstd", rstd, sdt)):
        _dev(t, n)
        if t.dtype != want:
            raise TypeError(f"layernorm_fwd: {n} must be {want}")
    ensure_device(x.device.index)
    _check("tg_layernorm_fwd", load().tg_layernorm_fwd(
        dtype_code(x), ptr(x), ptr(gamma), ptr(beta), ptr(y), ptr(mean), ptr(rstd), rows, cols,
        float(eps), stream_handle()))
    return y, mean, rstd


def layernorm_bwd(x, mean, rstd, gamma, dy, dx, dgamma, dbeta, accumulate_dx,
                  accumulate_params, dx_add=None):
    """dx (+)= LayerNorm input gradient; with dx_add (another buffer of dx's shape),
    dx = gradient + dx_add instead (accumulate_dx is then ignored)."""
    for n, t in (("x", x), ("dy", dy), ("dx", dx), ("mean", mean), ("rstd", rstd),
                 ("gamma", gamma)):
        _dev(t, n)
    _same("layernorm_bwd", x, dy, dx)
    if dx_add is not None:
        _dev(dx_add, "dx_add")
        _same("layernorm_bwd", x, dx_add)
    cols = gamma.numel()
    rows = x.numel() // cols
    lib = load()
    ensure_device(x.device.index)
    code = dtype_code(x)
    nbytes = lib.tg_layernorm_bwd_workspace(code, rows, cols)
    ws = workspace(nbytes, x.device)
    if dx_add is not None:
        _check("tg_layernorm_bwd_add", lib.tg_layernorm_bwd_add(
            code, ptr(x), ptr(mean), ptr(rstd), ptr(gamma), ptr(dy), ptr(dx_add), ptr(dx),
            ptr(dgamma), ptr(dbeta), rows, cols, int(bool(accumulate_params)), ptr(ws),
            ws.numel(), stream_handle()))
        return dx
    _check("tg_layernorm_bwd", lib.tg_layernorm_bwd(
        code, ptr(x), ptr(mean), ptr(rstd), ptr(gamma), ptr(dy), ptr(dx), ptr(dgamma),
        ptr(dbeta), rows, cols, int(bool(accumulate_dx)), int(bool(accumulate_params)), ptr(ws),
        ws.numel(), stream_handle()))
    return dx


def layernorm_bwd_partials(x, mean, rstd, gamma, dy, dx, accumulate_dx, dx_add=None):
    """layernorm_bwd for dx only, leaving the dgamma/dbeta partial rows for a later
    sum_partials2_group: returns (partials, K), partials a [2, K, cols] fp32 tensor
    (dgamma's rows first), or None (nothing done) where that finish does not cover the
    shape; the caller then runs layernorm_bwd."""
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return None
    for n, t in (("x", x), ("dy", dy), ("dx", dx), ("mean", mean), ("rstd", rstd),
                 ("gamma", gamma)):
        _dev(t, n)
    _same("layernorm_bwd", x, dy, dx)
    if dx_add is not None:
        _dev(dx_add, "dx_add")
        _same("layernorm_bwd", x, dx_add)
    cols = gamma.numel()
    rows = x.numel() // cols
    lib = load()
    code = dtype_code(x)
    K = lib.tg_layernorm_bwd_partials(code, ptr(x), ptr(dy), ptr(dx),
                                      ptr(dx_add) if dx_add is not None else None, rows, cols)
    if K <= 0:
        return None
    ensure_device(x.device.index)
    nbytes = lib.tg_layernorm_bwd_workspace(code, rows, cols)
    ws = torch.empty(max(int(nbytes), 8 * K * cols) // 4 + 1, dtype=torch.float32,
                     device=x.device)
    if dx_add is not None:
        _check("tg_layernorm_bwd_add", lib.tg_layernorm_bwd_add(
            code, ptr(x), ptr(mean), ptr(rstd), ptr(gamma), ptr(dy), ptr(dx_add), ptr(dx),
            None, None, rows, cols, 0, ptr(ws), ws.numel() * 4, stream_handle()))
    else:
        _check("tg_layernorm_bwd", lib.tg_layernorm_bwd(
            code, ptr(x), ptr(mean), ptr(rstd), ptr(gamma), ptr(dy), ptr(dx), None, None,
            rows, cols, int(bool(accumulate_dx)), 0, ptr(ws), ws.numel() * 4,
            stream_handle()))
    return ws[: 2 * K * cols].view(2, K, cols), K


def sum_partials2_group(parts, dgs, dbs, accs):
    """dgs[i] (+)= parts[i][0].sum(0) and dbs[i] (+)= parts[i][1].sum(0) for the
    [2, K, cols] partials of layernorm_bwd_partials, all in one launch (accs[i]: add);
    fp32 outputs, an output may be None."""
    n = len(parts)
    if n == 0:
        return
    for t, d, b in zip(parts, dgs, dbs):
        _dev(t, "partials")
        if t.dtype != torch.float32 or t.dim() != 3 or t.shape[0] != 2 or not t.is_contiguous():
            raise ValueError("sum_partials2_group: partials must be contiguous [2, K, cols] fp32")
        for o in (d, b):
            if o is not None and (o.dtype != torch.float32 or o.numel() != t.shape[2]
                                  or not o.is_contiguous()):
                raise ValueError("sum_partials2_group: outputs must be contiguous fp32 of "
                                 "cols elements")
    Ks = (ctypes.c_int64 * n)(*[t.shape[1] for t in parts])
    cs = (ctypes.c_int64 * n)(*[t.shape[2] for t in parts])
    acc = (ctypes.c_int * n)(*[int(bool(a)) for a in accs])
    ensure_device(parts[0].device.index)
    _check("tg_sum_partials2_group", load().tg_sum_partials2_group(
        n, _ptr_array(parts), Ks, cs, _ptr_array(dgs), _ptr_array(dbs), acc, stream_handle()))


def layernorm_bwd_noalloc(x, mean, rstd, gamma, dy, dx, dgamma, dbeta, accumulate_dx,
                          accumulate_params):
    """layernorm_bwd with the library's fixed device scratch in place of a workspace:
    allocates nothing.  Calls that overlap on one GPU share the scratch and race."""
    for n, t in (("x", x), ("dy", dy), ("dx", dx), ("mean", mean), ("rstd", rstd),
                 ("gamma", gamma)):
        _dev(t, n)
    _same("layernorm_bwd_noalloc", x, dy, dx)
    cols = gamma.numel()
    rows = x.numel() // cols
    ensure_device(x.device.index)
    _check("tg_layernorm_bwd_noalloc", load().tg_layernorm_bwd_noalloc(
        dtype_code(x), ptr(x), ptr(mean), ptr(rstd), ptr(gamma), ptr(dy), ptr(dx), ptr(dgamma),
        ptr(dbeta), rows, cols, int(bool(accumulate_dx)), int(bool(accumulate_params)),
        stream_handle()))
    return dx


def reduce_rows(g, out, accumulate):
    """out (+)= g.reshape(-1, out.numel()).sum(0)."""
    _dev(g, "g")
    _dev(out, "out")
    cols = out.numel()
    rows = g.numel() // cols if cols else 0
    if rows * cols != g.numel():
        raise ValueError("reduce_rows: grad numel is not a multiple of the target numel")
    lib = load()
    ensure_device(out.device.index)
    ws = workspace(lib.tg_reduce_rows_workspace(rows, cols), out.device)
    _check("tg_reduce_rows", lib.tg_reduce_rows(dtype_code(g), ptr(g), dtype_code(out), ptr(out),
                                                rows, cols, int(bool(accumulate)), ptr(ws),
                                                ws.numel(), stream_handle()))
    return out


# ---------------------------------------------------------------- batch norm
def _bn_shape(x, layout):
    if x.dim() != 4:
        raise ValueError(f"batch norm expects a 4-D input, got {tuple(x.shape)}")
    if layout == NHWC:
        N, H, W, C = x.shape
    else:
        N, C, H, W = x.shape
    return N, C, H * W


def batchnorm_fwd_train(x, gamma, beta, eps, momentum, running_mean, running_var, relu,
                        layout=NHWC):
    _dev(x, "x")
    if x.dtype != torch.float32:
        raise TypeError("batch norm kernels are fp32")
    N, C, HW = _bn_shape(x, layout)
    y = torch.empty_like(x)
    mean = torch.empty(C, dtype=torch.float32, device=x.device)
    rstd = torch.empty_like(mean)
    var = torch.empty_like(mean)
    lib = load()
    ensure_device(x.device.index)
    ws = workspace(lib.tg_batchnorm_workspace(layout, N, C, HW), x.device)
    _check("tg_batchnorm_fwd_train", lib.tg_batchnorm_fwd_train(
        layout, ptr(x), ptr(gamma), ptr(beta), ptr(y), ptr(mean), ptr(rstd), ptr(var),
        ptr(running_mean), ptr(running_var), float(momentum), N, C, HW, float(eps),
        int(bool(relu)), ptr(ws), ws.numel(), stream_handle()))
    return y, mean, rstd, var


def batchnorm_fwd_train_f64(x, gamma, beta, eps, momentum, running_mean, running_var, relu,
                            layout=NHWC):
    """fp64 training forward: y (fp64) and the batch mean, rstd, var (fp64, [C]); the
    running statistics (fp64 buffers, or None) take the EMA update in double."""
    _dev(x, "x")
    if x.dtype != torch.float64:
        raise TypeError("batchnorm_fwd_train_f64: x must be float64")
    for n, t in (("running_mean", running_mean), ("running_var", running_var)):
        if t is not None and (t.dtype != torch.float64 or not t.is_contiguous()):
            raise TypeError(f"batchnorm_fwd_train_f64: {n} must be a contiguous float64 buffer")
    N, C, HW = _bn_shape(x, layout)
    y = torch.empty_like(x)
    mean = torch.empty(C, dtype=torch.float64, device=x.device)
    rstd, var = torch.empty_like(mean), torch.empty_like(mean)
    ensure_device(x.device.index)
    _check("tg_batchnorm_fwd_train_f64", load().tg_batchnorm_fwd_train_f64(
        layout, ptr(x), ptr(gamma), ptr(beta), ptr(y), ptr(mean), ptr(rstd), ptr(var),
        ptr(running_mean), ptr(running_var), float(momentum), N, C, HW, float(eps),
        int(bool(relu)), stream_handle()))
    return y, mean, rstd, var


def batchnorm_bwd_stats(x, mean, rstd, gamma, beta, dy, dx, dgamma, dbeta, relu,
                        accumulate_dx, accumulate_params, layout=NHWC):
    """BatchNorm backward with the reference's full formula against given per-channel
    statistics (fp64 mean and rstd [C]): the fp64 path, and the eval-mode BatchNorm2D
    backward on the running statistics.  x, dy, dx fp32 or fp64."""
    for n, t in (("x", x), ("dy", dy), ("dx", dx), ("mean", mean), ("rstd", rstd)):
        _dev(t, n)
    _same("batchnorm_bwd_stats", x, dy, dx)
    if mean.dtype != torch.float64 or rstd.dtype != torch.float64:
        raise TypeError("batchnorm_bwd_stats: mean and rstd must be float64")
    N, C, HW = _bn_shape(x, layout)
    lib = load()
    ensure_device(x.device.index)
    ws = workspace(lib.tg_batchnorm_stats_workspace(C), x.device)
    _check("tg_batchnorm_bwd_stats", lib.tg_batchnorm_bwd_stats(
        dtype_code(x), layout, ptr(x), ptr(mean), ptr(rstd), ptr(gamma), ptr(beta), ptr(dy),
        ptr(dx), ptr(dgamma), ptr(dbeta), N, C, HW, int(bool(relu)), int(bool(accumulate_dx)),
        int(bool(accumulate_params)), ptr(ws), ws.numel(), stream_handle()))
    return dx


def batchnorm_bwd(x, mean, rstd, gamma, beta, dy, dx, dgamma, dbeta, relu, accumulate_dx,
                  accumulate_params, layout=NHWC):
    for n, t in (("x", x), ("dy", dy), ("dx", dx)):
        _dev(t, n)
    _same("batchnorm_bwd", x, dy, dx)
    N, C, HW = _bn_shape(x, layout)
    lib = load()
    ensure_device(x.device.index)
    ws = workspace(lib.tg_batchnorm_workspace(layout, N, C, HW), x.device)
    _check("tg_batchnorm_bwd", lib.tg_batchnorm_bwd(
        layout, ptr(x), ptr(mean), ptr(rstd), ptr(gamma), ptr(beta), ptr(dy), ptr(dx),
        ptr(dgamma), ptr(dbeta), N, C, HW, int(bool(relu)), int(bool(accumulate_dx)),
        int(bool(accumulate_params)), ptr(ws), ws.numel(), stream_handle()))
    return dx


# ---------------------------------------------------------------- multi-tensor
def _ptr_array(ts):
    arr = (ctypes.c_void_p * len(ts))()
    for i, t in enumerate(ts):
        arr[i] = t.data_ptr() if t is not None else 0
    return arr


def _numel_array(ts):
    arr = (ctypes.c_int64 * len(ts))()
    for i, t in enumerate(ts):
        arr[i] = t.numel()
    return arr


# Validated optimizer-state lists, keyed by their device addresses: the checks and the
# pointer arrays of params / exp_avg / exp_avg_sq (/ max_exp_avg_sq) are built once for
# a given set of buffers and reused on every later step with the same buffers.
_ADAM_STATE = {}


def _adam_state(params, exp_avg, exp_avg_sq, max_exp_avg_sq):
    key = (tuple(t.data_ptr() for t in params), tuple(t.data_ptr() for t in exp_avg),
           tuple(t.data_ptr() for t in exp_avg_sq),
           tuple(t.data_ptr() for t in max_exp_avg_sq) if max_exp_avg_sq else None)
    st = _ADAM_STATE.get(key)
    if st is not None and all(p.numel() == n for p, n in zip(params, st[1])):
        return st
    groups = (params, exp_avg, exp_avg_sq) + ((max_exp_avg_sq,) if max_exp_avg_sq else ())
    pdt = params[0].dtype
    if pdt not in (torch.float32, torch.float64):
        raise TypeError("adam_step: fp32 or fp64 tensors required")
    for group in groups:
        if len(group) != len(params):
            raise ValueError("adam_step: param/state list lengths differ")
        for t in group:
            _dev(t, "adam operand")
            if t.dtype != pdt:
                raise TypeError(f"adam_step: every tensor of one step must be {pdt}")
    numels = [p.numel() for p in params]
    for p, m, v in zip(params, exp_avg, exp_avg_sq):
        if not (p.numel() == m.numel() == v.numel()):
            raise ValueError("adam_step: param/grad/state sizes differ")
    if len(_ADAM_STATE) >= 16:
        _ADAM_STATE.clear()
    st = ((_ptr_array(params), _ptr_array(exp_avg), _ptr_array(exp_avg_sq),
           _ptr_array(max_exp_avg_sq) if max_exp_avg_sq else None), numels,
          _numel_array(params))
    _ADAM_STATE[key] = st
    return st


def adam_step(params, grads, exp_avg, exp_avg_sq, max_exp_avg_sq, lr, beta1, beta2, eps,
              weight_decay, bias_correction1, bias_correction2, lowp=None):
    """Multi-tensor Adam/AdamW step.  `lowp`, if given, is a list parallel to `params`
    of None or a contiguous fp16/bf16 tensor of the param's size (one dtype for the
    list) that receives the updated param rounded to that dtype in the same pass."""
    adam_prepare(params, grads, exp_avg, exp_avg_sq, max_exp_avg_sq, lowp)(
        lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2)


def adam_prepare(params, grads, exp_avg, exp_avg_sq, max_exp_avg_sq, lowp=None):
    """The checks and pointer arrays of adam_step for these buffers, done now; returns
    launch(lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2,
    gmul=(1.0, 1.0)), which only enqueues the kernel.  An optimizer prepares while the
    device is still busy and launches after the last host read-back of the step.  gmul
    (fp32 params): the gradients are read as (g * gmul[0]) * gmul[1] (scalings still
    pending on them)."""
    n = len(params)
    if n == 0:
        return lambda *a: None
    arrs, numels, numel_arr = _adam_state(params, exp_avg, exp_avg_sq, max_exp_avg_sq)
    if len(grads) != n:
        raise ValueError("adam_step: param/grad list lengths differ")
    pdt = params[0].dtype
    for g, k in zip(grads, numels):
        _dev(g, "adam operand")
        if g.dtype != pdt:
            raise TypeError(f"adam_step: gradients must be {pdt} like their params")
        if g.numel() != k:
            raise ValueError("adam_step: param/grad/state sizes differ")
    dev = params[0].device.index
    garr = _ptr_array(grads)
    keep = (list(grads),)  # the pointer array's buffers stay alive with the launcher
    lib = load()
    if pdt == torch.float64:
        if lowp is not None and any(t is not None for t in lowp):
            raise TypeError("adam_step: low-precision copies are for fp32 params")
        fn, extra, name = lib.tg_adam_step_f64, (), "tg_adam_step_f64"
    elif lowp is not None and any(t is not None for t in lowp):
        if len(lowp) != n:
            raise ValueError("adam_step: lowp list length differs from params")
        lp = [t for t in lowp if t is not None]
        dt = lp[0].dtype
        for p, t in zip(params, lowp):
            if t is None:
                continue
            _dev(t, "adam low-precision copy")
            if t.dtype != dt or dt not in (torch.float16, torch.bfloat16):
                raise TypeError("adam_step: low-precision copies must share one fp16/bf16 dtype")
            if t.numel() != p.numel() or not t.is_contiguous():
                raise ValueError("adam_step: low-precision copy must be contiguous and of its "
                                 "param's size")
        fn, extra, name = lib.tg_adam_step_lowp, (dtype_code(lp[0]), _ptr_array(lowp)), \
            "tg_adam_step_lowp"
        keep = keep + (list(lowp),)
    else:
        fn, extra, name = lib.tg_adam_step, (), "tg_adam_step"
    scaled_extra = extra if extra else (0, None)

    def launch(lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2,
               gmul=(1.0, 1.0)):
        ensure_device(dev)
        hyper = (float(lr), float(beta1), float(beta2), float(eps), float(weight_decay),
                 float(bias_correction1), float(bias_correction2))
        if tuple(gmul) != (1.0, 1.0):
            if pdt != torch.float32:
                raise TypeError("adam_step: gradient multipliers are for fp32 params")
            _check("tg_adam_step_scaled", lib.tg_adam_step_scaled(
                n, arrs[0], garr, arrs[1], arrs[2], arrs[3], numel_arr, *hyper,
                float(gmul[0]), float(gmul[1]), *scaled_extra, stream_handle()))
            return keep
        _check(name, fn(n, arrs[0], garr, arrs[1], arrs[2], arrs[3], numel_arr, *hyper, *extra,
                        stream_handle()))
        return keep
    return launch


def _group_by_dtype(ts):
    groups = {}
    for i, t in enumerate(ts):
        groups.setdefault(t.dtype, []).append(i)
    return groups


# Per-device buffers reused by the multi-tensor checks (flags, norm results and
# partials): allocating them anew on every call costs more host time than the calls
# themselves, and that host time sits between two read-backs with the GPU idle.
_SCRATCH = {}


def _scratch(key, nbytes, device):
    k = (key, device, stream_handle())  # per stream: calls on one stream are ordered
    t = _SCRATCH.get(k)
    if t is None or t.numel() < nbytes:
        t = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
        _SCRATCH[k] = t
    return t


def unscale_check(grads, mul, write=True, readback=True):
    """Scale grads in place by `mul`; return per-tensor flags (host list of ints):
    bit 0 = non-finite before scaling, bit 1 = non-finite after.  With readback False
    nothing is read back (no host synchronisation) and None is returned."""
    n = len(grads)
    if n == 0:
        return []
    for t in grads:
        _dev(t, "grad")
    dev = grads[0].device
    ensure_device(dev.index)
    flags = _scratch("flags", 4 * n, dev)[: 4 * n].view(torch.int32)
    out = [0] * n
    lib = load()
    groups = _group_by_dtype(grads)
    off = 0
    for dt, idx in groups.items():
        sub = [grads[i] for i in idx]
        fl = flags[off: off + len(sub)]
        off += len(sub)
        _check("tg_unscale_check", lib.tg_unscale_check(
            len(sub), dtype_code(sub[0]), _ptr_array(sub), _numel_array(sub), float(mul),
            int(bool(write)), ptr(fl), stream_handle()))
    if not readback:
        return None
    host = flags.cpu().tolist()
    off = 0
    for dt, idx in groups.items():
        for j, i in enumerate(idx):
            out[i] = host[off + j]
        off += len(idx)
    return out


def unscale_deferred(grads, mul):
    """GradScaler.unscale_ without a synchronisation: grads *= mul, every tensor that
    held or now holds a non-finite value zeroed on the device, and the per-tensor
    flags copied to host memory behind an event.  Returns resolve(), which waits for
    that copy and returns the flags (host list of ints, as unscale_check's) — at no
    cost once the stream has been synchronised for another read-back."""
    n = len(grads)
    if n == 0:
        return lambda: []
    for t in grads:
        _dev(t, "grad")
    dev = grads[0].device
    ensure_device(dev.index)
    # a fresh device buffer per call (not the shared scratch): a later call must not
    # overwrite flags that are still being copied out
    flags = torch.empty(n, dtype=torch.int32, device=dev)
    lib = load()
    groups = _group_by_dtype(grads)
    off = 0
    for dt, idx in groups.items():
        sub = [grads[i] for i in idx]
        fl = flags[off: off + len(sub)]
        off += len(sub)
        gp, ne = _ptr_array(sub), _numel_array(sub)
        _check("tg_unscale_check", lib.tg_unscale_check(
            len(sub), dtype_code(sub[0]), gp, ne, float(mul), 1, ptr(fl), stream_handle()))
        _check("tg_zero_flagged", lib.tg_zero_flagged(
            len(sub), dtype_code(sub[0]), gp, ne, ptr(fl), stream_handle()))
    host = torch.empty(n, dtype=torch.int32, pin_memory=True)
    host.copy_(flags, non_blocking=True)
    flags_keep = [flags]  # held until the copy is known to be done
    ev = torch.cuda.Event()
    ev.record()

    def resolve():
        ev.synchronize()
        del flags_keep[:]
        h = host.tolist()
        out = [0] * n
        o = 0
        for dt, idx in groups.items():
            for j, i in enumerate(idx):
                out[i] = h[o + j]
            o += len(idx)
        return out
    return resolve


def unscale_norm_deferred(grads, mul):
    """unscale_deferred without writing the scaled values: the gradients keep their
    contents (the caller applies `mul` later), every tensor that holds or would hold a
    non-finite value is zeroed on the device, and the squared L2 norm the unscaled,
    zeroed gradients would have is formed in the same pass (bit for bit the value
    grad_norm(kind 0) would return after unscale_deferred).  fp32/fp16/bf16 only.
    Returns resolve() -> (flags, sum of squares), which waits for one asynchronous
    device-to-host copy."""
    n = len(grads)
    if n == 0:
        return lambda: ([], 0.0)
    for t in grads:
        _dev(t, "grad")
        if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise TypeError(f"unscale_norm_deferred: unsupported dtype {t.dtype}")
    dev = grads[0].device
    ensure_device(dev.index)
    lib = load()
    groups = list(_group_by_dtype(grads).items())
    ng = len(groups)
    # per call: the flags and group sums (fresh, a later call must not overwrite them
    # while they are being copied out)
    buf = torch.empty(8 * ng + 4 * n, dtype=torch.uint8, device=dev)
    vals = buf[: 8 * ng].view(torch.float64)
    fls = buf[8 * ng:].view(torch.int32)
    off = 0
    for gi, (dt, idx) in enumerate(groups):
        sub = [grads[i] for i in idx]
        gp, ne = _ptr_array(sub), _numel_array(sub)
        fl = fls[off: off + len(sub)]
        off += len(sub)
        nb = lib.tg_unscale_norm_workspace(len(sub), ne)
        ws = _scratch(("unscalenorm", gi), nb, dev)
        _check("tg_unscale_norm", lib.tg_unscale_norm(
            len(sub), dtype_code(sub[0]), gp, ne, float(mul), ptr(fl), ptr(vals[gi:gi + 1]),
            ptr(ws), ws.numel(), stream_handle()))
        _check("tg_zero_flagged", lib.tg_zero_flagged(
            len(sub), dtype_code(sub[0]), gp, ne, ptr(fl), stream_handle()))
    host = torch.empty(buf.numel(), dtype=torch.uint8, pin_memory=True)
    host.copy_(buf, non_blocking=True)
    keep = [buf]
    ev = torch.cuda.Event()
    ev.record()

    done = []

    def resolve():
        # the first call waits and reads; later calls return the same result
        if done:
            return done[0]
        ev.synchronize()
        del keep[:]
        hv = host[: 8 * ng].view(torch.float64).tolist()
        hf = host[8 * ng:].view(torch.int32).tolist()
        if ng == 1:
            out, total = hf, float(hv[0])
        else:
            out = [0] * n
            total = 0.0
            o = 0
            for gi, (dt, idx) in enumerate(groups):
                total += float(hv[gi])
                for j, i in enumerate(idx):
                    out[i] = hf[o + j]
                o += len(idx)
        done.append((out, total))
        return done[0]
    return resolve


def grad_norm(grads, norm_kind, p=2.0):
    """Return (value, flags): value = sum g^2 (kind 0), max|g| (1) or sum|g|^p (2)
    over finite entries, as a Python float; flags[i] bit 0 = tensor i non-finite."""
    n = len(grads)
    if n == 0:
        return 0.0, []
    for t in grads:
        _dev(t, "grad")
    dev = grads[0].device
    ensure_device(dev.index)
    lib = load()
    groups = list(_group_by_dtype(grads).items())
    # one buffer for every group's result (fp64 value, 8 bytes) and flags (4 bytes each):
    # a single device-to-host copy
    buf = _scratch("norm", 8 * len(groups) + 4 * n, dev)[: 8 * len(groups) + 4 * n]
    vals = buf[: 8 * len(groups)].view(torch.float64)
    fls = buf[8 * len(groups):].view(torch.int32)
    off = 0
    for gi, (dt, idx) in enumerate(groups):
        sub = [grads[i] for i in idx]
        numel = _numel_array(sub)
        nb = lib.tg_grad_norm_workspace(len(sub), numel)
        ws = _scratch(("normws", gi), nb, dev)
        _check("tg_grad_norm", lib.tg_grad_norm(
            len(sub), dtype_code(sub[0]), _ptr_array(sub), numel, int(norm_kind), float(p),
            ptr(vals[gi:gi + 1]), ptr(fls[off: off + len(sub)]), ptr(ws), ws.numel(),
            stream_handle()))
        off += len(sub)
    host = buf.cpu()
    hv = host[: 8 * len(groups)].view(torch.float64).tolist()
    hf = host[8 * len(groups):].view(torch.int32).tolist()
    total = 0.0
    flags_out = [0] * n
    off = 0
    for gi, (dt, idx) in enumerate(groups):
        v = float(hv[gi])
        total = max(total, v) if norm_kind == 1 else total + v
        for j, i in enumerate(idx):
            flags_out[i] = hf[off + j]
        off += len(idx)
    return total, flags_out


def zero_nonfinite(grads):
    if not grads:
        return
    lib = load()
    ensure_device(grads[0].device.index)
    for dt, idx in _group_by_dtype(grads).items():
        sub = [grads[i] for i in idx]
        _check("tg_zero_nonfinite", lib.tg_zero_nonfinite(
            len(sub), dtype_code(sub[0]), _ptr_array(sub), _numel_array(sub), stream_handle()))


def scale_(grads, mul):
    """g *= mul for every tensor (no checks needed by the caller, no read-back)."""
    if grads:
        unscale_check(grads, mul, write=True, readback=False)


# ---------------------------------------------------------------- GEMM
def gemm(a, b, c, trans_a=False, trans_b=False, alpha=1.0, beta=0.0, M=None, N=None, K=None,
         lda=None, ldb=None, ldc=None, stride_a=0, stride_b=0, stride_c=0, batch=1):
    """Row-major batched GEMM on raw contiguous buffers; see include/tgbwd.h."""
    lib = load()
    ensure_device(c.device.index)
    if a.dtype != b.dtype:
        raise TypeError(f"gemm: A and B dtypes differ ({a.dtype} vs {b.dtype})")
    if c.dtype not in (torch.float32, a.dtype):
        raise TypeError(f"gemm: C must be float32 or {a.dtype}, got {c.dtype}")
    _check("tg_gemm", lib.tg_gemm(
        dtype_code(a), dtype_code(c), int(bool(trans_a)), int(bool(trans_b)), M, N, K,
        float(alpha), ptr(a), lda, stride_a, ptr(b), ldb, stride_b, float(beta), ptr(c), ldc,
        stride_c, batch, stream_handle()))
    return c


def gemm_bias(a, b, bias, out, trans_b=False):
    """out = a @ op(b) + bias (a [M, K], b [K, N] or, transposed, [N, K]; bias fp32 [N])."""
    for n, t in (("a", a), ("b", b), ("bias", bias), ("out", out)):
        _dev(t, n)
    M, K = a.shape
    N = b.shape[0] if trans_b else b.shape[1]
    if (b.shape[1] if trans_b else b.shape[0]) != K:
        raise ValueError(f"gemm_bias: inner dims differ ({tuple(a.shape)} @ {tuple(b.shape)})")
    if bias.dtype != torch.float32 or bias.numel() != N or tuple(out.shape) != (M, N):
        raise ValueError("gemm_bias: bias must be fp32 [N] and out [M, N]")
    if a.dtype != b.dtype or out.dtype not in (torch.float32, a.dtype):
        raise TypeError(f"gemm_bias: dtypes a={a.dtype} b={b.dtype} out={out.dtype}")
    ensure_device(out.device.index)
    return _gemm_bias_launch(a, b, bias, out, trans_b)


def _gemm_bias_launch(a, b, bias, out, trans_b):
    """gemm_bias without the argument checks, for callers that built the operands
    themselves (contiguous a [M, K], b [K, N] or [N, K], fp32 bias [N], out [M, N] on
    an initialised device)."""
    M, K = a.shape
    N = out.shape[1]
    _check("tg_gemm_bias", (_lib or load()).tg_gemm_bias(
        _TORCH_TO_CODE[a.dtype], _TORCH_TO_CODE[out.dtype], 0, 1 if trans_b else 0, M, N, K,
        1.0, a.data_ptr(), K, b.data_ptr(), b.shape[1], bias.data_ptr(), out.data_ptr(), N,
        stream_handle()))
    return out


def wgrad(x, g, dw, acc_w, db=None, acc_b=False):
    """dw (+)= x^T @ g and db (+)= g.sum(0) for x [K, M], g [K, N] contiguous (the weight
    and bias gradients of a Linear layer over K tokens); one GEMM pass over g for both
    with 16-bit operands."""
    for n, t in (("x", x), ("g", g), ("dw", dw)):
        _dev(t, n)
    if db is not None:
        _dev(db, "db")
    if x.dim() != 2 or g.dim() != 2 or x.shape[0] != g.shape[0]:
        raise ValueError(f"wgrad: x {tuple(x.shape)} and g {tuple(g.shape)} must be [K, M], [K, N]")
    if x.dtype != g.dtype:
        raise TypeError(f"wgrad: x and g dtypes differ ({x.dtype} vs {g.dtype})")
    K, M = x.shape
    N = g.shape[1]
    if not (x.is_contiguous() and g.is_contiguous()):
        raise ValueError("wgrad: x and g must be contiguous")
    if tuple(dw.shape) != (M, N) or not dw.is_contiguous():
        raise ValueError(f"wgrad: dw must be a contiguous [{M}, {N}] buffer")
    if db is not None and (db.numel() != N or not db.is_contiguous()):
        raise ValueError(f"wgrad: db must be a contiguous buffer of {N} elements")
    lib = load()
    ensure_device(dw.device.index)
    ws = workspace(lib.tg_gemm_wgrad_workspace(dtype_code(x), M, N, K, int(db is not None)),
                   dw.device)
    _check("tg_gemm_wgrad", lib.tg_gemm_wgrad(
        dtype_code(x), M, N, K, ptr(x), M, ptr(g), N, dtype_code(dw), ptr(dw), N,
        int(bool(acc_w)), dtype_code(db) if db is not None else 0,
        ptr(db) if db is not None else None, int(bool(acc_b)), ptr(ws), ws.numel(),
        stream_handle()))
    return dw



def _wgrad_launch(x, g, dw, acc_w, db, acc_b):
    """wgrad without the argument checks, for callers that built the operands
    themselves (contiguous x [K, M] and g [K, N], dw [M, N] and db [N] contiguous, one
    device); the workspace is this stream's reusable scratch (calls on one stream run in
    order, and the workspace is consumed within the call)."""
    K, M = x.shape
    N = g.shape[1]
    lib = _lib or load()
    code = _TORCH_TO_CODE[x.dtype]
    has_b = db is not None
    ws = _scratch("wgrad", lib.tg_gemm_wgrad_workspace(code, M, N, K, 1 if has_b else 0),
                  x.device)
    _check("tg_gemm_wgrad", lib.tg_gemm_wgrad(
        code, M, N, K, x.data_ptr(), M, g.data_ptr(), N, _TORCH_TO_CODE[dw.dtype],
        dw.data_ptr(), N, 1 if acc_w else 0, _TORCH_TO_CODE[db.dtype] if has_b else 0,
        db.data_ptr() if has_b else None, 1 if acc_b else 0, ws.data_ptr(), ws.numel(),
        stream_handle()))
    return dw


def wgrad_group(xs, gs, dws, acc_ws, dbs=None, acc_bs=None):
    """wgrad for n members at once: dws[i] (+)= xs[i]^T @ gs[i] and dbs[i] (+)=
    gs[i].sum(0) (dbs None, or an entry None: no bias).  The members share xs' shape
    [K, M]; each gs[i] is [K, N_i] with its own N_i.  16-bit members whose tiles together
    fill the CUs run as one launch; the gradient buffers must be distinct."""
    n = len(xs)
    if not (len(gs) == len(dws) == len(acc_ws) == n):
        raise ValueError("wgrad_group: xs, gs, dws and acc_ws differ in length")
    if n == 0:
        return
    dbs = list(dbs) if dbs is not None else [None] * n
    acc_bs = list(acc_bs) if acc_bs is not None else [False] * n
    if len(dbs) != n or len(acc_bs) != n:
        raise ValueError("wgrad_group: dbs and acc_bs must have one entry per member")
    x0, g0 = xs[0], gs[0]
    if x0.dim() != 2 or g0.dim() != 2 or x0.shape[0] != g0.shape[0]:
        raise ValueError(f"wgrad_group: x {tuple(x0.shape)} and g {tuple(g0.shape)} must be "
                         "[K, M], [K, N]")
    K, M = x0.shape
    dbt = next((d.dtype for d in dbs if d is not None), None)
    seen = set()
    Ns = []
    for x, g, dw, db in zip(xs, gs, dws, dbs):
        for nm, t in (("x", x), ("g", g), ("dw", dw)):
            _dev(t, nm)
        if tuple(x.shape) != (K, M) or g.dim() != 2 or g.shape[0] != K:
            raise ValueError("wgrad_group: members differ in K or M")
        N = g.shape[1]
        Ns.append(N)
        if x.dtype != x0.dtype or g.dtype != x0.dtype or dw.dtype != dws[0].dtype:
            raise TypeError("wgrad_group: members differ in dtype")
        if not (x.is_contiguous() and g.is_contiguous()):
            raise ValueError("wgrad_group: x and g must be contiguous")
        if tuple(dw.shape) != (M, N) or not dw.is_contiguous():
            raise ValueError(f"wgrad_group: dw must be a contiguous [{M}, {N}] buffer")
        targets = [dw]
        if db is not None:
            _dev(db, "db")
            if db.numel() != N or not db.is_contiguous() or db.dtype != dbt:
                raise ValueError(f"wgrad_group: db must be a contiguous {dbt} buffer of {N} "
                                 "elements")
            targets.append(db)
        for t in targets:
            if t.data_ptr() in seen:
                raise ValueError("wgrad_group: two members write one gradient buffer")
            seen.add(t.data_ptr())
    lib = load()
    dev = dws[0].device
    ensure_device(dev.index)
    with_b = dbt is not None
    accw = (ctypes.c_int * n)(*[int(bool(a)) for a in acc_ws])
    accb = (ctypes.c_int * n)(*[int(bool(a)) for a in acc_bs])
    if len(set(Ns)) == 1:
        N = Ns[0]
        ws = workspace(lib.tg_gemm_wgrad_group_workspace(dtype_code(x0), n, M, N, K,
                                                         int(with_b)), dev)
        _check("tg_gemm_wgrad_group", lib.tg_gemm_wgrad_group(
            dtype_code(x0), n, M, N, K, _ptr_array(xs), M, _ptr_array(gs), N,
            dtype_code(dws[0]), _ptr_array(dws), N, accw, _TORCH_TO_CODE[dbt] if with_b else 0,
            _ptr_array(dbs) if with_b else None, accb, ptr(ws), ws.numel(), stream_handle()))
        return
    na = (ctypes.c_int64 * n)(*Ns)
    ws = workspace(lib.tg_gemm_wgrad_group_n_workspace(dtype_code(x0), n, M, na, K,
                                                       int(with_b)), dev)
    _check("tg_gemm_wgrad_group_n", lib.tg_gemm_wgrad_group_n(
        dtype_code(x0), n, M, na, K, _ptr_array(xs), M, _ptr_array(gs), na, dtype_code(dws[0]),
        _ptr_array(dws), na, accw, _TORCH_TO_CODE[dbt] if with_b else 0,
        _ptr_array(dbs) if with_b else None, accb, ptr(ws), ws.numel(), stream_handle()))

_CUS = {}


def _num_cus(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CUS[idx]


def _split_k(M, N, K, device):
    """K-split factor for GEMMs whose output has too few 128x128 tiles for two per CU
    (e.g. weight gradients [1024, 1024] or [1024, 4096] over 8192 tokens; measured on
    the MI355X: [1024, 4096] 102 -> 86 us with two K halves).  Returns 1 or s with
    K % s == 0 and (K/s) % 64 == 0."""
    tiles = ((M + 127) // 128) * ((N + 127) // 128)
    cus = _num_cus(device)
    if K >= 16384 and tiles < 4 * cus:
        # very long K (the tied head's input gradient over a 32000-word vocabulary:
        # 676 -> 563 us in two halves)
        want = 2
    elif tiles >= 2 * cus or K < 2048:
        return 1
    else:
        want = min(-(-2 * cus // tiles), K // 1024)
    for s_ in range(want, 1, -1):
        if K % s_ == 0 and (K // s_) % 64 == 0:
            return s_
    return 1


def matmul2d(a, b, out=None, trans_a=False, trans_b=False, alpha=1.0, beta=0.0, out_dtype=None):
    """out (= or +=) op(a) @ op(b) for 2-D contiguous a, b.

    Output shapes with few tiles and a long K run as a K-split batched GEMM into
    fp32 partials followed by the deterministic column-sum kernel."""
    _dev(a, "a")
    _dev(b, "b")
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    Kb = b.shape[1] if trans_b else b.shape[0]
    N = b.shape[0] if trans_b else b.shape[1]
    if K != Kb:
        raise ValueError(f"matmul2d: inner dims differ ({K} vs {Kb})")
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype or a.dtype, device=a.device)
        beta = 0.0
    _dev(out, "out")
    if tuple(out.shape) != (M, N):
        raise ValueError(f"matmul2d: out shape {tuple(out.shape)} != {(M, N)}")
    lda, ldb = a.shape[1], b.shape[1]
    s_ = (_split_k(M, N, K, a.device)
          if (alpha == 1.0 and beta in (0.0, 1.0) and a.dtype != torch.float64) else 1)
    if s_ > 1:
        kc = K // s_
        parts = torch.empty(s_, M, N, dtype=torch.float32, device=a.device)
        sa = kc * M if trans_a else kc
        sb = kc if trans_b else kc * N
        gemm(a, b, parts, trans_a, trans_b, 1.0, 0.0, M, N, kc, lda, ldb, N, sa, sb, M * N, s_)
        reduce_rows(parts.view(s_, M * N), out.view(M * N), beta == 1.0)
        return out
    return gemm(a, b, out, trans_a, trans_b, alpha, beta, M, N, K, lda, ldb, N)


# ---------------------------------------------------------------- attention
def _fa_in(t, layout):
    """True if t (B, H, S, D) has the strides of `layout` on every dimension longer
    than 1 (0: contiguous (B, H, S, D); 1: contiguous (B, S, H, D) memory)."""
    if t.dim() != 4:
        return False
    B, H, S, D = t.shape
    want = (H * S * D, S * D, D, 1) if layout == 0 else (S * H * D, D, H * D, 1)
    return all(n == 1 or st == w for n, st, w in zip(t.shape, t.stride(), want))


def fa_layout(t):
    """0 if t (B, H, S, D) is contiguous, 1 if it is the (0, 2, 1, 3) view of a contiguous
    (B, S, H, D) tensor, else None."""
    if _fa_in(t, 0):
        return 0
    if _fa_in(t, 1):
        return 1
    return None


def fa_empty(B, H, S, D, dtype, device, layout):
    """Uninitialised (B, H, S, D) tensor in the given memory layout."""
    if layout == 1:
        return torch.empty(B, S, H, D, dtype=dtype, device=device).permute(0, 2, 1, 3)
    return torch.empty(B, H, S, D, dtype=dtype, device=device)


def _fa_dev(t, name, layout):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a torch device tensor")
    if not _fa_in(t, layout):
        raise ValueError(f"{name} must be in layout {layout} "
                         "(0: contiguous (B,H,S,D); 1: (B,S,H,D) memory)")


def flash_attn_fwd(q, k, v, scale, causal, layout=0):
    """o, lse = FlashAttention forward of (B, H, S, D) q/k/v in `layout`; o is returned in
    the same layout, lse as (B, H, Sq) fp32."""
    for n, t in (("q", q), ("k", k), ("v", v)):
        _fa_dev(t, n, layout)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    if k.shape != (B, H, Sk, D) or v.shape != (B, H, Sk, D):
        raise ValueError(f"flash_attn: k/v shape mismatch {tuple(k.shape)} {tuple(v.shape)}")
    o = fa_empty(B, H, Sq, D, q.dtype, q.device, layout)
    ensure_device(q.device.index)
    if q.dtype == torch.float64:
        # fp64: scores of a chunk of heads materialised in a workspace, fp64 GEMMs, lse in
        # double
        lse = torch.empty(B, H, Sq, dtype=torch.float64, device=q.device)
        lib = load()
        ws = workspace(lib.tg_flash_attn_f64_workspace(B, H, Sq, Sk), q.device)
        _check("tg_flash_attn_fwd_f64", lib.tg_flash_attn_fwd_f64(
            ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, H, Sq, Sk, D, float(scale),
            int(bool(causal)), int(layout), ptr(ws), ws.numel(), stream_handle()))
        return o, lse
    lse = torch.empty(B, H, Sq, dtype=torch.float32, device=q.device)
    _check("tg_flash_attn_fwd", load().tg_flash_attn_fwd_layout(
        dtype_code(q), ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, H, Sq, Sk, D, float(scale),
        int(bool(causal)), int(layout), stream_handle()))
    return o, lse


def flash_attn_bwd(q, k, v, o, do, lse, dq, dk, dv, scale, causal, accumulate, layout=0):
    for n, t in (("q", q), ("k", k), ("v", v), ("o", o), ("do", do), ("dq", dq), ("dk", dk),
                 ("dv", dv)):
        _fa_dev(t, n, layout)
    _dev(lse, "lse")
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    lib = load()
    ensure_device(q.device.index)
    if q.dtype == torch.float64:
        if lse.dtype != torch.float64:
            raise TypeError("flash_attn_bwd: fp64 inputs need the fp64 lse of the forward")
        ws = workspace(lib.tg_flash_attn_f64_workspace(B, H, Sq, Sk), q.device)
        _check("tg_flash_attn_bwd_f64", lib.tg_flash_attn_bwd_f64(
            ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse), ptr(dq), ptr(dk), ptr(dv), B, H,
            Sq, Sk, D, float(scale), int(bool(causal)), int(layout), int(bool(accumulate)),
            ptr(ws), ws.numel(), stream_handle()))
        return
    ws = workspace(lib.tg_flash_attn_bwd_workspace(B, H, Sq, Sk, D), q.device)
    _check("tg_flash_attn_bwd", lib.tg_flash_attn_bwd_layout(
        dtype_code(q), ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse), ptr(dq), ptr(dk),
        ptr(dv), B, H, Sq, Sk, D, float(scale), int(bool(causal)), int(bool(accumulate)),
        int(layout), ptr(ws), ws.numel(), stream_handle()))


def _qkv_dev(qkv, heads):
    if not isinstance(qkv, torch.Tensor) or not qkv.is_cuda:
        raise TypeError("qkv must be a torch device tensor")
    if qkv.dim() != 3 or qkv.shape[2] % (3 * heads) or not qkv.is_contiguous():
        raise ValueError(f"qkv must be a contiguous (B, S, 3*H*D) tensor with H = {heads}, "
                         f"got {tuple(qkv.shape)}")
    B, S, C3 = qkv.shape
    return B, S, C3 // (3 * heads)


def flash_attn_fwd_qkv(qkv, heads, scale, causal):
    """o, lse = self-attention of the packed projection qkv (B, S, 3*H*D): columns
    [0, HD) hold the query heads, [HD, 2HD) the keys, [2HD, 3HD) the values, head h at
    h*D within each.  o is (B, S, H*D) (heads merged), lse (B, H, S) fp32."""
    B, S, D = _qkv_dev(qkv, heads)
    if qkv.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"flash_attn_fwd_qkv: unsupported dtype {qkv.dtype}")
    o = torch.empty(B, S, heads * D, dtype=qkv.dtype, device=qkv.device)
    lse = torch.empty(B, heads, S, dtype=torch.float32, device=qkv.device)
    ensure_device(qkv.device.index)
    _check("tg_flash_attn_fwd_qkv", load().tg_flash_attn_fwd_qkv(
        dtype_code(qkv), ptr(qkv), ptr(o), ptr(lse), B, heads, S, D, float(scale),
        int(bool(causal)), stream_handle()))
    return o, lse


def flash_attn_bwd_qkv(qkv, o, do, lse, dqkv, heads, scale, causal, accumulate):
    """dqkv (+)= the gradient of flash_attn_fwd_qkv: dq, dk, dv in qkv's column order."""
    B, S, D = _qkv_dev(qkv, heads)
    _qkv_dev(dqkv, heads)
    for n, t in (("o", o), ("do", do)):
        if not t.is_cuda or tuple(t.shape) != (B, S, heads * D) or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous ({B}, {S}, {heads * D}) device tensor")
    for n, t in (("o", o), ("do", do), ("dqkv", dqkv)):
        if t.dtype != qkv.dtype:
            raise TypeError(f"flash_attn_bwd_qkv: {n} dtype {t.dtype} != {qkv.dtype}")
    if tuple(dqkv.shape) != tuple(qkv.shape):
        raise ValueError("flash_attn_bwd_qkv: dqkv shape differs from qkv")
    _dev(lse, "lse")
    lib = load()
    ensure_device(qkv.device.index)
    ws = workspace(lib.tg_flash_attn_bwd_workspace(B, heads, S, S, D), qkv.device)
    _check("tg_flash_attn_bwd_qkv", lib.tg_flash_attn_bwd_qkv(
        dtype_code(qkv), ptr(qkv), ptr(o), ptr(do), ptr(lse), ptr(dqkv), B, heads, S, D,
        float(scale), int(bool(causal)), int(bool(accumulate)), ptr(ws), ws.numel(),
        stream_handle()))


def cross_entropy_fwd(logits, targets, label_smoothing=0.0):
    """Per-row log-sum-exp and loss of logits [N, C] against int64 targets [N]:
    returns (lse, loss), both fp32 [N] (fp64 for fp64 logits)."""
    _dev(logits, "logits")
    _dev(targets, "targets")
    if logits.dim() != 2 or not logits.is_contiguous():
        raise ValueError("cross_entropy: logits must be a contiguous [N, C] tensor")
    if targets.dtype != torch.int64 or targets.numel() != logits.shape[0]:
        raise ValueError("cross_entropy: targets must be int64 [N]")
    N, C = logits.shape
    sdt = torch.float64 if logits.dtype == torch.float64 else torch.float32
    lse = torch.empty(N, dtype=sdt, device=logits.device)
    loss = torch.empty(N, dtype=sdt, device=logits.device)
    ensure_device(logits.device.index)
    if logits.dtype == torch.float64:
        _check("tg_cross_entropy_fwd_f64", load().tg_cross_entropy_fwd_f64(
            ptr(logits), ptr(targets), N, C, float(label_smoothing), ptr(lse), ptr(loss),
            stream_handle()))
        return lse, loss
    _check("tg_cross_entropy_fwd", load().tg_cross_entropy_fwd(
        dtype_code(logits), ptr(logits), ptr(targets), N, C, float(label_smoothing), ptr(lse),
        ptr(loss), stream_handle()))
    return lse, loss


def cross_entropy_fwd_grad_ok(logits):
    """Whether cross_entropy_fwd_grad takes these logits (fp32/fp16/bf16, 16-byte
    aligned rows of at most the kernel's register-resident width)."""
    if logits.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return False
    if logits.dim() != 2 or not logits.is_contiguous() or logits.data_ptr() % 16:
        return False
    C = logits.shape[1]
    v = 16 // logits.element_size()
    return C % v == 0 and C <= load().tg_cross_entropy_fwd_grad_max_classes(dtype_code(logits))


def cross_entropy_fwd_grad(logits, targets, scale):
    """cross_entropy_fwd (no label smoothing) and the gradient (softmax - onehot) * scale
    in the logits' dtype, from one read of the logits: returns (lse, loss, grad), bit for
    bit cross_entropy_fwd's results and what cross_entropy_bwd would write."""
    _dev(logits, "logits")
    _dev(targets, "targets")
    if not cross_entropy_fwd_grad_ok(logits):
        raise ValueError("cross_entropy_fwd_grad: logits not supported (see "
                         "cross_entropy_fwd_grad_ok)")
    if targets.dtype != torch.int64 or targets.numel() != logits.shape[0]:
        raise ValueError("cross_entropy: targets must be int64 [N]")
    N, C = logits.shape
    lse = torch.empty(N, dtype=torch.float32, device=logits.device)
    loss = torch.empty(N, dtype=torch.float32, device=logits.device)
    grad = torch.empty_like(logits)
    ensure_device(logits.device.index)
    _check("tg_cross_entropy_fwd_grad", load().tg_cross_entropy_fwd_grad(
        dtype_code(logits), ptr(logits), ptr(targets), N, C, ptr(lse), ptr(loss), float(scale),
        ptr(grad), stream_handle()))
    return lse, loss, grad


def cross_entropy_bwd(logits, targets, lse, grad, scale, accumulate, label_smoothing=0.0):
    """grad (+)= (softmax(logits) - target distribution) * scale."""
    for n, t in (("logits", logits), ("targets", targets), ("lse", lse), ("grad", grad)):
        _dev(t, n)
    if grad.shape != logits.shape or not grad.is_contiguous():
        raise ValueError("cross_entropy: grad must be contiguous with the logits' shape")
    N, C = logits.shape
    if logits.dtype == torch.float64:
        if grad.dtype != torch.float64 or lse.dtype != torch.float64:
            raise TypeError("cross_entropy: fp64 logits need an fp64 gradient and lse")
        _check("tg_cross_entropy_bwd_f64", load().tg_cross_entropy_bwd_f64(
            ptr(logits), ptr(targets), ptr(lse), N, C, float(label_smoothing), float(scale),
            ptr(grad), int(bool(accumulate)), stream_handle()))
        return
    _check("tg_cross_entropy_bwd", load().tg_cross_entropy_bwd(
        dtype_code(logits), ptr(logits), ptr(targets), ptr(lse), N, C, float(label_smoothing),
        float(scale), dtype_code(grad), ptr(grad), int(bool(accumulate)), stream_handle()))


def embedding_fwd(weight, indices, out_dtype=None):
    """weight[indices] (indices int64 of any shape) as a new [..., dim] tensor of
    out_dtype (default: weight's)."""
    _dev(weight, "weight")
    _dev(indices, "indices")
    if weight.dim() != 2 or indices.dtype != torch.int64:
        raise ValueError("embedding_fwd: weight must be [V, dim] and indices int64")
    V, dim = weight.shape
    out = torch.empty(*indices.shape, dim, dtype=out_dtype or weight.dtype, device=weight.device)
    ensure_device(weight.device.index)
    _check("tg_embedding_fwd", load().tg_embedding_fwd(
        dtype_code(weight), ptr(weight), ptr(indices), indices.numel(), dim, V, dtype_code(out),
        ptr(out), stream_handle()))
    return out


def embedding_bwd(dout, indices, grad, accumulate):
    """grad[indices[i]] (+)= dout[i]: dout [..., dim] with indices [...] (int64),
    grad [num_embeddings, dim]."""
    for n, t in (("dout", dout), ("indices", indices), ("grad", grad)):
        _dev(t, n)
    if indices.dtype != torch.int64:
        raise TypeError("embedding_bwd: indices must be int64")
    V, dim = grad.shape
    n = indices.numel()
    if dout.numel() != n * dim:
        raise ValueError(f"embedding_bwd: dout has {dout.numel()} elements for {n} x {dim}")
    lib = load()
    ensure_device(grad.device.index)
    ws = workspace(lib.tg_embedding_bwd_workspace(n, V), grad.device)
    _check("tg_embedding_bwd", lib.tg_embedding_bwd(
        dtype_code(dout), ptr(dout), ptr(indices), n, dim, dtype_code(grad), ptr(grad), V,
        int(bool(accumulate)), ptr(ws), ws.numel(), stream_handle()))


def transpose_add(src, dst, alpha=1.0):
    """dst += alpha * src.T for a contiguous 2-D src [R, C] and dst [C, R]."""
    _dev(src, "src")
    _dev(dst, "dst")
    R, C = src.shape
    if tuple(dst.shape) != (C, R):
        raise ValueError(f"transpose_add: dst {tuple(dst.shape)} is not {(C, R)}")
    ensure_device(dst.device.index)
    _check("tg_transpose_add", load().tg_transpose_add(
        dtype_code(src), ptr(src), R, C, dtype_code(dst), ptr(dst), float(alpha),
        stream_handle()))
