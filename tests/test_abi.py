"""The C-ABI library builds for gfx950, loads without a GPU and exports every
function include/tgbwd.h declares, with ctypes signatures for each.  CPU only."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "tgbwd.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_hot_path():
    names = declared()
    for must in ("tg_gelu_bwd", "tg_silu_bwd", "tg_softmax_bwd", "tg_layernorm_bwd",
                 "tg_batchnorm_bwd", "tg_flash_attn_bwd", "tg_gemm", "tg_adam_step",
                 "tg_unscale_check", "tg_grad_norm", "tg_reduce_rows"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from tensor_gpu_v2 import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"libtgbwd.so lacks {missing}"


def test_ctypes_signatures_cover_header():
    from tensor_gpu_v2 import _lib
    assert set(declared()) == set(_lib.SIGNATURES), (
        set(declared()) ^ set(_lib.SIGNATURES))
    _lib.load()  # binds every symbol; raises if one is missing


def test_library_is_built_for_gfx950():
    from tensor_gpu_v2 import _lib
    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_error_path_without_gpu_work():
    # argument validation happens before any device call
    from tensor_gpu_v2 import _lib
    lib = _lib.load()
    st = lib.tg_softmax_bwd(0, None, None, None, -1, 4, 0, None)
    assert st == -1 and b"negative" in lib.tg_last_error()
    assert lib.tg_gemm(0, 0, 0, 0, -1, 1, 1, 1.0, None, 1, 0, None, 1, 0, 0.0, None, 1, 0, 1,
                       None) == -1
    assert lib.tg_version() >= 10000


def test_every_entry_point_rejects_invalid_arguments():
    """Every status-returning entry point refuses NULL pointers (sizes 1) and negative
    sizes (pointers NULL) with a nonzero status and a message, before any device work
    (so this runs without a GPU).  Capability queries (int results that are counts) are
    not status functions and are left out."""
    import ctypes
    from tensor_gpu_v2 import _lib
    lib = _lib.load()
    skip = {"tg_init", "tg_stream_sync", "tg_cross_entropy_fwd_grad_max_classes"}
    ints = (ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int32)
    checked = 0
    for name, (res, args) in sorted(_lib.SIGNATURES.items()):
        if res is not ctypes.c_int or name in skip:
            continue
        for size in (-1, 1):
            vals = [size if a in ints else 1.0 if a in (ctypes.c_float, ctypes.c_double)
                    else None for a in args]
            st = getattr(lib, name)(*vals)
            assert st != 0, f"{name} accepted {'negative sizes' if size < 0 else 'NULL pointers'}"
            assert lib.tg_last_error(), name
            checked += 1
    assert checked >= 100
