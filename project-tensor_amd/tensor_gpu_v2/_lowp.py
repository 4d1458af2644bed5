"""Low-precision copies of parameters for autocast, kept between forwards.

Under autocast the reference casts every fp32 weight a forward reads to fp16
(_core.py:185-191), so each step pays one cast pass per weight.  Here the cast of a
leaf parameter is kept and reused until the parameter changes:

* in-place torch operations on the parameter (or any view of it) advance torch's
  version counter, which the entry records; a changed counter means a fresh cast;
* the Adam/AdamW update (the one engine path that writes parameters with a kernel,
  which torch's counter does not see) rewrites the copy in the same pass
  (tg_adam_step_lowp) and drops every other cached view of the same storage.

Entries are grouped by storage so the optimizer finds them without a scan.  An entry
holds a weak reference to its source tensor: a freed parameter never validates one.
"""
import weakref

import torch

# storage address -> {(offset, shape, stride, dtype): (weakref(source), version, copy)}
_CACHE = {}
_MAX_STORAGES = 4096
# Bumped on every change to the set of cached entries; refresh_targets reuses its last
# answer for the same parameters while it is unchanged.
_GEN = [0]
_LAST = {}


def _storage_key(d):
    return d.untyped_storage().data_ptr()


def _view_key(d, dtype):
    return (d.storage_offset(), tuple(d.shape), tuple(d.stride()), dtype)


def _valid(entry):
    src = entry[0]()
    return src is not None and src._version == entry[1]


def cast(d, dtype):
    """`d` (a contiguous parameter tensor) as `dtype`, from the cache when current."""
    sk = _storage_key(d)
    views = _CACHE.get(sk)
    vk = _view_key(d, dtype)
    if views is not None:
        e = views.get(vk)
        if e is not None and _valid(e):
            return e[2]
    lp = d.to(dtype)
    _GEN[0] += 1
    if views is None:
        if len(_CACHE) >= _MAX_STORAGES:
            _purge()
        views = _CACHE.setdefault(sk, {})
    views[vk] = (weakref.ref(d), d._version, lp)
    return lp


def _purge():
    _GEN[0] += 1
    for sk in list(_CACHE):
        views = _CACHE[sk]
        for vk in [k for k, e in views.items() if e[0]() is None]:
            del views[vk]
        if not views:
            del _CACHE[sk]


def refresh_targets(params):
    """For an optimizer pass that rewrites `params` (contiguous fp32 tensors) with a
    kernel: returns a list parallel to `params` holding, for each, the cached copy the
    pass should rewrite (one low-precision dtype for the whole list) or None.  Every
    other cached view of those storages is dropped, since the pass changes the data
    under it without advancing torch's version counter."""
    out = [None] * len(params)
    if not _CACHE:
        return out
    key = tuple(p.data_ptr() for p in params)
    last = _LAST.get(key)
    if last is not None and last[0] == _GEN[0]:
        return list(last[1])
    dt = None
    for i, p in enumerate(params):
        views = _CACHE.get(_storage_key(p))
        if not views:
            continue
        keep = None
        for cand in (torch.float16, torch.bfloat16):
            vk = _view_key(p, cand)
            e = views.get(vk)
            if e is not None and _valid(e) and (dt is None or dt == cand):
                keep = (vk, e)
                dt = cand
                break
        views.clear()
        if keep is not None:
            views[keep[0]] = keep[1]
            out[i] = keep[1][2]
    _GEN[0] += 1
    _LAST.clear()
    _LAST[key] = (_GEN[0], out)
    return list(out)


def clear():
    """Drop every cached copy."""
    _CACHE.clear()
    _LAST.clear()
    _GEN[0] += 1
