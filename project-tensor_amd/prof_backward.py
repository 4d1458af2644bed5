"""Run the C1 (README MLP) and C5 (GPT) training steps with each phase in its own
roctx range, for a rocprofv3 kernel trace that shows which kernels each phase
launches:

    rocprofv3 --kernel-trace --marker-trace -f csv -d <dir> -o bwd -- \
        python3 project-tensor_amd/prof_backward.py
    python3 project-tensor_amd/prof_summary.py ranges <dir>

Arguments select the configurations (default C1 C5); "closures" runs one backward
per op of the pointwise / log_softmax / max / advanced-index closures.

Phases (range names): "<cfg>.forward", "<cfg>.backward" (seed through the last
gradient closure; for C5 also sync_tied_gradients), "<cfg>.optimizer" (unscale,
clip, optimizer step).  The device is synchronised at both ends of every range, so
the kernels a range launches also run inside it.  One warm-up step runs first
(outside any range) so one-time work (weight casts, code-object loading) is not
attributed to a phase.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import tensor_gpu_v2 as tg  # noqa: E402
from tensor_gpu_v2 import _lib  # noqa: E402


class _phase:
    def __init__(self, name):
        self.name = name

    def __enter__(self):
        torch.cuda.synchronize()
        torch.cuda.nvtx.range_push(self.name)

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        torch.cuda.nvtx.range_pop()


def c1(tag):
    np.random.seed(0)
    x = tg.Tensor(np.random.randn(32, 784).astype(np.float32), requires_grad=False)
    l1, l2 = tg.Linear(784, 256), tg.Linear(256, 10)
    params = [l1.w, l1.b, l2.w, l2.b]
    opt = tg.Adam(params, lr=1e-3)
    for ranged in (False, True):
        for p in params:
            p.zero_grad()
        with (_phase(f"{tag}.forward") if ranged else _null()):
            loss = l2(l1(x).gelu()).mean()
        with (_phase(f"{tag}.backward") if ranged else _null()):
            loss.backward()
        with (_phase(f"{tag}.optimizer") if ranged else _null()):
            opt.step()


def c5(tag):
    from gpt_harness import GPT, Trainer, synthetic_batch
    model = GPT()
    tr = Trainer(model)
    ids, targets = synthetic_batch()
    for ranged in (False, True):
        tr.opt.zero_grad()
        for p in model.parameters():
            p.zero_grad()
        with (_phase(f"{tag}.forward") if ranged else _null()):
            with tg.autocast():
                logits = model(ids)
                loss = tr.loss_fn(logits, targets)
            scaled = tr.scaler.scale(loss)
        with (_phase(f"{tag}.backward") if ranged else _null()):
            scaled.backward()
            tg.sync_tied_gradients(model)
        with (_phase(f"{tag}.optimizer") if ranged else _null()):
            tr.scaler.unscale_(tr.opt)
            tg.clip_grad_norm_(tr.params, tr.clip)
            tr.scaler.step(tr.opt)
            tr.scaler.update()


def closures(tag):
    """One backward phase per op whose closure runs on tg_unary_bwd,
    tg_log_softmax_bwd, tg_max_bwd or tg_index_add_sorted (fp32 [256, 1024] input;
    each loss is a .sum() so the seed and the sum's backward fill are the other
    kernels in the phase)."""
    rng = np.random.default_rng(0)
    xv = (np.abs(rng.standard_normal((256, 1024))) + 0.1).astype(np.float32)
    bv = (np.abs(rng.standard_normal((256, 1024))) + 0.5).astype(np.float32)
    idx = rng.integers(0, 256, 4096)
    ops = {
        "relu": lambda x, b: x.relu(), "leaky_relu": lambda x, b: x.leaky_relu(0.1),
        "swish": lambda x, b: x.swish(1.5), "sigmoid": lambda x, b: x.sigmoid(),
        "tanh": lambda x, b: x.tanh(), "exp": lambda x, b: x.exp(),
        "log": lambda x, b: x.log(), "pow": lambda x, b: x ** 3.0,
        "truediv": lambda x, b: x / b, "log_softmax": lambda x, b: x.log_softmax(-1),
        "max": lambda x, b: x.max(axis=1), "min": lambda x, b: x.min(axis=0),
        "getitem_array": lambda x, b: x[idx], "getitem_mask": lambda x, b: x[xv > 1.0],
    }
    for name, f in ops.items():
        for ranged in (False, True):
            x = tg.Tensor(xv)
            b = tg.Tensor(bv)
            loss = f(x, b).sum()
            with (_phase(f"{tag}.{name}.backward") if ranged else _null()):
                loss.backward()


class _null:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


def main():
    _lib.ensure_device(0)
    which = sys.argv[1:] or ["C1", "C5"]
    if "C1" in which:
        c1("C1")
    if "C5" in which:
        c5("C5")
    if "closures" in which:
        closures("closures")
    torch.cuda.synchronize()
    print("prof_backward: done", flush=True)


if __name__ == "__main__":
    main()
