"""libtgbwd's GEMM (tg_gemm through _lib.matmul2d) against torch.matmul (hipBLASLt on
ROCm) on the C5 GPT shapes and 8192^3, fp16 in / fp32 accumulate.

    python3 project-tensor_amd/gemm_compare.py [--reps N] [--rounds R]

Each shape is timed with HIP events over N back-to-back calls, alternating the two
libraries for R rounds (clocks and power drift between back-to-back runs, so the
median of the rounds is reported).  Layouts as the step uses them: forward x @ W
(NN), input gradient dC @ W^T (NT), weight gradient x^T @ dC (TN, fp32 output; hipBLASLt writes fp16 there, as
torch has no fp16 x fp16 -> fp32 matmul).
"""
import argparse
import os
import statistics
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from tensor_gpu_v2 import _lib as L  # noqa: E402

# (name, M, N, K, trans_a, trans_b, out dtype)
SHAPES = [
    ("o fwd 8192x1024x1024", 8192, 1024, 1024, False, False, torch.float16),
    ("qkv fwd 8192x3072x1024", 8192, 3072, 1024, False, False, torch.float16),
    ("qkv dA 8192x1024x3072 (NT)", 8192, 1024, 3072, False, True, torch.float16),
    ("fc1 fwd 8192x4096x1024", 8192, 4096, 1024, False, False, torch.float16),
    ("fc2 fwd 8192x1024x4096", 8192, 1024, 4096, False, False, torch.float16),
    ("head fwd 8192x32000x1024", 8192, 32000, 1024, False, True, torch.float16),
    ("fc1 dA 8192x1024x4096 (NT)", 8192, 1024, 4096, False, True, torch.float16),
    ("o dW 1024x1024x8192 (TN)", 1024, 1024, 8192, True, False, torch.float32),
    ("qkv dW 1024x3072x8192 (TN)", 1024, 3072, 8192, True, False, torch.float32),
    ("fc1 dW 1024x4096x8192 (TN)", 1024, 4096, 8192, True, False, torch.float32),
    ("head dA 8192x1024x32000", 8192, 1024, 32000, False, False, torch.float16),
    ("square 8192x8192x8192", 8192, 8192, 8192, False, False, torch.float16),
]


def _time(fn, reps):
    for _ in range(2):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3  # us


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--only", default="", help="run the shapes whose name contains this")
    ap.add_argument("--ours-only", action="store_true", help="skip the hipBLASLt runs")
    a = ap.parse_args()
    L.ensure_device(0)
    g = torch.Generator(device="cuda").manual_seed(0)
    print(f"{'shape':32s} {'libtgbwd us':>11s} {'TFLOP/s':>8s} {'hipBLASLt us':>12s} "
          f"{'TFLOP/s':>8s} {'ratio':>6s}")
    for name, M, N, K, ta, tb, odt in SHAPES:
        if a.only and a.only not in name:
            continue
        A = torch.randn((K, M) if ta else (M, K), device="cuda", generator=g).half()
        B = torch.randn((N, K) if tb else (K, N), device="cuda", generator=g).half()
        C = torch.empty(M, N, device="cuda", dtype=odt)
        Aop, Bop = (A.t() if ta else A), (B.t() if tb else B)
        ours, ref = [], []
        for _ in range(a.rounds):
            ours.append(_time(lambda: L.matmul2d(A, B, out=C, trans_a=ta, trans_b=tb), a.reps))
            # torch has no fp16 x fp16 -> fp32 matmul: the weight-gradient shapes run
            # hipBLASLt with an fp16 output (half the output bytes libtgbwd writes)
            Ch = C if odt == torch.float16 else torch.empty(M, N, device="cuda",
                                                             dtype=torch.float16)
            if not a.ours_only:
                ref.append(_time(lambda: torch.matmul(Aop, Bop, out=Ch), a.reps))
        o, r = statistics.median(ours), (statistics.median(ref) if ref else float("nan"))
        fl = 2 * M * N * K
        print(f"{name:32s} {o:11.1f} {fl / o / 1e6:8.0f} {r:12.1f} {fl / r / 1e6:8.0f} "
              f"{r / o:6.2f}", flush=True)


if __name__ == "__main__":
    main()
