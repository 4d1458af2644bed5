"""libtgbwd's FlashAttention (tg_flash_attn_fwd / tg_flash_attn_bwd through _lib) against
torch.nn.functional.scaled_dot_product_attention on the same GPU, fp16 (B, H, S, D)
contiguous inputs: the C4 shapes (B 8, H 16, S 2048, head dim 64 and 128, causal and
not) and the GPT step's attention (S 1024, head dim 64).

    python3 project-tensor_amd/flash_compare.py [--reps N] [--rounds R]

Each case is timed with HIP events over N back-to-back calls, alternating the two
implementations for R rounds (median reported).  torch's backward is timed as its
forward + backward through autograd minus its no-grad forward.  FLOP counts: forward
4·B·H·S²·D, backward 10·B·H·S²·D (the five GEMM-equivalents of the reference count),
halved for causal masking.
"""
import argparse
import os
import statistics
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from tensor_gpu_v2 import _lib as L  # noqa: E402

CASES = [(8, 16, 2048, 64), (8, 16, 2048, 128), (8, 16, 1024, 64)]


def _time(fn, reps):
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps * 1e3  # us


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--rounds", type=int, default=5)
    a = ap.parse_args()
    L.ensure_device(0)
    sdpa = torch.nn.functional.scaled_dot_product_attention
    print(f"{'case':34s} {'ours us':>9s} {'TF/s':>6s} {'torch us':>9s} {'TF/s':>6s} {'ratio':>6s}")
    for B, H, S, D in CASES:
        for causal in (False, True):
            g = torch.Generator(device="cuda").manual_seed(S + D)
            q, k, v, do = (torch.randn(B, H, S, D, device="cuda", generator=g).half()
                           for _ in range(4))
            sc = D ** -0.5
            o, lse = L.flash_attn_fwd(q, k, v, sc, causal)
            dq, dk, dv = (torch.empty_like(q) for _ in range(3))
            qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))

            def ours_f():
                L.flash_attn_fwd(q, k, v, sc, causal)

            def ours_b():
                L.flash_attn_bwd(q, k, v, o, do, lse, dq, dk, dv, sc, causal, False)

            def torch_f():
                with torch.no_grad():
                    sdpa(q, k, v, is_causal=causal)

            def torch_fb():
                sdpa(qq, kk, vv, is_causal=causal).backward(do)
            for fn in (ours_f, ours_b, torch_f, torch_fb):
                fn()
            torch.cuda.synchronize()
            t = {n: [] for n in ("of", "ob", "tf", "tfb")}
            for _ in range(a.rounds):
                t["of"].append(_time(ours_f, a.reps))
                t["tf"].append(_time(torch_f, a.reps))
                t["ob"].append(_time(ours_b, a.reps))
                t["tfb"].append(_time(torch_fb, a.reps))
            m = {n: statistics.median(v) for n, v in t.items()}
            half = 0.5 if causal else 1.0
            ffl, bfl = 4 * B * H * S * S * D * half, 10 * B * H * S * S * D * half
            tb = m["tfb"] - m["tf"]
            name = f"S={S} D={D} {'causal' if causal else 'full'}"
            for what, ours, theirs, fl in (("fwd", m["of"], m["tf"], ffl), ("bwd", m["ob"], tb, bfl)):
                print(f"{name + ' ' + what:34s} {ours:9.1f} {fl / ours / 1e6:6.0f} {theirs:9.1f} "
                      f"{fl / theirs / 1e6:6.0f} {theirs / ours:6.2f}", flush=True)


if __name__ == "__main__":
    main()
