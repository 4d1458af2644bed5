"""Benchmark of the tensor_gpu_v2 backward engine on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAMES]

Headline workload: one "step" = GELU backward and SiLU
backward on fp32 [8192, 8192], softmax backward on fp32 [16384, 4096] and
LayerNorm backward on fp32 [16384, 4096] (x, dy ~ N(0,1); softmax logits
~ N(0, 2); gamma ~ N(1, .02)), inputs resident in HBM.  `value` is the step's
algorithmic HBM bytes (read every input once, write every output once: 12 B per
element for each of the four) divided by the step's wall time: GB/s.

Per-kernel durations come from HIP events recorded on the stream the kernels
run on (torch's current stream, which every libtgbwd launch uses), around each
launch inside the timed region.  Other configurations (the C1 README MLP step,
BatchNorm-ReLU NHWC, AdamW, GradScaler unscale, the C5 GEMMs, FlashAttention
backward, the GPT step) are reported under "components" with their own roofline
fractions.

The CPU baseline times the NumPy oracle (the reference's CPU algorithm) on the
host's threads: the C2 step at full shape is `cpu_baseline.value`; C1, C3, C4 (fp32,
scaled from a batch of heads) and C5 (one layer scaled to four, plus head, loss,
embedding and AdamW) are under `cpu_baseline.configs`.
"""
import argparse
import json
import os
import sys
import time

# BLAS threads of the CPU baseline: the job's share of the host (OMP_NUM_THREADS when
# the environment sets it), else every core; set before NumPy loads its BLAS.
_THREADS = os.environ.get("OMP_NUM_THREADS") or str(os.cpu_count() or 1)
os.environ.setdefault("OMP_NUM_THREADS", _THREADS)
os.environ.setdefault("OPENBLAS_NUM_THREADS", _THREADS)

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "project-tensor_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0

# Measured HBM traffic per launch of the headline kernels: profiles/c2_traffic.txt
# holds lines `traffic <kernel> <bytes>` made by project-tensor_amd/prof_summary.py
# from two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) scaled by a copy of known
# size.  Each headline op maps to the kernels it launches.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "c2_traffic.txt")
OP_KERNELS = {"gelu_bwd": ["k_act_bwd<float,0,"], "silu_bwd": ["k_act_bwd<float,1,"],
              "softmax_bwd": ["k_softmax_bwd_reg<float,"],
              "layernorm_bwd": ["k_ln_bwd_reg<float,", "k_colsum<float,"]}


def measured_traffic(op):
    """HBM bytes per launch of a headline op from the committed counter summary, or
    None when the summary or one of the op's kernels is missing."""
    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    table = {}
    for ln in lines:
        f = ln.split()
        if len(f) >= 3 and f[0] == "traffic":
            table[f[1]] = float(f[2])
    total = 0.0
    for prefix in OP_KERNELS.get(op, []):
        hits = [v for k, v in table.items() if k.startswith(prefix)]
        if not hits:
            return None
        total += hits[0]
    return round(total) if OP_KERNELS.get(op) else None


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--only", default="", help="comma list of component names")
    return ap.parse_args()


class Timed:
    """A named launch sequence with its algorithmic byte/flop count, timed by HIP
    events on the current stream."""

    def __init__(self, name, fn, work, unit, peak):
        self.name, self.fn, self.work, self.unit, self.peak = name, fn, work, unit, peak
        self.ms = []

    def run(self, record):
        import torch
        if record:
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            self.fn()
            e.record()
            self.ms.append((s, e))
        else:
            self.fn()

    def avg_ms(self):
        # The first timed launch can find the GPU idle, so its window also holds the
        # host-side argument preparation; later launches are queued behind their
        # predecessor and their windows hold device time only.
        ms = self.ms[1:] if len(self.ms) > 1 else self.ms
        return sum(s.elapsed_time(e) for s, e in ms) / max(1, len(ms))

    def summary(self):
        ms = self.avg_ms()
        if self.unit == "GB/s":
            ach = self.work / (ms * 1e-3) / 1e9
        else:
            ach = self.work / (ms * 1e-3) / 1e12
        return {"ms": round(ms, 5), "achieved": round(ach, 2), "unit": self.unit,
                "peak": self.peak, "frac": round(ach / self.peak, 4), "work": self.work}


def c2_ops(torch, L):
    """The headline step's four backward ops on inputs resident in HBM."""
    g = torch.Generator(device="cuda").manual_seed(0)
    dev = "cuda"
    n = 8192 * 8192
    x = torch.randn(8192, 8192, device=dev, generator=g)
    dy = torch.randn(8192, 8192, device=dev, generator=g)
    dx = torch.empty_like(x)
    logits = torch.randn(16384, 4096, device=dev, generator=g) * 2
    y = torch.softmax(logits, -1)
    dys = torch.randn(16384, 4096, device=dev, generator=g)
    dxs = torch.empty_like(y)
    xl = torch.randn(16384, 4096, device=dev, generator=g)
    gam = 1 + 0.02 * torch.randn(4096, device=dev, generator=g)
    bet = 0.02 * torch.randn(4096, device=dev, generator=g)
    _, mean, rstd = L.layernorm_fwd(xl, gam, bet, 1e-5)
    dyl = torch.randn(16384, 4096, device=dev, generator=g)
    dxl = torch.empty_like(xl)
    dgam = torch.empty_like(gam)
    dbet = torch.empty_like(bet)
    lib = L.load()
    ws_ln = L.workspace(lib.tg_layernorm_bwd_workspace(0, 16384, 4096), dev)
    s = L.stream_handle
    p = L.ptr

    def gelu():
        L._check("gelu", lib.tg_gelu_bwd(0, p(x), p(dy), p(dx), n, 0, s()))

    def silu():
        L._check("silu", lib.tg_silu_bwd(0, p(x), p(dy), p(dx), n, 0, s()))

    def softmax():
        L._check("softmax", lib.tg_softmax_bwd(0, p(y), p(dys), p(dxs), 16384, 4096, 0, s()))

    def layernorm():
        L._check("ln", lib.tg_layernorm_bwd(0, p(xl), p(mean), p(rstd), p(gam), p(dyl), p(dxl),
                                            p(dgam), p(dbet), 16384, 4096, 0, 0, p(ws_ln),
                                            ws_ln.numel(), s()))

    for t in (x, dy, dx):
        _need(t, n, "act")
    for t in (y, dys, dxs, xl, dyl, dxl):
        _need(t, 16384 * 4096, "row op")
    b = 12 * n
    return [Timed("gelu_bwd", gelu, b, "GB/s", HBM_PEAK_GBS),
            Timed("silu_bwd", silu, b, "GB/s", HBM_PEAK_GBS),
            Timed("softmax_bwd", softmax, 12 * 16384 * 4096, "GB/s", HBM_PEAK_GBS),
            Timed("layernorm_bwd", layernorm, 12 * 16384 * 4096 + 4 * (2 * 16384 + 3 * 4096),
                  "GB/s", HBM_PEAK_GBS)]


def _need(t, numel, what):
    """Host-side check that a raw launch's extent fits the buffer it touches."""
    if t.numel() < numel:
        raise ValueError(f"{what}: buffer of {t.numel()} elements, launch needs {numel}")


def _op_bn(torch, L, g):
    """C3: FusedBatchNormReLU backward, NHWC [64, 56, 56, 256]; 20 B/elem (x and dy read
    twice, dx written once)."""
    lib, s, p = L.load(), L.stream_handle, L.ptr
    N, H, W, C = 64, 56, 56, 256
    x = torch.randn(N, H, W, C, device="cuda", generator=g)
    gam = 1 + 0.1 * torch.randn(C, device="cuda", generator=g)
    bet = 0.1 * torch.randn(C, device="cuda", generator=g)
    rm, rv = torch.zeros(C, device="cuda"), torch.ones(C, device="cuda")
    _, mean, rstd, _ = L.batchnorm_fwd_train(x, gam, bet, 1e-5, 0.1, rm, rv, True, L.NHWC)
    dy = torch.randn_like(x)
    dx = torch.empty_like(x)
    dg, db = torch.empty_like(gam), torch.empty_like(bet)
    ws = L.workspace(lib.tg_batchnorm_workspace(0, N, C, H * W), "cuda")
    for t in (x, dy, dx):
        _need(t, N * H * W * C, "bn")

    def run():
        L._check("bn", lib.tg_batchnorm_bwd(0, p(x), p(mean), p(rstd), p(gam), p(bet), p(dy),
                                            p(dx), p(dg), p(db), N, C, H * W, 1, 0, 0, p(ws),
                                            ws.numel(), s()))
    return Timed("bn_relu_bwd_nhwc", run, 20 * x.numel(), "GB/s", HBM_PEAK_GBS)


NPARAM = 83_200_000


def _op_adam(torch, L, g):
    """C5-sized AdamW over 48 fp32 tensors totalling 83.2M params: 28 B/param."""
    sizes = [NPARAM // 48] * 47 + [NPARAM - 47 * (NPARAM // 48)]
    ps = [torch.randn(n, device="cuda", generator=g) for n in sizes]
    gs = [torch.randn(n, device="cuda", generator=g) * 1e-3 for n in sizes]
    ms = [torch.zeros(n, device="cuda") for n in sizes]
    vs = [torch.zeros(n, device="cuda") for n in sizes]

    def run():
        L.adam_step(ps, gs, ms, vs, None, 3e-4, 0.9, 0.999, 1e-8, 0.1, 0.1, 0.001)
    return Timed("adamw_step", run, 28 * NPARAM, "GB/s", HBM_PEAK_GBS)


def _op_unscale(torch, L, g):
    """GradScaler unscale + non-finite check over 83.2M fp32 grads: 8 B/param."""
    lib, s, p = L.load(), L.stream_handle, L.ptr
    sizes = [NPARAM // 48] * 48
    gs = [torch.randn(n, device="cuda", generator=g) for n in sizes]
    flags = torch.empty(len(gs), dtype=torch.int32, device="cuda")
    arr, num = L._ptr_array(gs), L._numel_array(gs)

    def run():
        L._check("unscale", lib.tg_unscale_check(len(gs), 0, arr, num, 1.0, 1, p(flags), s()))
    return Timed("unscale_check", run, 8 * sum(sizes), "GB/s", HBM_PEAK_GBS)


def _op_unscale_norm(torch, L, g):
    """GradScaler unscale check + the clip's L2 norm in one read-only pass over 83.2M
    fp32 grads (the unscale itself left pending for AdamW): 4 B/param."""
    lib, s, p = L.load(), L.stream_handle, L.ptr
    sizes = [NPARAM // 48] * 48
    gs = [torch.randn(n, device="cuda", generator=g) for n in sizes]
    flags = torch.empty(len(gs), dtype=torch.int32, device="cuda")
    out = torch.empty(1, dtype=torch.float64, device="cuda")
    arr, num = L._ptr_array(gs), L._numel_array(gs)
    ws = L.workspace(lib.tg_unscale_norm_workspace(len(gs), num), "cuda")

    def run():
        L._check("unscale_norm", lib.tg_unscale_norm(len(gs), 0, arr, num, 1.0 / 65536,
                                                     p(flags), p(out), p(ws), ws.numel(), s()))
    return Timed("unscale_norm", run, 4 * sum(sizes), "GB/s", HBM_PEAK_GBS)


def _op_gemm(torch, L, g):
    """C5 FC1 backward (8192 tokens, 1024 -> 4096), fp16 in, fp32 accumulate:
    dA = dC W^T and dW = A^T dC, 4*M*N*K flops."""
    M, K, N = 8192, 1024, 4096
    a = torch.randn(M, K, device="cuda", generator=g).half()
    w = torch.randn(K, N, device="cuda", generator=g).half()
    dc = torch.randn(M, N, device="cuda", generator=g).half()
    da = torch.empty(M, K, device="cuda", dtype=torch.float16)
    dw = torch.empty(K, N, device="cuda", dtype=torch.float32)

    def run():
        L.matmul2d(dc, w, out=da, trans_b=True)
        L.matmul2d(a, dc, out=dw, trans_a=True)
    return Timed("gemm_fc1_bwd", run, 4 * M * N * K, "TFLOP/s", FP16_PEAK_TFLOPS)


FP32_PEAK_TFLOPS = 157.3


def _op_flash(torch, L, g, d, causal, dt=None):
    """C4: FlashAttention backward, B=8, H=16, S=2048, fp16; 10*B*H*S^2*d flops
    (halved when causal).  With dt = float32: the same shape in fp32 (the reference's
    default dtype) on the fp32 matrix cores, against their 157.3 TFLOP/s."""
    B, H, S = 8, 16, 2048
    dt = dt or torch.float16
    q, k, v, do = (torch.randn(B, H, S, d, device="cuda", generator=g).to(dt) for _ in range(4))
    o, lse = L.flash_attn_fwd(q, k, v, d ** -0.5, causal)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    def run():
        L.flash_attn_bwd(q, k, v, o, do, lse, dq, dk, dv, d ** -0.5, causal, False)
    flops = 10 * B * H * S * S * d // (2 if causal else 1)
    fp32 = dt == torch.float32
    return Timed(f"flash_bwd{'_fp32' if fp32 else ''}_d{d}{'_causal' if causal else ''}", run,
                 flops, "TFLOP/s", FP32_PEAK_TFLOPS if fp32 else FP16_PEAK_TFLOPS)


def _op_gpt(torch, L, g):
    """C5: one GPT training step (vocab 32000 tied, d 1024, 16 heads, 4 layers, batch 8 x
    seq 1024, fp16 autocast, GradScaler, CE, backward, tied sync, unscale, clip 1.0,
    AdamW).  Work = 6 * params * tokens (dense) + causal attention fwd+bwd flops."""
    from gpt_harness import GPT, Trainer, synthetic_batch
    model = GPT()
    tr = Trainer(model)
    # the synthetic batch is resident in HBM, like every other workload's inputs
    ids, targets = (L.to_device(a) for a in synthetic_batch())
    nparam = sum(p.size for p in tr.params)
    B, T, H, hd, layers = 8, 1024, 16, 64, 4
    flops = 6 * nparam * B * T + layers * 14 * B * H * T * T * hd // 2

    def run():
        tr.step(ids, targets)
    return Timed("gpt_step", run, flops, "TFLOP/s", FP16_PEAK_TFLOPS)


def _op_mlp(torch, L, g):
    """C1: the README MLP, x fp32 [32, 784] -> Linear(784, 256) -> GELU -> Linear(256, 10),
    loss = out.mean(), full backward and one Adam step (lr 1e-3) through the tensor_gpu_v2
    API; a latency-bound step (launches), reported in ms.  Work = 3 x 2 x 32 x
    (784*256 + 256*10) flops (forward, dA, dB)."""
    import numpy as np
    import tensor_gpu_v2 as tg
    np.random.seed(0)
    x = tg.Tensor(np.random.randn(32, 784).astype(np.float32), requires_grad=False)
    l1, l2 = tg.Linear(784, 256), tg.Linear(256, 10)
    params = [l1.w, l1.b, l2.w, l2.b]
    opt = tg.Adam(params, lr=1e-3)

    def run():
        for p in params:
            p.zero_grad()
        loss = l2(l1(x).gelu()).mean()
        loss.backward()
        opt.step()
    return Timed("mlp_step", run, 3 * 2 * 32 * (784 * 256 + 256 * 10), "TFLOP/s",
                 FP16_PEAK_TFLOPS)


def _op_ce(torch, L, g):
    """C5 cross-entropy over fp16 logits [8192, 32000]: forward (row statistics and
    losses) then backward (gradient written in fp16).  Algorithmic bytes: the logits
    read twice and the gradient written once, 3 x 524 MB."""
    N, C = 8192, 32000
    x = (torch.randn(N, C, device="cuda", generator=g) * 2).half()
    y = torch.randint(0, C, (N,), device="cuda", generator=g)
    grad = torch.empty_like(x)
    _need(grad, N * C, "ce")

    def run():
        lse, loss = L.cross_entropy_fwd(x, y)
        L.cross_entropy_bwd(x, y, lse, grad, 1.0 / N, False)
    return Timed("cross_entropy_fwd_bwd", run, 3 * 2 * N * C, "GB/s", HBM_PEAK_GBS)


def _op_ce_one_pass(torch, L, g):
    """The same cross-entropy as the engine runs it when a backward follows (its gradient
    does not depend on the upstream one): statistics, losses and the fp16 gradient from
    one read of the logits.  Algorithmic bytes: 2 x 524 MB."""
    N, C = 8192, 32000
    x = (torch.randn(N, C, device="cuda", generator=g) * 2).half()
    y = torch.randint(0, C, (N,), device="cuda", generator=g)

    def run():
        L.cross_entropy_fwd_grad(x, y, 1.0 / N)
    return Timed("cross_entropy_one_pass", run, 2 * 2 * N * C, "GB/s", HBM_PEAK_GBS)


def _op_embedding(torch, L, g):
    """C5 embedding backward: fp32 output gradient [8192, 1024] scattered into a fresh
    [32000, 1024] fp32 gradient (deterministic sorted scatter-add; untouched rows
    zeroed).  Algorithmic bytes: write every gradient row once, read dout and the
    indices once."""
    V, dim, n = 32000, 1024, 8192
    idx = torch.randint(0, V, (n,), device="cuda", generator=g)
    dout = torch.randn(n, dim, device="cuda", generator=g)
    grad = torch.empty(V, dim, device="cuda")

    def run():
        L.embedding_bwd(dout, idx, grad, False)
    work = V * dim * 4 + n * dim * 4 + n * 8
    return Timed("embedding_bwd", run, work, "GB/s", HBM_PEAK_GBS)


def _op_ln_c5(torch, L, g):
    """C5 LayerNorm backward: fp16 [8192, 1024] (one of the step's nine), dx accumulated
    into the residual gradient as in the pre-LN block.  Algorithmic bytes: read x, dy
    and the old dx, write dx (8 B per element), plus the fp32 row statistics."""
    R, C = 8192, 1024
    x = torch.randn(R, C, device="cuda", generator=g).half()
    gam = 1 + 0.02 * torch.randn(C, device="cuda", generator=g)
    bet = 0.02 * torch.randn(C, device="cuda", generator=g)
    _, mean, rstd = L.layernorm_fwd(x, gam, bet, 1e-5)
    dy = torch.randn(R, C, device="cuda", generator=g).half()
    dx = torch.randn(R, C, device="cuda", generator=g).half()
    dg, db = torch.empty_like(gam), torch.empty_like(bet)
    lib, s, p = L.load(), L.stream_handle, L.ptr
    ws = L.workspace(lib.tg_layernorm_bwd_workspace(1, R, C), "cuda")
    for t in (x, dy, dx):
        _need(t, R * C, "ln c5")

    def run():  # the raw entry point with a prepared workspace (a ~20 us op)
        L._check("ln", lib.tg_layernorm_bwd(1, p(x), p(mean), p(rstd), p(gam), p(dy), p(dx),
                                            p(dg), p(db), R, C, 1, 0, p(ws), ws.numel(), s()))
    return Timed("layernorm_bwd_c5_fp16", run, 8 * R * C + 8 * R, "GB/s", HBM_PEAK_GBS)


def _op_tied(torch, L, g):
    """C5 tied-weight transfer: embedding.grad [32000, 1024] += head.grad.T, fp32.
    Algorithmic bytes: read both, write the source gradient (3 x 131 MB)."""
    V, dim = 32000, 1024
    src = torch.randn(dim, V, device="cuda", generator=g)
    dst = torch.randn(V, dim, device="cuda", generator=g)

    def run():
        L.transpose_add(src, dst)
    return Timed("tied_grad_sync", run, 3 * V * dim * 4, "GB/s", HBM_PEAK_GBS)


def _copy_floors(torch, L, nbytes):
    """Same-box floors of a memory-bound op: a plain copy moving the op's algorithmic
    byte count (half read, half written) in one launch, by libtgbwd's tg_axpby with
    beta 0 (read x, write y, 16-byte vectors) and by a device-to-device hipMemcpy
    (ROCm's blit kernel, through torch's copy_).  At the component sizes a launch's
    ramp-up and drain are a visible share of its time, so the faster of the two is
    the ceiling a single kernel of that size reaches on this box, not 8 TB/s."""
    n = max(1, nbytes // 8)
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)

    def axpby():
        L.axpby(x, y, 1.0, 0.0)

    def memcpy():
        y.copy_(x)
    return [Timed("copy_axpby", axpby, n * 8, "GB/s", HBM_PEAK_GBS),
            Timed("copy_memcpy", memcpy, n * 8, "GB/s", HBM_PEAK_GBS)]


def component_ops(torch, L, only):
    """Other configurations, each built in its own scope on HBM-resident inputs."""
    g = torch.Generator(device="cuda").manual_seed(1)
    builders = [("mlp_step", lambda: _op_mlp(torch, L, g)),
                ("bn_relu_bwd_nhwc", lambda: _op_bn(torch, L, g)),
                ("adamw_step", lambda: _op_adam(torch, L, g)),
                ("unscale_check", lambda: _op_unscale(torch, L, g)),
                ("unscale_norm", lambda: _op_unscale_norm(torch, L, g)),
                ("gemm_fc1_bwd", lambda: _op_gemm(torch, L, g)),
                ("cross_entropy_fwd_bwd", lambda: _op_ce(torch, L, g)),
                ("cross_entropy_one_pass", lambda: _op_ce_one_pass(torch, L, g)),
                ("embedding_bwd", lambda: _op_embedding(torch, L, g)),
                ("layernorm_bwd_c5_fp16", lambda: _op_ln_c5(torch, L, g)),
                ("tied_grad_sync", lambda: _op_tied(torch, L, g)),
                ("gpt_step", lambda: _op_gpt(torch, L, g))]
    for d in (64, 128):
        for causal in (False, True):
            builders.append((f"flash_bwd_d{d}{'_causal' if causal else ''}",
                             lambda d=d, causal=causal: _op_flash(torch, L, g, d, causal)))
    builders.append(("flash_bwd_fp32_d64",
                     lambda: _op_flash(torch, L, g, 64, False, torch.float32)))
    for name, build in builders:
        if only and name not in only:
            continue
        try:
            op = build()
        except RuntimeError as e:
            if "not implemented" in str(e):
                continue
            raise
        yield op


def _cpu_threads():
    """Host threads for the CPU baseline: the process's OMP_NUM_THREADS when set (the
    share of the host a job gets), else every core os.cpu_count() reports."""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "")))
    except ValueError:
        return os.cpu_count() or 1


def _median_s(fn, warmup=2, reps=5):
    import statistics
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _log(msg):
    print(f"cpu_baseline: {msg}", file=sys.stderr, flush=True)


def cpu_baseline():
    """The reference's CPU algorithm (the NumPy oracle, fp32) timed on the host: per
    config the median of 5 runs after 2 warm-ups (C5: 3 after 1), at the configured
    shapes.  NumPy's elementwise ufuncs run on one thread, so row-, channel- and
    head-independent work is split over a pool of host threads (ufuncs release the
    GIL); BLAS calls use OPENBLAS/OMP_NUM_THREADS threads.  C4 runs in fp32 (NumPy has
    no fast fp16 matmul): a thread-pool batch of heads is timed and scaled to the 128
    heads.  C5 is one transformer layer forward + backward timed and scaled to the
    step (4 layers), plus the head, loss, embedding and optimizer pieces."""
    import concurrent.futures as cf

    import numpy as np

    import oracle as O
    T = _cpu_threads()
    pool = cf.ThreadPoolExecutor(T)
    rng = np.random.default_rng(0)

    def rows(fn, n, *arrs):
        """fn over T row chunks of the arrays in the pool; returns the chunk results."""
        cuts = np.linspace(0, n, T + 1).astype(int)
        futs = [pool.submit(fn, *(a[c0:c1] for a in arrs)) for c0, c1 in zip(cuts[:-1], cuts[1:])
                if c1 > c0]
        return [f.result() for f in futs]

    out = {"threads": T, "os_cpu_count": os.cpu_count()}
    # ---- C2 at full shape
    c2 = {}
    x = rng.standard_normal((8192, 8192)).astype(np.float32)
    dy = rng.standard_normal((8192, 8192)).astype(np.float32)
    for name, fn in (("gelu_bwd", O.gelu_bwd), ("silu_bwd", O.silu_bwd)):
        _log(f"C2 {name} [8192,8192]")
        t = _median_s(lambda: rows(fn, 8192, x, dy))
        c2[name] = {"ms": round(t * 1e3, 1), "GB/s": round(12 * x.size / t / 1e9, 2)}
    del x, dy
    lg = (rng.standard_normal((16384, 4096)) * 2).astype(np.float32)
    y = np.concatenate(rows(O.softmax_fwd, 16384, lg))
    del lg
    dys = rng.standard_normal((16384, 4096)).astype(np.float32)
    _log("C2 softmax_bwd [16384,4096]")
    t = _median_s(lambda: rows(O.softmax_bwd, 16384, y, dys))
    c2["softmax_bwd"] = {"ms": round(t * 1e3, 1), "GB/s": round(12 * y.size / t / 1e9, 2)}
    del y
    xl = rng.standard_normal((16384, 4096)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    b = (0.02 * rng.standard_normal(4096)).astype(np.float32)
    parts = rows(lambda a: O.layernorm_fwd(a, g, b), 16384, xl)
    xh = np.concatenate([p[1] for p in parts])
    var = np.concatenate([p[3] for p in parts])
    del parts, xl

    def ln_bwd():
        res = rows(lambda a, v, d: O.layernorm_bwd(a, v, g, d), 16384, xh, var, dys)
        return sum(r[1] for r in res), sum(r[2] for r in res)  # dgamma, dbeta partials
    _log("C2 layernorm_bwd [16384,4096]")
    t = _median_s(ln_bwd)
    c2["layernorm_bwd"] = {"ms": round(t * 1e3, 1), "GB/s": round(12 * xh.size / t / 1e9, 2)}
    del xh, var, dys
    step_s = sum(v["ms"] for v in c2.values()) / 1e3
    out["C2"] = c2
    value = 3221405696 / step_s / 1e9
    # ---- C1: the README MLP step (forward, backward, Adam), BLAS threads
    _log("C1 MLP step")
    np.random.seed(0)
    xm = np.random.randn(32, 784).astype(np.float32)
    w1 = (np.random.randn(784, 256) * np.sqrt(2 / 784)).astype(np.float32)
    w2 = (np.random.randn(256, 10) * np.sqrt(2 / 256)).astype(np.float32)
    z1, z2 = np.zeros(256, np.float32), np.zeros(10, np.float32)
    t = _median_s(lambda: O.mlp_step(xm, w1, z1, w2, z2, dtype=np.float32))
    out["C1_mlp_step_ms"] = round(t * 1e3, 3)
    # ---- C3: BatchNorm-ReLU backward NHWC, channels split over the pool
    _log("C3 BN-ReLU bwd NHWC [64,56,56,256]")
    xb = rng.standard_normal((64, 56, 56, 256)).astype(np.float32)
    gb = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    bb = (0.1 * rng.standard_normal(256)).astype(np.float32)
    dyb = rng.standard_normal((64, 56, 56, 256)).astype(np.float32)
    cuts = np.linspace(0, 256, T + 1).astype(int)
    chunks = [(c0, c1) for c0, c1 in zip(cuts[:-1], cuts[1:]) if c1 > c0]
    caches = [O.batchnorm_relu_fwd_nhwc(xb[..., c0:c1], gb[c0:c1], bb[c0:c1])[1]
              for c0, c1 in chunks]
    del xb

    def bn_bwd():
        fs = [pool.submit(O.batchnorm_relu_bwd_nhwc, dyb[..., c0:c1], gb[c0:c1], cc)
              for (c0, c1), cc in zip(chunks, caches)]
        return [f.result() for f in fs]
    t = _median_s(bn_bwd)
    out["C3_bn_relu_bwd"] = {"ms": round(t * 1e3, 1), "GB/s": round(20 * dyb.size / t / 1e9, 2)}
    del caches, dyb
    # ---- C4: FlashAttention bwd fp32, T heads at once, scaled to B*H = 128
    c4 = {}
    for d in (64, 128):
        qh = [rng.standard_normal((1, 1, 2048, d)).astype(np.float32) for _ in range(4 * T)]
        for causal in (False, True):
            name = f"flash_bwd_d{d}{'_causal' if causal else ''}"
            _log(f"C4 {name} fp32, {T} heads in parallel")

            def heads():
                fs = [pool.submit(O.flash_attention_bwd, *qh[4 * i:4 * i + 4], causal)
                      for i in range(T)]
                return [f.result() for f in fs]
            t = _median_s(heads) * 128 / T
            flops = 10 * 128 * 2048 * 2048 * d // (2 if causal else 1)
            c4[name] = {"ms": round(t * 1e3, 1), "TFLOP/s": round(flops / t / 1e12, 4)}
    out["C4_fp32_extrapolated"] = c4
    # ---- C5: one layer forward + backward (scaled x4) + head, loss, embedding, AdamW
    out["C5"] = _cpu_c5(O, np, pool, T, rows, rng)
    pool.shutdown()
    return {"value": round(value, 3), "unit": "GB/s", "cores": T, "kind": "port",
            "sample": (f"NumPy oracle fp32 on {T} host threads (os.cpu_count() "
                       f"{os.cpu_count()}): the C2 step at full shape (median of 5 after 2 "
                       "warm-ups per op); other configs under 'configs'"),
            "configs": out}


def _cpu_c5(O, np, pool, T, rows, rng):
    """C5 on the host: one pre-LN decoder layer at batch 8 x seq 1024, d 1024, 16 heads
    (forward and backward with the oracle's formulas and NumPy matmuls), timed and
    scaled to the 4 layers, plus the tied head (logits GEMM and its two gradient
    GEMMs), cross-entropy forward + backward over [8192, 32000], the embedding
    backward and the AdamW step over the 83.2 M parameters."""
    N, C, H, hd, V = 8192, 1024, 16, 64, 32000

    def w(*shape):
        return (rng.standard_normal(shape) * 0.02).astype(np.float32)
    h0 = rng.standard_normal((N, C)).astype(np.float32)
    wq, wk, wv, wo, w1, w2 = w(C, C), w(C, C), w(C, C), w(C, C), w(C, 4 * C), w(4 * C, C)
    g1 = np.ones(C, np.float32)
    z = np.zeros(C, np.float32)

    def attn_heads(fn, *arrs):
        """fn per (batch, head) on (1, 1, 1024, 64) slices, over the pool."""
        sl = [(b, hh) for b in range(8) for hh in range(H)]
        split = [a.reshape(8, 1024, H, hd) for a in arrs]
        fs = [pool.submit(fn, *(s[b, :, hh][None, None] for s in split)) for b, hh in sl]
        return [f.result() for f in fs]

    def layer():
        a, xh1, _, var1 = O.layernorm_fwd(h0, g1, z)
        q, k, v = a @ wq, a @ wk, a @ wv
        outs = attn_heads(lambda qq, kk, vv: O.flash_attention_fwd(qq, kk, vv, True)[0], q, k, v)
        o = np.stack([r[0, 0] for r in outs]).reshape(8, H, 1024, hd).transpose(0, 2, 1, 3)
        o = np.ascontiguousarray(o).reshape(N, C)
        h1 = h0 + o @ wo
        m, xh2, _, var2 = O.layernorm_fwd(h1, g1, z)
        f = m @ w1
        gl = np.concatenate(rows(O.gelu_fwd, N, f))
        dh = rng.standard_normal((N, C)).astype(np.float32) * 1e-3  # upstream gradient
        # backward (the weight gradients are computed and dropped)
        _ = gl.T @ dh                            # dW2
        dgl = dh @ w2.T                          # gradient of the GELU output
        df = np.concatenate(rows(O.gelu_bwd, N, f, dgl))
        _ = m.T @ df
        dm = df @ w1.T
        dh1 = dh + np.concatenate([r[0] for r in rows(lambda x, vv, d: O.layernorm_bwd(
            x, vv, g1, d), N, xh2, var2, dm)])
        _ = o.T @ dh1
        do = dh1 @ wo.T
        grads = attn_heads(lambda qq, kk, vv, dd: O.flash_attention_bwd(qq, kk, vv, dd, True),
                           q, k, v, do)
        def merge(j):
            t = np.stack([r[j][0, 0] for r in grads]).reshape(8, H, 1024, hd)
            return np.ascontiguousarray(t.transpose(0, 2, 1, 3)).reshape(N, C)
        dq, dk, dv = merge(0), merge(1), merge(2)
        da = dq @ wq.T + dk @ wk.T + dv @ wv.T
        _ = a.T @ dq, a.T @ dk, a.T @ dv
        return np.concatenate([r[0] for r in rows(lambda x, vv, d: O.layernorm_bwd(
            x, vv, g1, d), N, xh1, var1, da)])

    _log("C5 one layer fwd+bwd (8 x 1024 tokens, d 1024, 16 heads)")
    t_layer = _median_s(layer, warmup=1, reps=3)
    hf = rng.standard_normal((N, C)).astype(np.float32)
    E = w(V, C)
    tg = rng.integers(0, V, N)

    def head_loss():
        logits = hf @ E.T
        res = rows(lambda lg, tt: O.cross_entropy_bwd(O.cross_entropy_fwd(lg, tt)[1], tt), N,
                   logits, tg)
        dl = np.concatenate(res)
        return dl @ E, dl.T @ hf
    _log("C5 head GEMMs + cross-entropy [8192, 32000]")
    t_head = _median_s(head_loss, warmup=1, reps=3)
    _log("C5 embedding bwd + AdamW (83.2 M params)")
    dout = rng.standard_normal((N, C)).astype(np.float32)
    t_emb = _median_s(lambda: O.embedding_bwd(tg, dout, V), warmup=1, reps=3)
    sizes = [83_200_000 // 48] * 48
    ps = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    gs = [(rng.standard_normal(n) * 1e-3).astype(np.float32) for n in sizes]
    ms = [np.zeros(n, np.float32) for n in sizes]

    def adamw():
        fs = [pool.submit(O.adam_step, p, gg, mm, mm, 1, 3e-4, (0.9, 0.999), 1e-8, 0.1)
              for p, gg, mm in zip(ps, gs, ms)]
        return [f.result() for f in fs]
    t_adam = _median_s(adamw, warmup=1, reps=3)
    step = 4 * t_layer + t_head + t_emb + t_adam
    return {"layer_fwd_bwd_ms": round(t_layer * 1e3, 1), "head_and_loss_ms": round(t_head * 1e3, 1),
            "embedding_bwd_ms": round(t_emb * 1e3, 1), "adamw_ms": round(t_adam * 1e3, 1),
            "step_ms_estimate": round(step * 1e3, 1),
            "note": "step = 4 x layer + head/loss + embedding + AdamW (extrapolated)"}


CALIB_BYTES = 256 << 20


def calibration_copy(torch):
    """Three plain device copies of CALIB_BYTES (read CALIB_BYTES, write CALIB_BYTES).
    Under rocprofv3 --pmc they give the scale between the FETCH_SIZE / WRITE_SIZE
    counters and true bytes, used to turn the counters of the kernels into HBM
    traffic."""
    src = torch.ones(CALIB_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


WARM_MS = 50.0


def _warm(torch, op, calls):
    """Untimed runs of op: at least `calls` of them and at least WARM_MS of wall time.
    The GPU clock ramps up over the first tens of milliseconds of work after an idle
    gap (a 0.5 ms FlashAttention backward runs ~15 % slower in its first ten calls), so
    a fixed small count would time part of the ramp."""
    n, t0 = 0, time.perf_counter()
    while n < max(1, calls) or (time.perf_counter() - t0) * 1e3 < WARM_MS:
        op.run(False)
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def main():
    a = _args()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not measured)"}))
        sys.exit(2)
    import torch

    from tensor_gpu_v2 import _lib as L

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    L.ensure_device(0)
    calibration_copy(torch)
    ops = c2_ops(torch, L)
    for _ in range(a.warmup):
        for op in ops:
            op.run(False)
    torch.cuda.synchronize()
    # One event before each step and one after each op: consecutive ops share the
    # boundary event, so each op's window is its launches plus one event's overhead.
    t0 = time.perf_counter()
    for _ in range(a.steps):
        prev = torch.cuda.Event(enable_timing=True)
        prev.record()
        for op in ops:
            op.fn()
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            op.ms.append((prev, ev))
            prev = ev
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_bytes = sum(op.work for op in ops)
    ms_step = wall / a.steps * 1e3
    value = step_bytes / (wall / a.steps) / 1e9
    per = {op.name: op.summary() for op in ops}
    dom = max(ops, key=lambda o: o.avg_ms())
    ds = dom.summary()
    del ops
    torch.cuda.empty_cache()

    comps = {}
    if not a.no_components:
        only = set(x for x in a.only.split(",") if x)
        for op in component_ops(torch, L, only):
            _warm(torch, op, a.warmup)
            for _ in range(max(3, a.steps // 2) + 1):
                op.run(True)
            torch.cuda.synchronize()
            comps[op.name] = op.summary()
            if op.unit == "GB/s":
                best = None
                for fl in _copy_floors(torch, L, op.work):
                    _warm(torch, fl, a.warmup)
                    for _ in range(max(3, a.steps // 2) + 1):
                        fl.run(True)
                    torch.cuda.synchronize()
                    if best is None or fl.avg_ms() < best[0]:
                        best = (fl.avg_ms(), fl.name)
                comps[op.name]["copy_floor_ms"] = round(best[0], 5)
                comps[op.name]["copy_floor_kernel"] = best[1]
                comps[op.name]["frac_of_copy_floor"] = round(best[0] / comps[op.name]["ms"], 4)
            del op
            torch.cuda.empty_cache()

    rec = {
        "metric": "fused-grad-kernel HBM GB/s (% peak); FlashAttention bwd TFLOP/s; step ms",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) inputs of the configured shapes, resident in HBM)",
        "config": {"workload": "C2: GELU+SiLU bwd fp32 [8192,8192], softmax+LayerNorm bwd fp32 "
                               "[16384,4096]", "step_bytes": step_bytes},
        "roofline": {"bound": "hbm", "kernel": dom.name, "achieved": ds["achieved"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ds["frac"],
                     "traffic": measured_traffic(dom.name)},
        "kernels": per,
        "components": comps,
    }
    if not a.no_cpu:
        rec["cpu_baseline"] = cpu_baseline()
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
