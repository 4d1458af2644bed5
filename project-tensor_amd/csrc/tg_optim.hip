// Multi-tensor optimizer and gradient-hygiene kernels:
//   Adam / AdamW step (decoupled weight decay applied first, optional AMSGrad),
//   GradScaler unscale with non-finite detection,
//   global gradient norm (L2, Linf, Lp) ignoring non-finite entries,
//   in-place scaling and zeroing of non-finite entries.
//
// One launch covers up to kMaxT tensors: the host packs tensor pointers and
// sizes into the kernel argument block and assigns each workgroup a fixed chunk
// of one tensor, so a whole model's update is a handful of launches regardless
// of the parameter count.  Each element is touched once (Adam: 28 B/param fp32).
#include "tg_common.h"

#include <vector>

namespace {

constexpr int kBlock = 256;
constexpr int kMaxT = 24;
constexpr int64_t kChunk = kBlock * 4 * 4;  // elements per workgroup (16 per thread)

struct MtArgs {
  void* a[kMaxT];  // param / grad
  void* b[kMaxT];  // grad (Adam) / unused
  void* c[kMaxT];  // exp_avg
  void* d[kMaxT];  // exp_avg_sq
  void* e[kMaxT];  // max_exp_avg_sq (AMSGrad) or null
  int64_t n[kMaxT];
  int64_t first_block[kMaxT + 1];
  int fidx[kMaxT];  // index of each tensor in the caller's list (flag slot)
  int ntensors;
};

__device__ __forceinline__ int find_tensor(const MtArgs& A, int64_t blk) {
  int t = 0;
  while (t + 1 < A.ntensors && A.first_block[t + 1] <= blk) ++t;
  return t;
}

// ---------------------------------------------------------------------------
// Adam/AdamW, reference order (_nn.py:1413-1442, _training.py:2198-2220):
//   p -= lr*wd*p (if wd != 0); m = b1*m + (1-b1)*g; v = b2*v + (1-b2)*g^2;
//   mhat = m/bc1; vhat = v/bc2; [vmax = max(vmax, vhat)]; p -= lr*mhat/(sqrt(v*)+eps)
struct AdamConsts {
  float lr, b1, omb1, b2, omb2, eps, lrwd, bc1, bc2;
  int decay;
};

template <bool AMS>
__global__ __launch_bounds__(kBlock) void k_adam(MtArgs A, AdamConsts K) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t start = (blockIdx.x - A.first_block[t]) * kChunk;
  float* __restrict__ p = (float*)A.a[t];
  const float* __restrict__ g = (const float*)A.b[t];
  float* __restrict__ m = (float*)A.c[t];
  float* __restrict__ v = (float*)A.d[t];
  float* __restrict__ vm = (float*)A.e[t];
  const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) |
                     reinterpret_cast<uintptr_t>(m) | reinterpret_cast<uintptr_t>(v) |
                     (AMS ? reinterpret_cast<uintptr_t>(vm) : 0)) & 15) == 0;
  auto upd = [&](float& pp, float gg, float& mm, float& vv, float* vmx) {
    if (K.decay) pp -= K.lrwd * pp;
    mm = K.b1 * mm + K.omb1 * gg;
    vv = K.b2 * vv + K.omb2 * (gg * gg);
    const float mh = mm / K.bc1;
    float vh = vv / K.bc2;
    if (AMS) {
      vh = fmaxf(*vmx, vh);
      *vmx = vh;
    }
    pp -= K.lr * mh / (sqrtf(vh) + K.eps);
  };
  if (vec && start + kChunk <= n) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = start + ((int64_t)u * kBlock + threadIdx.x) * 4;
      float4 P = *reinterpret_cast<float4*>(p + i);
      const float4 G = *reinterpret_cast<const float4*>(g + i);
      float4 Mv = *reinterpret_cast<float4*>(m + i);
      float4 Vv = *reinterpret_cast<float4*>(v + i);
      float4 VM = AMS ? *reinterpret_cast<float4*>(vm + i) : make_float4(0, 0, 0, 0);
      upd(P.x, G.x, Mv.x, Vv.x, &VM.x);
      upd(P.y, G.y, Mv.y, Vv.y, &VM.y);
      upd(P.z, G.z, Mv.z, Vv.z, &VM.z);
      upd(P.w, G.w, Mv.w, Vv.w, &VM.w);
      *reinterpret_cast<float4*>(p + i) = P;
      *reinterpret_cast<float4*>(m + i) = Mv;
      *reinterpret_cast<float4*>(v + i) = Vv;
      if (AMS) *reinterpret_cast<float4*>(vm + i) = VM;
    }
  } else {
    const int64_t end = start + kChunk < n ? start + kChunk : n;
    for (int64_t i = start + threadIdx.x; i < end; i += kBlock) {
      float P = p[i], Mv = m[i], Vv = v[i], VM = AMS ? vm[i] : 0.f;
      upd(P, g[i], Mv, Vv, &VM);
      p[i] = P;
      m[i] = Mv;
      v[i] = Vv;
      if (AMS) vm[i] = VM;
    }
  }
}

// ---------------------------------------------------------------------------
// g' = g*mul (stored if WRITE).  flags[t] |= 1 if any g is non-finite,
// |= 2 if any g' is non-finite (GradScaler.unscale_, _nn.py:1795-1833).
template <typename T, bool WRITE>
__global__ __launch_bounds__(kBlock) void k_scale_check(MtArgs A, float mul, int* flags) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t start = (blockIdx.x - A.first_block[t]) * kChunk;
  const int64_t end = start + kChunk < n ? start + kChunk : n;
  T* __restrict__ g = (T*)A.a[t];
  int f = 0;
  for (int64_t i = start + threadIdx.x; i < end; i += kBlock) {
    const float x = tg_to_float(g[i]);
    const float y = x * mul;
    if (!isfinite(x)) f |= 1;
    const T yt = tg_from_float<T>(y);
    if (!isfinite(tg_to_float(yt))) f |= 2;
    if (WRITE) g[i] = yt;
  }
  // wave-level OR, then one atomic per wave that found something
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) f |= __shfl_xor(f, off, 64);
  if ((threadIdx.x & 63) == 0 && f) atomicOr(flags + A.fidx[t], f);
}

// Per-block partial of the gradient norm over finite entries.
// KIND 0: sum g^2, 1: max |g|, 2: sum |g|^p.  Non-finite entries set flags bit 1.
template <typename T, int KIND>
__global__ __launch_bounds__(kBlock) void k_norm_partial(MtArgs A, float p, double* part,
                                                         int64_t part_base, int* flags) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t start = (blockIdx.x - A.first_block[t]) * kChunk;
  const int64_t end = start + kChunk < n ? start + kChunk : n;
  const T* __restrict__ g = (const T*)A.a[t];
  double acc = 0.0;
  int f = 0;
  for (int64_t i = start + threadIdx.x; i < end; i += kBlock) {
    const float x = tg_to_float(g[i]);
    if (!isfinite(x)) {
      f = 1;
      continue;
    }
    const float ax = fabsf(x);
    if (KIND == 0) acc += (double)ax * (double)ax;
    else if (KIND == 1) acc = fmax(acc, (double)ax);
    else acc += pow((double)ax, (double)p);
  }
  __shared__ double red[4];
  if (KIND == 1) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc = fmax(acc, __shfl_xor(acc, off, 64));
  } else {
    acc = tg_wave_sum_d(acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) f |= __shfl_xor(f, off, 64);
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = acc;
    if (f) atomicOr(flags + A.fidx[t], f);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    part[part_base + blockIdx.x] = KIND == 1 ? fmax(fmax(red[0], red[1]), fmax(red[2], red[3]))
                                             : (red[0] + red[1]) + (red[2] + red[3]);
  }
}

// Deterministic single-block reduction of the partials.
template <int KIND>
__global__ __launch_bounds__(kBlock) void k_norm_final(const double* part, int64_t n,
                                                       double* out) {
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock)
    acc = KIND == 1 ? fmax(acc, part[i]) : acc + part[i];
  __shared__ double red[kBlock];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s)
      red[threadIdx.x] = KIND == 1 ? fmax(red[threadIdx.x], red[threadIdx.x + s])
                                   : red[threadIdx.x] + red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = red[0];
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_zero_nonfinite(MtArgs A) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t start = (blockIdx.x - A.first_block[t]) * kChunk;
  const int64_t end = start + kChunk < n ? start + kChunk : n;
  T* __restrict__ g = (T*)A.a[t];
  for (int64_t i = start + threadIdx.x; i < end; i += kBlock)
    if (!isfinite(tg_to_float(g[i]))) g[i] = tg_from_float<T>(0.f);
}

__global__ void k_zero_ints(int* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

// Split a tensor list into launches of at most kMaxT tensors; calls fn(args, nblocks,
// first tensor index) per launch.  Empty tensors are skipped.
template <typename F>
int for_each_launch(int ntensors, void* const* a, void* const* b, void* const* c,
                    void* const* d, void* const* e, const int64_t* numel, F&& fn) {
  MtArgs A{};
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (A.ntensors > 0) {
      A.first_block[A.ntensors] = blocks;
      if (blocks > 0x7fffffff) {
        tg_set_error("multi-tensor launch: too many blocks");
        return TG_ERR_INVALID;
      }
      int st = fn(A, blocks);
      if (st) return st;
    }
    A = MtArgs{};
    blocks = 0;
    return TG_OK;
  };
  for (int i = 0; i < ntensors; ++i) {
    if (numel[i] < 0) {
      tg_set_error("multi-tensor: negative numel for tensor %d", i);
      return TG_ERR_INVALID;
    }
    if (numel[i] == 0) continue;
    if (A.ntensors == kMaxT) {
      int st = flush();
      if (st) return st;
    }
    const int k = A.ntensors++;
    A.a[k] = a ? a[i] : nullptr;
    A.b[k] = b ? b[i] : nullptr;
    A.c[k] = c ? c[i] : nullptr;
    A.d[k] = d ? d[i] : nullptr;
    A.e[k] = e ? e[i] : nullptr;
    A.n[k] = numel[i];
    A.fidx[k] = i;
    A.first_block[k] = blocks;
    blocks += (numel[i] + kChunk - 1) / kChunk;
  }
  return flush();
}

int64_t total_blocks(int ntensors, const int64_t* numel) {
  int64_t b = 0;
  for (int i = 0; i < ntensors; ++i)
    if (numel[i] > 0) b += (numel[i] + kChunk - 1) / kChunk;
  return b;
}

}  // namespace

TG_EXPORT int tg_adam_step(int ntensors, float* const* params, const float* const* grads,
                           float* const* exp_avg, float* const* exp_avg_sq,
                           float* const* max_exp_avg_sq, const int64_t* numel, double lr,
                           double beta1, double beta2, double eps, double weight_decay,
                           double bias_correction1, double bias_correction2, void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_adam_step: negative tensor count");
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(params && grads && exp_avg && exp_avg_sq && numel, "tg_adam_step: null list");
  for (int i = 0; i < ntensors; ++i)
    TG_REQUIRE(numel[i] == 0 || (params[i] && grads[i] && exp_avg[i] && exp_avg_sq[i] &&
                                 (!max_exp_avg_sq || max_exp_avg_sq[i])),
               "tg_adam_step: null pointer for tensor %d", i);
  hipStream_t s = tg_stream(stream);
  const bool ams = max_exp_avg_sq != nullptr;
  // Scalars are combined in double and rounded once to fp32, as the reference's
  // Python-float hyper-parameters are when they meet fp32 arrays (1 - beta2 in
  // particular must not be formed from an already-rounded fp32 beta2).
  AdamConsts K;
  K.lr = (float)lr;
  K.b1 = (float)beta1;
  K.omb1 = (float)(1.0 - beta1);
  K.b2 = (float)beta2;
  K.omb2 = (float)(1.0 - beta2);
  K.eps = (float)eps;
  K.lrwd = (float)(lr * weight_decay);
  K.decay = weight_decay != 0.0;
  K.bc1 = (float)bias_correction1;
  K.bc2 = (float)bias_correction2;
  return for_each_launch(
      ntensors, (void* const*)params, (void* const*)grads, (void* const*)exp_avg,
      (void* const*)exp_avg_sq, (void* const*)max_exp_avg_sq, numel,
      [&](const MtArgs& A, int64_t nb) {
        if (ams)
          k_adam<true><<<(unsigned)nb, kBlock, 0, s>>>(A, K);
        else
          k_adam<false><<<(unsigned)nb, kBlock, 0, s>>>(A, K);
        return tg_check_launch("tg_adam_step");
      });
}

// Multiply every gradient by `mul` (when write != 0) and report non-finite values:
// flags[i] (device int array, cleared here first) gets bit 0 if tensor i held a
// non-finite value on entry and bit 1 if it holds one after scaling.
TG_EXPORT int tg_unscale_check(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                               float mul, int write, int* flags, void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_unscale_check: negative tensor count");
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(grads && numel && flags, "tg_unscale_check: null argument");
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16,
             "tg_unscale_check: unsupported dtype %d", dtype);
  hipStream_t s = tg_stream(stream);
  k_zero_ints<<<1, kBlock, 0, s>>>(flags, ntensors);
  return for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, numel,
                         [&](const MtArgs& A, int64_t nb) {
#define L(T, W) k_scale_check<T, W><<<(unsigned)nb, kBlock, 0, s>>>(A, mul, flags)
                           if (dtype == TG_F32) { if (write) L(float, true); else L(float, false); }
                           else if (dtype == TG_F16) { if (write) L(tg_half, true); else L(tg_half, false); }
                           else { if (write) L(tg_bf16, true); else L(tg_bf16, false); }
#undef L
                           return tg_check_launch("tg_unscale_check");
                         });
}

TG_EXPORT size_t tg_grad_norm_workspace(int ntensors, const int64_t* numel) {
  if (ntensors <= 0 || !numel) return sizeof(double);
  const int64_t b = total_blocks(ntensors, numel);
  return (size_t)(b > 0 ? b : 1) * sizeof(double);
}

// Global norm over all gradients, skipping non-finite entries (equivalent to
// zeroing them first, as clip_grad_norm_ does, _nn.py:1588-1596):
//   norm_kind 0: out[0] = sum g^2;  1: out[0] = max |g|;  2: out[0] = sum |g|^p.
// flags[i] (cleared here) gets bit 0 if tensor i has a non-finite entry.
TG_EXPORT int tg_grad_norm(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                           int norm_kind, float p, double* out, int* flags, void* workspace,
                           size_t workspace_bytes, void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_grad_norm: negative tensor count");
  TG_REQUIRE(out && flags, "tg_grad_norm: null output");
  TG_REQUIRE(norm_kind >= 0 && norm_kind <= 2, "tg_grad_norm: bad norm kind %d", norm_kind);
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16,
             "tg_grad_norm: unsupported dtype %d", dtype);
  hipStream_t s = tg_stream(stream);
  const int64_t nb_total = ntensors > 0 ? total_blocks(ntensors, numel) : 0;
  const size_t need = (size_t)(nb_total > 0 ? nb_total : 1) * sizeof(double);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("tg_grad_norm: workspace of %zu bytes needed", need);
    return TG_ERR_WORKSPACE;
  }
  double* part = (double*)workspace;
  if (ntensors > 0) k_zero_ints<<<1, kBlock, 0, s>>>(flags, ntensors);
  int64_t part_base = 0;
  int st = TG_OK;
  if (ntensors > 0)
    st = for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, numel,
                         [&](const MtArgs& A, int64_t nb) {
#define L(T, K) k_norm_partial<T, K><<<(unsigned)nb, kBlock, 0, s>>>(A, p, part, part_base, flags)
#define LK(T) if (norm_kind == 0) L(T, 0); else if (norm_kind == 1) L(T, 1); else L(T, 2);
                           if (dtype == TG_F32) { LK(float) }
                           else if (dtype == TG_F16) { LK(tg_half) }
                           else { LK(tg_bf16) }
#undef LK
#undef L
                           part_base += nb;
                           return tg_check_launch("tg_grad_norm");
                         });
  if (st) return st;
  if (norm_kind == 1)
    k_norm_final<1><<<1, kBlock, 0, s>>>(part, nb_total, out);
  else
    k_norm_final<0><<<1, kBlock, 0, s>>>(part, nb_total, out);
  return tg_check_launch("tg_grad_norm final");
}

// Replace non-finite gradient entries by zero.
TG_EXPORT int tg_zero_nonfinite(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                                void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_zero_nonfinite: negative tensor count");
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(grads && numel, "tg_zero_nonfinite: null argument");
  hipStream_t s = tg_stream(stream);
  return for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, numel,
                         [&](const MtArgs& A, int64_t nb) {
                           if (dtype == TG_F32) k_zero_nonfinite<float><<<(unsigned)nb, kBlock, 0, s>>>(A);
                           else if (dtype == TG_F16) k_zero_nonfinite<tg_half><<<(unsigned)nb, kBlock, 0, s>>>(A);
                           else if (dtype == TG_BF16) k_zero_nonfinite<tg_bf16><<<(unsigned)nb, kBlock, 0, s>>>(A);
                           else {
                             tg_set_error("tg_zero_nonfinite: unsupported dtype %d", dtype);
                             return (int)TG_ERR_UNSUPPORTED;
                           }
                           return tg_check_launch("tg_zero_nonfinite");
                         });
}
