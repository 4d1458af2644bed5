// Cross-entropy over logits [N, C] with integer targets, reference
// CrossEntropyLoss (_nn.py:1128-1185):
//   p = softmax(x) per row; loss_i = -log(p[t_i] + 1e-10)
//   (label smoothing s: loss_i = -sum_c w_c log(p_c + 1e-10), w = s/C + (1-s) onehot)
//   backward: grad (+)= (p - w) * scale, scale = 1/N for the mean reduction; the
//   reference applies it without the loss's upstream gradient (_nn.py:1168-1180).
//
// One workgroup per row.  The forward streams the row once, each thread keeping an
// online (max, sum of exp) pair over its elements, merged across the workgroup; it
// stores the row's log-sum-exp for the backward, which streams the row once more
// (rows in reverse launch order) and writes the gradient.  Arithmetic is fp32; the
// gradient is rounded to its storage dtype once (for fp16 logits, (p - w)/N below
// fp16's range rounds to zero as in the reference's fp16 arithmetic).  A target in
// [-C, 0) counts from the end (the reference's NumPy indexing); one outside [-C, C)
// yields a NaN loss and an all-(p*scale) gradient row instead of an out-of-bounds
// access.
#include "tg_common.h"

namespace {

__device__ __forceinline__ int64_t wrap_target(int64_t t, int64_t C) { return t < 0 ? t + C : t; }

// 512-thread workgroups (one row each): measured 5 % faster than 256 for the one-pass
// and the two-pass forms at [8192, 32000] fp16 (half the serial work per thread).
constexpr int kBlock = 512;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 2^x by the hardware v_exp_f32 alone.  The arguments are <= 0 (values relative to a
// running maximum); results below the normal range flush to zero, which changes no
// sum of terms relative to a maximum term of 1 and no gradient rounded to fp16.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  s = s * fexp2(m - mn) + s2 * fexp2(m2 - mn);
  m = mn;
}

// Maximum over U 16-byte vectors, as fp32.  fp16 pairs use the packed half
// maximum (exact: the maximum of fp16 values is one of them).
template <typename T, int U>
__device__ __forceinline__ float vec_max(const tg_vec16<T> (&v)[U]) {
  constexpr int V = tg_vec16<T>::N;
  if constexpr (sizeof(T) == 2 && __is_same(T, tg_half)) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 acc = {(tg_half)-INFINITY, (tg_half)-INFINITY};
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < V; j += 2) {
        const h2 p = {v[u].v[j], v[u].v[j + 1]};
        acc = __builtin_elementwise_max(acc, p);
      }
    return fmaxf((float)acc.x, (float)acc.y);
  } else {
    float r = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < V; ++j) r = fmaxf(r, tg_to_float(v[u].v[j]));
    return r;
  }
}

// Online (max, sum) of x*log2e over this thread's elements of a row.
template <typename T, bool VEC>
__device__ __forceinline__ void row_stats(const T* __restrict__ x, int64_t C, float& m,
                                          float& s) {
  m = -INFINITY;
  s = 0.f;
  if (VEC) {
    // U vectors per step, all loads issued before the first is used.  The thread's
    // running maximum m (log2 units) is raised once per step to cover the step's
    // elements (s rescaled by one exp2), then every element costs one fused
    // multiply-add, one exp2 and one add.  Elements past the row end read as -inf.
    constexpr int V = tg_vec16<T>::N, U = 4;
    const int64_t nv = C / V;
    for (int64_t i0 = threadIdx.x; i0 < nv; i0 += U * kBlock) {
      tg_vec16<T> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (i0 + u * kBlock < nv) v[u] = tg_load16(x + (i0 + u * kBlock) * V);
        else
#pragma unroll
          for (int j = 0; j < V; ++j) v[u].v[j] = tg_from_float<T>(-INFINITY);
      }
      const float vm = vec_max<T, U>(v) * kLog2e;
      const float mn = fmaxf(m, vm);
      const float mref = mn == -INFINITY ? 0.f : mn;
      s *= fexp2(m - mref);
      m = mn;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < V; ++j) s += fexp2(fmaf(tg_to_float(v[u].v[j]), kLog2e, -mref));
    }
  } else {
    for (int64_t i = threadIdx.x; i < C; i += kBlock) lse_merge(m, s, tg_to_float(x[i]) * kLog2e, 1.f);
  }
}

// Row log-sum-exp (natural log) over the workgroup; every thread gets it.
__device__ __forceinline__ float block_lse(float m, float s) {
  __shared__ float rm[kBlock / 64], rs[kBlock / 64];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
    lse_merge(m, s, m2, s2);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    rm[wave] = m;
    rs[wave] = s;
  }
  __syncthreads();
  m = rm[0];
  s = rs[0];
#pragma unroll
  for (int w = 1; w < kBlock / 64; ++w) lse_merge(m, s, rm[w], rs[w]);
  __syncthreads();
  return (m + log2f(s)) * kLn2;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void k_ce_fwd(const T* __restrict__ X,
                                                   const int64_t* __restrict__ tgt, int64_t C,
                                                   float smooth, float* __restrict__ lse_out,
                                                   float* __restrict__ loss_out) {
  const int64_t row = blockIdx.x;
  const T* x = X + row * C;
  float m, s;
  row_stats<T, VEC>(x, C, m, s);
  const float lse = block_lse(m, s);
  const int64_t t = wrap_target(tgt[row], C);
  const bool valid = t >= 0 && t < C;
  float sum_log = 0.f;
  if (smooth > 0.f) {
    // sum_c log(p_c + 1e-10): second pass over the row
    for (int64_t i = threadIdx.x; i < C; i += kBlock)
      sum_log += logf(expf(tg_to_float(x[i]) - lse) + 1e-10f);
    float v[1] = {sum_log};
    __shared__ float red[kBlock / 64];
    tg_block_sum<kBlock / 64, 1>(v, red);
    sum_log = v[0];
  }
  if (threadIdx.x == 0) {
    lse_out[row] = lse;
    float loss = NAN;
    if (valid) {
      const float lpt = logf(expf(tg_to_float(x[t]) - lse) + 1e-10f);
      loss = smooth > 0.f ? -((smooth / (float)C) * sum_log + (1.f - smooth) * lpt) : -lpt;
    }
    loss_out[row] = loss;
  }
}

template <typename T, typename TG, bool ACC, bool VEC, bool NTS>
__global__ __launch_bounds__(kBlock) void k_ce_bwd(const T* __restrict__ X,
                                                   const int64_t* __restrict__ tgt,
                                                   const float* __restrict__ lse_in, int64_t C,
                                                   float smooth, float scale, TG* __restrict__ G,
                                                   int rev) {
  // rev: rows in reverse launch order, so the first rows processed are the ones the
  // forward read last (still in the memory-side cache when the backward follows it).
  const int64_t row = rev ? (int64_t)gridDim.x - 1 - blockIdx.x : (int64_t)blockIdx.x;
  const T* x = X + row * C;
  TG* g = G + row * C;
  const float l2 = lse_in[row] * kLog2e;
  const int64_t t = wrap_target(tgt[row], C);
  const float wu = smooth / (float)C;  // weight of every class
  const float wt = 1.f - smooth;       // extra weight of the target
  const float wus = wu * scale, wts = wt * scale;
  if constexpr (VEC) {
    constexpr int V = tg_vec16<T>::N;
    static_assert(sizeof(T) == sizeof(TG), "vector path needs equal element sizes");
    constexpr int U = 4;
    const int64_t nv = C / V;
    // The thread whose vectors hold the target writes its element once more, after its
    // own loop store of it (same thread, same address: the later store wins), with the
    // target weight included; it reads the old value first when accumulating.
    const bool own = t >= 0 && t < C && (t / V) % kBlock == threadIdx.x;
    const float old_t = (ACC && own) ? tg_to_float(g[t]) : 0.f;
    for (int64_t i0 = threadIdx.x; i0 < nv; i0 += U * kBlock) {
      tg_vec16<T> v[U];
      tg_vec16<TG> o[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = i0 + u * kBlock;
        if (i < nv) {
          v[u] = tg_load16(x + i * V);
          if (ACC) o[u] = tg_load16(g + i * V);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = i0 + u * kBlock;
        if (i < nv) {
          // (p - wu)*scale as p*scale - wu*scale; the target element is rewritten below
#pragma unroll
          for (int j = 0; j < V; ++j) {
            float r = fmaf(fexp2(fmaf(tg_to_float(v[u].v[j]), kLog2e, -l2)), scale, -wus);
            if (ACC) r += tg_to_float(o[u].v[j]);
            o[u].v[j] = tg_from_float<TG>(r);
          }
          tg_st16<NTS>(g + i * V, o[u]);
        }
      }
    }
    if (own) {
      float r = fmaf(fexp2(fmaf(tg_to_float(x[t]), kLog2e, -l2)), scale, -wus) - wts;
      if (ACC) r += old_t;
      g[t] = tg_from_float<TG>(r);
    }
  } else {
    for (int64_t c = threadIdx.x; c < C; c += kBlock) {
      const float p = fexp2(fmaf(tg_to_float(x[c]), kLog2e, -l2));
      float r = (p - wu - (c == t ? wt : 0.f)) * scale;
      if (ACC) r += tg_to_float(g[c]);
      g[c] = tg_from_float<TG>(r);
    }
  }
}

// Forward and gradient in one pass (no label smoothing; the gradient does not depend on
// the loss's upstream gradient): the row stays in registers, kFgVec 16-byte vectors per
// thread at vector indices tid + k*kBlock, which the statistics visit in the steps of
// row_stats (4 vectors at a time), so the log-sum-exp, the loss and the gradient are
// bit for bit those of k_ce_fwd followed by k_ce_bwd.  Reads the logits once instead of
// twice.
constexpr int kFgVec = 4096 / kBlock;  // 16-byte vectors per thread: 32768 fp16 classes
template <typename T, bool NTS>
__global__ __launch_bounds__(kBlock) void k_ce_fwd_grad(const T* __restrict__ X,
                                                        const int64_t* __restrict__ tgt,
                                                        int64_t C, float* __restrict__ lse_out,
                                                        float* __restrict__ loss_out, float scale,
                                                        T* __restrict__ G) {
  constexpr int V = tg_vec16<T>::N, U = 4;
  const int64_t row = blockIdx.x;
  const T* x = X + row * C;
  T* g = G + row * C;
  const int nv = (int)(C / V);
  tg_vec16<T> v[kFgVec];
#pragma unroll
  for (int k = 0; k < kFgVec; ++k) {
    const int i = threadIdx.x + k * kBlock;
    if (i < nv) v[k] = tg_ld16<NTS>(x + (int64_t)i * V);  // read once: non-temporal when large
    else
#pragma unroll
      for (int j = 0; j < V; ++j) v[k].v[j] = tg_from_float<T>(-INFINITY);
  }
  float m = -INFINITY, s = 0.f;
#pragma unroll
  for (int k0 = 0; k0 < kFgVec; k0 += U) {
    if (threadIdx.x + k0 * kBlock >= nv) break;  // row_stats stops at the same step
    tg_vec16<T> w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = v[k0 + u];
    const float vm = vec_max<T, U>(w) * kLog2e;
    const float mn = fmaxf(m, vm);
    const float mref = mn == -INFINITY ? 0.f : mn;
    s *= fexp2(m - mref);
    m = mn;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < V; ++j) s += fexp2(fmaf(tg_to_float(w[u].v[j]), kLog2e, -mref));
  }
  const float lse = block_lse(m, s);
  const int64_t t = wrap_target(tgt[row], C);
  const bool valid = t >= 0 && t < C;
  if (threadIdx.x == 0) {
    lse_out[row] = lse;
    loss_out[row] = valid ? -logf(expf(tg_to_float(x[t]) - lse) + 1e-10f) : NAN;
  }
  const float l2 = lse * kLog2e;
#pragma unroll
  for (int k = 0; k < kFgVec; ++k) {
    const int i = threadIdx.x + k * kBlock;
    if (i < nv) {
      tg_vec16<T> o;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        // p*scale rounded, then the target's -scale: the two roundings of k_ce_bwd (not
        // contracted into one fused multiply-add)
#pragma clang fp contract(off)
        float r = fexp2(fmaf(tg_to_float(v[k].v[j]), kLog2e, -l2)) * scale;
        if (valid && (int64_t)i * V + j == t) r -= scale;
        o.v[j] = tg_from_float<T>(r);
      }
      tg_st16<NTS>(g + (int64_t)i * V, o);
    }
  }
}

template <typename T>
int fwd_t(const void* x, const int64_t* tg, int64_t N, int64_t C, float smooth, float* lse,
          float* loss, hipStream_t s) {
  constexpr int V = tg_vec16<T>::N;
  const bool vec = tg_aligned16(x) && C % V == 0;
  if (vec)
    k_ce_fwd<T, true><<<(unsigned)N, kBlock, 0, s>>>((const T*)x, tg, C, smooth, lse, loss);
  else
    k_ce_fwd<T, false><<<(unsigned)N, kBlock, 0, s>>>((const T*)x, tg, C, smooth, lse, loss);
  return tg_check_launch("tg_cross_entropy_fwd");
}

template <typename T, typename TG>
int bwd_t(const void* x, const int64_t* tg, const float* lse, int64_t N, int64_t C, float smooth,
          float scale, void* g, int acc, hipStream_t s) {
  constexpr int V = tg_vec16<T>::N;
  const bool vec = sizeof(T) == sizeof(TG) && tg_aligned16(x) && tg_aligned16(g) && C % V == 0;
  const int rev = 1;
  // a gradient too large to stay cached is written non-temporally (measured: fwd+bwd
  // 0.30 -> 0.27 ms at [8192, 32000] fp16; cached stores were flushed during the next kernel)
  const bool nts = (int64_t)sizeof(TG) * N * C >= (128ll << 20);
#define L(ACC, VEC)                                                                         \
  if (nts) k_ce_bwd<T, TG, ACC, VEC, true><<<(unsigned)N, kBlock, 0, s>>>((const T*)x, tg, lse, C, smooth, scale, (TG*)g, rev); \
  else k_ce_bwd<T, TG, ACC, VEC, false><<<(unsigned)N, kBlock, 0, s>>>((const T*)x, tg, lse, C, smooth, \
                                                           scale, (TG*)g, rev)
  if constexpr (sizeof(T) == sizeof(TG)) {
    if (vec) {
      if (acc) L(true, true);
      else L(false, true);
      return tg_check_launch("tg_cross_entropy_bwd");
    }
  }
  if (acc) L(true, false);
  else L(false, false);
#undef L
  return tg_check_launch("tg_cross_entropy_bwd");
}

int check(int64_t N, int64_t C, float smooth, const char* who) {
  TG_REQUIRE(N >= 0 && C > 0, "%s: bad shape N=%lld C=%lld", who, (long long)N, (long long)C);
  TG_REQUIRE(N <= 0x7fffffff, "%s: N=%lld too large", who, (long long)N);
  TG_REQUIRE(smooth >= 0.f && smooth < 1.f, "%s: label_smoothing %g outside [0, 1)", who,
             (double)smooth);
  return TG_OK;
}

}  // namespace

TG_EXPORT int tg_cross_entropy_fwd(int dtype, const void* logits, const int64_t* targets,
                                   int64_t N, int64_t C, float label_smoothing, float* lse,
                                   float* loss, void* stream) {
  int st = check(N, C, label_smoothing, "tg_cross_entropy_fwd");
  if (st) return st;
  if (N == 0) return TG_OK;
  TG_REQUIRE(logits && targets && lse && loss, "tg_cross_entropy_fwd: null pointer");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: return fwd_t<float>(logits, targets, N, C, label_smoothing, lse, loss, s);
    case TG_F16: return fwd_t<tg_half>(logits, targets, N, C, label_smoothing, lse, loss, s);
    case TG_BF16: return fwd_t<tg_bf16>(logits, targets, N, C, label_smoothing, lse, loss, s);
  }
  tg_set_error("tg_cross_entropy_fwd: unsupported dtype %d (fp64: tg_cross_entropy_fwd_f64)",
               dtype);
  return TG_ERR_UNSUPPORTED;
}

TG_EXPORT int tg_cross_entropy_fwd_grad_max_classes(int dtype) {
  switch (dtype) {
    case TG_F32: return kFgVec * kBlock * tg_vec16<float>::N;
    case TG_F16:
    case TG_BF16: return kFgVec * kBlock * tg_vec16<tg_half>::N;
  }
  return 0;
}

TG_EXPORT int tg_cross_entropy_fwd_grad(int dtype, const void* logits, const int64_t* targets,
                                        int64_t N, int64_t C, float* lse, float* loss,
                                        float scale, void* grad, void* stream) {
  int st = check(N, C, 0.f, "tg_cross_entropy_fwd_grad");
  if (st) return st;
  if (N == 0) return TG_OK;
  TG_REQUIRE(logits && targets && lse && loss && grad, "tg_cross_entropy_fwd_grad: null pointer");
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16,
             "tg_cross_entropy_fwd_grad: unsupported dtype %d", dtype);
  const int V = dtype == TG_F32 ? 4 : 8;
  TG_REQUIRE(C % V == 0 && C <= tg_cross_entropy_fwd_grad_max_classes(dtype) &&
                 tg_aligned16(logits) && tg_aligned16(grad),
             "tg_cross_entropy_fwd_grad: needs 16-byte aligned rows of at most %d classes, "
             "a multiple of %d (C = %lld)",
             tg_cross_entropy_fwd_grad_max_classes(dtype), V, (long long)C);
  hipStream_t s = tg_stream(stream);
  const int64_t esz = dtype == TG_F32 ? 4 : 2;
  const bool nts = esz * N * C >= (128ll << 20);
#define L(T)                                                                                  \
  if (nts) k_ce_fwd_grad<T, true><<<(unsigned)N, kBlock, 0, s>>>((const T*)logits, targets, C, \
                                                                 lse, loss, scale, (T*)grad); \
  else k_ce_fwd_grad<T, false><<<(unsigned)N, kBlock, 0, s>>>((const T*)logits, targets, C,   \
                                                              lse, loss, scale, (T*)grad)
  if (dtype == TG_F32) L(float);
  else if (dtype == TG_F16) L(tg_half);
  else L(tg_bf16);
#undef L
  return tg_check_launch("tg_cross_entropy_fwd_grad");
}

TG_EXPORT int tg_cross_entropy_bwd(int dtype, const void* logits, const int64_t* targets,
                                   const float* lse, int64_t N, int64_t C, float label_smoothing,
                                   float scale, int dtype_grad, void* grad, int accumulate,
                                   void* stream) {
  int st = check(N, C, label_smoothing, "tg_cross_entropy_bwd");
  if (st) return st;
  if (N == 0) return TG_OK;
  TG_REQUIRE(logits && targets && lse && grad, "tg_cross_entropy_bwd: null pointer");
  hipStream_t s = tg_stream(stream);
#define D2(TX)                                                                                 \
  switch (dtype_grad) {                                                                        \
    case TG_F32: return bwd_t<TX, float>(logits, targets, lse, N, C, label_smoothing, scale,   \
                                         grad, accumulate, s);                                 \
    case TG_F16: return bwd_t<TX, tg_half>(logits, targets, lse, N, C, label_smoothing, scale, \
                                           grad, accumulate, s);                               \
    case TG_BF16: return bwd_t<TX, tg_bf16>(logits, targets, lse, N, C, label_smoothing,       \
                                            scale, grad, accumulate, s);                       \
  }                                                                                            \
  break;
  switch (dtype) {
    case TG_F32: D2(float)
    case TG_F16: D2(tg_half)
    case TG_BF16: D2(tg_bf16)
  }
#undef D2
  tg_set_error("tg_cross_entropy_bwd: unsupported dtype combination %d/%d", dtype, dtype_grad);
  return TG_ERR_UNSUPPORTED;
}
