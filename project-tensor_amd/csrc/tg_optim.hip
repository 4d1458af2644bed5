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
constexpr int kMaxT = 56;  // tensors per launch: 68 B each in the kernel argument block (< 4 KiB)
constexpr int kEPT = 16;                     // elements per thread (grad kernels)
constexpr int64_t kChunk = kBlock * kEPT;    // elements per workgroup
// Norm reductions: each workgroup covers kNormSub consecutive chunks (all loads issued
// first), so the single-block final reduction has half the partials.
constexpr int kNormSub = 2;  // measured: 4 no faster, 8 slower (longer final tail)
constexpr int64_t kNormChunk = kNormSub * kChunk;
// Adam streams four inputs and three outputs: two 16-byte vectors per operand and
// thread in 64-thread workgroups, with non-temporal loads and stores (measured 0.73 of
// peak; one vector per thread 0.69, four 0.67, 256-thread workgroups 0.66).
constexpr int kAdamEPT = 8;
constexpr int kAdamBlock = 64;
constexpr int64_t kAdamChunk = kAdamBlock * kAdamEPT;
// Unscale (one stream in, one out): one 16-byte vector per thread.
template <typename T> constexpr int kScaleEPT = 16 / (int)sizeof(T);
template <typename T> constexpr int64_t kScaleChunk = (int64_t)kBlock * kScaleEPT<T>;

struct MtArgs {
  void* a[kMaxT];  // param / grad
  void* b[kMaxT];  // grad (Adam) / unused
  void* c[kMaxT];  // exp_avg
  void* d[kMaxT];  // exp_avg_sq
  void* e[kMaxT];  // max_exp_avg_sq (AMSGrad) or null
  void* f[kMaxT];  // low-precision copy of the updated param (Adam) or null
  int64_t n[kMaxT];
  int first_block[kMaxT + 1];  // entries past the last tensor hold INT32_MAX
  int fidx[kMaxT];  // index of each tensor in the caller's list (flag slot)
  int ntensors;
};

// Largest t with first_block[t] <= blk (binary search; tensors are in block order).
__device__ __forceinline__ int find_tensor(const MtArgs& A, int blk) {
  int lo = 0, hi = A.ntensors - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (A.first_block[mid] <= blk) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Chunk access.  Thread `tid` owns the elements start + (j*kBlock + tid)*PER + k
// (PER elements per 16-byte vector, j < kEPT/PER): every vector instruction of a
// wavefront covers 1 KiB of contiguous memory.  FULL chunks (whole chunk in range,
// 16-byte aligned base) use vector accesses; the others use scalar accesses with
// the same mapping and a bound check.
template <typename T, int EPT = kEPT, int BS = kBlock>
struct ChunkMap {
  static constexpr int PER = 16 / sizeof(T);
  static constexpr int NV = EPT / PER;
  static_assert(NV >= 1, "chunk smaller than one vector");
  __device__ static int64_t at(int64_t start, int j) {
    return start + ((int64_t)j * BS + threadIdx.x) * PER;
  }
};

template <typename T, bool FULL, int EPT = kEPT, bool NT = false, int BS = kBlock>
__device__ __forceinline__ void load_chunk(const T* __restrict__ p, int64_t start, int64_t end,
                                           float (&x)[EPT]) {
  using M = ChunkMap<T, EPT, BS>;
  if (FULL) {
    tg_vec16<T> v[M::NV];
#pragma unroll
    for (int j = 0; j < M::NV; ++j) v[j] = tg_ld16<NT>(p + M::at(start, j));
#pragma unroll
    for (int j = 0; j < M::NV; ++j)
#pragma unroll
      for (int k = 0; k < M::PER; ++k) x[j * M::PER + k] = tg_to_float(v[j].v[k]);
  } else {
#pragma unroll
    for (int j = 0; j < M::NV; ++j)
#pragma unroll
      for (int k = 0; k < M::PER; ++k) {
        const int64_t i = M::at(start, j) + k;
        x[j * M::PER + k] = i < end ? tg_to_float(p[i]) : 0.f;
      }
  }
}

template <typename T, bool FULL, int EPT = kEPT, bool NT = false, int BS = kBlock>
__device__ __forceinline__ void store_chunk(T* __restrict__ p, int64_t start, int64_t end,
                                            const float (&x)[EPT]) {
  using M = ChunkMap<T, EPT, BS>;
#pragma unroll
  for (int j = 0; j < M::NV; ++j) {
    if (FULL) {
      tg_vec16<T> v;
#pragma unroll
      for (int k = 0; k < M::PER; ++k) v.v[k] = tg_from_float<T>(x[j * M::PER + k]);
      tg_st16<NT>(p + M::at(start, j), v);
    } else {
#pragma unroll
      for (int k = 0; k < M::PER; ++k) {
        const int64_t i = M::at(start, j) + k;
        if (i < end) p[i] = tg_from_float<T>(x[j * M::PER + k]);
      }
    }
  }
}

__device__ __forceinline__ bool al16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// ---------------------------------------------------------------------------
// Adam/AdamW, reference order (_nn.py:1413-1442, _training.py:2198-2220):
//   p -= lr*wd*p (if wd != 0); m = b1*m + (1-b1)*g; v = b2*v + (1-b2)*g^2;
//   mhat = m/bc1; vhat = v/bc2; [vmax = max(vmax, vhat)]; p -= lr*mhat/(sqrt(v*)+eps)
// The divisions by the bias corrections are multiplications by their reciprocals
// (formed in double on the host) and the last one a reciprocal of the denominator:
// each differs from the division by at most one rounding.
// gm1, gm2: the gradient is read as (g * gm1) * gm2, two fp32 roundings, the values
// that scaling the gradient in place by gm1 and then by gm2 would leave (1, 1: g).
struct AdamConsts {
  float lr, b1, omb1, b2, omb2, eps, lrwd, ibc1, ibc2, gm1, gm2;
  int decay;
};

// The E fp32 elements a thread owns in an Adam chunk (ChunkMap<float, E, kAdamBlock>:
// groups of 4 at start + 4*(j*kAdamBlock + tid)), stored as low-precision values: one
// 8-byte store per group when FULL.
template <typename TL, bool FULL, int E>
__device__ __forceinline__ void store_lowp(TL* __restrict__ p, int64_t start, int64_t end,
                                           const float (&x)[E]) {
#pragma unroll
  for (int j = 0; j < E / 4; ++j) {
    const int64_t i0 = start + ((int64_t)j * kAdamBlock + threadIdx.x) * 4;
    if (FULL) {
      TL v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = tg_from_float<TL>(x[4 * j + k]);
      *reinterpret_cast<uint2*>(p + i0) = *reinterpret_cast<const uint2*>(v);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (i0 + k < end) p[i0 + k] = tg_from_float<TL>(x[4 * j + k]);
    }
  }
}

// LP: 0 = no low-precision copy, 1 = fp16 copy, 2 = bf16 copy of the updated param
// (written in the same pass, so the next autocast forward needs no cast launch).
template <bool AMS, bool FULL, int LP = 0>
__device__ __forceinline__ void adam_chunk(float* __restrict__ p, const float* __restrict__ g,
                                           float* __restrict__ m, float* __restrict__ v,
                                           float* __restrict__ vm, void* __restrict__ lp,
                                           int64_t start, int64_t end, const AdamConsts& K) {
  constexpr int E = kAdamEPT;
  float P[E], G[E], Mv[E], Vv[E], VM[E];
  load_chunk<float, FULL, E, true, kAdamBlock>(p, start, end, P);
  load_chunk<float, FULL, E, true, kAdamBlock>(g, start, end, G);
  load_chunk<float, FULL, E, true, kAdamBlock>(m, start, end, Mv);
  load_chunk<float, FULL, E, true, kAdamBlock>(v, start, end, Vv);
  if (AMS) load_chunk<float, FULL, E, true, kAdamBlock>(vm, start, end, VM);
#pragma unroll
  for (int i = 0; i < E; ++i) {
    float pp = P[i];
    if (K.decay) pp -= K.lrwd * pp;
    const float gg = (G[i] * K.gm1) * K.gm2;
    const float mm = K.b1 * Mv[i] + K.omb1 * gg;
    const float vv = K.b2 * Vv[i] + K.omb2 * (gg * gg);
    const float mh = mm * K.ibc1;
    float vh = vv * K.ibc2;
    if (AMS) {
      vh = fmaxf(VM[i], vh);
      VM[i] = vh;
    }
    pp -= K.lr * mh * __frcp_rn(sqrtf(vh) + K.eps);
    P[i] = pp;
    Mv[i] = mm;
    Vv[i] = vv;
  }
  store_chunk<float, FULL, E, true, kAdamBlock>(p, start, end, P);
  if (LP == 1 && lp) store_lowp<tg_half, FULL, E>((tg_half*)lp, start, end, P);
  if (LP == 2 && lp) store_lowp<tg_bf16, FULL, E>((tg_bf16*)lp, start, end, P);
  store_chunk<float, FULL, E, true, kAdamBlock>(m, start, end, Mv);
  store_chunk<float, FULL, E, true, kAdamBlock>(v, start, end, Vv);
  if (AMS) store_chunk<float, FULL, E, true, kAdamBlock>(vm, start, end, VM);
}

template <bool AMS, int LP = 0>
__global__ __launch_bounds__(kAdamBlock) void k_adam(MtArgs A, AdamConsts K) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t start = (blockIdx.x - A.first_block[t]) * kAdamChunk;
  const int64_t end = start + kAdamChunk < n ? start + kAdamChunk : n;
  float* p = (float*)A.a[t];
  const float* g = (const float*)A.b[t];
  float* m = (float*)A.c[t];
  float* v = (float*)A.d[t];
  float* vm = (float*)A.e[t];
  void* lp = LP ? A.f[t] : nullptr;
  const bool full = start + kAdamChunk <= n && al16(p) && al16(g) && al16(m) && al16(v) &&
                    (!AMS || al16(vm)) && (reinterpret_cast<uintptr_t>(lp) & 7) == 0;
  if (full) adam_chunk<AMS, true, LP>(p, g, m, v, vm, lp, start, end, K);
  else adam_chunk<AMS, false, LP>(p, g, m, v, vm, lp, start, end, K);
}

// ---------------------------------------------------------------------------
// g' = g*mul (stored if WRITE).  flags[t] |= 1 if any g is non-finite,
// |= 2 if any g' is non-finite (GradScaler.unscale_, _nn.py:1795-1833).
template <typename T, bool WRITE, bool FULL>
__device__ __forceinline__ int scale_check_chunk(T* __restrict__ g, int64_t start, int64_t end,
                                                 float mul) {
  constexpr int E = kScaleEPT<T>;
  float x[E], y[E];
  load_chunk<T, FULL, E, true>(g, start, end, x);
  int f = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    if (!isfinite(x[i])) f |= 1;
    // round through T so the post-check sees what is stored
    y[i] = tg_to_float(tg_from_float<T>(x[i] * mul));
    if (!isfinite(y[i])) f |= 2;
  }
  if (WRITE) store_chunk<T, FULL, E, true>(g, start, end, y);
  return f;
}

template <typename T, bool WRITE>
__global__ __launch_bounds__(kBlock) void k_scale_check(MtArgs A, float mul, int* flags) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  constexpr int64_t CH = kScaleChunk<T>;
  const int64_t start = (blockIdx.x - A.first_block[t]) * CH;
  const int64_t end = start + CH < n ? start + CH : n;
  T* g = (T*)A.a[t];
  int f = (start + CH <= n && al16(g)) ? scale_check_chunk<T, WRITE, true>(g, start, end, mul)
                                           : scale_check_chunk<T, WRITE, false>(g, start, end, mul);
  // wave-level OR, then one atomic per wave that found something
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) f |= __shfl_xor(f, off, 64);
  if ((threadIdx.x & 63) == 0 && f) atomicOr(flags + A.fidx[t], f);
}

// The kNormSub chunks of a norm workgroup from element `base` of a tensor of n
// elements, every load issued before any is used (entries past n read as 0).
template <typename T>
__device__ __forceinline__ void load_norm_chunks(const T* __restrict__ g, int64_t base,
                                                 int64_t n, float (&x)[kNormSub][kEPT]) {
#pragma unroll
  for (int c = 0; c < kNormSub; ++c) {
    const int64_t start = base + c * kChunk;
    const int64_t end = start + kChunk < n ? start + kChunk : n;
    if (start + kChunk <= n && al16(g)) {
      load_chunk<T, true, kEPT, true>(g, start, end, x[c]);
    } else if (start < n) {
      load_chunk<T, false>(g, start, end, x[c]);
    } else {
#pragma unroll
      for (int i = 0; i < kEPT; ++i) x[c][i] = 0.f;
    }
  }
}

// Per-block partial of the gradient norm over finite entries (kNormChunk elements).
// KIND 0: sum g^2, 1: max |g|, 2: sum |g|^p.  Non-finite entries set flags bit 1.
template <typename T, int KIND>
__global__ __launch_bounds__(kBlock) void k_norm_partial(MtArgs A, float p, double* part,
                                                         int64_t part_base, int* flags) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t base = (blockIdx.x - A.first_block[t]) * kNormChunk;
  const T* g = (const T*)A.a[t];
  float x[kNormSub][kEPT];
  load_norm_chunks<T>(g, base, n, x);
  double acc = 0.0;
  int f = 0;
  using M = ChunkMap<T>;
#pragma unroll
  for (int c = 0; c < kNormSub; ++c) {
    const int64_t start = base + c * kChunk;
    const int64_t end = start + kChunk < n ? start + kChunk : n;
#pragma unroll
    for (int i = 0; i < kEPT; ++i) {
      if (M::at(start, i / M::PER) + i % M::PER >= end) continue;  // past the tensor's end
      if (!isfinite(x[c][i])) {
        f = 1;
        continue;
      }
      const float ax = fabsf(x[c][i]);
      if (KIND == 0) acc += (double)ax * (double)ax;
      else if (KIND == 1) acc = fmax(acc, (double)ax);
      else acc += pow((double)ax, (double)p);
    }
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

// GradScaler.unscale_ followed by the squared gradient norm, read-only: flags as
// k_scale_check's (bit 0: g non-finite, bit 1: g*mul rounded through T non-finite)
// and the per-block partial sum of (g*mul)^2 over finite entries, with k_norm_partial's
// chunking and order (the value it would give after the in-place unscale); tidx[b]
// is the caller's index of block b's tensor, for the masked final reduction.
template <typename T, bool BFLAG>
__global__ __launch_bounds__(kBlock) void k_unscale_norm_partial(MtArgs A, float mul,
                                                                 double* part, int* tidx,
                                                                 int64_t part_base, int* flags,
                                                                 int* bflag) {
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t base = (blockIdx.x - A.first_block[t]) * kNormChunk;
  const T* g = (const T*)A.a[t];
  float x[kNormSub][kEPT];
  load_norm_chunks<T>(g, base, n, x);
  double acc = 0.0;
  int f = 0;
  using M = ChunkMap<T>;
#pragma unroll
  for (int c = 0; c < kNormSub; ++c) {
    const int64_t start = base + c * kChunk;
    const int64_t end = start + kChunk < n ? start + kChunk : n;
#pragma unroll
    for (int i = 0; i < kEPT; ++i) {
      if (M::at(start, i / M::PER) + i % M::PER >= end) continue;  // past the tensor's end
      if (!isfinite(x[c][i])) f |= 1;
      const float y = tg_to_float(tg_from_float<T>(x[c][i] * mul));
      if (!isfinite(y)) {
        f |= 2;
        continue;
      }
      const float ay = fabsf(y);
      acc += (double)ay * (double)ay;
    }
  }
  __shared__ double red[4];
  __shared__ int redf[4];
  acc = tg_wave_sum_d(acc);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) f |= __shfl_xor(f, off, 64);
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = acc;
    redf[threadIdx.x >> 6] = f;
    if (!BFLAG && f) atomicOr(flags + A.fidx[t], f);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    part[part_base + blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
    tidx[part_base + blockIdx.x] = A.fidx[t];
    if (BFLAG) bflag[part_base + blockIdx.x] = (redf[0] | redf[1]) | (redf[2] | redf[3]);
  }
}

// Deterministic single-block reduction of the partials: 1024 threads, each with
// kNF independent accumulators over a fixed stride (kNF loads in flight instead of
// one dependent chain), then a fixed-order tree.
constexpr int kNormFinal = 1024;
constexpr int kNF = 8;
// With tidx (k_unscale_norm_partial): a partial whose tensor is flagged counts as 0,
// the value it has once unscale_ has zeroed that tensor.  The flags of up to kFlagLds
// tensors live in LDS, so the mask is not a second dependent global load; with bflag
// (per-block flags of the partial kernel) they are also formed here, OR-ed per tensor
// in LDS and written to flags[] (no clearing launch, no global atomics).  Each thread
// sums kNF strided partials per round with every load issued first, the kNF sums are
// combined in a fixed tree, then within the wavefront (xor butterfly) and across the
// 16 wavefronts in order: deterministic.
constexpr int kFlagLds = 8192;
template <int KIND>
__global__ __launch_bounds__(kNormFinal) void k_norm_final(const double* part, int64_t n,
                                                           double* out,
                                                           const int* tidx = nullptr,
                                                           int* flags = nullptr,
                                                           int ntensors = 0,
                                                           const int* bflag = nullptr) {
  auto comb = [](double a, double b) { return KIND == 1 ? fmax(a, b) : a + b; };
  __shared__ int fl[kFlagLds];
  __shared__ double red[kNormFinal / 64];
  const bool lds = tidx && ntensors <= kFlagLds;
  if (lds) {
    if (bflag) {
      for (int i = threadIdx.x; i < ntensors; i += kNormFinal) fl[i] = 0;
      __syncthreads();
      for (int64_t b0 = threadIdx.x; b0 < n; b0 += (int64_t)kNormFinal * kNF) {
        int f[kNF];
#pragma unroll
        for (int u = 0; u < kNF; ++u) {
          const int64_t b = b0 + (int64_t)u * kNormFinal;
          f[u] = b < n ? bflag[b] : 0;
        }
#pragma unroll
        for (int u = 0; u < kNF; ++u)
          if (f[u]) atomicOr(&fl[tidx[b0 + (int64_t)u * kNormFinal]], f[u]);
      }
      __syncthreads();
      for (int i = threadIdx.x; i < ntensors; i += kNormFinal) flags[i] = fl[i];
    } else {
      for (int i = threadIdx.x; i < ntensors; i += kNormFinal) fl[i] = flags[i];
      __syncthreads();
    }
  }
  double acc[kNF];
#pragma unroll
  for (int u = 0; u < kNF; ++u) acc[u] = 0.0;
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += (int64_t)kNormFinal * kNF) {
    double v[kNF];
    int ti[kNF];
#pragma unroll
    for (int u = 0; u < kNF; ++u) {
      const int64_t i = i0 + (int64_t)u * kNormFinal;
      const bool ok = i < n;
      v[u] = ok ? part[i] : 0.0;
      ti[u] = (tidx && ok) ? tidx[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < kNF; ++u) {
      const bool masked = ti[u] >= 0 && (lds ? fl[ti[u]] : flags[ti[u]]);
      acc[u] = comb(acc[u], masked ? 0.0 : v[u]);
    }
  }
#pragma unroll
  for (int w = kNF / 2; w >= 1; w /= 2)
#pragma unroll
    for (int u = 0; u < w; ++u) acc[u] = comb(acc[u], acc[u + w]);
  double a = acc[0];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) a = comb(a, __shfl_xor(a, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) {
    double r = red[0];
#pragma unroll
    for (int w = 1; w < kNormFinal / 64; ++w) r = comb(r, red[w]);
    out[0] = r;
  }
}

// Non-finite entries become zero; a 16-byte vector is written back only if it held one.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_zero_nonfinite(MtArgs A) {
  using M = ChunkMap<T>;
  const int t = find_tensor(A, blockIdx.x);
  const int64_t n = A.n[t];
  const int64_t start = (blockIdx.x - A.first_block[t]) * kChunk;
  const int64_t end = start + kChunk < n ? start + kChunk : n;
  T* __restrict__ g = (T*)A.a[t];
  if (start + kChunk <= n && al16(g)) {
    tg_vec16<T> v[M::NV];
#pragma unroll
    for (int j = 0; j < M::NV; ++j) v[j] = tg_load16(g + M::at(start, j));
#pragma unroll
    for (int j = 0; j < M::NV; ++j) {
      bool bad = false;
#pragma unroll
      for (int k = 0; k < M::PER; ++k)
        if (!isfinite(tg_to_float(v[j].v[k]))) {
          v[j].v[k] = tg_from_float<T>(0.f);
          bad = true;
        }
      if (bad) tg_store16(g + M::at(start, j), v[j]);
    }
  } else {
    for (int64_t i = start + threadIdx.x; i < end; i += kBlock)
      if (!isfinite(tg_to_float(g[i]))) g[i] = tg_from_float<T>(0.f);
  }
}

// Every tensor whose flag is set is zeroed whole (GradScaler.unscale_ clearing a
// gradient that holds a non-finite value).  The flags are read once per block into
// LDS; with none set every block exits after that read.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_zero_flagged(MtArgs A, const int* __restrict__ flags) {
  __shared__ int fl[kMaxT];
  if (threadIdx.x < A.ntensors) fl[threadIdx.x] = flags[A.fidx[threadIdx.x]];
  __syncthreads();
  T z;
  if constexpr (sizeof(T) == 8) z = 0.0;
  else z = tg_from_float<T>(0.f);
  for (int t = 0; t < A.ntensors; ++t) {
    if (fl[t] == 0) continue;
    T* __restrict__ g = (T*)A.a[t];
    const int64_t n = A.n[t];
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock)
      g[i] = z;
  }
}

__global__ void k_zero_ints(int* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

// Split a tensor list into launches of at most kMaxT tensors; calls fn(args, nblocks,
// first tensor index) per launch.  Empty tensors are skipped.
template <typename F>
int for_each_launch(int ntensors, void* const* a, void* const* b, void* const* c,
                    void* const* d, void* const* e, void* const* f, const int64_t* numel,
                    F&& fn, int64_t chunk = kChunk) {
  MtArgs A{};
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (A.ntensors > 0) {
      for (int i = A.ntensors; i <= kMaxT; ++i) A.first_block[i] = 0x7fffffff;
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
    if (blocks + (numel[i] + chunk - 1) / chunk > 0x7fffffff) {
      tg_set_error("multi-tensor launch: too many blocks");
      return TG_ERR_INVALID;
    }
    const int k = A.ntensors++;
    A.a[k] = a ? a[i] : nullptr;
    A.b[k] = b ? b[i] : nullptr;
    A.c[k] = c ? c[i] : nullptr;
    A.d[k] = d ? d[i] : nullptr;
    A.e[k] = e ? e[i] : nullptr;
    A.f[k] = f ? f[i] : nullptr;
    A.n[k] = numel[i];
    A.fidx[k] = i;
    A.first_block[k] = (int)blocks;
    blocks += (numel[i] + chunk - 1) / chunk;
  }
  return flush();
}

int64_t total_blocks(int ntensors, const int64_t* numel, int64_t chunk = kChunk) {
  int64_t b = 0;
  for (int i = 0; i < ntensors; ++i)
    if (numel[i] > 0) b += (numel[i] + chunk - 1) / chunk;
  return b;
}

}  // namespace

namespace {

int adam_step_impl(const char* who, int ntensors, float* const* params,
                   const float* const* grads, float* const* exp_avg, float* const* exp_avg_sq,
                   float* const* max_exp_avg_sq, const int64_t* numel, double lr, double beta1,
                   double beta2, double eps, double weight_decay, double bias_correction1,
                   double bias_correction2, float gm1, float gm2, int lowp_dtype,
                   void* const* lowp, void* stream) {
  TG_REQUIRE(ntensors >= 0, "%s: negative tensor count", who);
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(params && grads && exp_avg && exp_avg_sq && numel, "%s: null list", who);
  for (int i = 0; i < ntensors; ++i)
    TG_REQUIRE(numel[i] == 0 || (params[i] && grads[i] && exp_avg[i] && exp_avg_sq[i] &&
                                 (!max_exp_avg_sq || max_exp_avg_sq[i])),
               "%s: null pointer for tensor %d", who, i);
  int lp = 0;
  if (lowp) {
    TG_REQUIRE(lowp_dtype == TG_F16 || lowp_dtype == TG_BF16,
               "%s: low-precision copies must be float16 or bfloat16 (dtype %d)", who,
               lowp_dtype);
    lp = lowp_dtype == TG_F16 ? 1 : 2;
  }
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
  K.ibc1 = (float)(1.0 / bias_correction1);
  K.ibc2 = (float)(1.0 / bias_correction2);
  K.gm1 = gm1;
  K.gm2 = gm2;
  return for_each_launch(
      ntensors, (void* const*)params, (void* const*)grads, (void* const*)exp_avg,
      (void* const*)exp_avg_sq, (void* const*)max_exp_avg_sq, lowp, numel,
      [&](const MtArgs& A, int64_t nb) {
#define L(AMS, LP) k_adam<AMS, LP><<<(unsigned)nb, kAdamBlock, 0, s>>>(A, K)
        if (ams) {
          if (lp == 1) L(true, 1); else if (lp == 2) L(true, 2); else L(true, 0);
        } else {
          if (lp == 1) L(false, 1); else if (lp == 2) L(false, 2); else L(false, 0);
        }
#undef L
        return tg_check_launch(who);
      },
      kAdamChunk);
}

}  // namespace

TG_EXPORT int tg_adam_step(int ntensors, float* const* params, const float* const* grads,
                           float* const* exp_avg, float* const* exp_avg_sq,
                           float* const* max_exp_avg_sq, const int64_t* numel, double lr,
                           double beta1, double beta2, double eps, double weight_decay,
                           double bias_correction1, double bias_correction2, void* stream) {
  return adam_step_impl("tg_adam_step", ntensors, params, grads, exp_avg, exp_avg_sq,
                        max_exp_avg_sq, numel, lr, beta1, beta2, eps, weight_decay,
                        bias_correction1, bias_correction2, 1.f, 1.f, 0, nullptr, stream);
}

// tg_adam_step that also writes each updated parameter, rounded to `lowp_dtype`
// (fp16 or bf16), to lowp[i] when lowp[i] is not null: the autocast copy of the
// weights refreshed in the same pass (2 B/param more written, no separate cast).
TG_EXPORT int tg_adam_step_lowp(int ntensors, float* const* params, const float* const* grads,
                                float* const* exp_avg, float* const* exp_avg_sq,
                                float* const* max_exp_avg_sq, const int64_t* numel, double lr,
                                double beta1, double beta2, double eps, double weight_decay,
                                double bias_correction1, double bias_correction2,
                                int lowp_dtype, void* const* lowp, void* stream) {
  TG_REQUIRE(lowp, "tg_adam_step_lowp: null copy list");
  return adam_step_impl("tg_adam_step_lowp", ntensors, params, grads, exp_avg, exp_avg_sq,
                        max_exp_avg_sq, numel, lr, beta1, beta2, eps, weight_decay,
                        bias_correction1, bias_correction2, 1.f, 1.f, lowp_dtype, lowp, stream);
}

// tg_adam_step(_lowp) reading each gradient as (g * grad_mul1) * grad_mul2: the gradients
// still hold the loss-scaled values, and the unscale factor and the clip factor are
// applied here, in the order and with the roundings of two in-place scalings.
TG_EXPORT int tg_adam_step_scaled(int ntensors, float* const* params, const float* const* grads,
                                  float* const* exp_avg, float* const* exp_avg_sq,
                                  float* const* max_exp_avg_sq, const int64_t* numel,
                                  double lr, double beta1, double beta2, double eps,
                                  double weight_decay, double bias_correction1,
                                  double bias_correction2, float grad_mul1, float grad_mul2,
                                  int lowp_dtype, void* const* lowp, void* stream) {
  return adam_step_impl("tg_adam_step_scaled", ntensors, params, grads, exp_avg, exp_avg_sq,
                        max_exp_avg_sq, numel, lr, beta1, beta2, eps, weight_decay,
                        bias_correction1, bias_correction2, grad_mul1, grad_mul2, lowp_dtype,
                        lowp, stream);
}

// Multiply every gradient by `mul` (when write != 0) and report non-finite values:
// flags[i] (device int array, cleared here first) gets bit 0 if tensor i held a
// non-finite value on entry and bit 1 if it holds one after scaling.
TG_EXPORT int tg_unscale_check(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                               float mul, int write, int* flags, void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_unscale_check: negative tensor count");
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(grads && numel && flags, "tg_unscale_check: null argument");
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16 || dtype == TG_F64,
             "tg_unscale_check: unsupported dtype %d", dtype);
  hipStream_t s = tg_stream(stream);
  if (dtype == TG_F64) return tg64_unscale_check(ntensors, grads, numel, mul, write, flags, s);
  k_zero_ints<<<1, kBlock, 0, s>>>(flags, ntensors);
  return for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, nullptr, numel,
                         [&](const MtArgs& A, int64_t nb) {
#define L(T, W) k_scale_check<T, W><<<(unsigned)nb, kBlock, 0, s>>>(A, mul, flags)
                           if (dtype == TG_F32) { if (write) L(float, true); else L(float, false); }
                           else if (dtype == TG_F16) { if (write) L(tg_half, true); else L(tg_half, false); }
                           else { if (write) L(tg_bf16, true); else L(tg_bf16, false); }
#undef L
                           return tg_check_launch("tg_unscale_check");
                         },
                         dtype == TG_F32 ? kScaleChunk<float> : kScaleChunk<tg_half>);
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
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16 || dtype == TG_F64,
             "tg_grad_norm: unsupported dtype %d", dtype);
  hipStream_t s = tg_stream(stream);
  const int64_t nb_total = ntensors > 0 ? total_blocks(ntensors, numel) : 0;
  const size_t need = (size_t)(nb_total > 0 ? nb_total : 1) * sizeof(double);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("tg_grad_norm: workspace of %zu bytes needed", need);
    return TG_ERR_WORKSPACE;
  }
  double* part = (double*)workspace;
  if (dtype == TG_F64)  // one partial per kChunk elements, as the workspace counts them
    return tg64_grad_norm(ntensors, grads, numel, norm_kind, p, kChunk, out, flags, part, s);
  if (ntensors > 0) k_zero_ints<<<1, kBlock, 0, s>>>(flags, ntensors);
  // (the workspace counts kChunk partials, at least the kNormChunk ones used here)
  const int64_t nparts = ntensors > 0 ? total_blocks(ntensors, numel, kNormChunk) : 0;
  int64_t part_base = 0;
  int st = TG_OK;
  if (ntensors > 0)
    st = for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, nullptr, numel,
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
                         },
                         kNormChunk);
  if (st) return st;
  if (norm_kind == 1)
    k_norm_final<1><<<1, kNormFinal, 0, s>>>(part, nparts, out);
  else
    k_norm_final<0><<<1, kNormFinal, 0, s>>>(part, nparts, out);
  return tg_check_launch("tg_grad_norm final");
}

TG_EXPORT size_t tg_unscale_norm_workspace(int ntensors, const int64_t* numel) {
  if (ntensors <= 0 || !numel) return 2 * sizeof(double);
  const int64_t b = total_blocks(ntensors, numel, kNormChunk);
  return (size_t)(b > 0 ? b : 1) * (sizeof(double) + 2 * sizeof(int)) + sizeof(double);
}

// Read-only form of GradScaler.unscale_ plus clip_grad_norm_'s reduction: flags[i]
// (cleared here) as tg_unscale_check's, and out[0] = the squared L2 norm the gradients
// would have after tg_unscale_check(mul, write) and tg_zero_flagged, bit for bit (the
// same chunks and order as tg_grad_norm, flagged tensors counting zero).  fp32, fp16,
// bf16.
TG_EXPORT int tg_unscale_norm(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                              float mul, int* flags, double* out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_unscale_norm: negative tensor count");
  TG_REQUIRE(out && flags, "tg_unscale_norm: null output");
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16,
             "tg_unscale_norm: unsupported dtype %d", dtype);
  TG_REQUIRE(ntensors == 0 || (grads && numel), "tg_unscale_norm: null argument");
  hipStream_t s = tg_stream(stream);
  const int64_t nb_total = ntensors > 0 ? total_blocks(ntensors, numel, kNormChunk) : 0;
  const size_t need = tg_unscale_norm_workspace(ntensors, numel);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("tg_unscale_norm: workspace of %zu bytes needed", need);
    return TG_ERR_WORKSPACE;
  }
  double* part = (double*)workspace;
  int* tidx = (int*)(part + (nb_total > 0 ? nb_total : 1));
  int* bflag = tidx + (nb_total > 0 ? nb_total : 1);
  // up to kFlagLds tensors: per-block flags OR-ed by the final kernel; beyond that,
  // cleared flags and per-wavefront atomics
  const bool bf = ntensors <= kFlagLds;
  if (ntensors > 0 && !bf) k_zero_ints<<<1, kBlock, 0, s>>>(flags, ntensors);
  int64_t part_base = 0;
  int st = TG_OK;
  if (ntensors > 0)
    st = for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, nullptr, numel,
                         [&](const MtArgs& A, int64_t nb) {
#define L(T, B) k_unscale_norm_partial<T, B><<<(unsigned)nb, kBlock, 0, s>>>(A, mul, part, tidx, part_base, flags, bflag)
#define LB(T) if (bf) L(T, true); else L(T, false)
                           if (dtype == TG_F32) LB(float);
                           else if (dtype == TG_F16) LB(tg_half);
                           else LB(tg_bf16);
#undef LB
#undef L
                           part_base += nb;
                           return tg_check_launch("tg_unscale_norm");
                         },
                         kNormChunk);
  if (st) return st;
  k_norm_final<0><<<1, kNormFinal, 0, s>>>(part, nb_total, out, tidx, flags, ntensors,
                                           bf ? bflag : nullptr);
  return tg_check_launch("tg_unscale_norm final");
}

// Zero every gradient i whose device flag flags[i] is non-zero (as set by
// tg_unscale_check), without a read-back.
TG_EXPORT int tg_zero_flagged(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                              const int* flags, void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_zero_flagged: negative tensor count");
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(grads && numel && flags, "tg_zero_flagged: null argument");
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16 || dtype == TG_F64,
             "tg_zero_flagged: unsupported dtype %d", dtype);
  hipStream_t s = tg_stream(stream);
  const unsigned grid = (unsigned)tg_num_cus();
  return for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, nullptr, numel,
                         [&](const MtArgs& A, int64_t) {
                           if (dtype == TG_F32) k_zero_flagged<float><<<grid, kBlock, 0, s>>>(A, flags);
                           else if (dtype == TG_F16) k_zero_flagged<tg_half><<<grid, kBlock, 0, s>>>(A, flags);
                           else if (dtype == TG_BF16) k_zero_flagged<tg_bf16><<<grid, kBlock, 0, s>>>(A, flags);
                           else k_zero_flagged<double><<<grid, kBlock, 0, s>>>(A, flags);
                           return tg_check_launch("tg_zero_flagged");
                         });
}

// Replace non-finite gradient entries by zero.
TG_EXPORT int tg_zero_nonfinite(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                                void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_zero_nonfinite: negative tensor count");
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(grads && numel, "tg_zero_nonfinite: null argument");
  hipStream_t s = tg_stream(stream);
  if (dtype == TG_F64) return tg64_zero_nonfinite(ntensors, grads, numel, s);
  return for_each_launch(ntensors, grads, nullptr, nullptr, nullptr, nullptr, nullptr, numel,
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
