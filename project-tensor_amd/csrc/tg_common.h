// Shared device helpers and host-side error plumbing for libtgbwd (gfx950 only).
//
// Every exported entry point returns an int status (TG_OK = 0, negative on error)
// and records a message retrievable with tg_last_error().  Kernels are launched
// asynchronously on the caller's stream; the library never synchronises except
// where an entry point documents a device->host result.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "tgbwd.h"

#define TG_EXPORT extern "C" __attribute__((visibility("default")))

enum tg_status {
  TG_OK = 0,
  TG_ERR_INVALID = -1,   // bad argument (shape, pointer, dtype)
  TG_ERR_HIP = -2,       // HIP runtime / launch error
  TG_ERR_UNSUPPORTED = -3,
  TG_ERR_WORKSPACE = -4, // workspace missing or too small
};

enum tg_dtype { TG_F32 = 0, TG_F16 = 1, TG_BF16 = 2, TG_F64 = 3 };

typedef _Float16 tg_half;
typedef __bf16 tg_bf16;

// ---- host-side error handling (defined in tg_runtime.hip) ----
void tg_set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int tg_check_launch(const char* what);

#define TG_REQUIRE(cond, ...)            \
  do {                                   \
    if (!(cond)) {                       \
      tg_set_error(__VA_ARGS__);         \
      return TG_ERR_INVALID;             \
    }                                    \
  } while (0)

static inline hipStream_t tg_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

static inline bool tg_aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

static inline int tg_dtype_size(int dt) {
  switch (dt) {
    case TG_F32: return 4;
    case TG_F16: return 2;
    case TG_BF16: return 2;
    case TG_F64: return 8;
    default: return 0;
  }
}

// ---- device helpers ----
__device__ __forceinline__ float tg_to_float(float v) { return v; }
__device__ __forceinline__ float tg_to_float(tg_half v) { return (float)v; }
__device__ __forceinline__ float tg_to_float(tg_bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T tg_from_float(float v);
template <> __device__ __forceinline__ float tg_from_float<float>(float v) { return v; }
template <> __device__ __forceinline__ tg_half tg_from_float<tg_half>(float v) { return (tg_half)v; }
template <> __device__ __forceinline__ tg_bf16 tg_from_float<tg_bf16>(float v) { return (tg_bf16)v; }

// v materialised as an fp32 value: the compiler cannot merge the operation that made
// it with a following conversion (e.g. an FMA and the fp32 -> fp16 rounding into one
// single-rounding mixed-precision instruction), so kernels that compute the same value
// and then round it round identically.
__device__ __forceinline__ float tg_f32(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// tanh-approx GELU derivative, reference formula (_core.py:493-507):
//   u = c0*(x + c1*x^3), t = tanh(u)
//   g = 0.5*(1+t) + 0.5*x*(1-t^2)*c0*(1+3*c1*x^2)
// tanh is evaluated from e = exp(-2|u|) in (0,1] so that neither (1+t) nor
// (1-t^2) = sech^2(u) loses precision to cancellation.
// Both functions evaluate without FMA contraction, so every kernel that inlines them
// (the activation kernels and the GEMM epilogues) computes the same values.
__device__ __forceinline__ float tg_gelu_grad(float x) {
#pragma clang fp contract(off)
  const float c0 = 0.7978845608028654f, c1 = 0.044715f;
  const float x2 = x * x;
  const float u = c0 * (x + c1 * x2 * x);
  const float e = __expf(-2.0f * fabsf(u));
  const float r = __builtin_amdgcn_rcpf(1.0f + e);  // 1 ulp, e in (0, 1]
  const float onept = (u >= 0.f) ? 1.0f + (1.0f - e) * r : 2.0f * e * r;  // 1 + tanh(u)
  const float sech2 = 4.0f * e * r * r;                                   // 1 - tanh(u)^2
  const float du = c0 * (1.0f + 3.0f * c1 * x2);
  return 0.5f * onept + 0.5f * x * sech2 * du;
}

__device__ __forceinline__ float tg_gelu_fwd(float x) {
#pragma clang fp contract(off)
  const float c0 = 0.7978845608028654f, c1 = 0.044715f;
  const float u = c0 * (x + c1 * x * x * x);
  const float e = __expf(-2.0f * fabsf(u));
  const float r = __builtin_amdgcn_rcpf(1.0f + e);  // 1 ulp, e in (0, 1]
  const float onept = (u >= 0.f) ? 1.0f + (1.0f - e) * r : 2.0f * e * r;
  return tg_f32(0.5f * x * onept);
}

// Sum across the 64 lanes of a wavefront (butterfly, every lane gets the total).
__device__ __forceinline__ float tg_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ double tg_wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float tg_wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide sum of NV values for a block of NW wavefronts, through LDS.
// `red` must hold NW*NV floats.  All threads receive the totals.
template <int NW, int NV>
__device__ __forceinline__ void tg_block_sum(float (&v)[NV], float* red) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = tg_wave_sum(v[i]);
  if (NW == 1) return;
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) red[wave * NV + i] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += red[w * NV + i];
    v[i] = s;
  }
  __syncthreads();
}

// 16-byte vector of T used for coalesced dwordx4 traffic.
template <typename T> struct tg_vec16 {
  static constexpr int N = 16 / sizeof(T);
  T v[N];
};

template <typename T>
__device__ __forceinline__ tg_vec16<T> tg_load16(const T* p) {
  tg_vec16<T> r;
  *reinterpret_cast<uint4*>(&r) = *reinterpret_cast<const uint4*>(p);
  return r;
}
// 16-byte load with the non-temporal hint (one dwordx4 with the nt bit): inputs
// streamed once, too large to stay in the caches, skip cache retention.  Measured on
// gfx950 for a two-in/one-out fp32 stream of 256 MiB operands: 6.0 TB/s with plain
// loads, 6.6 TB/s with non-temporal loads (both with non-temporal stores).
typedef unsigned tg_u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ tg_vec16<T> tg_load16_nt(const T* p) {
  tg_vec16<T> r;
  *reinterpret_cast<tg_u32x4*>(&r) =
      __builtin_nontemporal_load(reinterpret_cast<const tg_u32x4*>(p));
  return r;
}
template <typename T>
__device__ __forceinline__ void tg_store16(T* p, const tg_vec16<T>& r) {
  *reinterpret_cast<uint4*>(p) = *reinterpret_cast<const uint4*>(&r);
}

// 16-byte store with the non-temporal hint: streaming outputs that no later kernel
// reads soon skip the cache-retention path (measured 3-6% more HBM throughput for
// streaming kernels on gfx950).
template <typename T>
__device__ __forceinline__ void tg_store16_nt(T* p, const tg_vec16<T>& r) {
  __builtin_nontemporal_store(*reinterpret_cast<const tg_u32x4*>(&r),
                              reinterpret_cast<tg_u32x4*>(p));
}

// Load/store chosen at compile time: NT selects the non-temporal forms.
template <bool NT, typename T>
__device__ __forceinline__ tg_vec16<T> tg_ld16(const T* p) {
  if constexpr (NT) return tg_load16_nt(p);
  else return tg_load16(p);
}
template <bool NT, typename T>
__device__ __forceinline__ void tg_st16(T* p, const tg_vec16<T>& r) {
  if constexpr (NT) tg_store16_nt(p, r);
  else tg_store16(p, r);
}

// Number of CUs on the current device, cached per device by tg_runtime.
int tg_num_cus();

// fp64 implementations (tg_f64.hip) behind the entry points' TG_F64 cases.
int tg64_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, double alpha,
              const double* A, int64_t lda, int64_t sa, const double* B, int64_t ldb,
              int64_t sb, double beta, double* C, int64_t ldc, int64_t sc, int64_t batch,
              const double* bias, hipStream_t s);
int tg64_act_fwd(int kind, const void* x, void* y, int64_t n, hipStream_t s);
int tg64_act_bwd(int kind, const void* x, const void* dy, void* dx, int64_t n, int acc,
                 hipStream_t s);
int tg64_fill(void* y, int64_t n, double v, hipStream_t s);
int tg64_axpbyz(int dtype_x, const void* x, int dtype_y, const void* y, void* z, int64_t n,
                double alpha, double beta, hipStream_t s);
int tg64_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t s);
int tg64_softmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols,
                     int acc, hipStream_t s);
int tg64_layernorm_fwd(const void* x, const float* gamma, const float* beta, void* y,
                       void* mean, void* rstd, int64_t rows, int64_t cols, double eps,
                       hipStream_t s);
size_t tg64_layernorm_bwd_workspace(int64_t rows, int64_t cols);
int tg64_layernorm_bwd(const void* x, const void* mean, const void* rstd, const float* gamma,
                       const void* dy, void* dx, float* dgamma, float* dbeta, int64_t rows,
                       int64_t cols, int acc_dx, int acc_params, void* ws, hipStream_t s);
int tg64_reduce_rows(int dtype_in, const void* in, int dtype_out, void* out, int64_t rows,
                     int64_t cols, int acc, void* ws, size_t ws_bytes, hipStream_t s);
int tg64_unscale_check(int ntensors, void* const* grads, const int64_t* numel, double mul,
                       int write, int* flags, hipStream_t s);
int tg64_grad_norm(int ntensors, void* const* grads, const int64_t* numel, int kind, double p,
                   int64_t chunk, double* out, int* flags, double* part, hipStream_t s);
int tg64_zero_nonfinite(int ntensors, void* const* grads, const int64_t* numel, hipStream_t s);

// Deterministic fp32 column sums: out[c] (+)= sum_{k<K} in[k*cols + c], converted to
// dtype_out.  `scratch` must hold tg_sum_partials_scratch(K, cols, nb) bytes (may be
// null when that is 0).  tg_sum_partials2 finishes two stacked matrices [2][K][cols]
// into out0 and out1 in one launch (a null output is skipped).  Defined in
// tg_reduce.hip.
size_t tg_sum_partials_scratch(int64_t K, int64_t cols, int nb = 1);
// Whether tg_sum_partials2_group finishes K partial rows of `cols` columns (its members
// must be finished by the same arithmetic as tg_sum_partials2 would use).
bool tg_sum_partials_groupable(int64_t K, int64_t cols);
int tg_sum_partials(const float* in, int64_t K, int64_t cols, int dtype_out, void* out, int acc,
                    float* scratch, hipStream_t s);
int tg_sum_partials2(const float* in, int64_t K, int64_t cols, int dtype_out, void* out0,
                     void* out1, int acc, float* scratch, hipStream_t s);
