// Elementwise activation forward/backward (GELU tanh-approx, SiLU) and the
// generic grad-accumulate kernel (y = a*x + b*y with dtype conversion).
//
// Layout: flat contiguous arrays of n elements.  Traffic is issued as 16-byte
// (dwordx4) vectors, UNROLL vectors in flight per thread, one pass over the
// array; a 16-byte misaligned operand switches to the scalar variant.
#include "tg_common.h"

namespace {

constexpr int kThreads = 256;
// Activation kernels: 128-thread workgroups, one 16-byte vector per operand and thread
// (measured 2 % faster than 256 threads for a two-in/one-out fp32 stream).
constexpr int kActThreads = 128;

enum { OP_GELU = 0, OP_SILU = 1 };

// GELU value and derivative: tg_gelu_grad / tg_gelu_fwd (tg_common.h, shared with the
// GEMM epilogues so fused and separate passes give identical values).
__device__ __forceinline__ float gelu_grad(float x) { return tg_gelu_grad(x); }
__device__ __forceinline__ float gelu_fwd(float x) { return tg_gelu_fwd(x); }

// SiLU derivative, reference formula (_core.py:522-533): s*(1 + x*(1-s)),
// s = sigmoid(x).  1-s is formed as e*s with e = exp(-x) (no cancellation).
__device__ __forceinline__ float silu_grad(float x) {
  const float e = __expf(-x);
  const float s = __builtin_amdgcn_rcpf(1.0f + e);  // 1 ulp
  const float oms = (x >= 0.f) ? e * s : 1.0f - s;
  return s * (1.0f + x * oms);
}
__device__ __forceinline__ float silu_fwd(float x) {
  const float e = __expf(-x);
  return x / (1.0f + e);
}

template <int OP> __device__ __forceinline__ float act_grad(float x) {
  return OP == OP_GELU ? gelu_grad(x) : silu_grad(x);
}
template <int OP> __device__ __forceinline__ float act_fwd(float x) {
  return OP == OP_GELU ? gelu_fwd(x) : silu_fwd(x);
}

// dx (+)= dy * act'(x).  One 16-byte vector per operand and thread (the
// measured optimum for two-in/one-out streams); NT marks loads and stores
// non-temporal, chosen for operands too large to stay in the Infinity Cache.
constexpr int kUnrollBwd = 1;
constexpr int kUnrollFwd = 1;  // one-in/one-out: one 16-byte vector per thread as well
constexpr int64_t kNtBytes = 128ll << 20;

template <typename T, int OP, bool ACC, bool NT>
__global__ __launch_bounds__(kActThreads) void k_act_bwd(const T* __restrict__ x,
                                                      const T* __restrict__ dy,
                                                      T* __restrict__ dx, int64_t nvec,
                                                      int64_t n) {
  constexpr int V = tg_vec16<T>::N;
  const int64_t base = (int64_t)blockIdx.x * kActThreads * kUnrollBwd + threadIdx.x;
  tg_vec16<T> xv[kUnrollBwd], gv[kUnrollBwd], ov[kUnrollBwd];
#pragma unroll
  for (int u = 0; u < kUnrollBwd; ++u) {
    const int64_t i = base + (int64_t)u * kActThreads;
    if (i < nvec) {
      xv[u] = tg_ld16<NT>(x + i * V);
      gv[u] = tg_ld16<NT>(dy + i * V);
      if (ACC) ov[u] = tg_ld16<NT>(dx + i * V);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnrollBwd; ++u) {
    const int64_t i = base + (int64_t)u * kActThreads;
    if (i < nvec) {
      tg_vec16<T> r;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        // accumulation as one explicit FMA, rounded to fp32 then to T (the GEMM epilogue
        // that fuses this derivative rounds the same way)
        const float d = tg_to_float(gv[u].v[j]), a = act_grad<OP>(tg_to_float(xv[u].v[j]));
        const float g = tg_f32(ACC ? fmaf(d, a, tg_to_float(ov[u].v[j])) : d * a);
        r.v[j] = tg_from_float<T>(g);
      }
      tg_st16<NT>(dx + i * V, r);
    }
  }
  // scalar part: the tail of fewer than V elements, or every element when an operand is
  // not 16-byte aligned (nvec == 0); grid-stride over all blocks
  {
    const int64_t stride = (int64_t)gridDim.x * kActThreads;
    for (int64_t i = nvec * V + (int64_t)blockIdx.x * kActThreads + threadIdx.x; i < n;
         i += stride) {
      const float d = tg_to_float(dy[i]), a = act_grad<OP>(tg_to_float(x[i]));
      const float g = tg_f32(ACC ? fmaf(d, a, tg_to_float(dx[i])) : d * a);
      dx[i] = tg_from_float<T>(g);
    }
  }
}

template <typename T, int OP, bool NT>
__global__ __launch_bounds__(kActThreads) void k_act_fwd(const T* __restrict__ x,
                                                      T* __restrict__ y, int64_t nvec,
                                                      int64_t n) {
  constexpr int V = tg_vec16<T>::N;
  const int64_t base = (int64_t)blockIdx.x * kActThreads * kUnrollFwd + threadIdx.x;
  tg_vec16<T> xv[kUnrollFwd];
#pragma unroll
  for (int u = 0; u < kUnrollFwd; ++u) {
    const int64_t i = base + (int64_t)u * kActThreads;
    if (i < nvec) xv[u] = tg_ld16<NT>(x + i * V);
  }
#pragma unroll
  for (int u = 0; u < kUnrollFwd; ++u) {
    const int64_t i = base + (int64_t)u * kActThreads;
    if (i < nvec) {
      tg_vec16<T> r;
#pragma unroll
      for (int j = 0; j < V; ++j) r.v[j] = tg_from_float<T>(act_fwd<OP>(tg_to_float(xv[u].v[j])));
      tg_st16<NT>(y + i * V, r);
    }
  }
  {
    const int64_t stride = (int64_t)gridDim.x * kActThreads;
    for (int64_t i = nvec * V + (int64_t)blockIdx.x * kActThreads + threadIdx.x; i < n;
         i += stride)
      y[i] = tg_from_float<T>(act_fwd<OP>(tg_to_float(x[i])));
  }
}

// Grid size: one block per kActThreads*unroll vectors; misaligned operands run the
// scalar loop grid-stride over a capped grid.  -1 when the grid would exceed the
// 2^32 work-items a dispatch can hold.
int64_t act_blocks(bool vec, int64_t nvec, int64_t n, int unroll) {
  int64_t blocks;
  if (vec) {
    blocks = (nvec + kActThreads * unroll - 1) / (kActThreads * unroll);
  } else {
    blocks = (n + kActThreads - 1) / kActThreads;
    const int64_t cap = (int64_t)tg_num_cus() * 16;
    if (blocks > cap) blocks = cap;
  }
  if (blocks < 1) blocks = 1;
  return blocks * kActThreads > 0xffffffffll ? -1 : blocks;
}

template <typename T, int OP>
int launch_act_bwd(const void* x, const void* dy, void* dx, int64_t n, int acc, hipStream_t s) {
  constexpr int V = tg_vec16<T>::N;
  const bool vec = tg_aligned16(x) && tg_aligned16(dy) && tg_aligned16(dx);
  const int64_t nvec = vec ? n / V : 0;
  const int64_t blocks = act_blocks(vec, nvec, n, kUnrollBwd);
  if (blocks < 0) {
    tg_set_error("activation backward: n=%lld too large", (long long)n);
    return TG_ERR_INVALID;
  }
  const bool nt = (int64_t)sizeof(T) * n >= kNtBytes;
#define L(ACC, NT)                                                      \
  k_act_bwd<T, OP, ACC, NT><<<(unsigned)blocks, kActThreads, 0, s>>>(      \
      (const T*)x, (const T*)dy, (T*)dx, nvec, n)
  if (acc) { if (nt) L(true, true); else L(true, false); }
  else { if (nt) L(false, true); else L(false, false); }
#undef L
  return tg_check_launch(OP == OP_GELU ? "tg_gelu_bwd" : "tg_silu_bwd");
}

template <typename T, int OP>
int launch_act_fwd(const void* x, void* y, int64_t n, hipStream_t s) {
  constexpr int V = tg_vec16<T>::N;
  const bool vec = tg_aligned16(x) && tg_aligned16(y);
  const int64_t nvec = vec ? n / V : 0;
  const int64_t blocks = act_blocks(vec, nvec, n, kUnrollFwd);
  if (blocks < 0) {
    tg_set_error("activation forward: n=%lld too large", (long long)n);
    return TG_ERR_INVALID;
  }
  if ((int64_t)sizeof(T) * n >= kNtBytes)
    k_act_fwd<T, OP, true><<<(unsigned)blocks, kActThreads, 0, s>>>((const T*)x, (T*)y, nvec, n);
  else
    k_act_fwd<T, OP, false><<<(unsigned)blocks, kActThreads, 0, s>>>((const T*)x, (T*)y, nvec, n);
  return tg_check_launch(OP == OP_GELU ? "tg_gelu_fwd" : "tg_silu_fwd");
}

template <int OP>
int dispatch_bwd(int dtype, const void* x, const void* dy, void* dx, int64_t n, int acc,
                 void* stream) {
  TG_REQUIRE(n >= 0, "activation backward: negative n");
  if (n == 0) return TG_OK;
  TG_REQUIRE(x && dy && dx, "activation backward: null pointer");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: return launch_act_bwd<float, OP>(x, dy, dx, n, acc, s);
    case TG_F16: return launch_act_bwd<tg_half, OP>(x, dy, dx, n, acc, s);
    case TG_BF16: return launch_act_bwd<tg_bf16, OP>(x, dy, dx, n, acc, s);
    case TG_F64: return tg64_act_bwd(OP, x, dy, dx, n, acc, s);
  }
  tg_set_error("activation backward: unsupported dtype %d", dtype);
  return TG_ERR_UNSUPPORTED;
}

template <int OP>
int dispatch_fwd(int dtype, const void* x, void* y, int64_t n, void* stream) {
  TG_REQUIRE(n >= 0, "activation forward: negative n");
  if (n == 0) return TG_OK;
  TG_REQUIRE(x && y, "activation forward: null pointer");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: return launch_act_fwd<float, OP>(x, y, n, s);
    case TG_F16: return launch_act_fwd<tg_half, OP>(x, y, n, s);
    case TG_BF16: return launch_act_fwd<tg_bf16, OP>(x, y, n, s);
    case TG_F64: return tg64_act_fwd(OP, x, y, n, s);
  }
  tg_set_error("activation forward: unsupported dtype %d", dtype);
  return TG_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// v rounded to T; for fp16/bf16 through tg_f32, so that the rounding is never merged
// with the multiply before it into one single-rounding instruction in one code path
// (the scalar tail, say) and not in another (the vector body).
template <typename T>
__device__ __forceinline__ T tg_round(float v) {
  return tg_from_float<T>(sizeof(T) == 2 ? tg_f32(v) : v);
}

// ---------------------------------------------------------------------------
// z = alpha*x + beta*y   (beta == 0: y is not read; z == y is the in-place update).
// x and y may differ in dtype, z has y's; arithmetic is fp32 (fp64 when an operand is
// fp64), as fma(beta, y, alpha*x) in every code path.  Used for `grad += g`
// with a dtype cast, for scaling, and for the out-of-place accumulation into a
// gradient buffer that another node shares.
template <typename TX, typename TY>
__global__ __launch_bounds__(kThreads) void k_axpby(const TX* __restrict__ x, const TY* y,
                                                    TY* z, float alpha, float beta, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
    float v = alpha * tg_to_float(x[i]);
    if (beta != 0.f) v = fmaf(beta, tg_to_float(y[i]), v);
    z[i] = tg_round<TY>(v);
  }
}

// 8 consecutive elements through 16-byte accesses (two for fp32).
template <typename T>
__device__ __forceinline__ void ld8f(const T* p, float (&f)[8]) {
  constexpr int V = tg_vec16<T>::N;
#pragma unroll
  for (int h = 0; h < 8 / V; ++h) {
    const tg_vec16<T> v = tg_load16(p + h * V);
#pragma unroll
    for (int j = 0; j < V; ++j) f[h * V + j] = tg_to_float(v.v[j]);
  }
}
template <typename T>
__device__ __forceinline__ void st8f(T* p, const float (&f)[8]) {
  constexpr int V = tg_vec16<T>::N;
#pragma unroll
  for (int h = 0; h < 8 / V; ++h) {
    tg_vec16<T> v;
#pragma unroll
    for (int j = 0; j < V; ++j) v.v[j] = tg_round<T>(f[h * V + j]);
    tg_store16(p + h * V, v);
  }
}

// Vector form: n8 groups of 8 elements, then a scalar tail in block 0.
template <typename TX, typename TY, bool READ_Y>
__global__ __launch_bounds__(kThreads) void k_axpby8(const TX* __restrict__ x, const TY* y,
                                                     TY* z, float alpha, float beta, int64_t n8,
                                                     int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8; i += stride) {
    float a[8], b[8];
    ld8f(x + i * 8, a);
    if (READ_Y) ld8f(y + i * 8, b);
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = READ_Y ? fmaf(beta, b[j], alpha * a[j]) : alpha * a[j];
    st8f(z + i * 8, a);
  }
  if (blockIdx.x == 0) {
    for (int64_t i = n8 * 8 + threadIdx.x; i < n; i += kThreads) {
      float v = alpha * tg_to_float(x[i]);
      if (READ_Y) v = fmaf(beta, tg_to_float(y[i]), v);
      z[i] = tg_round<TY>(v);
    }
  }
}

template <typename TX, typename TY>
int launch_axpby(const void* x, const void* y, void* z, float a, float b, int64_t n,
                 hipStream_t s) {
  if (tg_aligned16(x) && tg_aligned16(y) && tg_aligned16(z)) {
    const int64_t n8 = n / 8;
    int64_t blocks = (n8 + kThreads - 1) / kThreads;
    const int64_t cap = (int64_t)tg_num_cus() * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    if (b != 0.f)
      k_axpby8<TX, TY, true><<<(unsigned)blocks, kThreads, 0, s>>>((const TX*)x, (const TY*)y,
                                                                   (TY*)z, a, b, n8, n);
    else
      k_axpby8<TX, TY, false><<<(unsigned)blocks, kThreads, 0, s>>>((const TX*)x, (const TY*)y,
                                                                    (TY*)z, a, b, n8, n);
    return tg_check_launch("tg_axpby");
  }
  int64_t blocks = (n + kThreads * 4 - 1) / (kThreads * 4);
  const int64_t cap = (int64_t)tg_num_cus() * 32;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  k_axpby<TX, TY><<<(unsigned)blocks, kThreads, 0, s>>>((const TX*)x, (const TY*)y, (TY*)z, a, b,
                                                       n);
  return tg_check_launch("tg_axpby");
}

template <typename T>
__global__ __launch_bounds__(kThreads) void k_fill(T* __restrict__ y, float v, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const T tv = tg_from_float<T>(v);
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) y[i] = tv;
}

}  // namespace

// ---- exported C-ABI ----

TG_EXPORT int tg_gelu_bwd(int dtype, const void* x, const void* dy, void* dx, int64_t n,
                          int accumulate, void* stream) {
  return dispatch_bwd<OP_GELU>(dtype, x, dy, dx, n, accumulate, stream);
}
TG_EXPORT int tg_silu_bwd(int dtype, const void* x, const void* dy, void* dx, int64_t n,
                          int accumulate, void* stream) {
  return dispatch_bwd<OP_SILU>(dtype, x, dy, dx, n, accumulate, stream);
}
TG_EXPORT int tg_gelu_fwd(int dtype, const void* x, void* y, int64_t n, void* stream) {
  return dispatch_fwd<OP_GELU>(dtype, x, y, n, stream);
}
TG_EXPORT int tg_silu_fwd(int dtype, const void* x, void* y, int64_t n, void* stream) {
  return dispatch_fwd<OP_SILU>(dtype, x, y, n, stream);
}

TG_EXPORT int tg_axpbyz(int dtype_x, const void* x, int dtype_y, const void* y, void* z,
                        int64_t n, float alpha, float beta, void* stream) {
  TG_REQUIRE(n >= 0, "tg_axpbyz: negative n");
  if (n == 0) return TG_OK;
  TG_REQUIRE(x && z && (y || beta == 0.f), "tg_axpbyz: null pointer");
  if (!y) y = z;
  hipStream_t s = tg_stream(stream);
#define TG_AXPBY_CASE(DX, TX, DY, TY) \
  if (dtype_x == DX && dtype_y == DY) return launch_axpby<TX, TY>(x, y, z, alpha, beta, n, s);
  TG_AXPBY_CASE(TG_F32, float, TG_F32, float)
  TG_AXPBY_CASE(TG_F32, float, TG_F16, tg_half)
  TG_AXPBY_CASE(TG_F32, float, TG_BF16, tg_bf16)
  TG_AXPBY_CASE(TG_F16, tg_half, TG_F32, float)
  TG_AXPBY_CASE(TG_F16, tg_half, TG_F16, tg_half)
  TG_AXPBY_CASE(TG_BF16, tg_bf16, TG_F32, float)
  TG_AXPBY_CASE(TG_BF16, tg_bf16, TG_BF16, tg_bf16)
#undef TG_AXPBY_CASE
  if (dtype_x == TG_F64 || dtype_y == TG_F64)  // fp64 arithmetic (tg_f64.hip)
    return tg64_axpbyz(dtype_x, x, dtype_y, y, z, n, alpha, beta, s);
  tg_set_error("tg_axpby: unsupported dtype pair (%d,%d)", dtype_x, dtype_y);
  return TG_ERR_UNSUPPORTED;
}

TG_EXPORT int tg_axpby(int dtype_x, const void* x, int dtype_y, void* y, int64_t n, float alpha,
                       float beta, void* stream) {
  TG_REQUIRE(y || n == 0, "tg_axpby: null pointer");
  return tg_axpbyz(dtype_x, x, dtype_y, y, y, n, alpha, beta, stream);
}

// Fill n elements with `value` (a kernel, not a memset node, so it is safe to
// record into a captured graph).
TG_EXPORT int tg_fill(int dtype, void* y, int64_t n, float value, void* stream) {
  TG_REQUIRE(n >= 0, "tg_fill: negative n");
  if (n == 0) return TG_OK;
  TG_REQUIRE(y, "tg_fill: null pointer");
  hipStream_t s = tg_stream(stream);
  int64_t blocks = (n + kThreads * 4 - 1) / (kThreads * 4);
  const int64_t cap = (int64_t)tg_num_cus() * 32;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  switch (dtype) {
    case TG_F32: k_fill<float><<<(unsigned)blocks, kThreads, 0, s>>>((float*)y, value, n); break;
    case TG_F16: k_fill<tg_half><<<(unsigned)blocks, kThreads, 0, s>>>((tg_half*)y, value, n); break;
    case TG_BF16: k_fill<tg_bf16><<<(unsigned)blocks, kThreads, 0, s>>>((tg_bf16*)y, value, n); break;
    case TG_F64: return tg64_fill(y, n, value, s);
    default:
      tg_set_error("tg_fill: unsupported dtype %d", dtype);
      return TG_ERR_UNSUPPORTED;
  }
  return tg_check_launch("tg_fill");
}
