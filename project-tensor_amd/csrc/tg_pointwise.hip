// Backward of the remaining pointwise / row / indexing ops of Tensor
// (reference tensor_gpu_v2/_core.py):
//   tg_unary_bwd       dx (+)= f'(x or y) * dy for ReLU (:1149-1157), LeakyReLU
//                      (:1159-1170), Swish (:1248-1260), sigmoid (:1262-1272), tanh
//                      (:1274-1282), exp, log and x ** p (:973-981; also a / b, which the
//                      reference forms as a * b ** -1, :993-995);
//   tg_log_softmax_bwd dx (+)= dy - exp(y) * sum_row(dy) (:1301-1314);
//   tg_max_bwd         the even split of max's gradient over the tied maxima
//                      (:1115-1132; min runs as -max(-x), :1134-1135);
//   tg_index_add_sorted the scatter-add of integer-array / mask __getitem__
//                      (:918-929), in the order NumPy's add.at uses.
//
// Every formula keeps the reference's operation order (no fused multiply-add, see the
// contract pragma): float and double data compute in their own precision; fp16 and
// bf16 data compute in fp32 and round once.
#include "tg_common.h"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;

enum {
  U_RELU = 0,     // dy * (y > 0), y = relu(x)
  U_LEAKY = 1,    // dy * (x >= 0 ? 1 : slope)
  U_SIGMOID = 2,  // y * (1 - y) * dy
  U_TANH = 3,     // (1 - y^2) * dy
  U_EXP = 4,      // y * dy
  U_LOG = 5,      // dy / x
  U_POW = 6,      // (p * x^(p-1)) * dy
  U_SWISH = 7,    // (s + p*x*s*(1 - s)) * dy, s = 1 / (1 + exp(-p*x))
  U_NOPS = 8
};

template <typename T> struct Acc { typedef float type; };
template <> struct Acc<double> { typedef double type; };

template <typename T> __device__ __forceinline__ typename Acc<T>::type up(T v) {
  return (typename Acc<T>::type)tg_to_float(v);
}
template <> __device__ __forceinline__ double up<double>(double v) { return v; }
// fp16/bf16: the fp32 value is materialised first (tg_f32), so the rounding to T cannot
// be merged with the operation before it into one single-rounding mixed-precision
// instruction in one code path and not in another (the vector body and the scalar loop
// then round every element alike).
template <typename T> __device__ __forceinline__ T down(typename Acc<T>::type v) {
  return tg_from_float<T>(sizeof(T) == 2 ? tg_f32(v) : v);
}
template <> __device__ __forceinline__ double down<double>(double v) { return v; }

__device__ __forceinline__ float tg_pow(float a, float b) { return powf(a, b); }
__device__ __forceinline__ double tg_pow(double a, double b) { return pow(a, b); }
__device__ __forceinline__ float tg_sqrt(float a) { return sqrtf(a); }
__device__ __forceinline__ float tg_exp(float a) { return expf(a); }
__device__ __forceinline__ double tg_exp(double a) { return exp(a); }
__device__ __forceinline__ double tg_sqrt(double a) { return sqrt(a); }

// x ** e with the exact forms NumPy's power uses for e in {0, 0.5, 1, 2, -1}
// (1, sqrt, x, x*x, 1/x); other exponents go through pow.
template <typename C>
__device__ __forceinline__ C powe(C x, C e, int ek) {
  switch (ek) {
    case 0: return (C)1;
    case 1: return x;
    case 2: return x * x;
    case 3: return tg_sqrt(x);
    case 4: return (C)1 / x;
  }
  return tg_pow(x, e);
}

// f'(.) * dy in the reference's order; a = x or y as the op needs (host picks).
template <int OP, typename C>
__device__ __forceinline__ C ugrad(C a, C g, C p, C pm1, int ek) {
  switch (OP) {
    case U_RELU: return (C)(a > (C)0 ? 1 : 0) * g;
    case U_LEAKY: return (a >= (C)0 ? (C)1 : p) * g;
    case U_SIGMOID: return a * ((C)1 - a) * g;
    case U_TANH: return ((C)1 - a * a) * g;
    case U_EXP: return a * g;
    case U_LOG: return g / a;
    case U_SWISH: {
      const C sv = (C)1 / ((C)1 + tg_exp(-p * a));
      return (sv + p * a * sv * ((C)1 - sv)) * g;
    }
    default: return (p * powe<C>(a, pm1, ek)) * g;
  }
}

// One 16-byte vector per operand and thread; then a scalar loop, grid-stride over all
// blocks, for the tail of fewer than V elements or, when an operand is not 16-byte
// aligned (nvec == 0), for every element.
template <typename T, int OP, bool ACC>
__global__ __launch_bounds__(kThreads) void k_unary_bwd(const T* __restrict__ a,
                                                        const T* __restrict__ dy,
                                                        T* __restrict__ dx, int64_t nvec,
                                                        int64_t n, double p, int ek) {
  typedef typename Acc<T>::type C;
  constexpr int V = tg_vec16<T>::N;
  const C pc = (C)p, pm1 = (C)(p - 1.0);
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < nvec) {
    const tg_vec16<T> av = tg_load16(a + i * V), gv = tg_load16(dy + i * V);
    tg_vec16<T> ov;
    if (ACC) ov = tg_load16(dx + i * V);
    tg_vec16<T> r;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      C v = ugrad<OP, C>(up<T>(av.v[j]), up<T>(gv.v[j]), pc, pm1, ek);
      if (ACC) v = up<T>(ov.v[j]) + v;
      r.v[j] = down<T>(v);
    }
    tg_store16(dx + i * V, r);
  }
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t k = nvec * V + i; k < n; k += stride) {
    C v = ugrad<OP, C>(up<T>(a[k]), up<T>(dy[k]), pc, pm1, ek);
    if (ACC) v = up<T>(dx[k]) + v;
    dx[k] = down<T>(v);
  }
}

template <typename T, int OP>
int launch_unary(const void* a, const void* dy, void* dx, int64_t n, double p, int ek, int acc,
                 hipStream_t s) {
  constexpr int V = tg_vec16<T>::N;
  const bool vec = tg_aligned16(a) && tg_aligned16(dy) && tg_aligned16(dx);
  const int64_t nvec = vec ? n / V : 0;
  // one block per kThreads vectors; misaligned operands: the scalar loop over a capped
  // grid
  int64_t blocks = vec ? (nvec + kThreads - 1) / kThreads : (n + kThreads - 1) / kThreads;
  if (!vec && blocks > (int64_t)tg_num_cus() * 16) blocks = (int64_t)tg_num_cus() * 16;
  if (blocks < 1) blocks = 1;
  if (blocks * kThreads > 0xffffffffll) {  // a dispatch holds at most 2^32 work-items
    tg_set_error("tg_unary_bwd: n=%lld too large", (long long)n);
    return TG_ERR_INVALID;
  }
  if (acc)
    k_unary_bwd<T, OP, true><<<(unsigned)blocks, kThreads, 0, s>>>(
        (const T*)a, (const T*)dy, (T*)dx, nvec, n, p, ek);
  else
    k_unary_bwd<T, OP, false><<<(unsigned)blocks, kThreads, 0, s>>>(
        (const T*)a, (const T*)dy, (T*)dx, nvec, n, p, ek);
  return TG_OK;
}

template <typename T>
int unary_t(int op, const void* a, const void* dy, void* dx, int64_t n, double p, int ek,
            int acc, hipStream_t s) {
  switch (op) {
    case U_RELU: return launch_unary<T, U_RELU>(a, dy, dx, n, p, ek, acc, s);
    case U_LEAKY: return launch_unary<T, U_LEAKY>(a, dy, dx, n, p, ek, acc, s);
    case U_SIGMOID: return launch_unary<T, U_SIGMOID>(a, dy, dx, n, p, ek, acc, s);
    case U_TANH: return launch_unary<T, U_TANH>(a, dy, dx, n, p, ek, acc, s);
    case U_EXP: return launch_unary<T, U_EXP>(a, dy, dx, n, p, ek, acc, s);
    case U_LOG: return launch_unary<T, U_LOG>(a, dy, dx, n, p, ek, acc, s);
    case U_SWISH: return launch_unary<T, U_SWISH>(a, dy, dx, n, p, ek, acc, s);
    default: return launch_unary<T, U_POW>(a, dy, dx, n, p, ek, acc, s);
  }
}

// ------------------------------------------------------------------ log_softmax
// One wavefront per row (four rows per workgroup): the row sum of dy by a butterfly,
// then dx (+)= dy - exp(y) * sum.  Rows are read with 16-byte vectors when the row
// length and the pointers allow, else element by element.
template <typename T, bool ACC, bool VEC>
__global__ __launch_bounds__(kThreads) void k_log_softmax_bwd(const T* __restrict__ y,
                                                              const T* __restrict__ dy,
                                                              T* __restrict__ dx, int64_t rows,
                                                              int64_t cols) {
  typedef typename Acc<T>::type C;
  constexpr int V = tg_vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* yr = y + row * cols;
  const T* gr = dy + row * cols;
  T* xr = dx + row * cols;
  C sum = 0;
  if (VEC) {
    for (int64_t c = (int64_t)lane * V; c < cols; c += 64 * V) {
      const tg_vec16<T> gv = tg_load16(gr + c);
#pragma unroll
      for (int j = 0; j < V; ++j) sum += up<T>(gv.v[j]);
    }
  } else {
    for (int64_t c = lane; c < cols; c += 64) sum += up<T>(gr[c]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if (VEC) {
    for (int64_t c = (int64_t)lane * V; c < cols; c += 64 * V) {
      const tg_vec16<T> yv = tg_load16(yr + c), gv = tg_load16(gr + c);
      tg_vec16<T> ov, r;
      if (ACC) ov = tg_load16(xr + c);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        C v = up<T>(gv.v[j]) - tg_exp(up<T>(yv.v[j])) * sum;
        if (ACC) v = up<T>(ov.v[j]) + v;
        r.v[j] = down<T>(v);
      }
      tg_store16(xr + c, r);
    }
  } else {
    for (int64_t c = lane; c < cols; c += 64) {
      C v = up<T>(gr[c]) - tg_exp(up<T>(yr[c])) * sum;
      if (ACC) v = up<T>(xr[c]) + v;
      xr[c] = down<T>(v);
    }
  }
}

template <typename T>
void log_softmax_t(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols, int acc,
                   hipStream_t s) {
  constexpr int V = tg_vec16<T>::N;
  const bool vec = cols % V == 0 && tg_aligned16(y) && tg_aligned16(dy) && tg_aligned16(dx);
  const unsigned blocks = (unsigned)((rows + kThreads / 64 - 1) / (kThreads / 64));
#define LS(A, VV)                                                                   \
  k_log_softmax_bwd<T, A, VV><<<blocks, kThreads, 0, s>>>((const T*)y, (const T*)dy, \
                                                          (T*)dx, rows, cols)
  if (acc) { if (vec) LS(true, true); else LS(true, false); }
  else { if (vec) LS(false, true); else LS(false, false); }
#undef LS
}

// ------------------------------------------------------------------ max over a row
// x viewed as [rows, cols] (the reduced axes last), r = the row maxima, g = their
// upstream gradient: dx (+)= (x == r) * g / count(x == r) per row, in the reference's
// order (mask * g) / count (_core.py:1115-1132).  One wavefront per row.
template <typename T, bool ACC>
__global__ __launch_bounds__(kThreads) void k_max_bwd(const T* __restrict__ x,
                                                      const T* __restrict__ r,
                                                      const T* __restrict__ g,
                                                      T* __restrict__ dx, int64_t rows,
                                                      int64_t cols) {
  typedef typename Acc<T>::type C;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  T* dr = dx + row * cols;
  const C rv = up<T>(r[row]), gv = up<T>(g[row]);
  int64_t cnt = 0;
  for (int64_t c = lane; c < cols; c += 64) cnt += up<T>(xr[c]) == rv ? 1 : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
  const C cc = (C)cnt;
  for (int64_t c = lane; c < cols; c += 64) {
    C v = ((up<T>(xr[c]) == rv ? (C)1 : (C)0) * gv) / cc;
    if (ACC) v = up<T>(dr[c]) + v;
    dr[c] = down<T>(v);
  }
}

template <typename T>
void max_bwd_t(const void* x, const void* r, const void* g, void* dx, int64_t rows, int64_t cols,
               int acc, hipStream_t s) {
  const unsigned blocks = (unsigned)((rows + kThreads / 64 - 1) / (kThreads / 64));
  if (acc)
    k_max_bwd<T, true><<<blocks, kThreads, 0, s>>>((const T*)x, (const T*)r, (const T*)g,
                                                   (T*)dx, rows, cols);
  else
    k_max_bwd<T, false><<<blocks, kThreads, 0, s>>>((const T*)x, (const T*)r, (const T*)g,
                                                    (T*)dx, rows, cols);
}

// ------------------------------------------------------------------ index scatter-add
// grad[target[s]] += sum of src[order[j]] for j in [start[s], start[s+1]), summed in
// j order with T's rounding at every step (NumPy's add.at adds the selected elements
// one by one in index order into a zero array of the tensor's dtype; the reference
// then adds that array to the gradient).  target holds distinct flat indices and
// order is a stable sort of the selected elements by flat index, so each segment
// lists one target's elements in their original order.  One thread per target: no
// two threads write the same element and the result does not depend on scheduling.
template <typename T>
__global__ __launch_bounds__(kThreads) void k_index_add_sorted(T* __restrict__ grad,
                                                               int64_t nseg,
                                                               const int64_t* __restrict__ target,
                                                               const int64_t* __restrict__ start,
                                                               const int64_t* __restrict__ order,
                                                               const T* __restrict__ src) {
  const int64_t sidx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (sidx >= nseg) return;
  const int64_t j1 = start[sidx + 1];
  T acc = down<T>(0);
  for (int64_t j = start[sidx]; j < j1; ++j) acc = down<T>(up<T>(acc) + up<T>(src[order[j]]));
  const int64_t t = target[sidx];
  grad[t] = down<T>(up<T>(grad[t]) + up<T>(acc));
}

template <typename T>
void index_add_t(void* grad, int64_t nseg, const int64_t* target, const int64_t* start,
                 const int64_t* order, const void* src, hipStream_t s) {
  const unsigned blocks = (unsigned)((nseg + kThreads - 1) / kThreads);
  k_index_add_sorted<T><<<blocks, kThreads, 0, s>>>((T*)grad, nseg, target, start, order,
                                                    (const T*)src);
}

}  // namespace

TG_EXPORT int tg_unary_bwd(int dtype, int op, const void* a, const void* dy, void* dx, int64_t n,
                           double param, int accumulate, void* stream) {
  TG_REQUIRE(n >= 0, "tg_unary_bwd: negative n");
  TG_REQUIRE(op >= 0 && op < U_NOPS, "tg_unary_bwd: unknown op %d", op);
  if (n == 0) return TG_OK;
  TG_REQUIRE(a && dy && dx, "tg_unary_bwd: null pointer");
  TG_REQUIRE(n / kThreads < 0x7fffffffll, "tg_unary_bwd: n=%lld too large", (long long)n);
  hipStream_t s = tg_stream(stream);
  // exponent p - 1 of the power rule, by its exact form
  const double e = param - 1.0;
  const int ek = e == 0.0 ? 0 : e == 1.0 ? 1 : e == 2.0 ? 2 : e == 0.5 ? 3 : e == -1.0 ? 4 : 5;
  int st;
  switch (dtype) {
    case TG_F32: st = unary_t<float>(op, a, dy, dx, n, param, ek, accumulate, s); break;
    case TG_F16: st = unary_t<tg_half>(op, a, dy, dx, n, param, ek, accumulate, s); break;
    case TG_BF16: st = unary_t<tg_bf16>(op, a, dy, dx, n, param, ek, accumulate, s); break;
    case TG_F64: st = unary_t<double>(op, a, dy, dx, n, param, ek, accumulate, s); break;
    default:
      tg_set_error("tg_unary_bwd: unsupported dtype %d", dtype);
      return TG_ERR_UNSUPPORTED;
  }
  if (st != TG_OK) return st;
  return tg_check_launch("tg_unary_bwd");
}

TG_EXPORT int tg_log_softmax_bwd(int dtype, const void* y, const void* dy, void* dx,
                                 int64_t rows, int64_t cols, int accumulate, void* stream) {
  TG_REQUIRE(rows >= 0 && cols >= 0, "tg_log_softmax_bwd: negative shape");
  if (rows == 0 || cols == 0) return TG_OK;
  TG_REQUIRE(y && dy && dx, "tg_log_softmax_bwd: null pointer");
  TG_REQUIRE(rows / (kThreads / 64) < 0x7fffffffll, "tg_log_softmax_bwd: too many rows");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: log_softmax_t<float>(y, dy, dx, rows, cols, accumulate, s); break;
    case TG_F16: log_softmax_t<tg_half>(y, dy, dx, rows, cols, accumulate, s); break;
    case TG_BF16: log_softmax_t<tg_bf16>(y, dy, dx, rows, cols, accumulate, s); break;
    case TG_F64: log_softmax_t<double>(y, dy, dx, rows, cols, accumulate, s); break;
    default:
      tg_set_error("tg_log_softmax_bwd: unsupported dtype %d", dtype);
      return TG_ERR_UNSUPPORTED;
  }
  return tg_check_launch("tg_log_softmax_bwd");
}

TG_EXPORT int tg_index_add_sorted(int dtype, void* grad, int64_t nseg, const int64_t* target,
                                  const int64_t* start, const int64_t* order, const void* src,
                                  void* stream) {
  TG_REQUIRE(nseg >= 0, "tg_index_add_sorted: negative segment count");
  if (nseg == 0) return TG_OK;
  TG_REQUIRE(grad && target && start && order && src, "tg_index_add_sorted: null pointer");
  TG_REQUIRE(nseg / kThreads < 0x7fffffffll, "tg_index_add_sorted: too many segments");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: index_add_t<float>(grad, nseg, target, start, order, src, s); break;
    case TG_F16: index_add_t<tg_half>(grad, nseg, target, start, order, src, s); break;
    case TG_BF16: index_add_t<tg_bf16>(grad, nseg, target, start, order, src, s); break;
    case TG_F64: index_add_t<double>(grad, nseg, target, start, order, src, s); break;
    default:
      tg_set_error("tg_index_add_sorted: unsupported dtype %d", dtype);
      return TG_ERR_UNSUPPORTED;
  }
  return tg_check_launch("tg_index_add_sorted");
}

TG_EXPORT int tg_max_bwd(int dtype, const void* x, const void* r, const void* g, void* dx,
                         int64_t rows, int64_t cols, int accumulate, void* stream) {
  TG_REQUIRE(rows >= 0 && cols >= 0, "tg_max_bwd: negative shape");
  if (rows == 0 || cols == 0) return TG_OK;
  TG_REQUIRE(x && r && g && dx, "tg_max_bwd: null pointer");
  TG_REQUIRE(rows / (kThreads / 64) < 0x7fffffffll, "tg_max_bwd: too many rows");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: max_bwd_t<float>(x, r, g, dx, rows, cols, accumulate, s); break;
    case TG_F16: max_bwd_t<tg_half>(x, r, g, dx, rows, cols, accumulate, s); break;
    case TG_BF16: max_bwd_t<tg_bf16>(x, r, g, dx, rows, cols, accumulate, s); break;
    case TG_F64: max_bwd_t<double>(x, r, g, dx, rows, cols, accumulate, s); break;
    default:
      tg_set_error("tg_max_bwd: unsupported dtype %d", dtype);
      return TG_ERR_UNSUPPORTED;
  }
  return tg_check_launch("tg_max_bwd");
}
