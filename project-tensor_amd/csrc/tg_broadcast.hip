// Strided broadcast multiply with optional reduction: the gradient bookkeeping of the
// autograd closures that is neither a GEMM nor a fused row kernel.
//
//   out[o(i)] (+)= alpha * sum over i in `shape` of a[a(i)] * b[b(i)]
//
// over one N-d index space `shape`, where a(i), b(i), o(i) are offsets given by
// per-dimension element strides.  An input stride of 0 broadcasts that input along the
// dimension; an output stride of 0 sums the dimension away.  With that one form:
//   * Tensor._unbroadcast (_core.py:1380-1424): a = grad, b absent, out strides 0 on
//     the summed axes;
//   * __mul__ backward (_core.py:955-968): a = upstream grad, b = the other operand
//     (broadcast strides), out = this operand's grad, summed where it was broadcast;
//   * sum / mean backward (_core.py:1075-1100): a = upstream grad with stride 0 along
//     the reduced axes (a broadcast fill), alpha = 1 or 1/n;
//   * strided copies and casts of gradient buffers (a head-merge relayout, a permuted
//     gradient made contiguous, a dtype change on accumulation).
//
// The host drops size-1 dimensions, orders the kept (output) dimensions by output
// stride and the summed ones by a's stride, and merges neighbours that stay linear.
// Three kernels then cover the shapes:
//   * no summed dimension: one thread per output element (grid-stride);
//   * summed dimension innermost in memory (row-like): one wavefront per output
//     element, lanes walking the summed space in order, or a whole workgroup when that
//     space is large and the outputs few;
//   * kept dimension innermost (column-like): a workgroup covers 64 consecutive output
//     elements with 4 lane groups splitting the summed space, combined through LDS.
// Sums run in fp32 (fp64 when any operand is fp64) in a fixed order: results are
// deterministic.  Operand dtypes are runtime arguments (uniform branches), so one
// kernel serves every mix of fp32 / fp16 / bf16 / fp64.
#include "tg_common.h"

#include <algorithm>

namespace {

constexpr int kMaxDims = 8;

struct Dims {
  int n;
  int64_t size[kMaxDims];
  int64_t sa[kMaxDims], sb[kMaxDims], so[kMaxDims];
};

struct Operands {
  const void* a;
  const void* b;  // may be null: treated as 1
  void* out;
  int da, db, dout;
};

template <typename AT>
__device__ __forceinline__ AT ld(const void* p, int dt, int64_t i) {
  switch (dt) {
    case TG_F16: return (AT)(float)reinterpret_cast<const tg_half*>(p)[i];
    case TG_BF16: return (AT)(float)reinterpret_cast<const tg_bf16*>(p)[i];
    case TG_F64: return (AT)reinterpret_cast<const double*>(p)[i];
    default: return (AT)reinterpret_cast<const float*>(p)[i];
  }
}

template <typename AT>
__device__ __forceinline__ void st(void* p, int dt, int64_t i, AT v) {
  switch (dt) {
    case TG_F16: reinterpret_cast<tg_half*>(p)[i] = (tg_half)(float)v; break;
    case TG_BF16: reinterpret_cast<tg_bf16*>(p)[i] = (tg_bf16)(float)v; break;
    case TG_F64: reinterpret_cast<double*>(p)[i] = (double)v; break;
    default: reinterpret_cast<float*>(p)[i] = (float)v; break;
  }
}

// Offsets of linear index j (innermost dimension first) in a, b and out.
__device__ __forceinline__ void offsets(const Dims& d, int64_t j, int64_t& oa, int64_t& ob,
                                        int64_t& oo) {
  oa = ob = oo = 0;
  for (int k = 0; k < d.n; ++k) {
    const int64_t q = j / d.size[k];
    const int64_t r = j - q * d.size[k];
    oa += r * d.sa[k];
    ob += r * d.sb[k];
    oo += r * d.so[k];
    j = q;
  }
}

// Sum of a*b over the summed space R from base offsets (ba, bb), at linear indices
// t = t0, t0+step, ... < nred (each decoded into R's dimensions).
template <typename AT>
__device__ __forceinline__ AT sum_range(const Operands& op, const Dims& R, int64_t nred,
                                        int64_t ba, int64_t bb, int64_t t0, int64_t step) {
  AT acc = (AT)0;
  for (int64_t t = t0; t < nred; t += step) {
    int64_t oa, ob, oo;
    offsets(R, t, oa, ob, oo);
    const AT x = ld<AT>(op.a, op.da, ba + oa);
    acc += op.b ? x * ld<AT>(op.b, op.db, bb + ob) : x;
  }
  return acc;
}

template <typename AT>
__device__ __forceinline__ void finish(const Operands& op, int64_t oo, AT v, AT alpha, int acc) {
  v *= alpha;
  if (acc) v += ld<AT>(op.out, op.dout, oo);
  st<AT>(op.out, op.dout, oo, v);
}

// No summed dimension: one thread per output element.
template <typename AT>
__global__ __launch_bounds__(256) void k_bcast_elem(Operands op, Dims K, int64_t nout, AT alpha,
                                                    int acc, int have_input) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < nout; j += stride) {
    int64_t oa, ob, oo;
    offsets(K, j, oa, ob, oo);
    AT v = (AT)0;
    if (have_input) {
      v = ld<AT>(op.a, op.da, oa);
      if (op.b) v *= ld<AT>(op.b, op.db, ob);
    }
    finish<AT>(op, oo, v, alpha, acc);
  }
}

// Summed space innermost: W wavefronts per output element (W = 1: four outputs per
// 256-thread workgroup; W = 4: one output per workgroup).
template <typename AT, int W>
__global__ __launch_bounds__(256) void k_bcast_rows(Operands op, Dims K, Dims R, int64_t nout,
                                                    int64_t nred, AT alpha, int acc) {
  __shared__ AT red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t j = W == 1 ? (int64_t)blockIdx.x * 4 + wave : (int64_t)blockIdx.x;
  if (j >= nout) return;  // uniform per wavefront (W = 1) or per workgroup (W = 4)
  int64_t ba, bb, bo;
  offsets(K, j, ba, bb, bo);
  const int64_t t0 = W == 1 ? lane : threadIdx.x;
  AT v = sum_range<AT>(op, R, nred, ba, bb, t0, 64 * W);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if (W > 1) {
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = (AT)0;
#pragma unroll
    for (int w = 0; w < W; ++w) v += red[w];
  }
  if (threadIdx.x == 0 || (W == 1 && lane == 0)) finish<AT>(op, bo, v, alpha, acc);
}

// Kept dimension innermost: 64 consecutive outputs per workgroup, 4 lane groups each
// summing every 4th element of the summed space, combined in a fixed order.
template <typename AT>
__global__ __launch_bounds__(256) void k_bcast_cols(Operands op, Dims K, Dims R, int64_t nout,
                                                    int64_t nred, AT alpha, int acc) {
  __shared__ AT part[4][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.x * 64 + lane;
  AT v = (AT)0;
  int64_t bo = 0;
  if (j < nout) {
    int64_t ba, bb;
    offsets(K, j, ba, bb, bo);
    v = sum_range<AT>(op, R, nred, ba, bb, grp, 4);
  }
  part[grp][lane] = v;
  __syncthreads();
  if (grp == 0 && j < nout) {
    const AT s = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
    finish<AT>(op, bo, s, alpha, acc);
  }
}

struct Dim1 {
  int64_t size, sa, sb, so;
};

// Merge neighbours (inner i, outer i+1) whose strides stay linear.
int merge(Dim1* d, int n) {
  int m = 0;
  for (int i = 0; i < n; ++i) {
    if (m > 0) {
      Dim1& p = d[m - 1];
      if (d[i].sa == p.sa * p.size && d[i].sb == p.sb * p.size && d[i].so == p.so * p.size) {
        p.size *= d[i].size;
        continue;
      }
    }
    d[m++] = d[i];
  }
  return m;
}

Dims pack(const Dim1* d, int n) {
  Dims r{};
  r.n = n;
  for (int i = 0; i < n; ++i) {
    r.size[i] = d[i].size;
    r.sa[i] = d[i].sa;
    r.sb[i] = d[i].sb;
    r.so[i] = d[i].so;
  }
  return r;
}

int64_t iabs(int64_t v) { return v < 0 ? -v : v; }

template <typename AT>
int launch(const Operands& op, const Dims& K, const Dims& R, int64_t nout, int64_t nred,
           double alpha, int acc, hipStream_t s) {
  const AT al = (AT)alpha;
  if (nred <= 1) {
    int64_t blocks = (nout + 255) / 256;
    const int64_t cap = (int64_t)tg_num_cus() * 16;
    if (blocks > cap) blocks = cap;
    k_bcast_elem<AT><<<(unsigned)std::max<int64_t>(blocks, 1), 256, 0, s>>>(op, K, nout, al, acc,
                                                                            nred == 1);
    return tg_check_launch("tg_broadcast_mul_sum");
  }
  const bool rows = K.n == 0 || iabs(R.sa[0]) < iabs(K.sa[0]) ||
                    (iabs(R.sa[0]) == iabs(K.sa[0]) && R.size[0] > K.size[0]);
  if (rows) {
    if (nred >= 8192 && nout < 2048)
      k_bcast_rows<AT, 4><<<(unsigned)nout, 256, 0, s>>>(op, K, R, nout, nred, al, acc);
    else
      k_bcast_rows<AT, 1><<<(unsigned)((nout + 3) / 4), 256, 0, s>>>(op, K, R, nout, nred, al, acc);
  } else {
    k_bcast_cols<AT><<<(unsigned)((nout + 63) / 64), 256, 0, s>>>(op, K, R, nout, nred, al, acc);
  }
  return tg_check_launch("tg_broadcast_mul_sum");
}

}  // namespace

TG_EXPORT int tg_broadcast_mul_sum(int ndim, const int64_t* shape, int dtype_a, const void* a,
                                   const int64_t* strides_a, int dtype_b, const void* b,
                                   const int64_t* strides_b, int dtype_out, void* out,
                                   const int64_t* strides_out, double alpha, int accumulate,
                                   void* stream) {
  TG_REQUIRE(ndim >= 0 && ndim <= 16, "tg_broadcast_mul_sum: ndim %d outside [0, 16]", ndim);
  TG_REQUIRE(ndim == 0 || (shape && strides_a && strides_out),
             "tg_broadcast_mul_sum: null shape or strides");
  TG_REQUIRE(!b || ndim == 0 || strides_b, "tg_broadcast_mul_sum: null strides for b");
  TG_REQUIRE(tg_dtype_size(dtype_a) && tg_dtype_size(dtype_out) && (!b || tg_dtype_size(dtype_b)),
             "tg_broadcast_mul_sum: unsupported dtype");
  Dim1 kept[16], red[16];
  int nk = 0, nr = 0;
  int64_t nout = 1, nred = 1;
  for (int i = 0; i < ndim; ++i) {
    TG_REQUIRE(shape[i] >= 0, "tg_broadcast_mul_sum: negative extent");
    if (shape[i] == 1) continue;
    Dim1 d{shape[i], strides_a[i], b ? strides_b[i] : 0, strides_out[i]};
    if (d.so == 0) {
      red[nr++] = d;
      nred *= d.size;
    } else {
      kept[nk++] = d;
      nout *= d.size;
    }
  }
  if (nout == 0) return TG_OK;
  TG_REQUIRE(out && (a || nred == 0), "tg_broadcast_mul_sum: null pointer");
  // innermost first: kept dimensions by output stride, summed ones by a's stride
  std::sort(kept, kept + nk, [](const Dim1& x, const Dim1& y) { return iabs(x.so) < iabs(y.so); });
  std::sort(red, red + nr, [](const Dim1& x, const Dim1& y) { return iabs(x.sa) < iabs(y.sa); });
  nk = merge(kept, nk);
  nr = merge(red, nr);
  TG_REQUIRE(nk <= kMaxDims && nr <= kMaxDims,
             "tg_broadcast_mul_sum: more than %d non-mergeable dimensions", kMaxDims);
  const Dims K = pack(kept, nk), R = pack(red, nr);
  Operands op{a, b, out, dtype_a, b ? dtype_b : TG_F32, dtype_out};
  hipStream_t s = tg_stream(stream);
  const bool f64 = dtype_a == TG_F64 || (b && dtype_b == TG_F64) || dtype_out == TG_F64;
  // an empty summed space (nred == 0) writes 0 (or leaves out unchanged with accumulate)
  return f64 ? launch<double>(op, K, R, nout, nred, alpha, accumulate, s)
             : launch<float>(op, K, R, nout, nred, alpha, accumulate, s);
}
