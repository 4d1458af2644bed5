// fp64 kernels: the reference's CuPy/NumPy path runs float64 data in float64 (a user's
// np.random.randn array stays float64, _core.py:173-193), so fp64 tensors are computed in
// double here, not rounded through fp32.  These are straightforward kernels (fp64 is not
// on the benchmarked path): the matrix product on the fp64 matrix cores, wavefront-per-
// row softmax / LayerNorm, column sums in fixed order (deterministic), grid-stride
// elementwise ops.  The entry points of the other files dispatch here for dtype TG_F64.
//
// Formulas follow the reference's array-module (xp) fallbacks, which are the ones that
// float64 data takes: GELU _core.py:1192-1206, SiLU :1235-1243, softmax :1286-1297,
// LayerNorm _nn.py:900-942, Adam _nn.py:1413-1442.
#include "tg_common.h"

namespace {

constexpr int kT = 256;

int64_t grid_for(int64_t n, int64_t per_block) {
  int64_t b = (n + per_block - 1) / per_block;
  const int64_t cap = (int64_t)tg_num_cus() * 16;
  if (b > cap) b = cap;
  return b < 1 ? 1 : b;
}

// ---------------------------------------------------------------- GEMM
// C[b] = alpha * op(A[b]) op(B[b]) + beta * C[b], all double.  Block tile 64 x 64 x 16,
// four waves of 32 x 32, each 2 x 2 v_mfma_f64_16x16x4f64 tiles.  For that instruction
// lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and holds D[l / 16 + 4 r][l % 16],
// r = 0..3.  Operands are staged k-major in LDS (rows padded by one element).
typedef double f64x4 __attribute__((ext_vector_type(4)));

template <bool TA, bool TB>
__global__ __launch_bounds__(kT) void k64_gemm(int64_t M, int64_t N, int64_t K, double alpha,
                                               const double* __restrict__ A, int64_t lda,
                                               int64_t sa, const double* __restrict__ B,
                                               int64_t ldb, int64_t sb, double beta,
                                               double* __restrict__ C, int64_t ldc, int64_t sc,
                                               const double* __restrict__ bias) {
  __shared__ double As[16][64 + 1];
  __shared__ double Bs[16][64 + 1];
  const int64_t bz = blockIdx.z;
  A += bz * sa;
  B += bz * sb;
  C += bz * sc;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  f64x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
    // consecutive threads walk the operand's contiguous dimension
#pragma unroll
    for (int e = tid; e < 1024; e += kT) {
      const int mm = TA ? e % 64 : e / 16, kk = TA ? e / 64 : e % 16;
      const int64_t gm = m0 + mm, gk = k0 + kk;
      As[kk][mm] = (gm < M && gk < K) ? (TA ? A[gk * lda + gm] : A[gm * lda + gk]) : 0.0;
    }
#pragma unroll
    for (int e = tid; e < 1024; e += kT) {
      const int nn = TB ? e / 16 : e % 64, kk = TB ? e % 16 : e / 64;
      const int64_t gn = n0 + nn, gk = k0 + kk;
      Bs[kk][nn] = (gn < N && gk < K) ? (TB ? B[gn * ldb + gk] : B[gk * ldb + gn]) : 0.0;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 16; ks += 4) {
      const int kk = ks + (lane >> 4);
      double a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[kk][wm + 16 * i + (lane & 15)];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[kk][wn + 16 * j + (lane & 15)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn + 16 * j + (lane & 15);
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm + 16 * i + (lane >> 4) + 4 * r;
        if (row >= M) continue;
        double v = alpha * acc[i][j][r];
        if (bias) v += bias[col];
        double* pc = C + row * ldc + col;
        if (beta != 0.0) v += beta * *pc;
        *pc = v;
      }
    }
}

// ---------------------------------------------------------------- elementwise
constexpr double kSqrt2OverPi = 0.7978845608028654;
constexpr double kGeluC = 0.044715;

__global__ __launch_bounds__(kT) void k64_act_fwd(int kind, const double* __restrict__ x,
                                                  double* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kT) {
    const double v = x[i];
    if (kind == 0) {
      y[i] = v * (0.5 * (1.0 + tanh(kSqrt2OverPi * (v + kGeluC * v * v * v))));
    } else {
      y[i] = v * (1.0 / (1.0 + exp(-v)));
    }
  }
}

__global__ __launch_bounds__(kT) void k64_act_bwd(int kind, const double* __restrict__ x,
                                                  const double* __restrict__ dy,
                                                  double* __restrict__ dx, int64_t n, int acc) {
  for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kT) {
    const double v = x[i];
    double d;
    if (kind == 0) {
      const double t = tanh(kSqrt2OverPi * (v + kGeluC * v * v * v));
      const double dinner = kSqrt2OverPi * (1.0 + 3.0 * kGeluC * v * v);
      d = 0.5 * (1.0 + t) + 0.5 * v * (1.0 - t * t) * dinner;
    } else {
      const double s = 1.0 / (1.0 + exp(-v));
      d = s * (1.0 + v * (1.0 - s));
    }
    const double g = d * dy[i];
    dx[i] = acc ? dx[i] + g : g;
  }
}

template <typename TX, typename TY, typename TZ>
__global__ __launch_bounds__(kT) void k64_axpbyz(const TX* __restrict__ x, const TY* y,
                                                 TZ* z, int64_t n, double alpha, double beta) {
  for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kT) {
    double v = alpha * (double)x[i];
    if (beta != 0.0) v += beta * (double)y[i];
    z[i] = (TZ)v;
  }
}

__global__ __launch_bounds__(kT) void k64_fill(double* __restrict__ y, int64_t n, double v) {
  for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kT)
    y[i] = v;
}

// ---------------------------------------------------------------- row kernels
// One wavefront per row, four rows per block.
__global__ __launch_bounds__(kT) void k64_softmax_fwd(const double* __restrict__ x,
                                                      double* __restrict__ y, int64_t rows,
                                                      int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const double* xr = x + r * cols;
  double* yr = y + r * cols;
  double m = -INFINITY;
  for (int64_t c = lane; c < cols; c += 64) m = fmax(m, xr[c]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmax(m, __shfl_xor(m, off, 64));
  double s = 0.0;
  for (int64_t c = lane; c < cols; c += 64) s += exp(xr[c] - m);
  s = tg_wave_sum_d(s);
  for (int64_t c = lane; c < cols; c += 64) yr[c] = exp(xr[c] - m) / s;
}

__global__ __launch_bounds__(kT) void k64_softmax_bwd(const double* __restrict__ y,
                                                      const double* __restrict__ dy,
                                                      double* __restrict__ dx, int64_t rows,
                                                      int64_t cols, int acc) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t o = r * cols;
  double s = 0.0;
  for (int64_t c = lane; c < cols; c += 64) s += dy[o + c] * y[o + c];
  s = tg_wave_sum_d(s);
  for (int64_t c = lane; c < cols; c += 64) {
    const double g = y[o + c] * (dy[o + c] - s);
    dx[o + c] = acc ? dx[o + c] + g : g;
  }
}

// LayerNorm forward over the last axis (population variance, two passes as xp.var).
__global__ __launch_bounds__(kT) void k64_ln_fwd(const double* __restrict__ x,
                                                 const float* __restrict__ gamma,
                                                 const float* __restrict__ beta,
                                                 double* __restrict__ y, double* __restrict__ mean,
                                                 double* __restrict__ rstd, int64_t rows,
                                                 int64_t cols, double eps) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const double* xr = x + r * cols;
  double s = 0.0;
  for (int64_t c = lane; c < cols; c += 64) s += xr[c];
  const double mu = tg_wave_sum_d(s) / (double)cols;
  double q = 0.0;
  for (int64_t c = lane; c < cols; c += 64) {
    const double d = xr[c] - mu;
    q += d * d;
  }
  const double var = tg_wave_sum_d(q) / (double)cols;
  const double sd = sqrt(var + eps);
  for (int64_t c = lane; c < cols; c += 64)
    y[r * cols + c] = (double)gamma[c] * ((xr[c] - mu) / sd) + (double)beta[c];
  if (lane == 0) {
    mean[r] = mu;
    rstd[r] = 1.0 / sd;
  }
}

// dx (+)= rstd * (g - mean(g) - xhat * mean(g * xhat)), g = dy * gamma.
__global__ __launch_bounds__(kT) void k64_ln_bwd_dx(const double* __restrict__ x,
                                                    const double* __restrict__ mean,
                                                    const double* __restrict__ rstd,
                                                    const float* __restrict__ gamma,
                                                    const double* __restrict__ dy,
                                                    double* __restrict__ dx, int64_t rows,
                                                    int64_t cols, int acc) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t o = r * cols;
  const double mu = mean[r], rs = rstd[r];
  double s1 = 0.0, s2 = 0.0;
  for (int64_t c = lane; c < cols; c += 64) {
    const double g = dy[o + c] * (double)gamma[c];
    s1 += g;
    s2 += g * ((x[o + c] - mu) * rs);
  }
  const double mg = tg_wave_sum_d(s1) / (double)cols, mgx = tg_wave_sum_d(s2) / (double)cols;
  for (int64_t c = lane; c < cols; c += 64) {
    const double xh = (x[o + c] - mu) * rs;
    const double v = rs * (dy[o + c] * (double)gamma[c] - mg - xh * mgx);
    dx[o + c] = acc ? dx[o + c] + v : v;
  }
}

// Column sums in fixed order: stage 1 sums row chunk `blockIdx.y` of each column (one
// thread per column), stage 2 sums the chunks in order.  Mode 0: sum in[r][c]; mode 1:
// the LayerNorm parameter sums sum dy*xhat (into part) and sum dy (into part2).
template <typename TI>
__global__ __launch_bounds__(kT) void k64_colsum_part(const TI* __restrict__ in, int64_t rows,
                                                      int64_t cols, int64_t per,
                                                      double* __restrict__ part,
                                                      const double* __restrict__ x,
                                                      const double* __restrict__ mean,
                                                      const double* __restrict__ rstd,
                                                      double* __restrict__ part2) {
  const int64_t c = (int64_t)blockIdx.x * kT + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * per;
  const int64_t r1 = r0 + per < rows ? r0 + per : rows;
  double s = 0.0, s2 = 0.0;
  for (int64_t r = r0; r < r1; ++r) {
    const double v = (double)in[r * cols + c];
    if (x) {
      s += v * ((x[r * cols + c] - mean[r]) * rstd[r]);
      s2 += v;
    } else {
      s += v;
    }
  }
  part[(int64_t)blockIdx.y * cols + c] = s;
  if (x) part2[(int64_t)blockIdx.y * cols + c] = s2;
}

template <typename TO>
__global__ __launch_bounds__(kT) void k64_colsum_final(const double* __restrict__ part,
                                                       int64_t nparts, int64_t cols,
                                                       TO* __restrict__ out, int acc) {
  const int64_t c = (int64_t)blockIdx.x * kT + threadIdx.x;
  if (c >= cols || !out) return;
  double s = 0.0;
  for (int64_t k = 0; k < nparts; ++k) s += part[k * cols + c];
  if (acc) s += (double)out[c];
  out[c] = (TO)s;
}

// ---------------------------------------------------------------- Adam / AdamW
struct Adam64 {
  double lr, b1, omb1, b2, omb2, eps, lrwd, ibc1, ibc2;
  int decay, ams;
};

__global__ __launch_bounds__(kT) void k64_adam(double* __restrict__ p, const double* __restrict__ g,
                                               double* __restrict__ m, double* __restrict__ v,
                                               double* __restrict__ vm, int64_t n, Adam64 K) {
  for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kT) {
    double pp = p[i];
    if (K.decay) pp -= K.lrwd * pp;  // decoupled decay before the moments (AdamW)
    const double gg = g[i];
    const double mm = K.b1 * m[i] + K.omb1 * gg;
    const double vv = K.b2 * v[i] + K.omb2 * (gg * gg);
    const double mh = mm * K.ibc1;
    double vh = vv * K.ibc2;
    if (K.ams) {
      vh = fmax(vm[i], vh);
      vm[i] = vh;
    }
    p[i] = pp - K.lr * mh / (sqrt(vh) + K.eps);
    m[i] = mm;
    v[i] = vv;
  }
}

// ---------------------------------------------------------------- cross-entropy
// One block per row (CrossEntropyLoss, _nn.py:1136-1182, as tg_ce.hip in double):
// lse = log sum exp x; loss = -log(p_t + 1e-10), or with label smoothing s
// -((s/C) sum_c log(p_c + 1e-10) + (1 - s) log(p_t + 1e-10)); NaN for a target outside
// [0, C).  Backward: grad (+)= (p - w) * scale, w = s/C + (1 - s) [c == t].
__device__ double block_reduce_d(double v, bool is_max) {
  __shared__ double red[kT / 64];
  if (is_max) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
  } else {
    v = tg_wave_sum_d(v);
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = red[0];
  for (int w = 1; w < kT / 64; ++w) r = is_max ? fmax(r, red[w]) : r + red[w];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kT) void k64_ce_fwd(const double* __restrict__ X,
                                                 const int64_t* __restrict__ tgt, int64_t C,
                                                 double smooth, double* __restrict__ lse_out,
                                                 double* __restrict__ loss_out) {
  const int64_t row = blockIdx.x;
  const double* x = X + row * C;
  double m = -INFINITY;
  for (int64_t i = threadIdx.x; i < C; i += kT) m = fmax(m, x[i]);
  m = block_reduce_d(m, true);
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < C; i += kT) s += exp(x[i] - m);
  const double lse = m + log(block_reduce_d(s, false));
  double sum_log = 0.0;
  if (smooth > 0.0) {
    for (int64_t i = threadIdx.x; i < C; i += kT) sum_log += log(exp(x[i] - lse) + 1e-10);
    sum_log = block_reduce_d(sum_log, false);
  }
  if (threadIdx.x == 0) {
    const int64_t t = tgt[row] < 0 ? tgt[row] + C : tgt[row];  // [-C, 0) wraps
    double loss = NAN;
    if (t >= 0 && t < C) {
      const double lpt = log(exp(x[t] - lse) + 1e-10);
      loss = smooth > 0.0 ? -((smooth / (double)C) * sum_log + (1.0 - smooth) * lpt) : -lpt;
    }
    lse_out[row] = lse;
    loss_out[row] = loss;
  }
}

__global__ __launch_bounds__(kT) void k64_ce_bwd(const double* __restrict__ X,
                                                 const int64_t* __restrict__ tgt,
                                                 const double* __restrict__ lse_in, int64_t C,
                                                 double smooth, double scale,
                                                 double* __restrict__ G, int acc) {
  const int64_t row = blockIdx.x;
  const double* x = X + row * C;
  double* g = G + row * C;
  const double lse = lse_in[row];
  const int64_t t = tgt[row] < 0 ? tgt[row] + C : tgt[row];  // [-C, 0) wraps
  const double wu = smooth / (double)C, wt = 1.0 - smooth;
  for (int64_t i = threadIdx.x; i < C; i += kT) {
    const double w = wu + (i == t ? wt : 0.0);
    const double v = (exp(x[i] - lse) - w) * scale;
    g[i] = acc ? g[i] + v : v;
  }
}

// ---------------------------------------------------------------- GradScaler / clipping
// g' = g * mul (stored if write); flags[t] |= 1 if some g is non-finite, |= 2 if some g'
// is (GradScaler.unscale_, _nn.py:1795-1833).
__global__ __launch_bounds__(kT) void k64_scale_check(double* __restrict__ g, int64_t n,
                                                      double mul, int write, int* flags, int t) {
  int f = 0;
  for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kT) {
    const double x = g[i];
    if (!isfinite(x)) f |= 1;
    const double y = x * mul;
    if (!isfinite(y)) f |= 2;
    if (write) g[i] = y;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) f |= __shfl_xor(f, off, 64);
  if ((threadIdx.x & 63) == 0 && f) atomicOr(flags + t, f);
}

// Block partials of the norm over finite entries (kind 0: sum g^2, 1: max |g|, 2: sum
// |g|^p) into part[base + blockIdx.x]; a non-finite entry sets flags[t] bit 0.
__global__ __launch_bounds__(kT) void k64_norm_partial(const double* __restrict__ g, int64_t n,
                                                       int64_t chunk, int kind, double p,
                                                       double* __restrict__ part, int64_t base,
                                                       int* flags, int t) {
  const int64_t start = (int64_t)blockIdx.x * chunk;
  const int64_t end = start + chunk < n ? start + chunk : n;
  double acc = 0.0;
  int f = 0;
  for (int64_t i = start + threadIdx.x; i < end; i += kT) {
    const double x = g[i];
    if (!isfinite(x)) {
      f = 1;
      continue;
    }
    const double ax = fabs(x);
    if (kind == 0) acc += ax * ax;
    else if (kind == 1) acc = fmax(acc, ax);
    else acc += pow(ax, p);
  }
  __shared__ double red[kT / 64];
  if (kind == 1) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc = fmax(acc, __shfl_xor(acc, off, 64));
  } else {
    acc = tg_wave_sum_d(acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) f |= __shfl_xor(f, off, 64);
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = acc;
    if (f) atomicOr(flags + t, 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double r = red[0];
    for (int w = 1; w < kT / 64; ++w) r = kind == 1 ? fmax(r, red[w]) : r + red[w];
    part[base + blockIdx.x] = r;
  }
}

// Fixed-order combination of the partials: thread i takes partials i, i + kT, ...; the
// per-thread values are then combined in thread order by thread 0.
__global__ __launch_bounds__(kT) void k64_norm_final(const double* __restrict__ part, int64_t n,
                                                     int kind, double* out) {
  __shared__ double red[kT];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kT)
    acc = kind == 1 ? fmax(acc, part[i]) : acc + part[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double r = red[0];
    for (int k = 1; k < kT; ++k) r = kind == 1 ? fmax(r, red[k]) : r + red[k];
    out[0] = r;
  }
}

__global__ __launch_bounds__(kT) void k64_zero_nonfinite(double* __restrict__ g, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kT)
    if (!isfinite(g[i])) g[i] = 0.0;
}

__global__ void k64_zero_ints(int* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

// ---------------------------------------------------------------- attention
// fp64 FlashAttention (flash_attention on float64 data, _core.py:1686-1870, which runs in
// the input dtype): scores of a chunk of heads are materialised in a workspace (the
// reference materialises them per 64-query block) and the products run as batched fp64
// GEMMs.  Row softmax of S (one wavefront per row of a [rows = heads * Sq, Sk] chunk),
// P written over S; query i keeps keys j <= i under causal masking (the reference's
// -1e9 fill gives those keys exactly zero weight in double).  lse = m + log(sum).
__global__ __launch_bounds__(kT) void k64_fa_softmax(double* __restrict__ S,
                                                     double* __restrict__ lse, int64_t rows,
                                                     int64_t Sq, int64_t Sk, int causal) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t i = r % Sq;
  double* row = S + r * Sk;
  const int64_t kend = causal ? (i + 1 < Sk ? i + 1 : Sk) : Sk;
  double m = -INFINITY;
  for (int64_t c = lane; c < kend; c += 64) m = fmax(m, row[c]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmax(m, __shfl_xor(m, off, 64));
  double s = 0.0;
  for (int64_t c = lane; c < kend; c += 64) s += exp(row[c] - m);
  s = tg_wave_sum_d(s);
  for (int64_t c = lane; c < Sk; c += 64) row[c] = c < kend ? exp(row[c] - m) / s : 0.0;
  if (lane == 0) lse[r] = m + log(s);
}

// P = exp(S - lse) (masked keys 0), in place, for the backward.
__global__ __launch_bounds__(kT) void k64_fa_p(double* __restrict__ S,
                                               const double* __restrict__ lse, int64_t rows,
                                               int64_t Sq, int64_t Sk, int causal) {
  const int64_t n = rows * Sk;
  for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < n; e += (int64_t)gridDim.x * kT) {
    const int64_t r = e / Sk, c = e % Sk;
    S[e] = (causal && c > r % Sq) ? 0.0 : exp(S[e] - lse[r]);
  }
}

// dS = P * (dP - rowsum(P * dP)) * scale, written over dP (the reference's row term,
// _core.py:1818-1847).
__global__ __launch_bounds__(kT) void k64_fa_ds(const double* __restrict__ P,
                                                double* __restrict__ dP, int64_t rows,
                                                int64_t Sk, double scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const double* pr = P + r * Sk;
  double* dr = dP + r * Sk;
  double t = 0.0;
  for (int64_t c = lane; c < Sk; c += 64) t += pr[c] * dr[c];
  t = tg_wave_sum_d(t);
  for (int64_t c = lane; c < Sk; c += 64) dr[c] = pr[c] * (dr[c] - t) * scale;
}

// ---------------------------------------------------------------- batch norm
// fp64 BatchNorm(+ReLU) training forward/backward (FusedBatchNormReLU / BatchNorm2D on
// float64 data, _nn.py:794-833, :701-736), following the reference's formulas in
// double; gamma/beta are the module's fp32 parameters.  One workgroup per channel
// reduces over the m = N*HW elements of the channel (layout 0: [m, C]; 1: NCHW).
__device__ __forceinline__ int64_t bn_at(int layout, int64_t j, int64_t c, int64_t C,
                                         int64_t HW) {
  return layout == 0 ? j * C + c : ((j / HW) * C + c) * HW + j % HW;
}

__device__ __forceinline__ double block_sum_d(double v, double* red) {
  v = tg_wave_sum_d(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < kT / 64; ++w) t += red[w];
  return t;
}

// mean, var (population, two passes as xp.var), rstd = 1/sqrt(var + eps), running EMA
__global__ __launch_bounds__(kT) void k64_bn_stats(int layout, const double* __restrict__ x,
                                                   int64_t C, int64_t HW, int64_t m, double eps,
                                                   double momentum, double* __restrict__ mean,
                                                   double* __restrict__ var,
                                                   double* __restrict__ rstd,
                                                   double* __restrict__ rmean,
                                                   double* __restrict__ rvar) {
  __shared__ double red[kT / 64];
  const int64_t c = blockIdx.x;
  double s = 0.0;
  for (int64_t j = threadIdx.x; j < m; j += kT) s += x[bn_at(layout, j, c, C, HW)];
  const double mu = block_sum_d(s, red) / (double)m;
  double q = 0.0;
  for (int64_t j = threadIdx.x; j < m; j += kT) {
    const double d = x[bn_at(layout, j, c, C, HW)] - mu;
    q += d * d;
  }
  const double v = block_sum_d(q, red) / (double)m;
  if (threadIdx.x == 0) {
    mean[c] = mu;
    if (var) var[c] = v;
    rstd[c] = 1.0 / sqrt(v + eps);
    if (rmean) rmean[c] = (1.0 - momentum) * rmean[c] + momentum * mu;
    if (rvar) rvar[c] = (1.0 - momentum) * rvar[c] + momentum * v;
  }
}

// y = [relu](gamma * ((x - mean) * rstd) + beta)
__global__ __launch_bounds__(kT) void k64_bn_apply(int layout, const double* __restrict__ x,
                                                   const float* __restrict__ gamma,
                                                   const float* __restrict__ beta,
                                                   const double* __restrict__ mean,
                                                   const double* __restrict__ rstd,
                                                   double* __restrict__ y, int64_t n, int64_t C,
                                                   int64_t HW, int relu) {
  for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < n; e += (int64_t)gridDim.x * kT) {
    const int64_t c = layout == 0 ? e % C : (e / HW) % C;
    double v = (double)gamma[c] * ((x[e] - mean[c]) * rstd[c]) + (double)beta[c];
    y[e] = relu ? fmax(v, 0.0) : v;
  }
}

// Backward per channel (_nn.py:812-833, :720-736), for float64 data and for the
// eval-mode BatchNorm2D backward (which the reference runs with the same formula on the
// running statistics): T is the data type, every sum is in double.
// dout = dy*[out > 0]; dgamma += sum dout*xn,
// dbeta += sum dout (rounded into the fp32 gradients as the reference's in-place add on
// float32 arrays does); coefficients of dx = dxn*rstd + dvar*(2/m)*xc + dmean/m with
// dxn = dout*gamma, dvar = sum(dxn*xc)*(-0.5)*rstd^3,
// dmean = sum(dxn*(-rstd)) + dvar*(-2/m)*sum(xc).
template <typename T>
__global__ __launch_bounds__(kT) void k64_bn_bwd_sums(
    int layout, const T* __restrict__ x, const double* __restrict__ mean,
    const double* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, const T* __restrict__ dy, int64_t C, int64_t HW,
    int64_t m, int relu, float* __restrict__ dgamma, float* __restrict__ dbeta, int acc_params,
    double* __restrict__ coef) {
  __shared__ double red[kT / 64];
  const int64_t c = blockIdx.x;
  const double mu = mean[c], rs = rstd[c], g = (double)gamma[c], b = (double)beta[c];
  double s_dxn = 0.0, s_dn = 0.0, s_d = 0.0, s_dxc = 0.0, s_xc = 0.0;
  for (int64_t j = threadIdx.x; j < m; j += kT) {
    const int64_t e = bn_at(layout, j, c, C, HW);
    const double xc = (double)x[e] - mu, xn = xc * rs;
    double d = (double)dy[e];
    if (relu && !(g * xn + b > 0.0)) d = 0.0;
    s_dn += d * xn;
    s_d += d;
    s_dxc += d * g * xc;
    s_dxn += d * g * (-rs);
    s_xc += xc;
  }
  s_dn = block_sum_d(s_dn, red);
  s_d = block_sum_d(s_d, red);
  s_dxc = block_sum_d(s_dxc, red);
  s_dxn = block_sum_d(s_dxn, red);
  s_xc = block_sum_d(s_xc, red);
  if (threadIdx.x == 0) {
    if (dgamma) dgamma[c] = (float)(acc_params ? (double)dgamma[c] + s_dn : s_dn);
    if (dbeta) dbeta[c] = (float)(acc_params ? (double)dbeta[c] + s_d : s_d);
    const double dvar = s_dxc * -0.5 * (rs * rs * rs);
    const double dmean = s_dxn + dvar * (-2.0 / (double)m) * s_xc;
    coef[3 * c] = dvar * (2.0 / (double)m);
    coef[3 * c + 1] = dmean / (double)m;
    coef[3 * c + 2] = 0.0;
  }
}

template <typename T>
__global__ __launch_bounds__(kT) void k64_bn_bwd_dx(int layout, const T* __restrict__ x,
                                                    const double* __restrict__ mean,
                                                    const double* __restrict__ rstd,
                                                    const float* __restrict__ gamma,
                                                    const float* __restrict__ beta,
                                                    const T* __restrict__ dy,
                                                    const double* __restrict__ coef,
                                                    T* __restrict__ dx, int64_t n,
                                                    int64_t C, int64_t HW, int relu, int acc) {
  for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < n; e += (int64_t)gridDim.x * kT) {
    const int64_t c = layout == 0 ? e % C : (e / HW) % C;
    const double rs = rstd[c], g = (double)gamma[c];
    const double xc = (double)x[e] - mean[c];
    double d = (double)dy[e];
    if (relu && !(g * (xc * rs) + (double)beta[c] > 0.0)) d = 0.0;
    const double v = d * g * rs + coef[3 * c] * xc + coef[3 * c + 1];
    dx[e] = (T)(acc ? (double)dx[e] + v : v);
  }
}

}  // namespace

// ---------------------------------------------------------------- internal entry points
int tg64_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, double alpha,
              const double* A, int64_t lda, int64_t sa, const double* B, int64_t ldb,
              int64_t sb, double beta, double* C, int64_t ldc, int64_t sc, int64_t batch,
              const double* bias, hipStream_t s) {
  dim3 g((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64), (unsigned)batch);
#define L(TA_, TB_) \
  k64_gemm<TA_, TB_><<<g, kT, 0, s>>>(M, N, K, alpha, A, lda, sa, B, ldb, sb, beta, C, ldc, sc, bias)
  if (!trans_a && !trans_b) L(false, false);
  else if (!trans_a && trans_b) L(false, true);
  else if (trans_a && !trans_b) L(true, false);
  else L(true, true);
#undef L
  return tg_check_launch("tg_gemm (fp64)");
}

int tg64_act_fwd(int kind, const void* x, void* y, int64_t n, hipStream_t s) {
  k64_act_fwd<<<(unsigned)grid_for(n, kT * 4), kT, 0, s>>>(kind, (const double*)x, (double*)y, n);
  return tg_check_launch("activation forward (fp64)");
}

int tg64_act_bwd(int kind, const void* x, const void* dy, void* dx, int64_t n, int acc,
                 hipStream_t s) {
  k64_act_bwd<<<(unsigned)grid_for(n, kT * 4), kT, 0, s>>>(kind, (const double*)x,
                                                           (const double*)dy, (double*)dx, n, acc);
  return tg_check_launch("activation backward (fp64)");
}

int tg64_fill(void* y, int64_t n, double v, hipStream_t s) {
  k64_fill<<<(unsigned)grid_for(n, kT * 4), kT, 0, s>>>((double*)y, n, v);
  return tg_check_launch("tg_fill (fp64)");
}

int tg64_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t s) {
  k64_softmax_fwd<<<(unsigned)((rows + 3) / 4), kT, 0, s>>>((const double*)x, (double*)y, rows,
                                                             cols);
  return tg_check_launch("tg_softmax_fwd (fp64)");
}

int tg64_softmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols,
                     int acc, hipStream_t s) {
  k64_softmax_bwd<<<(unsigned)((rows + 3) / 4), kT, 0, s>>>(
      (const double*)y, (const double*)dy, (double*)dx, rows, cols, acc);
  return tg_check_launch("tg_softmax_bwd (fp64)");
}

int tg64_layernorm_fwd(const void* x, const float* gamma, const float* beta, void* y,
                       void* mean, void* rstd, int64_t rows, int64_t cols, double eps,
                       hipStream_t s) {
  k64_ln_fwd<<<(unsigned)((rows + 3) / 4), kT, 0, s>>>((const double*)x, gamma, beta,
                                                        (double*)y, (double*)mean,
                                                        (double*)rstd, rows, cols, eps);
  return tg_check_launch("tg_layernorm_fwd (fp64)");
}

// Row chunks of the fp64 column sums: enough column-thread blocks to fill the CUs, at
// least 64 rows per chunk, at most 256 chunks.
int64_t tg64_colsum_parts(int64_t rows, int64_t cols) {
  const int64_t cb = (cols + kT - 1) / kT;
  int64_t want = (4 * (int64_t)tg_num_cus() + cb - 1) / cb;
  const int64_t maxp = (rows + 63) / 64;
  if (want > maxp) want = maxp;
  if (want > 256) want = 256;
  return want < 1 ? 1 : want;
}

size_t tg64_layernorm_bwd_workspace(int64_t rows, int64_t cols) {
  return (size_t)(2 * tg64_colsum_parts(rows, cols) * cols) * sizeof(double);
}

int tg64_layernorm_bwd(const void* x, const void* mean, const void* rstd, const float* gamma,
                       const void* dy, void* dx, float* dgamma, float* dbeta, int64_t rows,
                       int64_t cols, int acc_dx, int acc_params, void* ws, hipStream_t s) {
  k64_ln_bwd_dx<<<(unsigned)((rows + 3) / 4), kT, 0, s>>>(
      (const double*)x, (const double*)mean, (const double*)rstd, gamma, (const double*)dy,
      (double*)dx, rows, cols, acc_dx);
  int st = tg_check_launch("tg_layernorm_bwd (fp64)");
  if (st || (!dgamma && !dbeta)) return st;
  const int64_t np = tg64_colsum_parts(rows, cols), per = (rows + np - 1) / np;
  double* pg = (double*)ws;
  double* pb = pg + np * cols;
  dim3 g1((unsigned)((cols + kT - 1) / kT), (unsigned)np);
  k64_colsum_part<double><<<g1, kT, 0, s>>>((const double*)dy, rows, cols, per, pg,
                                            (const double*)x, (const double*)mean,
                                            (const double*)rstd, pb);
  const unsigned g2 = (unsigned)((cols + kT - 1) / kT);
  k64_colsum_final<float><<<g2, kT, 0, s>>>(pg, np, cols, dgamma, acc_params);
  k64_colsum_final<float><<<g2, kT, 0, s>>>(pb, np, cols, dbeta, acc_params);
  return tg_check_launch("tg_layernorm_bwd (fp64) parameters");
}

// out[c] (+)= sum_r in[r][c] with in fp64 (out fp64 or fp32) or out fp64 (in fp32).
int tg64_reduce_rows(int dtype_in, const void* in, int dtype_out, void* out, int64_t rows,
                     int64_t cols, int acc, void* ws, size_t ws_bytes, hipStream_t s) {
  int64_t np = tg64_colsum_parts(rows, cols);
  const int64_t fit = (int64_t)(ws_bytes / (sizeof(double) * (size_t)cols));
  if (np > fit) np = fit;
  if (np < 1) {
    tg_set_error("tg_reduce_rows (fp64): workspace of %zu bytes needed, got %zu",
                 (size_t)cols * sizeof(double), ws_bytes);
    return TG_ERR_WORKSPACE;
  }
  const int64_t per = (rows + np - 1) / np;
  double* part = (double*)ws;
  dim3 g1((unsigned)((cols + kT - 1) / kT), (unsigned)np);
  if (dtype_in == TG_F64)
    k64_colsum_part<double><<<g1, kT, 0, s>>>((const double*)in, rows, cols, per, part, nullptr,
                                              nullptr, nullptr, nullptr);
  else
    k64_colsum_part<float><<<g1, kT, 0, s>>>((const float*)in, rows, cols, per, part, nullptr,
                                             nullptr, nullptr, nullptr);
  const unsigned g2 = (unsigned)((cols + kT - 1) / kT);
  if (dtype_out == TG_F64)
    k64_colsum_final<double><<<g2, kT, 0, s>>>(part, np, cols, (double*)out, acc);
  else
    k64_colsum_final<float><<<g2, kT, 0, s>>>(part, np, cols, (float*)out, acc);
  return tg_check_launch("tg_reduce_rows (fp64)");
}

// z = alpha x + beta y with z of y's dtype, any of fp64 / fp32 operands (one fp64).
int tg64_axpbyz(int dtype_x, const void* x, int dtype_y, const void* y, void* z, int64_t n,
                double alpha, double beta, hipStream_t s) {
  const unsigned g = (unsigned)grid_for(n, kT * 4);
#define L(TX, TY) \
  k64_axpbyz<TX, TY, TY><<<g, kT, 0, s>>>((const TX*)x, (const TY*)y, (TY*)z, n, alpha, beta)
  if (dtype_x == TG_F64 && dtype_y == TG_F64) L(double, double);
  else if (dtype_x == TG_F64 && dtype_y == TG_F32) L(double, float);
  else if (dtype_x == TG_F32 && dtype_y == TG_F64) L(float, double);
  else {
    tg_set_error("tg_axpbyz (fp64): unsupported dtype pair (%d,%d)", dtype_x, dtype_y);
    return TG_ERR_UNSUPPORTED;
  }
#undef L
  return tg_check_launch("tg_axpbyz (fp64)");
}

int tg64_unscale_check(int ntensors, void* const* grads, const int64_t* numel, double mul,
                       int write, int* flags, hipStream_t s) {
  k64_zero_ints<<<1, kT, 0, s>>>(flags, ntensors);
  for (int i = 0; i < ntensors; ++i) {
    if (numel[i] <= 0) continue;
    k64_scale_check<<<(unsigned)grid_for(numel[i], kT * 4), kT, 0, s>>>(
        (double*)grads[i], numel[i], mul, write, flags, i);
  }
  return tg_check_launch("tg_unscale_check (fp64)");
}

// chunk: elements per partial, the caller's (its workspace holds sum ceil(n / chunk)
// partials).
int tg64_grad_norm(int ntensors, void* const* grads, const int64_t* numel, int kind, double p,
                   int64_t chunk, double* out, int* flags, double* part, hipStream_t s) {
  k64_zero_ints<<<1, kT, 0, s>>>(flags, ntensors);
  int64_t base = 0;
  for (int i = 0; i < ntensors; ++i) {
    if (numel[i] <= 0) continue;
    const int64_t nb = (numel[i] + chunk - 1) / chunk;
    k64_norm_partial<<<(unsigned)nb, kT, 0, s>>>((const double*)grads[i], numel[i], chunk, kind,
                                                  p, part, base, flags, i);
    base += nb;
  }
  k64_norm_final<<<1, kT, 0, s>>>(part, base, kind, out);
  return tg_check_launch("tg_grad_norm (fp64)");
}

int tg64_zero_nonfinite(int ntensors, void* const* grads, const int64_t* numel, hipStream_t s) {
  for (int i = 0; i < ntensors; ++i) {
    if (numel[i] <= 0) continue;
    k64_zero_nonfinite<<<(unsigned)grid_for(numel[i], kT * 4), kT, 0, s>>>((double*)grads[i],
                                                                           numel[i]);
  }
  return tg_check_launch("tg_zero_nonfinite (fp64)");
}

// ---------------------------------------------------------------- exported
TG_EXPORT int tg_axpbyz64(int dtype_x, const void* x, int dtype_y, const void* y, void* z,
                          int64_t n, double alpha, double beta, void* stream) {
  TG_REQUIRE(n >= 0, "tg_axpbyz64: negative n");
  if (n == 0) return TG_OK;
  TG_REQUIRE(x && z && (y || beta == 0.0), "tg_axpbyz64: null pointer");
  if (!y) y = z;
  return tg64_axpbyz(dtype_x, x, dtype_y, y, z, n, alpha, beta, tg_stream(stream));
}

TG_EXPORT int tg_adam_step_f64(int ntensors, double* const* params, const double* const* grads,
                               double* const* exp_avg, double* const* exp_avg_sq,
                               double* const* max_exp_avg_sq, const int64_t* numel, double lr,
                               double beta1, double beta2, double eps, double weight_decay,
                               double bias_correction1, double bias_correction2, void* stream) {
  TG_REQUIRE(ntensors >= 0, "tg_adam_step_f64: negative tensor count");
  if (ntensors == 0) return TG_OK;
  TG_REQUIRE(params && grads && exp_avg && exp_avg_sq && numel, "tg_adam_step_f64: null list");
  Adam64 K{lr, beta1, 1.0 - beta1, beta2, 1.0 - beta2, eps, lr * weight_decay,
           1.0 / bias_correction1, 1.0 / bias_correction2, weight_decay != 0.0,
           max_exp_avg_sq != nullptr};
  hipStream_t s = tg_stream(stream);
  for (int i = 0; i < ntensors; ++i) {
    TG_REQUIRE(numel[i] >= 0, "tg_adam_step_f64: negative numel for tensor %d", i);
    if (numel[i] == 0) continue;
    TG_REQUIRE(params[i] && grads[i] && exp_avg[i] && exp_avg_sq[i] &&
                   (!K.ams || max_exp_avg_sq[i]),
               "tg_adam_step_f64: null pointer for tensor %d", i);
    k64_adam<<<(unsigned)grid_for(numel[i], kT * 4), kT, 0, s>>>(
        params[i], grads[i], exp_avg[i], exp_avg_sq[i], K.ams ? max_exp_avg_sq[i] : nullptr,
        numel[i], K);
  }
  return tg_check_launch("tg_adam_step_f64");
}

// Cross-entropy of fp64 logits with double scalars (label smoothing and the gradient
// scale 1/N are not exact in fp32); lse and loss are double.
TG_EXPORT int tg_cross_entropy_fwd_f64(const double* logits, const int64_t* targets, int64_t N,
                                       int64_t C, double label_smoothing, double* lse,
                                       double* loss, void* stream) {
  TG_REQUIRE(N >= 0 && C > 0 && N <= 0x7fffffff, "tg_cross_entropy_fwd_f64: bad shape");
  TG_REQUIRE(label_smoothing >= 0.0 && label_smoothing < 1.0,
             "tg_cross_entropy_fwd_f64: label_smoothing %g outside [0, 1)", label_smoothing);
  if (N == 0) return TG_OK;
  TG_REQUIRE(logits && targets && lse && loss, "tg_cross_entropy_fwd_f64: null pointer");
  k64_ce_fwd<<<(unsigned)N, kT, 0, tg_stream(stream)>>>(logits, targets, C, label_smoothing,
                                                        lse, loss);
  return tg_check_launch("tg_cross_entropy_fwd_f64");
}

TG_EXPORT int tg_cross_entropy_bwd_f64(const double* logits, const int64_t* targets,
                                       const double* lse, int64_t N, int64_t C,
                                       double label_smoothing, double scale, double* grad,
                                       int accumulate, void* stream) {
  TG_REQUIRE(N >= 0 && C > 0 && N <= 0x7fffffff, "tg_cross_entropy_bwd_f64: bad shape");
  TG_REQUIRE(label_smoothing >= 0.0 && label_smoothing < 1.0,
             "tg_cross_entropy_bwd_f64: label_smoothing %g outside [0, 1)", label_smoothing);
  if (N == 0) return TG_OK;
  TG_REQUIRE(logits && targets && lse && grad, "tg_cross_entropy_bwd_f64: null pointer");
  k64_ce_bwd<<<(unsigned)N, kT, 0, tg_stream(stream)>>>(logits, targets, lse, C,
                                                        label_smoothing, scale, grad,
                                                        accumulate);
  return tg_check_launch("tg_cross_entropy_bwd_f64");
}

// ---------------------------------------------------------------- fp64 attention entries
namespace {
constexpr int64_t kFa64Budget = (int64_t)256 << 20;  // bytes of scores per chunk buffer

int64_t fa64_heads_per_chunk(int64_t H, int64_t Sq, int64_t Sk) {
  const int64_t per = Sq * Sk * (int64_t)sizeof(double);
  int64_t hc = per > 0 ? kFa64Budget / per : H;
  if (hc < 1) hc = 1;
  return hc < H ? hc : H;
}

struct Fa64Geo {
  int64_t H, Sq, Sk, D;
  int layout;
  int64_t rs() const { return layout ? H * D : D; }
  int64_t hstride(int64_t S) const { return layout ? D : S * D; }
  int64_t head(int64_t b, int64_t h, int64_t S) const {
    return layout ? (b * S * H + h) * D : (b * H + h) * S * D;
  }
};

int fa64_check(const char* who, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
               int layout) {
  TG_REQUIRE(B >= 0 && H >= 0 && Sq >= 0 && Sk >= 0 && D > 0, "%s: bad shape", who);
  TG_REQUIRE(layout == 0 || layout == 1, "%s: layout %d", who, layout);
  TG_REQUIRE(H <= 65535 && (Sq + 63) / 64 <= 65535 && (Sk + 63) / 64 <= 65535,
             "%s: shape too large for the fp64 path", who);
  return TG_OK;
}
}  // namespace

TG_EXPORT size_t tg_flash_attn_f64_workspace(int64_t B, int64_t H, int64_t Sq, int64_t Sk) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0) return 0;
  return (size_t)(2 * fa64_heads_per_chunk(H, Sq, Sk) * Sq * Sk) * sizeof(double);
}

TG_EXPORT int tg_flash_attn_fwd_f64(const double* q, const double* k, const double* v,
                                    double* o, double* lse, int64_t B, int64_t H, int64_t Sq,
                                    int64_t Sk, int64_t D, double scale, int causal, int layout,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  int st = fa64_check("tg_flash_attn_fwd_f64", B, H, Sq, Sk, D, layout);
  if (st) return st;
  if (B == 0 || H == 0 || Sq == 0) return TG_OK;
  TG_REQUIRE(q && k && v && o && lse, "tg_flash_attn_fwd_f64: null pointer");
  hipStream_t s = tg_stream(stream);
  const Fa64Geo g{H, Sq, Sk, D, layout};
  if (Sk == 0) {  // no keys: zero output, log-sum-exp -inf
    for (int64_t b = 0; b < B; ++b)
      for (int64_t h = 0; h < H; ++h) {
        st = tg64_gemm(0, 0, Sq, D, 0, 1.0, nullptr, 1, 0, nullptr, 1, 0, 0.0,
                       o + g.head(b, h, Sq), g.rs(), 0, 1, nullptr, s);
        if (st) return st;
      }
    return tg64_fill(lse, B * H * Sq, -INFINITY, s);
  }
  const size_t need = tg_flash_attn_f64_workspace(B, H, Sq, Sk);
  TG_REQUIRE(workspace && workspace_bytes >= need,
             "tg_flash_attn_fwd_f64: workspace of %zu bytes needed", need);
  double* S = (double*)workspace;
  const int64_t hc = fa64_heads_per_chunk(H, Sq, Sk);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h0 = 0; h0 < H; h0 += hc) {
      const int64_t n = hc < H - h0 ? hc : H - h0;
      const int64_t oq = g.head(b, h0, Sq), ok = g.head(b, h0, Sk);
      st = tg64_gemm(0, 1, Sq, Sk, D, scale, q + oq, g.rs(), g.hstride(Sq), k + ok, g.rs(),
                     g.hstride(Sk), 0.0, S, Sk, Sq * Sk, n, nullptr, s);
      if (st) return st;
      k64_fa_softmax<<<(unsigned)((n * Sq + 3) / 4), kT, 0, s>>>(S, lse + (b * H + h0) * Sq,
                                                                 n * Sq, Sq, Sk, causal);
      st = tg_check_launch("tg_flash_attn_fwd_f64");
      if (st) return st;
      st = tg64_gemm(0, 0, Sq, D, Sk, 1.0, S, Sk, Sq * Sk, v + ok, g.rs(), g.hstride(Sk), 0.0,
                     o + oq, g.rs(), g.hstride(Sq), n, nullptr, s);
      if (st) return st;
    }
  return TG_OK;
}

TG_EXPORT int tg_flash_attn_bwd_f64(const double* q, const double* k, const double* v,
                                    const double* o, const double* dout, const double* lse,
                                    double* dq, double* dk, double* dv, int64_t B, int64_t H,
                                    int64_t Sq, int64_t Sk, int64_t D, double scale, int causal,
                                    int layout, int accumulate, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  (void)o;  // the row term is rowsum(P * dP), as the reference forms it
  int st = fa64_check("tg_flash_attn_bwd_f64", B, H, Sq, Sk, D, layout);
  if (st) return st;
  if (B == 0 || H == 0 || (Sq == 0 && Sk == 0)) return TG_OK;
  TG_REQUIRE(q && k && v && dout && lse && dq && dk && dv,
             "tg_flash_attn_bwd_f64: null pointer");
  hipStream_t s = tg_stream(stream);
  const Fa64Geo g{H, Sq, Sk, D, layout};
  const double beta = accumulate ? 1.0 : 0.0;
  if (Sq == 0 || Sk == 0) {  // empty product: dq (Sk == 0) or dk, dv (Sq == 0) are zero
    for (int64_t b = 0; b < B; ++b)
      for (int64_t h = 0; h < H; ++h) {
        if (Sq > 0)
          st = tg64_gemm(0, 0, Sq, D, 0, 1.0, nullptr, 1, 0, nullptr, 1, 0, beta,
                         dq + g.head(b, h, Sq), g.rs(), 0, 1, nullptr, s);
        if (!st && Sk > 0)
          st = tg64_gemm(0, 0, Sk, D, 0, 1.0, nullptr, 1, 0, nullptr, 1, 0, beta,
                         dk + g.head(b, h, Sk), g.rs(), 0, 1, nullptr, s);
        if (!st && Sk > 0)
          st = tg64_gemm(0, 0, Sk, D, 0, 1.0, nullptr, 1, 0, nullptr, 1, 0, beta,
                         dv + g.head(b, h, Sk), g.rs(), 0, 1, nullptr, s);
        if (st) return st;
      }
    return TG_OK;
  }
  const size_t need = tg_flash_attn_f64_workspace(B, H, Sq, Sk);
  TG_REQUIRE(workspace && workspace_bytes >= need,
             "tg_flash_attn_bwd_f64: workspace of %zu bytes needed", need);
  const int64_t hc = fa64_heads_per_chunk(H, Sq, Sk);
  double* P = (double*)workspace;
  double* dP = P + hc * Sq * Sk;
  const int64_t rs = g.rs(), hq = g.hstride(Sq), hk = g.hstride(Sk), ss = Sq * Sk;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h0 = 0; h0 < H; h0 += hc) {
      const int64_t n = hc < H - h0 ? hc : H - h0;
      const int64_t oq = g.head(b, h0, Sq), ok = g.head(b, h0, Sk);
      // P = exp(scale Q K^T - lse)
      st = tg64_gemm(0, 1, Sq, Sk, D, scale, q + oq, rs, hq, k + ok, rs, hk, 0.0, P, Sk, ss, n,
                     nullptr, s);
      if (st) return st;
      const int64_t e = n * ss;
      k64_fa_p<<<(unsigned)grid_for(e, kT * 4), kT, 0, s>>>(P, lse + (b * H + h0) * Sq, n * Sq,
                                                          Sq, Sk, causal);
      if ((st = tg_check_launch("tg_flash_attn_bwd_f64"))) return st;
      // dV (+)= P^T dO;  dP = dO V^T;  dS over dP;  dQ (+)= dS K;  dK (+)= dS^T Q
      st = tg64_gemm(1, 0, Sk, D, Sq, 1.0, P, Sk, ss, dout + oq, rs, hq, beta, dv + ok, rs, hk,
                     n, nullptr, s);
      if (!st)
        st = tg64_gemm(0, 1, Sq, Sk, D, 1.0, dout + oq, rs, hq, v + ok, rs, hk, 0.0, dP, Sk, ss,
                       n, nullptr, s);
      if (st) return st;
      k64_fa_ds<<<(unsigned)((n * Sq + 3) / 4), kT, 0, s>>>(P, dP, n * Sq, Sk, scale);
      if ((st = tg_check_launch("tg_flash_attn_bwd_f64"))) return st;
      st = tg64_gemm(0, 0, Sq, D, Sk, 1.0, dP, Sk, ss, k + ok, rs, hk, beta, dq + oq, rs, hq, n,
                     nullptr, s);
      if (!st)
        st = tg64_gemm(1, 0, Sk, D, Sq, 1.0, dP, Sk, ss, q + oq, rs, hq, beta, dk + ok, rs, hk,
                       n, nullptr, s);
      if (st) return st;
    }
  return TG_OK;
}

// ---------------------------------------------------------------- batch norm entries
TG_EXPORT size_t tg_batchnorm_stats_workspace(int64_t C) {
  return C > 0 ? (size_t)(3 * C) * sizeof(double) : 0;
}

TG_EXPORT int tg_batchnorm_fwd_train_f64(int layout, const double* x, const float* gamma,
                                         const float* beta, double* y, double* mean,
                                         double* rstd, double* var, double* running_mean,
                                         double* running_var, double momentum, int64_t N,
                                         int64_t C, int64_t HW, double eps, int relu,
                                         void* stream) {
  TG_REQUIRE(layout == 0 || layout == 1, "tg_batchnorm_fwd_train_f64: layout %d", layout);
  TG_REQUIRE(N >= 0 && C >= 0 && HW >= 0, "tg_batchnorm_fwd_train_f64: negative shape");
  const int64_t m = N * HW;
  if (C == 0) return TG_OK;
  TG_REQUIRE(m > 0, "tg_batchnorm_fwd_train_f64: no elements per channel");
  TG_REQUIRE(C <= 0x7fffffff, "tg_batchnorm_fwd_train_f64: too many channels");
  TG_REQUIRE(x && gamma && beta && y && mean && rstd, "tg_batchnorm_fwd_train_f64: null pointer");
  hipStream_t s = tg_stream(stream);
  k64_bn_stats<<<(unsigned)C, kT, 0, s>>>(layout, x, C, HW, m, eps, momentum, mean, var, rstd,
                                          running_mean, running_var);
  int st = tg_check_launch("tg_batchnorm_fwd_train_f64");
  if (st) return st;
  const int64_t n = m * C;
  k64_bn_apply<<<(unsigned)grid_for(n, kT * 4), kT, 0, s>>>(layout, x, gamma, beta, mean, rstd, y,
                                                            n, C, HW, relu);
  return tg_check_launch("tg_batchnorm_fwd_train_f64");
}

TG_EXPORT int tg_batchnorm_bwd_stats(int dtype, int layout, const void* x, const double* mean,
                                     const double* rstd, const float* gamma, const float* beta,
                                     const void* dy, void* dx, float* dgamma, float* dbeta,
                                     int64_t N, int64_t C, int64_t HW, int relu,
                                     int accumulate_dx, int accumulate_params, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  TG_REQUIRE(layout == 0 || layout == 1, "tg_batchnorm_bwd_stats: layout %d", layout);
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F64, "tg_batchnorm_bwd_stats: dtype %d", dtype);
  TG_REQUIRE(N >= 0 && C >= 0 && HW >= 0, "tg_batchnorm_bwd_stats: negative shape");
  const int64_t m = N * HW;
  if (C == 0) return TG_OK;
  TG_REQUIRE(m > 0, "tg_batchnorm_bwd_stats: no elements per channel");
  TG_REQUIRE(C <= 0x7fffffff, "tg_batchnorm_bwd_stats: too many channels");
  TG_REQUIRE(x && mean && rstd && gamma && beta && dy && dx, "tg_batchnorm_bwd_stats: null pointer");
  TG_REQUIRE(workspace && workspace_bytes >= tg_batchnorm_stats_workspace(C),
             "tg_batchnorm_bwd_stats: workspace of %zu bytes needed",
             tg_batchnorm_stats_workspace(C));
  hipStream_t s = tg_stream(stream);
  double* coef = (double*)workspace;
  const int64_t n = m * C;
#define BN(T)                                                                                   \
  k64_bn_bwd_sums<T><<<(unsigned)C, kT, 0, s>>>(layout, (const T*)x, mean, rstd, gamma, beta,   \
                                                (const T*)dy, C, HW, m, relu, dgamma, dbeta,    \
                                                accumulate_params, coef);                       \
  k64_bn_bwd_dx<T><<<(unsigned)grid_for(n, kT * 4), kT, 0, s>>>(                                \
      layout, (const T*)x, mean, rstd, gamma, beta, (const T*)dy, coef, (T*)dx, n, C, HW, relu,  \
      accumulate_dx)
  if (dtype == TG_F64) { BN(double); } else { BN(float); }
#undef BN
  return tg_check_launch("tg_batchnorm_bwd_stats");
}
