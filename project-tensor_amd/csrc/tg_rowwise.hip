// Row-wise kernels over a row-major [rows, cols] matrix:
//   softmax forward/backward along the last axis,
//   LayerNorm forward (saves mean, rstd) and backward (dx, dgamma, dbeta),
//   column sums (the unbroadcast reduction of a bias gradient).
//
// Register path: a row is split across TPR threads (a wavefront when TPR=64,
// the whole 256-thread block when TPR=256), each thread holding VPT 16-byte
// vectors, so every element of x/y/dy is read from HBM exactly once.  Row sums
// use wavefront butterflies plus one LDS exchange when TPR=256.  Shapes that do
// not fit (cols not a multiple of the vector width, misaligned, or very wide)
// take the looping wavefront-per-row path, which re-reads the row from cache.
#include "tg_common.h"

#include <mutex>

namespace {

constexpr int kBlock = 256;
// Outputs at least this large skip cache retention (non-temporal stores).
constexpr int64_t kNtBytes = 128ll << 20;

// ---------------------------------------------------------------------------
// Partial sums across the TPR threads of a row group.  For TPR == 256 the block
// is one group; `red` holds 4*NV floats.
template <int TPR, int NV>
__device__ __forceinline__ void group_sum(float (&v)[NV], float* red) {
  if (TPR == 64) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = tg_wave_sum(v[i]);
  } else {
    tg_block_sum<4, NV>(v, red);
  }
}
template <int TPR>
__device__ __forceinline__ float group_max(float v, float* red) {
  v = tg_wave_max(v);
  if (TPR == 64) return v;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}

// ============================ softmax ======================================
// Forward: y = exp(x - max) / sum(exp(x - max))   (_core.py:1286-1292)
template <typename T, int TPR, int VPT>
__global__ __launch_bounds__(kBlock) void k_softmax_fwd_reg(const T* __restrict__ x,
                                                            T* __restrict__ y, int64_t rows,
                                                            int cols) {
  constexpr int V = tg_vec16<T>::N;
  constexpr int G = kBlock / TPR;
  __shared__ float red[8];
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * G + threadIdx.x / TPR;
  const bool live = row < rows;
  const int nv = cols / V;
  const T* xr = x + (live ? row : 0) * (int64_t)cols;
  float xv[VPT][V];
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
    if (live && vi < nv) {
      tg_vec16<T> a = tg_load16(xr + vi * V);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        xv[k][j] = tg_to_float(a.v[j]);
        m = fmaxf(m, xv[k][j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) xv[k][j] = -INFINITY;
    }
  }
  m = group_max<TPR>(m, red);
  float s[1] = {0.f};
#pragma unroll
  for (int k = 0; k < VPT; ++k)
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float e = (xv[k][j] == -INFINITY) ? 0.f : __expf(xv[k][j] - m);
      xv[k][j] = e;
      s[0] += e;
    }
  group_sum<TPR, 1>(s, red);
  const float inv = 1.0f / s[0];
  if (!live) return;
  T* yr = y + row * (int64_t)cols;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
    if (vi < nv) {
      tg_vec16<T> o;
#pragma unroll
      for (int j = 0; j < V; ++j) o.v[j] = tg_from_float<T>(xv[k][j] * inv);
      tg_store16(yr + vi * V, o);
    }
  }
}

// Backward: dx (+)= y * (dy - sum(dy * y))   (_core.py:1294-1297)
template <typename T, int TPR, int VPT, bool ACC, bool NT>
__global__ __launch_bounds__(kBlock) void k_softmax_bwd_reg(const T* __restrict__ y,
                                                            const T* __restrict__ dy,
                                                            T* __restrict__ dx, int64_t rows,
                                                            int cols) {
  constexpr int V = tg_vec16<T>::N;
  constexpr int G = kBlock / TPR;
  __shared__ float red[8];
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * G + threadIdx.x / TPR;
  const bool live = row < rows;
  const int nv = cols / V;
  const int64_t off = (live ? row : 0) * (int64_t)cols;
  tg_vec16<T> yv[VPT], gv[VPT];
  float s[1] = {0.f};
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
    if (live && vi < nv) {
      yv[k] = tg_ld16<NT>(y + off + vi * V);
      gv[k] = tg_ld16<NT>(dy + off + vi * V);
#pragma unroll
      for (int j = 0; j < V; ++j) s[0] += tg_to_float(yv[k].v[j]) * tg_to_float(gv[k].v[j]);
    }
  }
  group_sum<TPR, 1>(s, red);
  if (!live) return;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
    if (vi < nv) {
      tg_vec16<T> o;
      if (ACC) o = tg_ld16<NT>(dx + off + vi * V);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float r = tg_to_float(yv[k].v[j]) * (tg_to_float(gv[k].v[j]) - s[0]);
        if (ACC) r += tg_to_float(o.v[j]);
        o.v[j] = tg_from_float<T>(r);
      }
      tg_st16<NT>(dx + off + vi * V, o);
    }
  }
}

// Looping wavefront-per-row variants for arbitrary cols.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_softmax_fwd_loop(const T* __restrict__ x,
                                                             T* __restrict__ y, int64_t rows,
                                                             int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  T* yr = y + row * cols;
  float m = -INFINITY;
  for (int64_t c = lane; c < cols; c += 64) m = fmaxf(m, tg_to_float(xr[c]));
  m = tg_wave_max(m);
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float v = tg_to_float(xr[c]);
    s += (v == -INFINITY) ? 0.f : __expf(v - m);
  }
  s = tg_wave_sum(s);
  const float inv = 1.0f / s;
  for (int64_t c = lane; c < cols; c += 64) {
    const float v = tg_to_float(xr[c]);
    yr[c] = tg_from_float<T>(((v == -INFINITY) ? 0.f : __expf(v - m)) * inv);
  }
}

template <typename T, bool ACC>
__global__ __launch_bounds__(kBlock) void k_softmax_bwd_loop(const T* __restrict__ y,
                                                             const T* __restrict__ dy,
                                                             T* __restrict__ dx, int64_t rows,
                                                             int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t off = row * cols;
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += tg_to_float(y[off + c]) * tg_to_float(dy[off + c]);
  s = tg_wave_sum(s);
  for (int64_t c = lane; c < cols; c += 64) {
    float r = tg_to_float(y[off + c]) * (tg_to_float(dy[off + c]) - s);
    if (ACC) r += tg_to_float(dx[off + c]);
    dx[off + c] = tg_from_float<T>(r);
  }
}

// Choose threads-per-row and vectors-per-thread for the register path.
// Returns false if the row does not fit the register path.
template <typename T>
bool pick_reg_shape(int64_t cols, bool aligned, int* tpr, int* vpt) {
  constexpr int V = tg_vec16<T>::N;
  if (!aligned || cols % V != 0 || cols <= 0) return false;
  const int64_t nv = cols / V;
  if (nv <= 64 * 4) {
    *tpr = 64;
    *vpt = nv <= 64 ? 1 : nv <= 128 ? 2 : 4;
    return true;
  }
  if (nv <= 256 * 8) {
    *tpr = 256;
    *vpt = nv <= 256 ? 1 : nv <= 512 ? 2 : nv <= 1024 ? 4 : 8;
    return true;
  }
  return false;
}

#define TG_REG_DISPATCH(KERNEL_LAUNCH)                   \
  switch (tpr * 16 + vpt) {                              \
    case 64 * 16 + 1: KERNEL_LAUNCH(64, 1); break;       \
    case 64 * 16 + 2: KERNEL_LAUNCH(64, 2); break;       \
    case 64 * 16 + 4: KERNEL_LAUNCH(64, 4); break;       \
    case 256 * 16 + 1: KERNEL_LAUNCH(256, 1); break;     \
    case 256 * 16 + 2: KERNEL_LAUNCH(256, 2); break;     \
    case 256 * 16 + 4: KERNEL_LAUNCH(256, 4); break;     \
    case 256 * 16 + 8: KERNEL_LAUNCH(256, 8); break;     \
  }

template <typename T>
int softmax_fwd_t(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t s) {
  int tpr = 0, vpt = 0;
  if (pick_reg_shape<T>(cols, tg_aligned16(x) && tg_aligned16(y), &tpr, &vpt)) {
    const int64_t g = kBlock / tpr;
    const unsigned blocks = (unsigned)((rows + g - 1) / g);
#define L(TPR, VPT) \
  k_softmax_fwd_reg<T, TPR, VPT><<<blocks, kBlock, 0, s>>>((const T*)x, (T*)y, rows, (int)cols)
    TG_REG_DISPATCH(L)
#undef L
  } else {
    k_softmax_fwd_loop<T><<<(unsigned)((rows + 3) / 4), kBlock, 0, s>>>((const T*)x, (T*)y, rows,
                                                                        cols);
  }
  return tg_check_launch("tg_softmax_fwd");
}

template <typename T>
int softmax_bwd_t(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols, int acc,
                  hipStream_t s) {
  int tpr = 0, vpt = 0;
  const bool al = tg_aligned16(y) && tg_aligned16(dy) && tg_aligned16(dx);
  if (pick_reg_shape<T>(cols, al, &tpr, &vpt)) {
    const int64_t g = kBlock / tpr;
    const unsigned blocks = (unsigned)((rows + g - 1) / g);
    const bool nt = (int64_t)sizeof(T) * rows * cols >= kNtBytes;
#define SMARGS (const T*)y, (const T*)dy, (T*)dx, rows, (int)cols
    if (acc) {
#define L(TPR, VPT)                                                                            \
  if (nt) k_softmax_bwd_reg<T, TPR, VPT, true, true><<<blocks, kBlock, 0, s>>>(SMARGS); \
  else k_softmax_bwd_reg<T, TPR, VPT, true, false><<<blocks, kBlock, 0, s>>>(SMARGS)
      TG_REG_DISPATCH(L)
#undef L
    } else {
#define L(TPR, VPT)                                                                             \
  if (nt) k_softmax_bwd_reg<T, TPR, VPT, false, true><<<blocks, kBlock, 0, s>>>(SMARGS); \
  else k_softmax_bwd_reg<T, TPR, VPT, false, false><<<blocks, kBlock, 0, s>>>(SMARGS)
      TG_REG_DISPATCH(L)
#undef L
    }
#undef SMARGS
  } else {
    const unsigned blocks = (unsigned)((rows + 3) / 4);
    if (acc)
      k_softmax_bwd_loop<T, true><<<blocks, kBlock, 0, s>>>((const T*)y, (const T*)dy, (T*)dx,
                                                            rows, cols);
    else
      k_softmax_bwd_loop<T, false><<<blocks, kBlock, 0, s>>>((const T*)y, (const T*)dy, (T*)dx,
                                                             rows, cols);
  }
  return tg_check_launch("tg_softmax_bwd");
}

// ============================ LayerNorm ====================================
// Forward (_nn.py:900-917): mean, population variance over the row,
// xhat = (x-mean)/sqrt(var+eps), y = gamma*xhat + beta.  Saves mean and
// rstd = 1/sqrt(var+eps) per row (fp32).
template <typename T, int TPR, int VPT>
__global__ __launch_bounds__(kBlock) void k_ln_fwd_reg(const T* __restrict__ x,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta,
                                                       T* __restrict__ y, float* __restrict__ mean,
                                                       float* __restrict__ rstd, int64_t rows,
                                                       int cols, float eps) {
  constexpr int V = tg_vec16<T>::N;
  constexpr int G = kBlock / TPR;
  __shared__ float red[8];
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * G + threadIdx.x / TPR;
  const bool live = row < rows;
  const int nv = cols / V;
  const int64_t off = (live ? row : 0) * (int64_t)cols;
  float xv[VPT][V];
  float s[1] = {0.f};
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
    if (live && vi < nv) {
      tg_vec16<T> a = tg_load16(x + off + vi * V);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        xv[k][j] = tg_to_float(a.v[j]);
        s[0] += xv[k][j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) xv[k][j] = 0.f;
    }
  }
  group_sum<TPR, 1>(s, red);
  const float mu = s[0] / (float)cols;
  float q[1] = {0.f};
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
    if (live && vi < nv) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float d = xv[k][j] - mu;
        q[0] += d * d;
      }
    }
  }
  group_sum<TPR, 1>(q, red);
  const float rs = 1.0f / sqrtf(q[0] / (float)cols + eps);
  if (!live) return;
  if (t == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
    if (vi < nv) {
      tg_vec16<T> o;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int c = vi * V + j;
        o.v[j] = tg_from_float<T>(gamma[c] * ((xv[k][j] - mu) * rs) + beta[c]);
      }
      tg_store16(y + off + vi * V, o);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_ln_fwd_loop(const T* __restrict__ x,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta,
                                                        T* __restrict__ y, float* __restrict__ mean,
                                                        float* __restrict__ rstd, int64_t rows,
                                                        int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t off = row * cols;
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += tg_to_float(x[off + c]);
  const float mu = tg_wave_sum(s) / (float)cols;
  float q = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float d = tg_to_float(x[off + c]) - mu;
    q += d * d;
  }
  const float rs = 1.0f / sqrtf(tg_wave_sum(q) / (float)cols + eps);
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
  for (int64_t c = lane; c < cols; c += 64)
    y[off + c] = tg_from_float<T>(gamma[c] * ((tg_to_float(x[off + c]) - mu) * rs) + beta[c]);
}

// Backward (_nn.py:921-942), with g = dy*gamma and xhat = (x-mean)*rstd:
//   dx (+)= rstd * (g - mean(g) - xhat * mean(g*xhat))
//   dgamma partial = sum_rows dy*xhat, dbeta partial = sum_rows dy
// Block b walks rows b, b+nblocks, ...; its threads own fixed columns, so the
// dgamma/dbeta partials stay in registers and are written once per block to
// part[b][0:cols] and part[nblocks + b][0:cols].  ACC: dx = (that) + dxin, where dxin
// is dx itself (accumulate in place) or another buffer (a gradient shared with another
// node, summed into this node's own buffer without copying it first); each element of
// dxin is read by the thread that writes that element of dx, before the write.
template <typename T, int TPR, int VPT, bool ACC, bool NT>
__global__ __launch_bounds__(kBlock) void k_ln_bwd_reg(
    const T* __restrict__ x, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gamma, const T* __restrict__ dy, T* dx, const T* dxin,
    float* __restrict__ part, int64_t rows, int cols) {
  constexpr int V = tg_vec16<T>::N;
  constexpr int G = kBlock / TPR;
  __shared__ float red[8];
  const int t = threadIdx.x % TPR;
  const int grp = threadIdx.x / TPR;
  const int nv = cols / V;
  float gam[VPT][V], pg[VPT][V], pb[VPT][V];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      gam[k][j] = (vi < nv) ? gamma[vi * V + j] : 0.f;
      pg[k][j] = 0.f;
      pb[k][j] = 0.f;
    }
  }
  const float inv_n = 1.0f / (float)cols;
  // Every group iterates the same number of times so block barriers stay uniform.
  const int64_t stride = (int64_t)gridDim.x * G;
  const int64_t iters = (rows + stride - 1) / stride;
  // Software pipeline: the next row's x/dy (and, when accumulating, the old dx, for
  // rows that leave room for it) and mean/rstd are loaded while the current row is
  // reduced and written; two rows ahead when that fits in registers.  Row buffers are whole structs copied by value, so
  // every register index is known at compile time.
  struct RowBuf {
    tg_vec16<T> x[VPT], y[VPT], o[ACC ? VPT : 1];
    float mu, rs;
  };
  constexpr bool kPreO = ACC && VPT <= 4;  // wider rows load the old dx late (no spill)
  // rows in flight per group: 2 where the registers allow (measured: 3 and 4 are slower
  // on the fp16 [8192, 1024] shape, 4 by a fifth)
  constexpr int kDepth = (ACC ? VPT <= 2 : VPT <= 4) ? 2 : 1;
  auto fetch = [&](int64_t it, RowBuf& b) {
    const int64_t row = it * stride + (int64_t)blockIdx.x * G + grp;
    if (row < rows) {
      const int64_t off = row * (int64_t)cols;
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int vi = t + k * TPR;
        if (vi < nv) {
          b.x[k] = tg_ld16<NT>(x + off + vi * V);
          b.y[k] = tg_ld16<NT>(dy + off + vi * V);
          if (kPreO) b.o[k] = tg_ld16<NT>(dxin + off + vi * V);
        }
      }
      b.mu = mean[row];
      b.rs = rstd[row];
    }
  };
  auto body = [&](int64_t it, const RowBuf& b) {
    const int64_t row = it * stride + (int64_t)blockIdx.x * G + grp;
    const bool live = row < rows;
    const int64_t off = (live ? row : 0) * (int64_t)cols;
    const float mu = b.mu, rs = b.rs;
    float xh[VPT][V], dyv[VPT][V];
    float sums[2] = {0.f, 0.f};
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int vi = t + k * TPR;
      if (live && vi < nv) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
          xh[k][j] = (tg_to_float(b.x[k].v[j]) - mu) * rs;
          dyv[k][j] = tg_to_float(b.y[k].v[j]);
          const float g = dyv[k][j] * gam[k][j];
          sums[0] += g;
          sums[1] += g * xh[k][j];
          pg[k][j] += dyv[k][j] * xh[k][j];
          pb[k][j] += dyv[k][j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < V; ++j) {
          xh[k][j] = 0.f;
          dyv[k][j] = 0.f;
        }
      }
    }
    group_sum<TPR, 2>(sums, red);
    if (live) {
      const float mg = sums[0] * inv_n, mgx = sums[1] * inv_n;
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int vi = t + k * TPR;
        if (vi < nv) {
          tg_vec16<T> o;
          if (ACC && !kPreO) o = tg_ld16<NT>(dxin + off + vi * V);
#pragma unroll
          for (int j = 0; j < V; ++j) {
            float r = rs * (dyv[k][j] * gam[k][j] - mg - xh[k][j] * mgx);
            if (ACC) r += tg_to_float(kPreO ? b.o[k].v[j] : o.v[j]);
            o.v[j] = tg_from_float<T>(r);
          }
          tg_st16<NT>(dx + off + vi * V, o);
        }
      }
    }
  };
  // kDepth row buffers in a ring (the loop is unrolled by kDepth, so each buffer's
  // registers are fixed): row it + kDepth is fetched as row it is processed
  RowBuf ring[kDepth], cur;
#pragma unroll
  for (int j = 0; j < kDepth; ++j)
    if (j < iters) fetch(j, ring[j]);
  for (int64_t it = 0; it < iters; it += kDepth) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      if (it + j < iters) {  // uniform across the block, as iters is
        cur = ring[j];
        if (it + j + kDepth < iters) fetch(it + j + kDepth, ring[j]);
        body(it + j, cur);
      }
    }
  }
  // Combine the G row groups of this block, then write the block partial.
  // (G > 1 only when TPR == 64; LDS holds G-1 groups' partials one vector at a time.)
  __shared__ float xch[2][kBlock / 64 - 1][64 * 8];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int vi = t + k * TPR;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      if (G > 1) {
        if (grp > 0) {
          xch[0][grp - 1][t * V + j] = pg[k][j];
          xch[1][grp - 1][t * V + j] = pb[k][j];
        }
      }
    }
    if (G > 1) {
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int j = 0; j < V; ++j)
#pragma unroll
          for (int q = 0; q < G - 1; ++q) {
            pg[k][j] += xch[0][q][t * V + j];
            pb[k][j] += xch[1][q][t * V + j];
          }
      }
      __syncthreads();
    }
    if (grp == 0 && vi < nv) {
      float* pgo = part + (int64_t)blockIdx.x * cols + vi * V;
      float* pbo = part + ((int64_t)gridDim.x + blockIdx.x) * cols + vi * V;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        pgo[j] = pg[k][j];
        pbo[j] = pb[k][j];
      }
    }
  }
}

// Generic LayerNorm backward: wavefront per row for dx; dgamma/dbeta partials
// go through a per-block LDS-free scheme: each block owns a row range and
// accumulates per-column sums with a column loop after its rows (re-reading them).
template <typename T, bool ACC>
__global__ __launch_bounds__(kBlock) void k_ln_bwd_dx_loop(
    const T* __restrict__ x, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gamma, const T* __restrict__ dy, T* dx, const T* dxin, int64_t rows,
    int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t off = row * cols;
  const float mu = mean[row], rs = rstd[row];
  float a = 0.f, b = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float xh = (tg_to_float(x[off + c]) - mu) * rs;
    const float g = tg_to_float(dy[off + c]) * gamma[c];
    a += g;
    b += g * xh;
  }
  const float mg = tg_wave_sum(a) / (float)cols, mgx = tg_wave_sum(b) / (float)cols;
  for (int64_t c = lane; c < cols; c += 64) {
    const float xh = (tg_to_float(x[off + c]) - mu) * rs;
    float r = rs * (tg_to_float(dy[off + c]) * gamma[c] - mg - xh * mgx);
    if (ACC) r += tg_to_float(dxin[off + c]);
    dx[off + c] = tg_from_float<T>(r);
  }
}

// dgamma/dbeta partials for the generic path: grid (ceil(cols/256), nsplit);
// part[split][c] = sum over the split's rows of dy*xhat, part[nsplit+split][c] of dy.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_ln_bwd_param_loop(
    const T* __restrict__ x, const float* __restrict__ mean, const float* __restrict__ rstd,
    const T* __restrict__ dy, float* __restrict__ part, int64_t rows, int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= cols) return;
  const int64_t nsplit = gridDim.y;
  const int64_t per = (rows + nsplit - 1) / nsplit;
  const int64_t r0 = blockIdx.y * per;
  const int64_t r1 = r0 + per < rows ? r0 + per : rows;
  float sg = 0.f, sb = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float d = tg_to_float(dy[r * cols + c]);
    sg += d * (tg_to_float(x[r * cols + c]) - mean[r]) * rstd[r];
    sb += d;
  }
  part[(int64_t)blockIdx.y * cols + c] = sg;
  part[(nsplit + blockIdx.y) * cols + c] = sb;
}

// ============================ column sums ==================================
// Stage 1: part[split][c] = sum over rows in split of in[r][c]   (grid: ctiles x nsplit)
template <typename TI>
__global__ __launch_bounds__(kBlock) void k_colsum_partial(const TI* __restrict__ in,
                                                           float* __restrict__ part, int64_t rows,
                                                           int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= cols) return;
  const int64_t nsplit = gridDim.y;
  const int64_t per = (rows + nsplit - 1) / nsplit;
  const int64_t r0 = blockIdx.y * per;
  const int64_t r1 = r0 + per < rows ? r0 + per : rows;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int64_t r = r0;
  for (; r + 4 <= r1; r += 4) {
    s0 += tg_to_float(in[(r + 0) * cols + c]);
    s1 += tg_to_float(in[(r + 1) * cols + c]);
    s2 += tg_to_float(in[(r + 2) * cols + c]);
    s3 += tg_to_float(in[(r + 3) * cols + c]);
  }
  for (; r < r1; ++r) s0 += tg_to_float(in[r * cols + c]);
  part[(int64_t)blockIdx.y * cols + c] = (s0 + s1) + (s2 + s3);
}

// Stage 1 with 16-byte loads, for a [rows, cols] input with cols % V == 0 and a
// 16-byte aligned base: a block covers 64 vector columns (one per lane, so a wave
// reads a contiguous 1 KiB row segment for 16-bit input); its 4 waves take rows
// r0+w, r0+w+4, ... of the block's split with four loads in flight; the wave sums
// are combined through LDS in a fixed order (deterministic).
template <typename TI>
__global__ __launch_bounds__(kBlock) void k_colsum_partial_v(const TI* __restrict__ in,
                                                             float* __restrict__ part,
                                                             int64_t rows, int64_t cols,
                                                             int64_t per) {
  constexpr int V = tg_vec16<TI>::N;
  constexpr int W = kBlock / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nvc = cols / V;
  const int64_t cv = (int64_t)blockIdx.x * 64 + lane;
  const int64_t r0 = (int64_t)blockIdx.y * per;
  const int64_t r1 = r0 + per < rows ? r0 + per : rows;
  float acc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) acc[j] = 0.f;
  if (cv < nvc) {
    const TI* p = in + cv * V;
    int64_t r = r0 + wave;
    for (; r + 3 * W < r1; r += 4 * W) {
      tg_vec16<TI> v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = tg_load16(p + (r + u * W) * cols);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < V; ++j) acc[j] += tg_to_float(v[u].v[j]);
    }
    for (; r < r1; r += W) {
      const tg_vec16<TI> v = tg_load16(p + r * cols);
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] += tg_to_float(v.v[j]);
    }
  }
  __shared__ float red[W - 1][V][64];
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < V; ++j) red[wave - 1][j][lane] = acc[j];
  }
  __syncthreads();
  if (wave == 0 && cv < nvc) {
#pragma unroll
    for (int w = 0; w < W - 1; ++w)
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] += red[w][j][lane];
    float* o = part + (int64_t)blockIdx.y * cols + cv * V;
#pragma unroll
    for (int j = 0; j < V; j += 4)
      *reinterpret_cast<float4*>(o + j) = make_float4(acc[j], acc[j + 1], acc[j + 2], acc[j + 3]);
  }
}

// Row splits of tg_reduce_rows: enough blocks to fill the CUs (counted in 512-column
// tiles, the vector kernel's width for 16-bit input) with at least 32 rows per split.
int64_t rr_splits(int64_t rows, int64_t cols) {
  const int64_t ctiles = (cols + 511) / 512;
  int64_t want = (4 * (int64_t)tg_num_cus() + ctiles - 1) / ctiles;
  int64_t maxs = rows / 32;
  if (want > maxs) want = maxs;
  if (want > 2048) want = 2048;
  if (want < 1) want = 1;
  return want;
}

int64_t colsum_splits(int64_t rows, int64_t cols) {
  const int64_t ctiles = (cols + kBlock - 1) / kBlock;
  int64_t want = (4 * (int64_t)tg_num_cus() + ctiles - 1) / ctiles;
  int64_t maxs = rows / 16;
  if (want > maxs) want = maxs;
  if (want > 1024) want = 1024;
  if (want < 1) want = 1;
  return want;
}

// Row-groups per LayerNorm-backward launch (the number of dgamma/dbeta partials): one
// block per CU.  Measured on the MI355X against two and three per CU, one is faster at
// every shape tried (fewer partials to write and finish; the two-row prefetch keeps
// enough loads in flight).
int64_t ln_bwd_blocks(int64_t rows, int tpr) {
  const int64_t g = kBlock / tpr;
  int64_t want = (int64_t)tg_num_cus();
  const int64_t maxb = (rows + g - 1) / g;
  if (want > maxb) want = maxb;
  if (want < 1) want = 1;
  return want;
}

template <typename T>
int ln_fwd_t(const void* x, const float* gamma, const float* beta, void* y, float* mean,
             float* rstd, int64_t rows, int64_t cols, float eps, hipStream_t s) {
  int tpr = 0, vpt = 0;
  if (pick_reg_shape<T>(cols, tg_aligned16(x) && tg_aligned16(y), &tpr, &vpt)) {
    const int64_t g = kBlock / tpr;
    const unsigned blocks = (unsigned)((rows + g - 1) / g);
#define L(TPR, VPT)                                                                     \
  k_ln_fwd_reg<T, TPR, VPT><<<blocks, kBlock, 0, s>>>((const T*)x, gamma, beta, (T*)y, mean, \
                                                      rstd, rows, (int)cols, eps)
    TG_REG_DISPATCH(L)
#undef L
  } else {
    k_ln_fwd_loop<T><<<(unsigned)((rows + 3) / 4), kBlock, 0, s>>>(
        (const T*)x, gamma, beta, (T*)y, mean, rstd, rows, cols, eps);
  }
  return tg_check_launch("tg_layernorm_fwd");
}

struct LnBwdPlan {
  bool reg;
  int tpr, vpt;
  int64_t nparts;  // number of dgamma (and dbeta) partial rows in the workspace
};

template <typename T>
LnBwdPlan ln_bwd_plan(int64_t rows, int64_t cols, bool aligned) {
  LnBwdPlan p{};
  p.reg = pick_reg_shape<T>(cols, aligned, &p.tpr, &p.vpt);
  p.nparts = p.reg ? ln_bwd_blocks(rows, p.tpr) : colsum_splits(rows, cols);
  return p;
}

LnBwdPlan ln_bwd_plan_dt(int dtype, int64_t rows, int64_t cols, bool aligned) {
  switch (dtype) {
    case TG_F16: return ln_bwd_plan<tg_half>(rows, cols, aligned);
    case TG_BF16: return ln_bwd_plan<tg_bf16>(rows, cols, aligned);
    default: return ln_bwd_plan<float>(rows, cols, aligned);
  }
}

template <typename T>
int ln_bwd_t(const void* x, const float* mean, const float* rstd, const float* gamma,
             const void* dy, void* dx, const void* dxin, float* dgamma, float* dbeta,
             int64_t rows, int64_t cols,
             int acc_dx, int acc_params, float* part, const LnBwdPlan& p, hipStream_t s) {
  if (p.reg) {
    const unsigned blocks = (unsigned)p.nparts;
    const int tpr = p.tpr, vpt = p.vpt;
    const bool nt = (int64_t)sizeof(T) * rows * cols >= kNtBytes;
#define LNARGS \
  (const T*)x, mean, rstd, gamma, (const T*)dy, (T*)dx, (const T*)dxin, part, rows, (int)cols
    if (acc_dx) {
#define L(TPR, VPT)                                                                           \
  if (nt) k_ln_bwd_reg<T, TPR, VPT, true, true><<<blocks, kBlock, 0, s>>>(LNARGS); \
  else k_ln_bwd_reg<T, TPR, VPT, true, false><<<blocks, kBlock, 0, s>>>(LNARGS)
      TG_REG_DISPATCH(L)
#undef L
    } else {
#define L(TPR, VPT)                                                                            \
  if (nt) k_ln_bwd_reg<T, TPR, VPT, false, true><<<blocks, kBlock, 0, s>>>(LNARGS); \
  else k_ln_bwd_reg<T, TPR, VPT, false, false><<<blocks, kBlock, 0, s>>>(LNARGS)
      TG_REG_DISPATCH(L)
#undef L
    }
#undef LNARGS
  } else {
    const unsigned blocks = (unsigned)((rows + 3) / 4);
    if (acc_dx)
      k_ln_bwd_dx_loop<T, true><<<blocks, kBlock, 0, s>>>((const T*)x, mean, rstd, gamma,
                                                          (const T*)dy, (T*)dx, (const T*)dxin,
                                                          rows, cols);
    else
      k_ln_bwd_dx_loop<T, false><<<blocks, kBlock, 0, s>>>((const T*)x, mean, rstd, gamma,
                                                           (const T*)dy, (T*)dx, (const T*)dxin,
                                                           rows, cols);
    dim3 grid((unsigned)((cols + kBlock - 1) / kBlock), (unsigned)p.nparts);
    k_ln_bwd_param_loop<T><<<grid, kBlock, 0, s>>>((const T*)x, mean, rstd, (const T*)dy, part,
                                                   rows, cols);
  }
  int st = tg_check_launch("tg_layernorm_bwd");
  if (st) return st;
  if (!dgamma && !dbeta) return TG_OK;
  return tg_sum_partials2(part, p.nparts, cols, TG_F32, dgamma, dbeta, acc_params,
                          part + 2 * p.nparts * cols, s);
}

}  // namespace

// ============================ exported C-ABI ===============================

TG_EXPORT int tg_softmax_fwd(int dtype, const void* x, void* y, int64_t rows, int64_t cols,
                             void* stream) {
  TG_REQUIRE(rows >= 0 && cols >= 0, "tg_softmax_fwd: negative shape");
  if (rows == 0 || cols == 0) return TG_OK;
  TG_REQUIRE(x && y, "tg_softmax_fwd: null pointer");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: return softmax_fwd_t<float>(x, y, rows, cols, s);
    case TG_F16: return softmax_fwd_t<tg_half>(x, y, rows, cols, s);
    case TG_BF16: return softmax_fwd_t<tg_bf16>(x, y, rows, cols, s);
    case TG_F64: return tg64_softmax_fwd(x, y, rows, cols, s);
  }
  tg_set_error("tg_softmax_fwd: unsupported dtype %d", dtype);
  return TG_ERR_UNSUPPORTED;
}

TG_EXPORT int tg_softmax_bwd(int dtype, const void* y, const void* dy, void* dx, int64_t rows,
                             int64_t cols, int accumulate, void* stream) {
  TG_REQUIRE(rows >= 0 && cols >= 0, "tg_softmax_bwd: negative shape");
  if (rows == 0 || cols == 0) return TG_OK;
  TG_REQUIRE(y && dy && dx, "tg_softmax_bwd: null pointer");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: return softmax_bwd_t<float>(y, dy, dx, rows, cols, accumulate, s);
    case TG_F16: return softmax_bwd_t<tg_half>(y, dy, dx, rows, cols, accumulate, s);
    case TG_BF16: return softmax_bwd_t<tg_bf16>(y, dy, dx, rows, cols, accumulate, s);
    case TG_F64: return tg64_softmax_bwd(y, dy, dx, rows, cols, accumulate, s);
  }
  tg_set_error("tg_softmax_bwd: unsupported dtype %d", dtype);
  return TG_ERR_UNSUPPORTED;
}

TG_EXPORT int tg_layernorm_fwd(int dtype, const void* x, const float* gamma, const float* beta,
                               void* y, float* mean, float* rstd, int64_t rows, int64_t cols,
                               float eps, void* stream) {
  TG_REQUIRE(rows >= 0 && cols > 0, "tg_layernorm_fwd: bad shape");
  if (rows == 0) return TG_OK;
  TG_REQUIRE(x && gamma && beta && y && mean && rstd, "tg_layernorm_fwd: null pointer");
  hipStream_t s = tg_stream(stream);
  switch (dtype) {
    case TG_F32: return ln_fwd_t<float>(x, gamma, beta, y, mean, rstd, rows, cols, eps, s);
    case TG_F16: return ln_fwd_t<tg_half>(x, gamma, beta, y, mean, rstd, rows, cols, eps, s);
    case TG_BF16: return ln_fwd_t<tg_bf16>(x, gamma, beta, y, mean, rstd, rows, cols, eps, s);
    case TG_F64: return tg64_layernorm_fwd(x, gamma, beta, y, mean, rstd, rows, cols, eps, s);
  }
  tg_set_error("tg_layernorm_fwd: unsupported dtype %d", dtype);
  return TG_ERR_UNSUPPORTED;
}

TG_EXPORT size_t tg_layernorm_bwd_workspace(int dtype, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  if (dtype == TG_F64) return tg64_layernorm_bwd_workspace(rows, cols);
  // Alignment unknown at query time: size for the larger of the two plans.
  LnBwdPlan a = ln_bwd_plan_dt(dtype, rows, cols, true);
  LnBwdPlan b = ln_bwd_plan_dt(dtype, rows, cols, false);
  const int64_t np = a.nparts > b.nparts ? a.nparts : b.nparts;
  return (size_t)(2 * np * cols) * sizeof(float) + tg_sum_partials_scratch(np, cols, 2);
}

namespace {
// dx = LayerNorm dx (+ dxin when dxin is non-null; dxin may be dx itself).
int ln_bwd_entry(const char* who, int dtype, const void* x, const float* mean, const float* rstd,
                 const float* gamma, const void* dy, void* dx, const void* dxin, float* dgamma,
                 float* dbeta, int64_t rows, int64_t cols, int accumulate_params,
                 void* workspace, size_t workspace_bytes, void* stream) {
  TG_REQUIRE(rows >= 0 && cols > 0, "%s: bad shape", who);
  if (rows == 0) return TG_OK;
  TG_REQUIRE(x && mean && rstd && gamma && dy && dx, "%s: null pointer", who);
  hipStream_t s = tg_stream(stream);
  if (dtype == TG_F64) {
    const size_t need64 = tg64_layernorm_bwd_workspace(rows, cols);
    if ((dgamma || dbeta) && (!workspace || workspace_bytes < need64)) {
      tg_set_error("%s: workspace of %zu bytes needed, got %zu", who, need64,
                   workspace ? workspace_bytes : (size_t)0);
      return TG_ERR_WORKSPACE;
    }
    if (dxin && dxin != dx) {
      // the fp64 kernels accumulate in place: start dx from dxin
      const hipError_t e = hipMemcpyAsync(dx, dxin, (size_t)(rows * cols) * sizeof(double),
                                          hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) {
        tg_set_error("%s: hipMemcpyAsync: %s", who, hipGetErrorString(e));
        return TG_ERR_HIP;
      }
    }
    return tg64_layernorm_bwd(x, mean, rstd, gamma, dy, dx, dgamma, dbeta, rows, cols,
                              dxin != nullptr, accumulate_params, workspace, s);
  }
  const bool al = tg_aligned16(x) && tg_aligned16(dy) && tg_aligned16(dx) &&
                  (!dxin || tg_aligned16(dxin));
  LnBwdPlan p = ln_bwd_plan_dt(dtype, rows, cols, al);
  const size_t need =
      (size_t)(2 * p.nparts * cols) * sizeof(float) + tg_sum_partials_scratch(p.nparts, cols, 2);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("%s: workspace of %zu bytes needed, got %zu", who, need,
                 workspace ? workspace_bytes : (size_t)0);
    return TG_ERR_WORKSPACE;
  }
  float* part = (float*)workspace;
  const int acc = dxin != nullptr;
  switch (dtype) {
    case TG_F32:
      return ln_bwd_t<float>(x, mean, rstd, gamma, dy, dx, dxin, dgamma, dbeta, rows, cols, acc,
                             accumulate_params, part, p, s);
    case TG_F16:
      return ln_bwd_t<tg_half>(x, mean, rstd, gamma, dy, dx, dxin, dgamma, dbeta, rows, cols,
                               acc, accumulate_params, part, p, s);
    case TG_BF16:
      return ln_bwd_t<tg_bf16>(x, mean, rstd, gamma, dy, dx, dxin, dgamma, dbeta, rows, cols,
                               acc, accumulate_params, part, p, s);
  }
  tg_set_error("%s: unsupported dtype %d", who, dtype);
  return TG_ERR_UNSUPPORTED;
}
}  // namespace

TG_EXPORT int tg_layernorm_bwd(int dtype, const void* x, const float* mean, const float* rstd,
                               const float* gamma, const void* dy, void* dx, float* dgamma,
                               float* dbeta, int64_t rows, int64_t cols, int accumulate_dx,
                               int accumulate_params, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return ln_bwd_entry("tg_layernorm_bwd", dtype, x, mean, rstd, gamma, dy, dx,
                      accumulate_dx ? dx : nullptr, dgamma, dbeta, rows, cols,
                      accumulate_params, workspace, workspace_bytes, stream);
}

TG_EXPORT int64_t tg_layernorm_bwd_partials(int dtype, const void* x, const void* dy,
                                            const void* dx, const void* dx_add, int64_t rows,
                                            int64_t cols) {
  if (rows <= 0 || cols <= 0 || dtype == TG_F64) return -1;
  if (dtype != TG_F32 && dtype != TG_F16 && dtype != TG_BF16) return -1;
  const bool al = tg_aligned16(x) && tg_aligned16(dy) && tg_aligned16(dx) &&
                  (!dx_add || tg_aligned16(dx_add));
  const LnBwdPlan p = ln_bwd_plan_dt(dtype, rows, cols, al);
  return tg_sum_partials_groupable(p.nparts, cols) ? p.nparts : -1;
}

TG_EXPORT int tg_layernorm_bwd_add(int dtype, const void* x, const float* mean,
                                   const float* rstd, const float* gamma, const void* dy,
                                   const void* dx_add, void* dx, float* dgamma, float* dbeta,
                                   int64_t rows, int64_t cols, int accumulate_params,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  TG_REQUIRE(dx_add || rows == 0, "tg_layernorm_bwd_add: null dx_add");
  return ln_bwd_entry("tg_layernorm_bwd_add", dtype, x, mean, rstd, gamma, dy, dx, dx_add,
                      dgamma, dbeta, rows, cols, accumulate_params, workspace, workspace_bytes,
                      stream);
}

// ---- LayerNorm backward without a caller workspace -------------------------
// The dgamma/dbeta partial rows (and the staging of their column sum) live in this
// file-scope device array instead of a workspace argument.  Every GPU the library
// runs on holds its own copy until the process ends.  Host code must not pass the
// array's name to a kernel (on the host it names a stand-in, not device memory): the
// device address is looked up once per device and kept in g_ln_scratch.  Every
// partial row is written before it is read, so nothing needs clearing between calls.
static constexpr size_t kLnScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kLnScratchBytes];

static std::mutex g_ln_scratch_mu;
static void* g_ln_scratch[64];

static int ln_scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) {
    tg_set_error("tg_layernorm_bwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return TG_ERR_HIP;
  }
  std::lock_guard<std::mutex> lk(g_ln_scratch_mu);
  if (!g_ln_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      tg_set_error("tg_layernorm_bwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                   dev, hipGetErrorString(e));
      return TG_ERR_HIP;
    }
    g_ln_scratch[dev] = p;
  }
  *out = g_ln_scratch[dev];
  return TG_OK;
}

TG_EXPORT size_t tg_layernorm_bwd_noalloc_max_scratch(void) { return kLnScratchBytes; }

TG_EXPORT int tg_layernorm_bwd_noalloc(int dtype, const void* x, const float* mean,
                                       const float* rstd, const float* gamma, const void* dy,
                                       void* dx, float* dgamma, float* dbeta, int64_t rows,
                                       int64_t cols, int accumulate_dx, int accumulate_params,
                                       void* stream) {
  TG_REQUIRE(rows >= 0 && cols > 0, "tg_layernorm_bwd_noalloc: bad shape");
  if (rows == 0) return TG_OK;
  TG_REQUIRE(x && mean && rstd && gamma && dy && dx, "tg_layernorm_bwd_noalloc: null pointer");
  TG_REQUIRE(dtype == TG_F32 || dtype == TG_F16 || dtype == TG_BF16,
             "tg_layernorm_bwd_noalloc: unsupported dtype %d", dtype);
  const bool al = tg_aligned16(x) && tg_aligned16(dy) && tg_aligned16(dx);
  LnBwdPlan p = ln_bwd_plan_dt(dtype, rows, cols, al);
  const size_t need =
      (size_t)(2 * p.nparts * cols) * sizeof(float) + tg_sum_partials_scratch(p.nparts, cols, 2);
  if (need > kLnScratchBytes) {
    tg_set_error("tg_layernorm_bwd_noalloc: [%lld, %lld] needs %zu bytes of scratch, above the "
                 "fixed %zu; use tg_layernorm_bwd with a workspace",
                 (long long)rows, (long long)cols, need, kLnScratchBytes);
    return TG_ERR_INVALID;
  }
  void* ws = nullptr;
  int st = ln_scratch_ptr(&ws);
  if (st) return st;
  return tg_layernorm_bwd(dtype, x, mean, rstd, gamma, dy, dx, dgamma, dbeta, rows, cols,
                          accumulate_dx, accumulate_params, ws, kLnScratchBytes, stream);
}

TG_EXPORT size_t tg_reduce_rows_workspace(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int64_t ns = rr_splits(rows, cols);
  // sized for fp64 partials (the fp64 path keeps its partial sums in double)
  return (size_t)(ns * cols) * sizeof(double) + tg_sum_partials_scratch(ns, cols);
}

// out[c] (+)= sum_r in[r][c] for a row-major [rows, cols] input: the reduction that
// unbroadcasts a [.., cols] gradient onto a [cols] parameter (_core.py:1380-1424).
TG_EXPORT int tg_reduce_rows(int dtype_in, const void* in, int dtype_out, void* out,
                             int64_t rows, int64_t cols, int accumulate, void* workspace,
                             size_t workspace_bytes, void* stream) {
  TG_REQUIRE(rows >= 0 && cols >= 0, "tg_reduce_rows: negative shape");
  if (cols == 0) return TG_OK;
  TG_REQUIRE(out, "tg_reduce_rows: null output");
  hipStream_t s = tg_stream(stream);
  if (rows == 0) {
    if (accumulate) return TG_OK;
    // sum over zero rows is zero
    if (dtype_out == TG_F64) return tg64_fill(out, cols, 0.0, s);
    return tg_sum_partials(nullptr, 0, cols, dtype_out, out, 0, nullptr, s);
  }
  TG_REQUIRE(in, "tg_reduce_rows: null input");
  if (dtype_in == TG_F64 || dtype_out == TG_F64)  // fp64 sums in fixed order (tg_f64.hip)
    return tg64_reduce_rows(dtype_in, in, dtype_out, out, rows, cols, accumulate, workspace,
                            workspace_bytes, s);
  // A few fp32 rows over many columns (split-K GEMM partials): the finishing column
  // sum reads them directly, one launch instead of partials plus a copy.
  if (dtype_in == TG_F32 && rows <= 64 && cols >= 4096)
    return tg_sum_partials((const float*)in, rows, cols, dtype_out, out, accumulate, nullptr, s);
  const int64_t ns = rr_splits(rows, cols);
  const size_t need = (size_t)(ns * cols) * sizeof(float) + tg_sum_partials_scratch(ns, cols);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("tg_reduce_rows: workspace of %zu bytes needed, got %zu", need,
                 workspace ? workspace_bytes : (size_t)0);
    return TG_ERR_WORKSPACE;
  }
  float* part = (float*)workspace;
  const int64_t per = (rows + ns - 1) / ns;
  const int vw = dtype_in == TG_F32 ? 4 : 8;  // elements per 16-byte vector
  if ((dtype_in == TG_F32 || dtype_in == TG_F16 || dtype_in == TG_BF16) && cols % vw == 0 &&
      tg_aligned16(in)) {
    dim3 gv((unsigned)((cols / vw + 63) / 64), (unsigned)ns);
    switch (dtype_in) {
      case TG_F32: k_colsum_partial_v<float><<<gv, kBlock, 0, s>>>((const float*)in, part, rows, cols, per); break;
      case TG_F16: k_colsum_partial_v<tg_half><<<gv, kBlock, 0, s>>>((const tg_half*)in, part, rows, cols, per); break;
      default: k_colsum_partial_v<tg_bf16><<<gv, kBlock, 0, s>>>((const tg_bf16*)in, part, rows, cols, per); break;
    }
    int st = tg_check_launch("tg_reduce_rows");
    if (st) return st;
    return tg_sum_partials(part, ns, cols, dtype_out, out, accumulate, part + ns * cols, s);
  }
  dim3 grid((unsigned)((cols + kBlock - 1) / kBlock), (unsigned)ns);
  switch (dtype_in) {
    case TG_F32: k_colsum_partial<float><<<grid, kBlock, 0, s>>>((const float*)in, part, rows, cols); break;
    case TG_F16: k_colsum_partial<tg_half><<<grid, kBlock, 0, s>>>((const tg_half*)in, part, rows, cols); break;
    case TG_BF16: k_colsum_partial<tg_bf16><<<grid, kBlock, 0, s>>>((const tg_bf16*)in, part, rows, cols); break;
    default:
      tg_set_error("tg_reduce_rows: unsupported input dtype %d", dtype_in);
      return TG_ERR_UNSUPPORTED;
  }
  int st = tg_check_launch("tg_reduce_rows");
  if (st) return st;
  return tg_sum_partials(part, ns, cols, dtype_out, out, accumulate, part + ns * cols, s);
}
