// Training-mode BatchNorm(+ReLU) forward statistics and backward, fp32.
//
// Layouts: TG_NHWC (channel-last, a row-major [M = N*H*W, C] matrix) and TG_NCHW
// (the reference module's layout, [N][C][HW]).  Reference: FusedBatchNormReLU
// (_nn.py:750-836) and BatchNorm2D (_nn.py:681-747).
//
// Backward is two HBM passes, because dx needs full-batch per-channel sums:
//   pass 1 (reduce): per channel S1 = sum dy_m, S2 = sum dy_m*xhat, where
//           xhat = (x-mean)*rstd and dy_m = dy*[gamma*xhat+beta > 0] (ReLU mask
//           recomputed from x instead of reading the saved output);
//   pass 2 (apply):  dx (+)= gamma*rstd*(dy_m - S1/m - xhat*S2/m),
// which is the reference's dvar/dmean chain with sum(x - mean) = 0 folded in.
// dgamma (+)= S2 and dbeta (+)= S1.
//
// The ReLU mask is evaluated with contraction disabled, in the reference
// forward's operation order ((x-mean)*rstd, then *gamma, then +beta), so given the
// same mean/rstd it is bit-identical to the mask of the forward pass.
#include "tg_common.h"

namespace {

constexpr int kBlock = 256;
enum { TG_NHWC = 0, TG_NCHW = 1 };

__device__ __forceinline__ float bn_xhat(float x, float mu, float rs) {
#pragma clang fp contract(off)
  return (x - mu) * rs;
}
__device__ __forceinline__ bool bn_relu_on(float xh, float g, float b) {
#pragma clang fp contract(off)
  const float v = g * xh + b;
  return v > 0.f;
}
__device__ __forceinline__ float bn_affine(float xh, float g, float b) {
#pragma clang fp contract(off)
  return g * xh + b;
}

// ---------------------------------------------------------------------------
// NHWC channel reductions.  Block = 4 wavefronts; lane l of a wave owns channel
// vector (blockIdx.y*64 + l) (V channels), the 4 waves take interleaved rows of
// the block's row range; the block writes one partial per channel.
// MODE 0: sum x.  MODE 1: sum (x-mean)^2.  MODE 2 (backward): sum dy_m, sum dy_m*xhat.
template <int V, int MODE, bool NTL = false>
__global__ __launch_bounds__(kBlock) void k_nhwc_reduce(
    const float* __restrict__ x, const float* __restrict__ dy, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, int relu, float* __restrict__ part, int64_t M, int64_t C) {
  constexpr int NS = MODE == 2 ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c0 = ((int64_t)blockIdx.y * 64 + lane) * V;
  const bool cl = c0 < C;
  const int64_t nsplit = gridDim.x;
  const int64_t per = (M + nsplit - 1) / nsplit;
  const int64_t r0 = (int64_t)blockIdx.x * per;
  const int64_t r1 = r0 + per < M ? r0 + per : M;
  float mu[V], rs[V], g[V], b[V];
  float acc[NS][V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    mu[j] = (MODE >= 1 && cl) ? mean[c0 + j] : 0.f;
    rs[j] = (MODE == 2 && cl) ? rstd[c0 + j] : 0.f;
    g[j] = (MODE == 2 && cl) ? gamma[c0 + j] : 0.f;
    b[j] = (MODE == 2 && cl) ? beta[c0 + j] : 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) acc[s][j] = 0.f;
  }
  auto row = [&](int64_t r, float (&xv)[V], float (&dv)[V]) {
    if (V == 4) {
      const tg_vec16<float> a = tg_ld16<NTL>(x + r * C + c0);
#pragma unroll
      for (int j = 0; j < V; ++j) xv[j] = a.v[j];
      if (MODE == 2) {
        const tg_vec16<float> d = tg_ld16<NTL>(dy + r * C + c0);
#pragma unroll
        for (int j = 0; j < V; ++j) dv[j] = d.v[j];
      }
    } else {
      xv[0] = x[r * C + c0];
      if (MODE == 2) dv[0] = dy[r * C + c0];
    }
  };
  auto accum = [&](const float (&xv)[V], const float (&dv)[V]) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      if (MODE == 0) {
        acc[0][j] += xv[j];
      } else if (MODE == 1) {
        const float d = xv[j] - mu[j];
        acc[0][j] += d * d;
      } else {
        const float xh = bn_xhat(xv[j], mu[j], rs[j]);
        const float dm = (!relu || bn_relu_on(xh, g[j], b[j])) ? dv[j] : 0.f;
        acc[0][j] += dm;
        acc[1][j] += dm * xh;
      }
    }
  };
  if (cl) {
    // Four rows per wave in flight (all loads issued before any is used), then the
    // remaining rows one at a time.  The accumulation order per wave is the row order.
    constexpr int U = 4;
    int64_t r = r0 + wave;
    for (; r + 4 * (U - 1) < r1; r += 4 * U) {
      float xv[U][V], dv[U][V];
#pragma unroll
      for (int u = 0; u < U; ++u) row(r + 4 * u, xv[u], dv[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) accum(xv[u], dv[u]);
    }
    for (; r < r1; r += 4) {
      float xv[V], dv[V];
      row(r, xv, dv);
      accum(xv, dv);
    }
  }
  // combine the 4 waves through LDS
  __shared__ float red[4][NS][64 * V];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int j = 0; j < V; ++j) red[wave][s][lane * V + j] = acc[s][j];
  __syncthreads();
  if (wave == 0 && cl) {
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float t = (red[0][s][lane * V + j] + red[1][s][lane * V + j]) +
                        (red[2][s][lane * V + j] + red[3][s][lane * V + j]);
        if (c0 + j < C) part[((int64_t)blockIdx.x * NS + s) * C + c0 + j] = t;
      }
  }
}

// NCHW channel reductions: grid (nsplit, C); block reduces channel blockIdx.y over
// the images of its split, threads striding the contiguous HW run.
template <int V, int MODE>
__global__ __launch_bounds__(kBlock) void k_nchw_reduce(
    const float* __restrict__ x, const float* __restrict__ dy, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, int relu, float* __restrict__ part, int64_t N, int64_t C,
    int64_t HW) {
  constexpr int NS = MODE == 2 ? 2 : 1;
  const int64_t c = blockIdx.y;
  const int64_t nsplit = gridDim.x;
  const int64_t per = (N + nsplit - 1) / nsplit;
  const int64_t n0 = (int64_t)blockIdx.x * per;
  const int64_t n1 = n0 + per < N ? n0 + per : N;
  const float mu = MODE >= 1 ? mean[c] : 0.f;
  const float rs = MODE == 2 ? rstd[c] : 0.f;
  const float g = MODE == 2 ? gamma[c] : 0.f;
  const float b = MODE == 2 ? beta[c] : 0.f;
  float acc[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) acc[s] = 0.f;
  for (int64_t n = n0; n < n1; ++n) {
    const int64_t base = (n * C + c) * HW;
    for (int64_t h = (int64_t)threadIdx.x * V; h < HW; h += kBlock * V) {
      float xv[V], dv[V];
      if (V == 4) {
        const float4 a = *reinterpret_cast<const float4*>(x + base + h);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        if (MODE == 2) {
          const float4 d = *reinterpret_cast<const float4*>(dy + base + h);
          dv[0] = d.x; dv[1] = d.y; dv[2] = d.z; dv[3] = d.w;
        }
      } else {
        xv[0] = x[base + h];
        if (MODE == 2) dv[0] = dy[base + h];
      }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        if (MODE == 0) {
          acc[0] += xv[j];
        } else if (MODE == 1) {
          const float d = xv[j] - mu;
          acc[0] += d * d;
        } else {
          const float xh = bn_xhat(xv[j], mu, rs);
          const float dm = (!relu || bn_relu_on(xh, g, b)) ? dv[j] : 0.f;
          acc[0] += dm;
          acc[1] += dm * xh;
        }
      }
    }
  }
  __shared__ float red[4 * NS];
  tg_block_sum<4, NS>(acc, red);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int s = 0; s < NS; ++s) part[((int64_t)blockIdx.x * NS + s) * C + c] = acc[s];
  }
}

// Per-channel finalisation kernels over the reduced sums (one thread per channel).
// Forward mean: mean = S/m.
__global__ void k_bn_mean(const float* __restrict__ sums, float* __restrict__ mean, int64_t C,
                          float inv_m) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c < C) mean[c] = sums[c] * inv_m;
}
// Forward variance (population), rstd and the running-statistics EMA.
__global__ void k_bn_var(const float* __restrict__ sums, float* __restrict__ var,
                         float* __restrict__ rstd, const float* __restrict__ mean,
                         float* __restrict__ run_mean, float* __restrict__ run_var,
                         float momentum, int64_t C, float inv_m, float eps) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= C) return;
  const float v = sums[c] * inv_m;
  if (var) var[c] = v;
  rstd[c] = 1.0f / sqrtf(v + eps);
  if (run_mean) run_mean[c] = (1.0f - momentum) * run_mean[c] + momentum * mean[c];
  if (run_var) run_var[c] = (1.0f - momentum) * run_var[c] + momentum * v;
}

// Per-channel apply coefficients from the channel sums S1, S2 (sums[c], sums[C + c]),
// formed by the apply kernel itself (no separate per-channel launch):
// dx = P*dy_m - Q - R*xhat with P = gamma*rstd, Q = P*S1/m, R = P*S2/m.
__device__ __forceinline__ void bn_coef(const float* __restrict__ sums, float g, float rs,
                                        float inv_m, int64_t C, int64_t c, float& P, float& Q,
                                        float& R) {
  P = g * rs;
  Q = P * (sums[c] * inv_m);
  R = P * (sums[C + c] * inv_m);
}

// Elementwise apply kernels.  Channel of flat index i: NHWC i % C, NCHW (i / HW) % C.
// V = 4 needs all operands 16-byte aligned and (NHWC) C % 4 == 0 or (NCHW) HW % 4 == 0.
template <int LAYOUT, int V>
__device__ __forceinline__ int64_t chan_of(int64_t i, int64_t C, int64_t HW) {
  return LAYOUT == TG_NHWC ? (i % C) : ((i / HW) % C);
}

template <int LAYOUT, int V, bool ACC, bool CONST_CH, bool NTL = false>
__global__ __launch_bounds__(kBlock) void k_bn_bwd_apply(
    const float* __restrict__ x, const float* __restrict__ dy, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, const float* __restrict__ sums, float inv_m, int relu,
    float* __restrict__ dx, int64_t nvec, int64_t C, int64_t HW, bool nt,
    float* __restrict__ dgamma, float* __restrict__ dbeta, int acc_params) {
  // CONST_CH (NHWC, grid stride a multiple of C): every iteration of a thread
  // touches the same V channels, so their parameters are loaded once.
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  const int64_t iv0 = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  // dgamma (+)= S2, dbeta (+)= S1: one thread per channel
  for (int64_t c = iv0; c < C; c += stride) {
    if (dbeta) dbeta[c] = acc_params ? dbeta[c] + sums[c] : sums[c];
    if (dgamma) dgamma[c] = acc_params ? dgamma[c] + sums[C + c] : sums[C + c];
  }
  float pmu[V], prs[V], pg[V], pb[V], pP[V], pQ[V], pR[V];
  if (CONST_CH) {
    const int64_t cb = (iv0 * V) % C;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t c = cb + j;
      pmu[j] = mean[c]; prs[j] = rstd[c]; pg[j] = gamma[c]; pb[j] = beta[c];
      bn_coef(sums, pg[j], prs[j], inv_m, C, c, pP[j], pQ[j], pR[j]);
    }
  }
  for (int64_t iv = iv0; iv < nvec; iv += stride) {
    const int64_t i = iv * V;
    float xv[V], dv[V], ov[V];
    if (V == 4) {
      const tg_vec16<float> a = tg_ld16<NTL>(x + i), d = tg_ld16<NTL>(dy + i);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        xv[j] = a.v[j];
        dv[j] = d.v[j];
      }
      if (ACC) {
        const tg_vec16<float> o = tg_ld16<NTL>(dx + i);
#pragma unroll
        for (int j = 0; j < V; ++j) ov[j] = o.v[j];
      }
    } else {
      xv[0] = x[i];
      dv[0] = dy[i];
      if (ACC) ov[0] = dx[i];
    }
    if (!CONST_CH) {
      const int64_t cb = chan_of<LAYOUT, V>(i, C, HW);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int64_t c = LAYOUT == TG_NHWC ? cb + j : cb;
        pmu[j] = mean[c]; prs[j] = rstd[c]; pg[j] = gamma[c]; pb[j] = beta[c];
        bn_coef(sums, pg[j], prs[j], inv_m, C, c, pP[j], pQ[j], pR[j]);
      }
    }
    float r[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float xh = bn_xhat(xv[j], pmu[j], prs[j]);
      const float dm = (!relu || bn_relu_on(xh, pg[j], pb[j])) ? dv[j] : 0.f;
      r[j] = pP[j] * dm - pQ[j] - pR[j] * xh;
      if (ACC) r[j] += ov[j];
    }
    if (V == 4) {
      tg_vec16<float> o;
      o.v[0] = r[0]; o.v[1] = r[1]; o.v[2] = r[2]; o.v[3] = r[3];
      if (nt) tg_store16_nt(dx + i, o);
      else tg_store16(dx + i, o);
    } else {
      dx[i] = r[0];
    }
  }
}

template <int LAYOUT, int V>
__global__ __launch_bounds__(kBlock) void k_bn_fwd_apply(
    const float* __restrict__ x, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gamma, const float* __restrict__ beta, int relu,
    float* __restrict__ y, int64_t nvec, int64_t C, int64_t HW) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t iv = (int64_t)blockIdx.x * kBlock + threadIdx.x; iv < nvec; iv += stride) {
    const int64_t i = iv * V;
    float xv[V];
    if (V == 4) {
      const float4 a = *reinterpret_cast<const float4*>(x + i);
      xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
    } else {
      xv[0] = x[i];
    }
    float r[V];
    const int64_t cb = chan_of<LAYOUT, V>(i, C, HW);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t c = LAYOUT == TG_NHWC ? cb + j : cb;
      const float v = bn_affine(bn_xhat(xv[j], mean[c], rstd[c]), gamma[c], beta[c]);
      r[j] = (relu && !(v > 0.f)) ? 0.f : v;
    }
    if (V == 4)
      *reinterpret_cast<float4*>(y + i) = make_float4(r[0], r[1], r[2], r[3]);
    else
      y[i] = r[0];
  }
}

struct BnPlan {
  int64_t M;       // rows per channel = N*HW
  int64_t nsplit;  // partial count per channel
  int V;           // vector width of the reduction
  int64_t ctiles;  // NHWC channel tiles of 64*V
};

BnPlan bn_plan(int layout, int64_t N, int64_t C, int64_t HW, bool aligned) {
  BnPlan p{};
  p.M = N * HW;
  const int64_t cus = tg_num_cus();
  if (layout == TG_NHWC) {
    p.V = (aligned && C % 4 == 0) ? 4 : 1;
    p.ctiles = (C + 64 * p.V - 1) / (64 * p.V);
    int64_t want = (4 * cus + p.ctiles - 1) / p.ctiles;
    if (want > p.M / 16) want = p.M / 16;
    p.nsplit = want < 1 ? 1 : want;
  } else {
    p.V = (aligned && HW % 4 == 0) ? 4 : 1;
    p.ctiles = 0;
    int64_t want = (4 * cus + C - 1) / C;
    if (want > N) want = N;
    p.nsplit = want < 1 ? 1 : want;
  }
  return p;
}

// Workspace: partials [nsplit][2][C] | sums [2C] | 3C reserved | tree scratch
size_t bn_ws_bytes(const BnPlan& p, int64_t C) {
  return (size_t)(2 * p.nsplit * C + 5 * C) * sizeof(float) +
         tg_sum_partials_scratch(p.nsplit, 2 * C);
}

template <int MODE>
void launch_reduce(int layout, const BnPlan& p, const float* x, const float* dy,
                   const float* mean, const float* rstd, const float* gamma, const float* beta,
                   int relu, float* part, int64_t N, int64_t C, int64_t HW, hipStream_t s,
                   bool ntl = false) {
  if (layout == TG_NHWC) {
    dim3 grid((unsigned)p.nsplit, (unsigned)p.ctiles);
    if (p.V == 4 && ntl)
      k_nhwc_reduce<4, MODE, true><<<grid, kBlock, 0, s>>>(x, dy, mean, rstd, gamma, beta, relu,
                                                           part, p.M, C);
    else if (p.V == 4)
      k_nhwc_reduce<4, MODE><<<grid, kBlock, 0, s>>>(x, dy, mean, rstd, gamma, beta, relu, part,
                                                     p.M, C);
    else
      k_nhwc_reduce<1, MODE><<<grid, kBlock, 0, s>>>(x, dy, mean, rstd, gamma, beta, relu, part,
                                                     p.M, C);
  } else {
    dim3 grid((unsigned)p.nsplit, (unsigned)C);
    if (p.V == 4)
      k_nchw_reduce<4, MODE><<<grid, kBlock, 0, s>>>(x, dy, mean, rstd, gamma, beta, relu, part,
                                                     N, C, HW);
    else
      k_nchw_reduce<1, MODE><<<grid, kBlock, 0, s>>>(x, dy, mean, rstd, gamma, beta, relu, part,
                                                     N, C, HW);
  }
}

unsigned apply_blocks(int64_t nvec) {
  int64_t b = (nvec + kBlock - 1) / kBlock;
  const int64_t cap = (int64_t)tg_num_cus() * 64;
  if (b > cap) b = cap;
  return (unsigned)(b < 1 ? 1 : b);
}

int64_t gcd64(int64_t a, int64_t b) {
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// NHWC apply grid whose element stride (blocks*256*V) is a multiple of C, so each
// thread keeps one channel group; returns 0 when no such grid fits.
unsigned const_channel_blocks(int64_t nvec, int64_t C, int V) {
  const int64_t per_block = (int64_t)kBlock * V;
  const int64_t unit = C / gcd64(C, per_block);  // blocks per channel period
  int64_t b = apply_blocks(nvec);
  if (unit > b) return 0;
  b -= b % unit;
  return (unsigned)b;
}

int check_args(int layout, int64_t N, int64_t C, int64_t HW, const char* who) {
  TG_REQUIRE(layout == TG_NHWC || layout == TG_NCHW, "%s: unknown layout %d", who, layout);
  TG_REQUIRE(N > 0 && C > 0 && HW > 0, "%s: bad shape N=%lld C=%lld HW=%lld", who,
             (long long)N, (long long)C, (long long)HW);
  TG_REQUIRE(C <= 65535 || layout == TG_NHWC, "%s: C too large for NCHW grid", who);
  return TG_OK;
}

}  // namespace

TG_EXPORT size_t tg_batchnorm_workspace(int layout, int64_t N, int64_t C, int64_t HW) {
  if (N <= 0 || C <= 0 || HW <= 0) return 0;
  BnPlan a = bn_plan(layout, N, C, HW, true), b = bn_plan(layout, N, C, HW, false);
  const size_t x = bn_ws_bytes(a, C), y = bn_ws_bytes(b, C);
  return x > y ? x : y;
}

// Training forward: batch mean/var over (N,H,W) per channel, rstd, running-stat
// EMA (population variance, as the reference), y = [relu](gamma*xhat + beta).
TG_EXPORT int tg_batchnorm_fwd_train(int layout, const float* x, const float* gamma,
                                     const float* beta, float* y, float* mean, float* rstd,
                                     float* var, float* running_mean, float* running_var,
                                     float momentum, int64_t N, int64_t C, int64_t HW, float eps,
                                     int relu, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  int st = check_args(layout, N, C, HW, "tg_batchnorm_fwd_train");
  if (st) return st;
  TG_REQUIRE(x && gamma && beta && y && mean && rstd, "tg_batchnorm_fwd_train: null pointer");
  const bool al = tg_aligned16(x) && tg_aligned16(y);
  BnPlan p = bn_plan(layout, N, C, HW, al);
  const size_t need = bn_ws_bytes(p, C);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("tg_batchnorm_fwd_train: workspace of %zu bytes needed", need);
    return TG_ERR_WORKSPACE;
  }
  hipStream_t s = tg_stream(stream);
  float* part = (float*)workspace;
  float* sums = part + 2 * p.nsplit * C;
  float* scratch = sums + 5 * C;
  const float inv_m = 1.0f / (float)p.M;
  const unsigned cb = (unsigned)((C + kBlock - 1) / kBlock);
  launch_reduce<0>(layout, p, x, nullptr, nullptr, nullptr, nullptr, nullptr, relu, part, N, C,
                   HW, s);
  st = tg_sum_partials(part, p.nsplit, C, TG_F32, sums, 0, scratch, s);
  if (st) return st;
  k_bn_mean<<<cb, kBlock, 0, s>>>(sums, mean, C, inv_m);
  launch_reduce<1>(layout, p, x, nullptr, mean, nullptr, nullptr, nullptr, relu, part, N, C, HW,
                   s);
  st = tg_sum_partials(part, p.nsplit, C, TG_F32, sums, 0, scratch, s);
  if (st) return st;
  k_bn_var<<<cb, kBlock, 0, s>>>(sums, var, rstd, mean, running_mean, running_var, momentum, C,
                                 inv_m, eps);
  const int64_t n = N * C * HW;
  const bool vec = p.V == 4 && al;
  const int64_t nvec = vec ? n / 4 : n;
  const unsigned ab = apply_blocks(nvec);
  if (layout == TG_NHWC) {
    if (vec) k_bn_fwd_apply<TG_NHWC, 4><<<ab, kBlock, 0, s>>>(x, mean, rstd, gamma, beta, relu, y, nvec, C, HW);
    else k_bn_fwd_apply<TG_NHWC, 1><<<ab, kBlock, 0, s>>>(x, mean, rstd, gamma, beta, relu, y, nvec, C, HW);
  } else {
    if (vec) k_bn_fwd_apply<TG_NCHW, 4><<<ab, kBlock, 0, s>>>(x, mean, rstd, gamma, beta, relu, y, nvec, C, HW);
    else k_bn_fwd_apply<TG_NCHW, 1><<<ab, kBlock, 0, s>>>(x, mean, rstd, gamma, beta, relu, y, nvec, C, HW);
  }
  return tg_check_launch("tg_batchnorm_fwd_train");
}

// Backward (training statistics).  `beta` (the BN shift) is only read for the
// ReLU mask; pass relu = 0 for plain BatchNorm.
TG_EXPORT int tg_batchnorm_bwd(int layout, const float* x, const float* mean, const float* rstd,
                               const float* gamma, const float* beta, const float* dy,
                               float* dx, float* dgamma, float* dbeta, int64_t N, int64_t C,
                               int64_t HW, int relu, int accumulate_dx, int accumulate_params,
                               void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_args(layout, N, C, HW, "tg_batchnorm_bwd");
  if (st) return st;
  TG_REQUIRE(x && mean && rstd && gamma && beta && dy && dx, "tg_batchnorm_bwd: null pointer");
  const bool al = tg_aligned16(x) && tg_aligned16(dy) && tg_aligned16(dx);
  BnPlan p = bn_plan(layout, N, C, HW, al);
  const size_t need = bn_ws_bytes(p, C);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("tg_batchnorm_bwd: workspace of %zu bytes needed", need);
    return TG_ERR_WORKSPACE;
  }
  hipStream_t s = tg_stream(stream);
  float* part = (float*)workspace;
  float* sums = part + 2 * p.nsplit * C;
  float* scratch = sums + 5 * C;
  // x and dy too large to stay cached: both passes read them non-temporally
  const bool big = N * C * HW * (int64_t)sizeof(float) >= (128ll << 20);
  launch_reduce<2>(layout, p, x, dy, mean, rstd, gamma, beta, relu, part, N, C, HW, s, big);
  st = tg_sum_partials(part, p.nsplit, 2 * C, TG_F32, sums, 0, scratch, s);
  if (st) return st;
  const float inv_m = 1.0f / (float)p.M;
  const int64_t n = N * C * HW;
  const bool vec = p.V == 4 && al;
  const int64_t nvec = vec ? n / 4 : n;
  const unsigned ab = apply_blocks(nvec);
#define TG_BN_APPLY(LAY, VV, ACC, CC, NB)                                                    \
  do {                                                                                       \
  if (nt)                                                                                   \
    k_bn_bwd_apply<LAY, VV, ACC, CC, true><<<NB, kBlock, 0, s>>>(x, dy, mean, rstd, gamma, beta, \
        sums, inv_m, relu, dx, nvec, C, HW, nt, dgamma, dbeta, accumulate_params);           \
  else                                                                                       \
    k_bn_bwd_apply<LAY, VV, ACC, CC><<<NB, kBlock, 0, s>>>(x, dy, mean, rstd, gamma, beta,     \
        sums, inv_m, relu, dx, nvec, C, HW, nt, dgamma, dbeta, accumulate_params);           \
  } while (0)
  const bool nt = n * (int64_t)sizeof(float) >= (128ll << 20);  // output too large to keep cached
  const unsigned cc = (layout == TG_NHWC && vec) ? const_channel_blocks(nvec, C, 4) : 0;
  if (cc) {
    if (accumulate_dx) TG_BN_APPLY(TG_NHWC, 4, true, true, cc);
    else TG_BN_APPLY(TG_NHWC, 4, false, true, cc);
  } else if (layout == TG_NHWC) {
    if (vec) { if (accumulate_dx) TG_BN_APPLY(TG_NHWC, 4, true, false, ab); else TG_BN_APPLY(TG_NHWC, 4, false, false, ab); }
    else { if (accumulate_dx) TG_BN_APPLY(TG_NHWC, 1, true, false, ab); else TG_BN_APPLY(TG_NHWC, 1, false, false, ab); }
  } else {
    if (vec) { if (accumulate_dx) TG_BN_APPLY(TG_NCHW, 4, true, false, ab); else TG_BN_APPLY(TG_NCHW, 4, false, false, ab); }
    else { if (accumulate_dx) TG_BN_APPLY(TG_NCHW, 1, true, false, ab); else TG_BN_APPLY(TG_NCHW, 1, false, false, ab); }
  }
#undef TG_BN_APPLY
  return tg_check_launch("tg_batchnorm_bwd");
}
