// Deterministic column sums of fp32 partial-sum matrices: out[c] = sum_k in[k][c].
//
// Finishes every two-stage reduction in the library (LayerNorm dgamma/dbeta,
// BatchNorm channel sums, bias-gradient unbroadcast).  A block covers 64 columns
// (one per lane, so each wavefront reads a contiguous 256-byte row segment); its 16
// wavefronts split the rows round-robin and each keeps kU independent loads in
// flight, so one launch finishes up to kDirect partial rows in a handful of memory
// round trips.  The combine order (per-wave accumulators, then waves through LDS) is
// fixed, so results do not depend on scheduling.  Several matrices stacked as
// [nb][K][cols] (dgamma and dbeta partials) are finished by the same launch.
#include "tg_common.h"

namespace {

constexpr int kWaves = 16;
constexpr int kBlock = kWaves * 64;
constexpr int kU = 8;
constexpr int64_t kDirect = 2048;
constexpr int64_t kStage = 256;

struct Outs {
  void* p[2];
};

template <typename TO, bool FINAL, bool ACC>
__global__ __launch_bounds__(kBlock) void k_colsum(const float* __restrict__ in, int64_t K,
                                                   int64_t cols, int64_t rpb, Outs outs,
                                                   float* __restrict__ stage, int64_t nstage) {
  const int b = blockIdx.y;
  TO* out = reinterpret_cast<TO*>(outs.p[b]);
  if (FINAL && out == nullptr) return;  // uniform per block
  in += (int64_t)b * K * cols;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int64_t r0 = (int64_t)blockIdx.z * rpb;
  const int64_t r1 = r0 + rpb < K ? r0 + rpb : K;
  float acc[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) acc[u] = 0.f;
  if (c < cols) {
    int64_t r = r0 + wave;
    for (; r + (kU - 1) * kWaves < r1; r += kU * kWaves) {
#pragma unroll
      for (int u = 0; u < kU; ++u) acc[u] += in[(r + u * kWaves) * cols + c];
    }
#pragma unroll
    for (int u = 0; u < kU - 1; ++u)
      if (r + u * kWaves < r1) acc[u] += in[(r + u * kWaves) * cols + c];
  }
#pragma unroll
  for (int w = kU / 2; w >= 1; w /= 2)
#pragma unroll
    for (int u = 0; u < w; ++u) acc[u] += acc[u + w];
  __shared__ float red[kWaves][64];
  red[wave][lane] = acc[0];
  __syncthreads();
  if (wave == 0 && c < cols) {
    float v[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v[w] = red[w][lane];
#pragma unroll
    for (int w = kWaves / 2; w >= 1; w /= 2)
#pragma unroll
      for (int u = 0; u < w; ++u) v[u] += v[u + w];
    float s = v[0];
    if (FINAL) {
      if (ACC) s += tg_to_float(out[c]);
      out[c] = tg_from_float<TO>(s);
    } else {
      stage[((int64_t)b * nstage + blockIdx.z) * cols + c] = s;
    }
  }
}

// Few rows, many columns (split-K GEMM partials, small-batch bias gradients): one
// thread per 4 adjacent columns, rows summed in order with 4 loads in flight.
constexpr int64_t kNarrowK = 64;
constexpr int kNarrowBlock = 256;

template <typename TO, bool ACC, bool VEC>
__global__ __launch_bounds__(kNarrowBlock) void k_colsum_narrow(const float* __restrict__ in,
                                                                int64_t K, int64_t cols,
                                                                Outs outs) {
  const int b = blockIdx.y;
  TO* out = reinterpret_cast<TO*>(outs.p[b]);
  if (out == nullptr) return;
  in += (int64_t)b * K * cols;
  const int64_t c0 = ((int64_t)blockIdx.x * kNarrowBlock + threadIdx.x) * 4;
  if (c0 >= cols) return;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  if (VEC) {
    int64_t r = 0;
    for (; r + 4 <= K; r += 4) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4*>(in + (r + u) * cols + c0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a[0] += v[u].x;
        a[1] += v[u].y;
        a[2] += v[u].z;
        a[3] += v[u].w;
      }
    }
    for (; r < K; ++r) {
      const float4 v = *reinterpret_cast<const float4*>(in + r * cols + c0);
      a[0] += v.x;
      a[1] += v.y;
      a[2] += v.z;
      a[3] += v.w;
    }
  } else {
    for (int64_t r = 0; r < K; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c0 + j < cols) a[j] += in[r * cols + c0 + j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (c0 + j < cols) {
      float s = a[j];
      if (ACC) s += tg_to_float(out[c0 + j]);
      out[c0 + j] = tg_from_float<TO>(s);
    }
  }
}

template <typename TO>
void launch_final(const float* in, int64_t K, int64_t cols, int nb, Outs outs, int acc,
                  hipStream_t s) {
  if (K <= kNarrowK && cols >= 4096) {
    dim3 g((unsigned)((cols + 4 * kNarrowBlock - 1) / (4 * kNarrowBlock)), (unsigned)nb);
    const bool vec = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0;
#define L(A, V) k_colsum_narrow<TO, A, V><<<g, kNarrowBlock, 0, s>>>(in, K, cols, outs)
    if (acc) { if (vec) L(true, true); else L(true, false); }
    else { if (vec) L(false, true); else L(false, false); }
#undef L
    return;
  }
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)nb, 1);
  if (acc)
    k_colsum<TO, true, true><<<grid, kBlock, 0, s>>>(in, K, cols, K, outs, nullptr, 0);
  else
    k_colsum<TO, true, false><<<grid, kBlock, 0, s>>>(in, K, cols, K, outs, nullptr, 0);
}

int sum_partials(const float* in, int64_t K, int64_t cols, int dtype_out, Outs outs, int nb,
                 int acc, float* scratch, hipStream_t s) {
  if (cols <= 0) return TG_OK;
  if (K > kDirect) {
    const int64_t k1 = (K + kStage - 1) / kStage;
    dim3 grid((unsigned)((cols + 63) / 64), (unsigned)nb, (unsigned)k1);
    k_colsum<float, false, false><<<grid, kBlock, 0, s>>>(in, K, cols, kStage, outs, scratch, k1);
    in = scratch;
    K = k1;
  }
  switch (dtype_out) {
    case TG_F32: launch_final<float>(in, K, cols, nb, outs, acc, s); break;
    case TG_F16: launch_final<tg_half>(in, K, cols, nb, outs, acc, s); break;
    case TG_BF16: launch_final<tg_bf16>(in, K, cols, nb, outs, acc, s); break;
    default:
      tg_set_error("sum of partials: unsupported output dtype %d", dtype_out);
      return TG_ERR_UNSUPPORTED;
  }
  return tg_check_launch("sum of partials");
}

// Several finishes of two stacked partial matrices (dgamma, dbeta) in one launch:
// member m = blockIdx.z, with its own rows K, columns and outputs; the per-column
// arithmetic is k_colsum's final pass (the members' K within kDirect), so each output
// equals that member finished on its own.
constexpr int kGroupMax = 32;
struct ColsumGroup {
  const float* in[kGroupMax];
  int64_t K[kGroupMax], cols[kGroupMax];
  float* out[kGroupMax][2];
  unsigned acc;  // bit m: add member m's sums to its outputs
};

__global__ __launch_bounds__(kBlock) void k_colsum_group(const ColsumGroup g) {
  const int m = blockIdx.z, b = blockIdx.y;
  const int64_t cols = g.cols[m], K = g.K[m];
  float* out = g.out[m][b];
  if (out == nullptr || (int64_t)blockIdx.x * 64 >= cols) return;  // uniform per block
  const float* in = g.in[m] + (int64_t)b * K * cols;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  float acc[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) acc[u] = 0.f;
  if (c < cols) {
    int64_t r = wave;
    for (; r + (kU - 1) * kWaves < K; r += kU * kWaves) {
#pragma unroll
      for (int u = 0; u < kU; ++u) acc[u] += in[(r + u * kWaves) * cols + c];
    }
#pragma unroll
    for (int u = 0; u < kU - 1; ++u)
      if (r + u * kWaves < K) acc[u] += in[(r + u * kWaves) * cols + c];
  }
#pragma unroll
  for (int w = kU / 2; w >= 1; w /= 2)
#pragma unroll
    for (int u = 0; u < w; ++u) acc[u] += acc[u + w];
  __shared__ float red[kWaves][64];
  red[wave][lane] = acc[0];
  __syncthreads();
  if (wave == 0 && c < cols) {
    float v[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v[w] = red[w][lane];
#pragma unroll
    for (int w = kWaves / 2; w >= 1; w /= 2)
#pragma unroll
      for (int u = 0; u < w; ++u) v[u] += v[u + w];
    float sv = v[0];
    if ((g.acc >> m) & 1u) sv += out[c];
    out[c] = sv;
  }
}
}  // namespace

bool tg_sum_partials_groupable(int64_t K, int64_t cols) {
  return K >= 1 && K <= kDirect && !(K <= kNarrowK && cols >= 4096);
}

size_t tg_sum_partials_scratch(int64_t K, int64_t cols, int nb) {
  if (K <= kDirect) return 0;
  return (size_t)(nb * ((K + kStage - 1) / kStage) * cols) * sizeof(float);
}

int tg_sum_partials(const float* in, int64_t K, int64_t cols, int dtype_out, void* out, int acc,
                    float* scratch, hipStream_t s) {
  Outs o{{out, nullptr}};
  return sum_partials(in, K, cols, dtype_out, o, 1, acc, scratch, s);
}

int tg_sum_partials2(const float* in, int64_t K, int64_t cols, int dtype_out, void* out0,
                     void* out1, int acc, float* scratch, hipStream_t s) {
  Outs o{{out0, out1}};
  return sum_partials(in, K, cols, dtype_out, o, 2, acc, scratch, s);
}

TG_EXPORT int tg_sum_partials2_group(int n, const float* const* parts, const int64_t* K,
                                     const int64_t* cols, float* const* out0,
                                     float* const* out1, const int* acc, void* stream) {
  TG_REQUIRE(n >= 0, "tg_sum_partials2_group: negative count");
  if (n == 0) return TG_OK;
  TG_REQUIRE(parts && K && cols && out0 && out1, "tg_sum_partials2_group: null pointer array");
  for (int i = 0; i < n; ++i) {
    TG_REQUIRE(parts[i] && cols[i] > 0 && tg_sum_partials_groupable(K[i], cols[i]),
               "tg_sum_partials2_group: member %d: K = %lld rows of %lld columns not covered "
               "(1 <= K <= %lld, and not K <= %lld with 4096 or more columns)", i,
               (long long)K[i], (long long)cols[i], (long long)kDirect, (long long)kNarrowK);
  }
  hipStream_t s = tg_stream(stream);
  for (int g0 = 0; g0 < n; g0 += kGroupMax) {
    const int cnt = n - g0 < kGroupMax ? n - g0 : kGroupMax;
    ColsumGroup grp{};
    int64_t maxc = 0;
    for (int i = 0; i < cnt; ++i) {
      grp.in[i] = parts[g0 + i];
      grp.K[i] = K[g0 + i];
      grp.cols[i] = cols[g0 + i];
      grp.out[i][0] = out0[g0 + i];
      grp.out[i][1] = out1[g0 + i];
      if (acc && acc[g0 + i]) grp.acc |= 1u << i;
      maxc = cols[g0 + i] > maxc ? cols[g0 + i] : maxc;
    }
    dim3 grid((unsigned)((maxc + 63) / 64), 2, (unsigned)cnt);
    k_colsum_group<<<grid, kBlock, 0, s>>>(grp);
    const int st = tg_check_launch("tg_sum_partials2_group");
    if (st) return st;
  }
  return TG_OK;
}
