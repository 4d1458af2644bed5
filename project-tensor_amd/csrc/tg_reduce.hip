// Deterministic column sums of fp32 partial-sum matrices: out[c] = sum_k in[k][c].
//
// Used to finish every two-stage reduction in the library (LayerNorm dgamma/dbeta,
// BatchNorm channel sums, bias-gradient unbroadcast).  A block covers 64 columns
// (one per lane: each wavefront reads a contiguous 256-byte row segment) and its
// 4 wavefronts split the rows, combined through LDS in a fixed order.  More than
// kDirect rows go through one intermediate stage of kStage-row groups, so no lane
// walks a long serial chain and the grid stays wide enough to fill the CUs.
#include "tg_common.h"

namespace {

constexpr int kBlock = 256;
constexpr int64_t kDirect = 256;
constexpr int64_t kStage = 64;

template <typename TO, bool FINAL, bool ACC>
__global__ __launch_bounds__(kBlock) void k_rowsum(const float* __restrict__ in, int64_t K,
                                                   int64_t cols, int64_t rpb,
                                                   TO* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int64_t r0 = (int64_t)blockIdx.y * rpb;
  const int64_t r1 = r0 + rpb < K ? r0 + rpb : K;
  float a = 0.f, b = 0.f;
  if (c < cols) {
    int64_t r = r0 + wave;
    for (; r + 4 < r1; r += 8) {
      a += in[r * cols + c];
      b += in[(r + 4) * cols + c];
    }
    if (r < r1) a += in[r * cols + c];
  }
  __shared__ float red[4][64];
  red[wave][lane] = a + b;
  __syncthreads();
  if (wave == 0 && c < cols) {
    float s = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    if (FINAL) {
      if (ACC) s += tg_to_float(out[c]);
      out[c] = tg_from_float<TO>(s);
    } else {
      out[(int64_t)blockIdx.y * cols + c] = tg_from_float<TO>(s);
    }
  }
}

template <typename TO>
void launch_final(const float* in, int64_t K, int64_t cols, TO* out, int acc, hipStream_t s) {
  dim3 grid((unsigned)((cols + 63) / 64), 1);
  if (acc)
    k_rowsum<TO, true, true><<<grid, kBlock, 0, s>>>(in, K, cols, K, out);
  else
    k_rowsum<TO, true, false><<<grid, kBlock, 0, s>>>(in, K, cols, K, out);
}

}  // namespace

size_t tg_sum_partials_scratch(int64_t K, int64_t cols) {
  if (K <= kDirect) return 0;
  return (size_t)(((K + kStage - 1) / kStage) * cols) * sizeof(float);
}

int tg_sum_partials(const float* in, int64_t K, int64_t cols, int dtype_out, void* out, int acc,
                    float* scratch, hipStream_t s) {
  if (cols <= 0) return TG_OK;
  if (K > kDirect) {
    const int64_t k1 = (K + kStage - 1) / kStage;
    dim3 grid((unsigned)((cols + 63) / 64), (unsigned)k1);
    k_rowsum<float, false, false><<<grid, kBlock, 0, s>>>(in, K, cols, kStage, scratch);
    in = scratch;
    K = k1;
  }
  switch (dtype_out) {
    case TG_F32: launch_final<float>(in, K, cols, (float*)out, acc, s); break;
    case TG_F16: launch_final<tg_half>(in, K, cols, (tg_half*)out, acc, s); break;
    case TG_BF16: launch_final<tg_bf16>(in, K, cols, (tg_bf16*)out, acc, s); break;
    default:
      tg_set_error("sum of partials: unsupported output dtype %d", dtype_out);
      return TG_ERR_UNSUPPORTED;
  }
  return tg_check_launch("sum of partials");
}
