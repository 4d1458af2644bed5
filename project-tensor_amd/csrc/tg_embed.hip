// Embedding backward and the tied-weight gradient transfer.
//
// tg_embedding_bwd: grad[idx[i]] (+)= dout[i] (Embedding._backward, _nn.py:1083-1089,
// a scatter-add).  Deterministic: (index, position) pairs are radix-sorted (stable,
// rocPRIM), then one wavefront per run of equal indices sums the run's dout rows in
// their original order in fp32 and adds the sum to the gradient row once -- the
// order np.add.at uses, so fp32 results match it exactly.  Indices outside [0, V)
// are skipped.  Rows never indexed are left as they are (zeroed first when not
// accumulating).
//
// tg_transpose_add: dst[c][r] += alpha * src[r][c] through 64x64 LDS tiles
// (sync_tied_gradients, _training.py:264-284: source.grad += param.grad.T).
#include <rocprim/device/device_radix_sort.hpp>

#include "tg_common.h"

namespace {

constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void k_iota(int* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) p[i] = (int)i;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_fill_zero(T* __restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    p[i] = tg_from_float<T>(0.f);
}

// One wavefront per sorted position; a wave whose position starts a run of equal
// keys sums the run.  dim is processed in chunks of 64 lanes x 4 columns.
template <typename TD, typename TG>
__global__ __launch_bounds__(kBlock) void k_embed_seg(const int64_t* __restrict__ keys,
                                                      const int* __restrict__ pos, int64_t n,
                                                      const TD* __restrict__ dout, int64_t dim,
                                                      int64_t V, TG* __restrict__ grad) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  if (i >= n) return;
  const int64_t key = keys[i];
  if (i > 0 && keys[i - 1] == key) return;  // not the start of a run
  if (key < 0 || key >= V) return;
  int64_t end = i + 1;
  while (end < n && keys[end] == key) ++end;
  TG* grow = grad + key * dim;
  for (int64_t c0 = 0; c0 < dim; c0 += 64 * 4) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t j = i; j < end; ++j) {
      const TD* drow = dout + (int64_t)pos[j] * dim;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t c = c0 + u * 64 + lane;
        if (c < dim) acc[u] += tg_to_float(drow[c]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = c0 + u * 64 + lane;
      if (c < dim) grow[c] = tg_from_float<TG>(tg_to_float(grow[c]) + acc[u]);
    }
  }
}

template <typename TS, typename TD>
__global__ __launch_bounds__(kBlock) void k_transpose_add(const TS* __restrict__ src, int64_t R,
                                                          int64_t C, TD* __restrict__ dst,
                                                          float alpha) {
  __shared__ float tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int rr = ty + 4 * k;
    const int64_t r = r0 + rr, c = c0 + tx;
    tile[rr][tx] = (r < R && c < C) ? tg_to_float(src[r * C + c]) : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int cc = ty + 4 * k;
    const int64_t c = c0 + cc, r = r0 + tx;  // dst[c][r]
    if (c < C && r < R) {
      TD* p = dst + c * R + r;
      *p = tg_from_float<TD>(tg_to_float(*p) + alpha * tile[tx][cc]);
    }
  }
}

// fp32 transpose-add over whole 64 x 64 tiles (R and C multiples of 64, 16-byte
// aligned rows): 16-byte loads of src rows and 16-byte read-modify-writes of dst
// rows, all non-temporal (each element is touched once).
__global__ __launch_bounds__(kBlock) void k_transpose_add_v4(const float* __restrict__ src,
                                                             int64_t R, int64_t C,
                                                             float* __restrict__ dst,
                                                             float alpha) {
  __shared__ float tile[64][65];
  // blockIdx.x walks src rows (= dst columns): blocks running together cover one band
  // of dst rows contiguously instead of striding across dst rows R*4 bytes apart.
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int q = (threadIdx.x & 15) * 4, w = threadIdx.x >> 4;  // 16 x 16
  tg_vec16<float> v[4], o[4];  // both operands' loads in flight before the exchange
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = tg_load16_nt(src + (r0 + w + 16 * k) * C + c0 + q);
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = tg_load16_nt(dst + (c0 + w + 16 * k) * R + r0 + q);
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) tile[w + 16 * k][q + i] = v[k].v[i];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[k].v[i] += alpha * tile[q + i][w + 16 * k];
    tg_store16_nt(dst + (c0 + w + 16 * k) * R + r0 + q, o[k]);
  }
}

int sort_bits(int64_t V) {
  int b = 1;
  while (b < 63 && ((int64_t)1 << b) < V) ++b;
  return b;
}

size_t sort_temp_bytes(int64_t n, int64_t V) {
  size_t bytes = 0;
  (void)rocprim::radix_sort_pairs(nullptr, bytes, (const int64_t*)nullptr, (int64_t*)nullptr,
                                  (const int*)nullptr, (int*)nullptr, (size_t)n, 0,
                                  sort_bits(V));
  return bytes;
}

// Gather: out[i, :] = weight[idx[i], :] converted to the output dtype (negative
// indices wrap by V; rows of indices outside [-V, V) are zero).  8 elements per thread,
// 16-byte accesses when dim % 8 == 0 and both rows are 16-byte aligned.
template <typename TW, typename TO, bool VEC>
__global__ __launch_bounds__(kBlock) void k_embed_fwd(const TW* __restrict__ w,
                                                      const int64_t* __restrict__ idx, int64_t n,
                                                      int64_t dim, int64_t V,
                                                      TO* __restrict__ out) {
  const int64_t per = (dim + 7) / 8;  // 8-element groups per row
  const int64_t total = n * per;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t u = (int64_t)blockIdx.x * kBlock + threadIdx.x; u < total; u += stride) {
    const int64_t i = u / per, c = (u % per) * 8;
    int64_t r = idx[i];
    if (r < 0) r += V;
    const bool ok = r >= 0 && r < V;
    const TW* src = w + (ok ? r : 0) * dim + c;
    TO* dst = out + i * dim + c;
    float f[8];
    if (VEC) {
#pragma unroll
      for (int h = 0; h < 8 / tg_vec16<TW>::N; ++h) {
        const tg_vec16<TW> v = tg_load16(src + h * tg_vec16<TW>::N);
#pragma unroll
        for (int j = 0; j < tg_vec16<TW>::N; ++j) f[h * tg_vec16<TW>::N + j] = ok ? tg_to_float(v.v[j]) : 0.f;
      }
#pragma unroll
      for (int h = 0; h < 8 / tg_vec16<TO>::N; ++h) {
        tg_vec16<TO> o;
#pragma unroll
        for (int j = 0; j < tg_vec16<TO>::N; ++j) o.v[j] = tg_from_float<TO>(f[h * tg_vec16<TO>::N + j]);
        tg_store16(dst + h * tg_vec16<TO>::N, o);
      }
    } else {
      for (int j = 0; j < 8 && c + j < dim; ++j)
        dst[j] = tg_from_float<TO>(ok ? tg_to_float(src[j]) : 0.f);
    }
  }
}

template <typename TW, typename TO>
int embed_fwd_t(const void* w, const int64_t* idx, int64_t n, int64_t dim, int64_t V, void* out,
                hipStream_t s) {
  const int64_t total = n * ((dim + 7) / 8);
  int64_t blocks = (total + kBlock - 1) / kBlock;
  const int64_t cap = (int64_t)tg_num_cus() * 16;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  const bool vec = dim % 8 == 0 && tg_aligned16(w) && tg_aligned16(out);
  if (vec)
    k_embed_fwd<TW, TO, true><<<(unsigned)blocks, kBlock, 0, s>>>((const TW*)w, idx, n, dim, V,
                                                                  (TO*)out);
  else
    k_embed_fwd<TW, TO, false><<<(unsigned)blocks, kBlock, 0, s>>>((const TW*)w, idx, n, dim, V,
                                                                   (TO*)out);
  return tg_check_launch("tg_embedding_fwd");
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

template <typename TD, typename TG>
int embed_t(const void* dout, const int64_t* idx, int64_t n, int64_t dim, void* grad, int64_t V,
            int accumulate, char* ws, size_t ws_bytes, hipStream_t s) {
  if (!accumulate) {
    const int64_t total = V * dim;
    int64_t blocks = (total + kBlock - 1) / kBlock;
    if (blocks > (int64_t)tg_num_cus() * 16) blocks = (int64_t)tg_num_cus() * 16;
    if (blocks < 1) blocks = 1;
    k_fill_zero<TG><<<(unsigned)blocks, kBlock, 0, s>>>((TG*)grad, total);
  }
  if (n == 0) return tg_check_launch("tg_embedding_bwd");
  int64_t* keys_out = (int64_t*)ws;
  int* pos_in = (int*)(ws + align256(n * sizeof(int64_t)));
  int* pos_out = (int*)((char*)pos_in + align256(n * sizeof(int)));
  char* tmp = (char*)pos_out + align256(n * sizeof(int));
  size_t tmp_bytes = ws_bytes - (size_t)(tmp - ws);
  k_iota<<<(unsigned)((n + kBlock - 1) / kBlock), kBlock, 0, s>>>(pos_in, n);
  if (rocprim::radix_sort_pairs(tmp, tmp_bytes, idx, keys_out, pos_in, pos_out, (size_t)n, 0,
                                sort_bits(V), s) != hipSuccess) {
    tg_set_error("tg_embedding_bwd: radix sort failed");
    return TG_ERR_HIP;
  }
  k_embed_seg<TD, TG><<<(unsigned)((n + 3) / 4), kBlock, 0, s>>>(keys_out, pos_out, n,
                                                                   (const TD*)dout, dim, V,
                                                                   (TG*)grad);
  return tg_check_launch("tg_embedding_bwd");
}

}  // namespace

TG_EXPORT size_t tg_embedding_bwd_workspace(int64_t n_tokens, int64_t num_embeddings) {
  if (n_tokens <= 0) return 0;
  return align256(n_tokens * sizeof(int64_t)) + 2 * align256(n_tokens * sizeof(int)) +
         align256(sort_temp_bytes(n_tokens, num_embeddings > 1 ? num_embeddings : 2));
}

TG_EXPORT int tg_embedding_bwd(int dtype_dout, const void* dout, const int64_t* indices,
                               int64_t n_tokens, int64_t dim, int dtype_grad, void* grad,
                               int64_t num_embeddings, int accumulate, void* workspace,
                               size_t workspace_bytes, void* stream) {
  TG_REQUIRE(n_tokens >= 0 && dim > 0 && num_embeddings > 0, "tg_embedding_bwd: bad shape");
  TG_REQUIRE(n_tokens <= 0x7fffffff, "tg_embedding_bwd: too many tokens");
  TG_REQUIRE(grad && (n_tokens == 0 || (dout && indices)), "tg_embedding_bwd: null pointer");
  const size_t need = tg_embedding_bwd_workspace(n_tokens, num_embeddings);
  if (n_tokens > 0 && (!workspace || workspace_bytes < need)) {
    tg_set_error("tg_embedding_bwd: workspace of %zu bytes needed, got %zu", need,
                 workspace ? workspace_bytes : (size_t)0);
    return TG_ERR_WORKSPACE;
  }
  hipStream_t s = tg_stream(stream);
  char* ws = (char*)workspace;
#define G(TD)                                                                                  \
  switch (dtype_grad) {                                                                        \
    case TG_F32: return embed_t<TD, float>(dout, indices, n_tokens, dim, grad, num_embeddings, \
                                           accumulate, ws, workspace_bytes, s);                \
    case TG_F16: return embed_t<TD, tg_half>(dout, indices, n_tokens, dim, grad,               \
                                             num_embeddings, accumulate, ws, workspace_bytes,  \
                                             s);                                               \
    case TG_BF16: return embed_t<TD, tg_bf16>(dout, indices, n_tokens, dim, grad,              \
                                              num_embeddings, accumulate, ws, workspace_bytes, \
                                              s);                                              \
  }                                                                                            \
  break;
  switch (dtype_dout) {
    case TG_F32: G(float)
    case TG_F16: G(tg_half)
    case TG_BF16: G(tg_bf16)
  }
#undef G
  tg_set_error("tg_embedding_bwd: unsupported dtypes %d/%d", dtype_dout, dtype_grad);
  return TG_ERR_UNSUPPORTED;
}

TG_EXPORT int tg_embedding_fwd(int dtype_w, const void* weight, const int64_t* indices,
                               int64_t n_tokens, int64_t dim, int64_t num_embeddings,
                               int dtype_out, void* out, void* stream) {
  TG_REQUIRE(n_tokens >= 0 && dim >= 0 && num_embeddings > 0, "tg_embedding_fwd: bad shape");
  if (n_tokens == 0 || dim == 0) return TG_OK;
  TG_REQUIRE(weight && indices && out, "tg_embedding_fwd: null pointer");
  hipStream_t s = tg_stream(stream);
#define EF(TW)                                                                                 \
  switch (dtype_out) {                                                                         \
    case TG_F32: return embed_fwd_t<TW, float>(weight, indices, n_tokens, dim, num_embeddings, \
                                               out, s);                                        \
    case TG_F16: return embed_fwd_t<TW, tg_half>(weight, indices, n_tokens, dim,               \
                                                 num_embeddings, out, s);                      \
    case TG_BF16: return embed_fwd_t<TW, tg_bf16>(weight, indices, n_tokens, dim,              \
                                                  num_embeddings, out, s);                     \
  }                                                                                            \
  break;
  switch (dtype_w) {
    case TG_F32: EF(float)
    case TG_F16: EF(tg_half)
    case TG_BF16: EF(tg_bf16)
  }
#undef EF
  tg_set_error("tg_embedding_fwd: unsupported dtypes %d/%d", dtype_w, dtype_out);
  return TG_ERR_UNSUPPORTED;
}

TG_EXPORT int tg_transpose_add(int dtype_src, const void* src, int64_t rows, int64_t cols,
                               int dtype_dst, void* dst, float alpha, void* stream) {
  TG_REQUIRE(rows >= 0 && cols >= 0, "tg_transpose_add: negative shape");
  if (rows == 0 || cols == 0) return TG_OK;
  TG_REQUIRE(src && dst, "tg_transpose_add: null pointer");
  TG_REQUIRE((rows + 63) / 64 <= 65535, "tg_transpose_add: too many rows");
  hipStream_t s = tg_stream(stream);
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (dtype_src == TG_F32 && dtype_dst == TG_F32 && rows % 64 == 0 && cols % 64 == 0 &&
      cols / 64 <= 65535 && tg_aligned16(src) && tg_aligned16(dst)) {
    const dim3 gt((unsigned)(rows / 64), (unsigned)(cols / 64));
    k_transpose_add_v4<<<gt, kBlock, 0, s>>>((const float*)src, rows, cols, (float*)dst, alpha);
    return tg_check_launch("tg_transpose_add");
  }
#define T2(TS)                                                                                  \
  switch (dtype_dst) {                                                                          \
    case TG_F32: k_transpose_add<TS, float><<<grid, kBlock, 0, s>>>((const TS*)src, rows, cols, \
                                                                    (float*)dst, alpha);       \
      return tg_check_launch("tg_transpose_add");                                               \
    case TG_F16: k_transpose_add<TS, tg_half><<<grid, kBlock, 0, s>>>(                          \
        (const TS*)src, rows, cols, (tg_half*)dst, alpha);                                      \
      return tg_check_launch("tg_transpose_add");                                               \
    case TG_BF16: k_transpose_add<TS, tg_bf16><<<grid, kBlock, 0, s>>>(                         \
        (const TS*)src, rows, cols, (tg_bf16*)dst, alpha);                                      \
      return tg_check_launch("tg_transpose_add");                                               \
  }                                                                                             \
  break;
  switch (dtype_src) {
    case TG_F32: T2(float)
    case TG_F16: T2(tg_half)
    case TG_BF16: T2(tg_bf16)
  }
#undef T2
  tg_set_error("tg_transpose_add: unsupported dtypes %d/%d", dtype_src, dtype_dst);
  return TG_ERR_UNSUPPORTED;
}
