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

template <typename T>
__global__ __launch_bounds__(kBlock) void k_fill_zero(T* __restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    p[i] = tg_from_float<T>(0.f);
}

// Sort input: positions 0..n-1 and 32-bit keys, every index outside [0, V) mapped to
// the sentinel V (sorted after all valid keys, then skipped).  When not accumulating,
// also clears the per-row "touched" flags.
__global__ __launch_bounds__(kBlock) void k_embed_prep(const int64_t* __restrict__ idx,
                                                       int64_t n, int64_t V,
                                                       int* __restrict__ keys,
                                                       int* __restrict__ pos,
                                                       int* __restrict__ touched) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) {
    const int64_t k = idx[i];
    keys[i] = (k >= 0 && k < V) ? (int)k : (int)V;
    pos[i] = (int)i;
  }
  if (touched && i < V) touched[i] = 0;
}

// One wavefront per sorted position; a wave whose position starts a run of equal keys
// sums the run's dout rows in their original order (four rows in flight) and writes
// the gradient row: grad (+)= sum when accumulating, else grad = sum and the row is
// marked touched.  VEC: each lane owns PER = 16/sizeof(TD) adjacent columns (16-byte
// loads); else 4 columns 64 apart.
template <typename TD, typename TG, bool VEC>
__global__ __launch_bounds__(kBlock) void k_embed_seg(const int* __restrict__ keys,
                                                      const int* __restrict__ pos, int64_t n,
                                                      const TD* __restrict__ dout, int64_t dim,
                                                      int64_t V, int accumulate,
                                                      int* __restrict__ touched,
                                                      TG* __restrict__ grad) {
  constexpr int PER = VEC ? 16 / (int)sizeof(TD) : 4;
  constexpr int U = 4;
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  if (i >= n) return;
  const int key = keys[i];
  if (i > 0 && keys[i - 1] == key) return;  // not the start of a run
  if (key >= V) return;                     // sentinel: index outside [0, V)
  int64_t end = i + 1;
  while (end < n && keys[end] == key) ++end;
  TG* grow = grad + (int64_t)key * dim;
  auto col = [&](int64_t c0, int e) {
    return VEC ? c0 + (int64_t)lane * PER + e : c0 + (int64_t)e * 64 + lane;
  };
  for (int64_t c0 = 0; c0 < dim; c0 += 64 * PER) {
    float acc[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] = 0.f;
    auto load = [&](int64_t j, float (&v)[PER]) {
      const TD* drow = dout + (int64_t)pos[j] * dim;
      if (VEC) {
        if (col(c0, 0) < dim) {
          const tg_vec16<TD> t = tg_load16(drow + col(c0, 0));
#pragma unroll
          for (int e = 0; e < PER; ++e) v[e] = tg_to_float(t.v[e]);
        } else {
#pragma unroll
          for (int e = 0; e < PER; ++e) v[e] = 0.f;
        }
      } else {
#pragma unroll
        for (int e = 0; e < PER; ++e) v[e] = col(c0, e) < dim ? tg_to_float(drow[col(c0, e)]) : 0.f;
      }
    };
    int64_t j = i;
    for (; j + U <= end; j += U) {
      float v[U][PER];
#pragma unroll
      for (int u = 0; u < U; ++u) load(j + u, v[u]);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < PER; ++e) acc[e] += v[u][e];
    }
    for (; j < end; ++j) {
      float v[PER];
      load(j, v);
#pragma unroll
      for (int e = 0; e < PER; ++e) acc[e] += v[e];
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int64_t c = col(c0, e);
      if (c < dim)
        grow[c] = tg_from_float<TG>((accumulate ? tg_to_float(grow[c]) : 0.f) + acc[e]);
    }
  }
  if (!accumulate && lane == 0) touched[key] = 1;
}

// Zero every gradient row that no index touched (not accumulating): one wavefront per
// row, 16-byte non-temporal stores when rows are 16-byte multiples.
template <typename TG, bool VZ>
__global__ __launch_bounds__(kBlock) void k_embed_zero_rows(const int* __restrict__ touched,
                                                            int64_t V, int64_t dim,
                                                            TG* __restrict__ grad) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * (kBlock / 64);
  for (int64_t r = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6); r < V; r += stride) {
    if (touched[r]) continue;
    TG* grow = grad + r * dim;
    if (VZ) {
      constexpr int PER = 16 / (int)sizeof(TG);
      tg_vec16<TG> z;
#pragma unroll
      for (int e = 0; e < PER; ++e) z.v[e] = tg_from_float<TG>(0.f);
      for (int64_t c = (int64_t)lane * PER; c < dim; c += 64 * PER) tg_store16_nt(grow + c, z);
    } else {
      for (int64_t c = lane; c < dim; c += 64) grow[c] = tg_from_float<TG>(0.f);
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
  (void)rocprim::radix_sort_pairs(nullptr, bytes, (const int*)nullptr, (int*)nullptr,
                                  (const int*)nullptr, (int*)nullptr, (size_t)n, 0,
                                  sort_bits(V + 1));
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

// Workspace: keys_in, keys_out, pos_in, pos_out (n ints each), touched (V ints), then
// rocPRIM's radix-sort scratch.
size_t embed_ws(int64_t n, int64_t V, size_t* tmp_off) {
  const size_t fixed = 4 * align256(n * sizeof(int)) + align256(V * sizeof(int));
  if (tmp_off) *tmp_off = fixed;
  return fixed + align256(sort_temp_bytes(n, V));
}

template <typename TD, typename TG>
int embed_t(const void* dout, const int64_t* idx, int64_t n, int64_t dim, void* grad, int64_t V,
            int accumulate, char* ws, size_t ws_bytes, hipStream_t s) {
  if (n == 0) {  // nothing indexed: the gradient is zero (or unchanged)
    if (!accumulate) {
      const int64_t total = V * dim;
      int64_t blocks = (total + kBlock - 1) / kBlock;
      if (blocks > (int64_t)tg_num_cus() * 16) blocks = (int64_t)tg_num_cus() * 16;
      k_fill_zero<TG><<<(unsigned)(blocks < 1 ? 1 : blocks), kBlock, 0, s>>>((TG*)grad, total);
    }
    return tg_check_launch("tg_embedding_bwd");
  }
  size_t tmp_off = 0;
  embed_ws(n, V, &tmp_off);
  const size_t nb = align256(n * sizeof(int));
  int* keys_in = (int*)ws;
  int* keys_out = (int*)(ws + nb);
  int* pos_in = (int*)(ws + 2 * nb);
  int* pos_out = (int*)(ws + 3 * nb);
  int* touched = accumulate ? nullptr : (int*)(ws + 4 * nb);
  char* tmp = ws + tmp_off;
  size_t tmp_bytes = ws_bytes - tmp_off;
  const int64_t m = n > V ? n : V;
  k_embed_prep<<<(unsigned)((m + kBlock - 1) / kBlock), kBlock, 0, s>>>(idx, n, V, keys_in, pos_in,
                                                                        touched);
  if (rocprim::radix_sort_pairs(tmp, tmp_bytes, keys_in, keys_out, pos_in, pos_out, (size_t)n, 0,
                                sort_bits(V + 1), s) != hipSuccess) {
    tg_set_error("tg_embedding_bwd: radix sort failed");
    return TG_ERR_HIP;
  }
  constexpr int PER = 16 / (int)sizeof(TD);
  const bool vec = dim % PER == 0 && tg_aligned16(dout);
  const unsigned sb = (unsigned)((n + 3) / 4);
  if (vec)
    k_embed_seg<TD, TG, true><<<sb, kBlock, 0, s>>>(keys_out, pos_out, n, (const TD*)dout, dim, V,
                                                    accumulate, touched, (TG*)grad);
  else
    k_embed_seg<TD, TG, false><<<sb, kBlock, 0, s>>>(keys_out, pos_out, n, (const TD*)dout, dim,
                                                     V, accumulate, touched, (TG*)grad);
  if (!accumulate) {
    int64_t blocks = (V + 3) / 4;
    if (blocks > (int64_t)tg_num_cus() * 32) blocks = (int64_t)tg_num_cus() * 32;
    const bool vz = (dim * (int64_t)sizeof(TG)) % 16 == 0 && tg_aligned16(grad);
    if (vz)
      k_embed_zero_rows<TG, true><<<(unsigned)blocks, kBlock, 0, s>>>(touched, V, dim, (TG*)grad);
    else
      k_embed_zero_rows<TG, false><<<(unsigned)blocks, kBlock, 0, s>>>(touched, V, dim, (TG*)grad);
  }
  return tg_check_launch("tg_embedding_bwd");
}

}  // namespace

TG_EXPORT size_t tg_embedding_bwd_workspace(int64_t n_tokens, int64_t num_embeddings) {
  if (n_tokens <= 0) return 0;
  return embed_ws(n_tokens, num_embeddings > 1 ? num_embeddings : 1, nullptr);
}

TG_EXPORT int tg_embedding_bwd(int dtype_dout, const void* dout, const int64_t* indices,
                               int64_t n_tokens, int64_t dim, int dtype_grad, void* grad,
                               int64_t num_embeddings, int accumulate, void* workspace,
                               size_t workspace_bytes, void* stream) {
  TG_REQUIRE(n_tokens >= 0 && dim > 0 && num_embeddings > 0, "tg_embedding_bwd: bad shape");
  TG_REQUIRE(num_embeddings < 0x7fffffff, "tg_embedding_bwd: too many rows");
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
