// Embedding backward and the tied-weight gradient transfer.
//
// tg_embedding_bwd: grad[idx[i]] (+)= dout[i] (Embedding._backward, _nn.py:1083-1089,
// a scatter-add), deterministic, in the order np.add.at applies the tokens.  Up to 8192
// tokens: one launch of k_embed_band (each workgroup finds the tokens of its band of
// gradient rows and writes every row once).  More tokens: the tokens are sorted by
// (index, position) -- 64-bit
// keys index << 32 | position, all distinct -- with a radix sort of 8192-key chunks in
// LDS (stable, so equal indices keep their token order) and, for more tokens, merge
// passes of the sorted chunks.  One wavefront per run of equal indices then sums the
// run's dout rows in their original order in fp32 and writes the gradient row once --
// the order np.add.at uses, so fp32 results match it exactly.  When not accumulating,
// every gradient row is zeroed first; for up to 8192 tokens that fill runs in the same
// launch as the sort (one workgroup sorts, the others write zeros), so the sort's
// latency hides behind the fill.  Indices in [-V, 0) count from the end (NumPy
// indexing, as the reference's forward gathers); indices outside [-V, V) are skipped.
//
// tg_transpose_add: dst[c][r] += alpha * src[r][c] through 64x64 LDS tiles
// (sync_tied_gradients, _training.py:264-284: source.grad += param.grad.T).
#include "tg_common.h"

namespace {

constexpr int kBlock = 256;

// A dout element as added: fp32 for 16/32-bit dout; fp64 dout is added in double and the
// sum rounded to fp32 at every step, as np.add.at does on a float32 array.
__device__ __forceinline__ float tg_in(float v) { return v; }
__device__ __forceinline__ float tg_in(tg_half v) { return (float)v; }
__device__ __forceinline__ float tg_in(tg_bf16 v) { return (float)v; }
__device__ __forceinline__ double tg_in(double v) { return v; }
__device__ __forceinline__ void acc_add(float& a, float v) { a += v; }
__device__ __forceinline__ void acc_add(float& a, double v) { a = (float)((double)a + v); }
template <typename TD> using InT = decltype(tg_in(TD()));

constexpr int kSortThreads = 1024;

__device__ __forceinline__ int64_t wrap_index(int64_t k, int64_t V) { return k < 0 ? k + V : k; }
constexpr int kChunk = 8192;  // keys sorted per workgroup in LDS (two 64 KiB buffers)

// Sort keys: index << pb | position, with pb position bits (32 in 64-bit keys; in
// 32-bit keys, used when the index and position bits fit, the fewest that hold n - 1).
template <typename K>
__device__ __forceinline__ K sort_key(const int64_t* idx, int64_t i, int64_t V, int pb) {
  const int64_t k = wrap_index(idx[i], V);
  const K key = (k >= 0 && k < V) ? (K)k : (K)V;  // V: skipped
  return key << pb | (K)i;
}

// Each workgroup sorts one chunk of kChunk tokens by index in LDS and writes it to
// out[chunk]: a least-significant-digit radix sort on 8-bit digits of the index, which
// is stable, so equal indices keep their token order and the chunk ends sorted by the
// whole 64-bit key.  A pass: each wavefront owns 512 consecutive keys (8 rounds of 64);
// lanes holding the same digit are found with 8 ballots, so each key's rank among equal
// digits in its wavefront comes from a per-wavefront digit histogram; a scan over
// (digit, wavefront) gives every group's destination.  Workgroups from `nsort` on do
// not sort: they write zeros over `fill` (fill_n elements of type TG; none if null).
template <typename K, typename TG>
__global__ __launch_bounds__(kSortThreads) void k_embed_sort_chunk(const int64_t* __restrict__ idx,
                                                                   int64_t n, int64_t V, int pb,
                                                                   int passes, int nsort,
                                                                   K* __restrict__ out,
                                                                   TG* __restrict__ fill,
                                                                   int64_t fill_n) {
  if ((int)blockIdx.x >= nsort) {
    constexpr int PZ = 16 / (int)sizeof(TG);
    tg_vec16<TG> z;
#pragma unroll
    for (int e = 0; e < PZ; ++e) z.v[e] = tg_from_float<TG>(0.f);
    const bool al = (reinterpret_cast<uintptr_t>(fill) & 15) == 0;
    const int64_t nv = al ? fill_n / PZ : 0, fb = (int64_t)gridDim.x - nsort;
    const int64_t stride = fb * kSortThreads;
    const int64_t t0 = ((int64_t)blockIdx.x - nsort) * kSortThreads + threadIdx.x;
    for (int64_t v = t0; v < nv; v += stride) tg_store16_nt(fill + v * PZ, z);
    for (int64_t e = nv * PZ + t0; e < fill_n; e += stride) fill[e] = tg_from_float<TG>(0.f);
    return;
  }
  constexpr int kWaves = kSortThreads / 64, kPer = kChunk / kWaves, kRounds = kPer / 64;
  __shared__ K buf[2][kChunk];
  __shared__ int hist[kWaves][256];
  __shared__ int wtot[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t lt = (1ull << lane) - 1;
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  const int cnt = (int)(n - base < kChunk ? n - base : kChunk);
  for (int i = threadIdx.x; i < cnt; i += kSortThreads) buf[0][i] = sort_key<K>(idx, base + i, V, pb);
  int cur = 0;
  for (int pass = 0; pass < passes; ++pass, cur ^= 1) {
    const int sh = pb + 8 * pass;
    for (int d = lane; d < 256; d += 64) hist[w][d] = 0;
    __syncthreads();
    K val[kRounds];
    int dig[kRounds], rank[kRounds];
#pragma unroll
    for (int it = 0; it < kRounds; ++it) {
      const int i = w * kPer + it * 64 + lane;
      const bool ok = i < cnt;
      val[it] = ok ? buf[cur][i] : 0;
      const int d = (int)((val[it] >> sh) & 255);
      uint64_t m = __ballot(ok);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint64_t bb = __ballot((d >> b) & 1);
        m &= ((d >> b) & 1) ? bb : ~bb;
      }
      const int h = ok ? hist[w][d] : 0;
      dig[it] = d;
      rank[it] = h + __popcll(m & lt);
      if (ok && (m & lt) == 0) hist[w][d] = h + __popcll(m);  // the group's first lane
    }
    __syncthreads();
    // exclusive offsets in (digit, wavefront) order: threads 0..255 own one digit each
    int run = 0, inc = 0;
    if (threadIdx.x < 256) {
      const int d = threadIdx.x;
      for (int ww = 0; ww < kWaves; ++ww) {
        const int c = hist[ww][d];
        hist[ww][d] = run;
        run += c;
      }
      inc = run;  // inclusive scan of the digit totals within the wavefront
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off, 64);
        if (lane >= off) inc += y;
      }
      if (lane == 63) wtot[w] = inc;
    }
    __syncthreads();
    if (threadIdx.x < 256) {
      int add = inc - run;  // digits of lower wavefronts come first
      for (int ww = 0; ww < w; ++ww) add += wtot[ww];
      for (int ww = 0; ww < kWaves; ++ww) hist[ww][threadIdx.x] += add;
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kRounds; ++it) {
      const int i = w * kPer + it * 64 + lane;
      if (i < cnt) buf[cur ^ 1][hist[w][dig[it]] + rank[it]] = val[it];
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < cnt; i += kSortThreads) out[base + i] = buf[cur][i];
}

// One merge pass: adjacent sorted runs of `width` keys (all keys distinct) merged into
// runs of 2*width.  Each element's output position is its rank in its own run plus
// the number of keys of the partner run below it (binary search).
template <typename K>
__global__ __launch_bounds__(256) void k_embed_merge(const K* __restrict__ in, int64_t n,
                                                     int64_t width, K* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const K v = in[i];
  const int64_t pair = i / (2 * width) * (2 * width);
  const bool left = i - pair < width;
  const int64_t own0 = left ? pair : pair + width;
  int64_t o0 = left ? pair + width : pair;
  int64_t o1 = left ? pair + 2 * width : pair + width;
  if (o0 > n) o0 = n;
  if (o1 > n) o1 = n;
  int64_t lo = o0, hi = o1;  // first partner key > v (keys are distinct)
  while (lo < hi) {
    const int64_t m = (lo + hi) >> 1;
    if (in[m] < v) lo = m + 1;
    else hi = m;
  }
  out[pair + (i - own0) + (lo - o0)] = v;
}

// One wavefront per sorted position; a wave whose position starts a run of equal
// indices sums the run's dout rows in their original order (four rows in flight) and
// writes the gradient row once: grad (+)= sum.  VEC: each lane owns PER = 16/sizeof(TD)
// adjacent columns (16-byte loads); else 4 columns 64 apart.
template <typename K, typename TD, typename TG, bool VEC, bool VG>
__global__ __launch_bounds__(kBlock) void k_embed_seg(const K* __restrict__ sorted, int pb,
                                                      int64_t n, const TD* __restrict__ dout,
                                                      int64_t dim, int64_t V, int accumulate,
                                                      TG* __restrict__ grad) {
  constexpr int PER = VEC ? 16 / (int)sizeof(TD) : 4;
  constexpr int U = 4;
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  if (i >= n) return;
  const K pmask = ((K)1 << pb) - 1;
  const K key = sorted[i] >> pb;
  if (key >= (K)V) return;                            // index outside [0, V)
  if (i > 0 && (sorted[i - 1] >> pb) == key) return;  // not the start of a run
  int64_t end = i + 1;
  while (end < n && (sorted[end] >> pb) == key) ++end;
  TG* grow = grad + (int64_t)key * dim;
  auto col = [&](int64_t c0, int e) {
    return VEC ? c0 + (int64_t)lane * PER + e : c0 + (int64_t)e * 64 + lane;
  };
  for (int64_t c0 = 0; c0 < dim; c0 += 64 * PER) {
    float acc[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] = 0.f;
    using IT = InT<TD>;
    auto load = [&](int64_t j, IT (&v)[PER]) {
      const TD* drow = dout + (int64_t)(sorted[j] & pmask) * dim;
      if (VEC) {
        if (col(c0, 0) < dim) {
          const tg_vec16<TD> t = tg_load16(drow + col(c0, 0));
#pragma unroll
          for (int e = 0; e < PER; ++e) v[e] = tg_in(t.v[e]);
        } else {
#pragma unroll
          for (int e = 0; e < PER; ++e) v[e] = 0;
        }
      } else {
#pragma unroll
        for (int e = 0; e < PER; ++e) v[e] = col(c0, e) < dim ? tg_in(drow[col(c0, e)]) : (IT)0;
      }
    };
    int64_t j = i;
    for (; j + U <= end; j += U) {
      IT v[U][PER];
#pragma unroll
      for (int u = 0; u < U; ++u) load(j + u, v[u]);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < PER; ++e) acc_add(acc[e], v[u][e]);
    }
    for (; j < end; ++j) {
      IT v[PER];
      load(j, v);
#pragma unroll
      for (int e = 0; e < PER; ++e) acc_add(acc[e], v[e]);
    }
    if (VG && col(c0, 0) < dim) {  // PER adjacent outputs per lane as 16-byte stores
      constexpr int NG = tg_vec16<TG>::N;
#pragma unroll
      for (int h = 0; h < PER / NG; ++h) {
        TG* p = grow + col(c0, h * NG);
        tg_vec16<TG> o;
        if (accumulate) o = tg_load16(p);
#pragma unroll
        for (int e = 0; e < NG; ++e)
          o.v[e] = tg_from_float<TG>((accumulate ? tg_to_float(o.v[e]) : 0.f) + acc[h * NG + e]);
        tg_store16(p, o);
      }
    } else if (!VG) {
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const int64_t c = col(c0, e);
        if (c < dim)
          grow[c] = tg_from_float<TG>((accumulate ? tg_to_float(grow[c]) : 0.f) + acc[e]);
      }
    }
  }
}

// Up to kChunk tokens, one launch, no sort and no workspace: workgroup b owns the
// gradient rows [b*kBandRows, (b+1)*kBandRows) and writes each of them exactly once.
// Phase 1: wave w scans tokens [w*seg, (w+1)*seg) of the indices and keeps the ones
// that fall in the band in LDS, in token order (ballot compaction), as
// (row in band) << 16 | token.  The four wave lists read in wave order are therefore
// the band's tokens in token order.  Phase 2: wave w takes band rows w, w+4, ...; for
// each column chunk it walks the lists, and for every token of its row adds the dout
// row in token order (the order np.add.at applies them), then writes grad (+)= sum, or
// zeros for a row no token touches (nothing, when accumulating).
constexpr int kBandRows = 64;
constexpr int kBandThreads = 512;

template <typename TD, typename TG, bool VEC, bool VG>
__global__ __launch_bounds__(kBandThreads) void k_embed_band(const int64_t* __restrict__ idx, int n,
                                                       const TD* __restrict__ dout, int64_t dim,
                                                       int64_t V, int accumulate,
                                                       TG* __restrict__ grad) {
  constexpr int PER = VEC ? 16 / (int)sizeof(TD) : 4;
  constexpr int NW = kBandThreads / 64;
  __shared__ uint32_t list[kChunk];
  __shared__ int cnt[NW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * kBandRows;
  const int seg = (n + NW - 1) / NW;
  const int t0 = wave * seg, t1 = min(n, t0 + seg);
  uint32_t* wl = list + t0;
  const uint64_t below = (1ull << lane) - 1;
  // all of the wave's indices are loaded at once (seg <= kChunk / NW = 64 * KPL), so
  // the scan costs one memory round trip
  constexpr int KPL = kChunk / NW / 64;
  int64_t k[KPL];
#pragma unroll
  for (int u = 0; u < KPL; ++u) {
    const int i = t0 + u * 64 + lane;
    k[u] = i < t1 ? wrap_index(idx[i], V) : -1;
  }
  int c = 0;
#pragma unroll
  for (int u = 0; u < KPL; ++u) {
    const bool hit = k[u] >= r0 && k[u] < r0 + kBandRows && k[u] < V;
    const uint64_t m = __ballot(hit);
    if (hit) wl[c + __popcll(m & below)] = (uint32_t)(k[u] - r0) << 16 | (uint32_t)(u * 64 + lane);
    c += __popcll(m);
  }
  if (lane == 0) cnt[wave] = c;
  __syncthreads();
  int wc[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) wc[w] = cnt[w];
  auto col = [&](int64_t c0, int e) {
    return VEC ? c0 + (int64_t)lane * PER + e : c0 + (int64_t)e * 64 + lane;
  };
  for (int rl = wave; rl < kBandRows; rl += NW) {
    const int64_t row = r0 + rl;
    if (row >= V) break;
    bool any = false;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      for (int b = 0; b < wc[w] && !any; b += 64)
        any = __ballot(b + lane < wc[w] && (int)(list[w * seg + b + lane] >> 16) == rl) != 0;
    if (!any && accumulate) continue;
    TG* grow = grad + row * dim;
    // NCH column chunks of 64 * PER per pass: a token's loads for all of them are in
    // flight together
    constexpr int NCH = 4;
    for (int64_t c0 = 0; c0 < dim; c0 += NCH * 64 * PER) {
      float acc[NCH][PER];
#pragma unroll
      for (int q = 0; q < NCH; ++q)
#pragma unroll
        for (int e = 0; e < PER; ++e) acc[q][e] = 0.f;
      auto add = [&](int tok) {
        const TD* drow = dout + (int64_t)tok * dim;
        if (VEC) {
          tg_vec16<TD> t[NCH];
#pragma unroll
          for (int q = 0; q < NCH; ++q)
            if (col(c0 + q * 64 * PER, 0) < dim) t[q] = tg_load16(drow + col(c0 + q * 64 * PER, 0));
#pragma unroll
          for (int q = 0; q < NCH; ++q)
            if (col(c0 + q * 64 * PER, 0) < dim)
#pragma unroll
              for (int e = 0; e < PER; ++e) acc_add(acc[q][e], tg_in(t[q].v[e]));
        } else {
#pragma unroll
          for (int q = 0; q < NCH; ++q)
#pragma unroll
            for (int e = 0; e < PER; ++e) {
              const int64_t cc = col(c0 + q * 64 * PER, e);
              if (cc < dim) acc_add(acc[q][e], tg_in(drow[cc]));
            }
        }
      };
      if (any) {
#pragma unroll
        for (int w = 0; w < NW; ++w)
          for (int b = 0; b < wc[w]; b += 64) {
            const uint32_t e = b + lane < wc[w] ? list[w * seg + b + lane] : 0xffffffffu;
            uint64_t m = __ballot((int)(e >> 16) == rl);
            while (m) {  // tokens of this row in token order
              const int j = __builtin_ctzll(m);
              m &= m - 1;
              add(w * seg + (int)(__shfl(e, j, 64) & 0xffffu));
            }
          }
      }
#pragma unroll
      for (int q = 0; q < NCH; ++q) {
        const int64_t cq = c0 + q * 64 * PER;
        if (VG && col(cq, 0) < dim) {
          constexpr int NG = tg_vec16<TG>::N;
#pragma unroll
          for (int h = 0; h < PER / NG; ++h) {
            TG* p = grow + col(cq, h * NG);
            tg_vec16<TG> o;
            if (accumulate) o = tg_load16(p);
#pragma unroll
            for (int e = 0; e < NG; ++e)
              o.v[e] = tg_from_float<TG>((accumulate ? tg_to_float(o.v[e]) : 0.f) +
                                         acc[q][h * NG + e]);
            tg_store16(p, o);
          }
        } else if (!VG) {
#pragma unroll
          for (int e = 0; e < PER; ++e) {
            const int64_t cc = col(cq, e);
            if (cc < dim)
              grow[cc] =
                  tg_from_float<TG>((accumulate ? tg_to_float(grow[cc]) : 0.f) + acc[q][e]);
          }
        }
      }
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

// The same in double, for gradients where either side is float64 (the reference's
// source.grad += param.grad.T adds in the wider dtype and casts to the destination's).
template <typename TS, typename TD>
__global__ __launch_bounds__(kBlock) void k_transpose_add_d(const TS* __restrict__ src, int64_t R,
                                                            int64_t C, TD* __restrict__ dst,
                                                            double alpha) {
  __shared__ double tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int rr = ty + 4 * k;
    const int64_t r = r0 + rr, c = c0 + tx;
    tile[rr][tx] = (r < R && c < C) ? (double)src[r * C + c] : 0.0;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int cc = ty + 4 * k;
    const int64_t c = c0 + cc, r = r0 + tx;  // dst[c][r]
    if (c < C && r < R) {
      TD* p = dst + c * R + r;
      *p = (TD)((double)*p + alpha * tile[tx][cc]);
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

// Workspace: two n-key buffers of 64-bit keys (the sorted keys and the merge passes'
// partner); 32-bit keys use the front of each.
// (none up to kChunk tokens: the band kernel needs no scratch)
size_t embed_ws(int64_t n) { return n <= kChunk ? 0 : 2 * align256(n * sizeof(uint64_t)); }

int bits_for(int64_t v) {  // bits holding 0..v
  int b = 1;
  while (b < 63 && (v >> b) > 0) ++b;
  return b;
}

template <typename K, typename TD, typename TG>
int embed_k(const void* dout, const int64_t* idx, int64_t n, int64_t dim, void* grad, int64_t V,
            int accumulate, char* ws, int pb, hipStream_t s) {
  constexpr int PER = 16 / (int)sizeof(TD);
  const bool vec = dim % PER == 0 && tg_aligned16(dout);
  const bool vg = vec && (PER * sizeof(TG)) % 16 == 0 && (dim * sizeof(TG)) % 16 == 0 &&
                  tg_aligned16(grad);
  if (n <= kChunk) {
    if (n == 0 && accumulate) return TG_OK;
    const unsigned nb = (unsigned)((V + kBandRows - 1) / kBandRows);
#define BAND(VE, VGE)                                                                         \
  k_embed_band<TD, TG, VE, VGE><<<nb, kBandThreads, 0, s>>>(idx, (int)n, (const TD*)dout, dim, V, \
                                                      accumulate, (TG*)grad)
    if (vg) BAND(true, true);
    else if (vec) BAND(true, false);
    else BAND(false, false);
#undef BAND
    return tg_check_launch("tg_embedding_bwd");
  }
  const int64_t total = V * dim;
  int64_t fill_blocks = (total + 8 * kSortThreads - 1) / (8 * kSortThreads);
  if (fill_blocks > (int64_t)tg_num_cus() * 2) fill_blocks = (int64_t)tg_num_cus() * 2;
  if (fill_blocks < 1) fill_blocks = 1;
  if (n == 0) {  // nothing indexed: the gradient is zero (or unchanged)
    if (!accumulate)
      k_embed_sort_chunk<K, TG><<<(unsigned)fill_blocks, kSortThreads, 0, s>>>(
          nullptr, 0, V, pb, 0, 0, nullptr, (TG*)grad, total);
    return tg_check_launch("tg_embedding_bwd");
  }
  const size_t nb = align256(n * sizeof(uint64_t));
  K* buf[2] = {(K*)ws, (K*)(ws + nb)};
  const int64_t chunks = (n + kChunk - 1) / kChunk;
  const int passes = (bits_for(V) + 7) / 8;  // 8-bit digits of indices 0..V (V: skipped)
  // one chunk: the zero fill rides in the sort's launch; else it is its own launch
  const bool fused = !accumulate && chunks == 1;
  k_embed_sort_chunk<K, TG><<<(unsigned)(chunks + (fused ? fill_blocks : 0)), kSortThreads, 0, s>>>(
      idx, n, V, pb, passes, (int)chunks, buf[0], fused ? (TG*)grad : nullptr, fused ? total : 0);
  if (!accumulate && !fused)
    k_embed_sort_chunk<K, TG><<<(unsigned)fill_blocks, kSortThreads, 0, s>>>(
        nullptr, 0, V, pb, 0, 0, nullptr, (TG*)grad, total);
  int cur = 0;
  for (int64_t w = kChunk; w < n; w *= 2, cur ^= 1)
    k_embed_merge<K><<<(unsigned)((n + 255) / 256), 256, 0, s>>>(buf[cur], n, w, buf[cur ^ 1]);
  const unsigned sb = (unsigned)((n + 3) / 4);
#define SEG(VE, VGE)                                                                        \
  k_embed_seg<K, TD, TG, VE, VGE><<<sb, kBlock, 0, s>>>(buf[cur], pb, n, (const TD*)dout, dim, \
                                                        V, accumulate, (TG*)grad)
  if (vg) SEG(true, true);
  else if (vec) SEG(true, false);
  else SEG(false, false);
#undef SEG
  return tg_check_launch("tg_embedding_bwd");
}

template <typename TD, typename TG>
int embed_t(const void* dout, const int64_t* idx, int64_t n, int64_t dim, void* grad, int64_t V,
            int accumulate, char* ws, hipStream_t s) {
  const int pb = n > 1 ? bits_for(n - 1) : 1;
  if (bits_for(V) + pb <= 32)
    return embed_k<uint32_t, TD, TG>(dout, idx, n, dim, grad, V, accumulate, ws, pb, s);
  return embed_k<uint64_t, TD, TG>(dout, idx, n, dim, grad, V, accumulate, ws, 32, s);
}

}  // namespace

TG_EXPORT size_t tg_embedding_bwd_workspace(int64_t n_tokens, int64_t num_embeddings) {
  if (n_tokens <= 0) return 0;
  return embed_ws(n_tokens);
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
  if (need > 0 && (!workspace || workspace_bytes < need)) {
    tg_set_error("tg_embedding_bwd: workspace of %zu bytes needed, got %zu", need,
                 workspace ? workspace_bytes : (size_t)0);
    return TG_ERR_WORKSPACE;
  }
  hipStream_t s = tg_stream(stream);
  char* ws = (char*)workspace;
#define G(TD)                                                                              \
  switch (dtype_grad) {                                                                    \
    case TG_F32:                                                                           \
      return embed_t<TD, float>(dout, indices, n_tokens, dim, grad, num_embeddings,        \
                                accumulate, ws, s);                                        \
    case TG_F16:                                                                           \
      return embed_t<TD, tg_half>(dout, indices, n_tokens, dim, grad, num_embeddings,      \
                                  accumulate, ws, s);                                      \
    case TG_BF16:                                                                          \
      return embed_t<TD, tg_bf16>(dout, indices, n_tokens, dim, grad, num_embeddings,      \
                                  accumulate, ws, s);                                      \
  }                                                                                        \
  break;
  switch (dtype_dout) {
    case TG_F32: G(float)
    case TG_F16: G(tg_half)
    case TG_BF16: G(tg_bf16)
    case TG_F64: G(double)  // each row rounded to fp32, then added in fp32 (np.add.at)
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
  if (dtype_src == TG_F64 || dtype_dst == TG_F64) {
#define D2(TS, TD) \
  k_transpose_add_d<TS, TD><<<grid, kBlock, 0, s>>>((const TS*)src, rows, cols, (TD*)dst, (double)alpha)
    if (dtype_src == TG_F64 && dtype_dst == TG_F64) D2(double, double);
    else if (dtype_src == TG_F64 && dtype_dst == TG_F32) D2(double, float);
    else if (dtype_src == TG_F32 && dtype_dst == TG_F64) D2(float, double);
    else {
      tg_set_error("tg_transpose_add: unsupported dtypes %d/%d", dtype_src, dtype_dst);
      return TG_ERR_UNSUPPORTED;
    }
#undef D2
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
