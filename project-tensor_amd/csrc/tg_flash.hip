// FlashAttention forward and backward for gfx950, reference: flash_attention
// (_core.py:1686-1870).  Tuned kernels for fp16 / bf16 with head dim 64 or 128; generic
// kernels (fp32 matrix cores, any head dim up to 256) for fp32 and other head dims.
//
// Tensors are contiguous [B, H, S, D]; lse is [B, H, Sq] fp32 (natural log).
// causal masks key > query (top-left aligned, as the reference's col > row).
//
// MFMA layout facts used throughout (v_mfma_f32_32x32x16_{f16,bf16}, wave64):
//   A operand: lane (row = lane%32, half h = lane/32) supplies 8 k-elements,
//   B operand: lane (col = lane%32, half h) supplies 8 k-elements, the same k for
//              the same (h, element) as the A side,
//   C/D tile:  lane owns column lane%32 and rows 8*(r/4) + 4*h + r%4, r = 0..15.
// A C-layout tile T[rows][cols] can therefore feed a following MFMA either as the
// B operand (X * T, k = rows) or as the A operand of T^T (T^T * Y, k = rows) with
// no data movement, provided the other operand is read with the matching
// permutation of k.  For a 32-row tile and k-step s (0,1) the lane's 8 elements are
// its accumulator registers r = 8*s + e, i.e. rows 16*s + 8*(e/4) + 4*h + e%4.
// That other operand is read from LDS in that row order with transpose reads
// (ds_read_b64_tr_b16, see the backward tiles below).
//
// Forward: one workgroup = 128 queries (4 waves x 32), K/V tiles of 64 keys.
//   S^T = K Q^T (lane = query), online softmax per lane, O^T += V^T P^T.
// Backward (no atomics, two kernels):
//   k_fa_bwd_dkdv: one workgroup = 128 keys (4 waves x 32 keys), loop over query
//     tiles of 128: S = Q K^T (lane = key), P = exp(S*scale - lse), dP = dO V^T,
//     dS = P*(dP - D)*scale, dV += P^T dO, dK += dS^T Q (the factor scale is applied
//     to dK once, when it is stored).
//   k_fa_bwd_dq: one workgroup = 128 queries, loop over key tiles of 64:
//     S^T = K Q^T (lane = query), dP^T = V dO^T, dQ += dS K.
//   D = rowsum(dO * O) is formed by k_fa_bwd_dq (launched first) for its queries and
//   stored for k_fa_bwd_dkdv.
#include "tg_common.h"

#include <initializer_list>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Vec8;
template <> struct Vec8<tg_half> { typedef _Float16 type __attribute__((ext_vector_type(8))); };
template <> struct Vec8<tg_bf16> { typedef __bf16 type __attribute__((ext_vector_type(8))); };

__device__ __forceinline__ f32x16 mfma(Vec8<tg_half>::type a, Vec8<tg_half>::type b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma(Vec8<tg_bf16>::type a, Vec8<tg_bf16>::type b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

constexpr float kLog2e = 1.4426950408889634f;

// 2^x with the hardware v_exp_f32 (exp2(-inf) = 0; the softmax arguments here are
// <= 0 up to rounding, far from the overflow range).
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr int kThreads = 256;

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type ld8(const T* p) {
  return *reinterpret_cast<const typename Vec8<T>::type*>(p);
}

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type pack8(const float* v) {
  typename Vec8<T>::type r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (T)v[e];
  return r;
}

// Workgroup -> (tile, head) mapping.  Dispatch i lands on XCD i % 8.  The launch
// index is remapped so that XCD x gets the contiguous range [x*T/8, (x+1)*T/8) of a
// head-group-major order: groups of G heads (G divides the heads per XCD), and within
// a group tile-major order.  Each XCD then works on few heads at a time, so the
// workgroups of a head share its K/V or Q/dO re-reads in that XCD's L2; with G > 1
// (causal masking, where the callers make tile 0 the heaviest) the heaviest tiles of a
// group start first and the light ones fill in behind them (longest-first).  G = 0:
// no remap, every head tile-major (tile = index / heads, head = index % heads).
// Returns (tile, head).
__device__ __forceinline__ void fa_block(int64_t& tile, int64_t& head, int G) {
  const int64_t gx = gridDim.x, T = gx * gridDim.y;
  int64_t lin = (int64_t)blockIdx.y * gx + blockIdx.x;
  if (G == 0) {
    tile = lin / gridDim.y;
    head = lin % gridDim.y;
    return;
  }
  if (T % 8 == 0) lin = (lin % 8) * (T / 8) + lin / 8;
  const int64_t grp = lin / (G * gx), r = lin % (G * gx);
  tile = r / G;
  head = grp * G + r % G;
}

// Layout of Q/K/V/O/dO/dQ/dK/dV.  Logical [B, H, S, D]; in memory either
// contiguous [B, H, S, D] (bshd = 0: rows D elements apart) or [B, S, H, D] rows with
// head h at column h*D (bshd = 1: the head split of a projection, used without a
// transposing copy).  Under bshd the rows of Q/K/V/dQ/dK/dV are rsa elements apart and
// those of O/dO rso: H*D each for separate [B, S, H*D] tensors, rsa = 3*H*D for Q, K
// and V read from (and dQ, dK, dV written into) one packed [B, S, 3, H, D] projection.
// LSE and D stay [B, H, S].
struct FaLay {
  int64_t H;
  int bshd;
  int G;    // heads per dispatch group (fa_block)
  int rsa;  // row stride of Q, K, V, dQ, dK, dV
  int rso;  // row stride of O, dO
  __device__ __forceinline__ int64_t head(int64_t bh, int64_t S, int D, int rs) const {
    return bshd ? (bh / H) * S * rs + (bh % H) * D : bh * S * D;
  }
  __device__ __forceinline__ int64_t ha(int64_t bh, int64_t S, int D) const {
    return head(bh, S, D, rsa);
  }
  __device__ __forceinline__ int64_t ho(int64_t bh, int64_t S, int D) const {
    return head(bh, S, D, rso);
  }
};

// Row index (within a 32-row C tile) of accumulator register r for lane half h.
__device__ __forceinline__ int crow(int r, int h) { return ((r >> 2) << 3) + (h << 2) + (r & 3); }

// ============================================================================ backward
// Store of a wave's 32 x D accumulator tiles (rows row0.., C layout) through a wave-
// private LDS region st of 32 x D floats: each lane writes its column's 16 values, then
// reads back 8 consecutive values of one row and writes them with one 16-byte global
// store (plus one 16-byte load of the old values when accumulating), so every store
// instruction covers whole rows.  (Written straight from the C layout, the tiles need
// 16 two-byte stores per lane and tile, each covering two 64-byte row pieces: measured
// at about a quarter of the dK/dV kernel's time at d = 128.)  Columns of the rows with
// bit 2 set (lane half 1) are XOR-ed with 32 so the two lane halves write different
// banks.  out (+)= acc * mul, in fp32, then rounded to T.
template <typename T, int D>
__device__ __forceinline__ void store_tiles_staged(T* __restrict__ out, int64_t ld, int64_t row0,
                                                   int64_t nrows, const f32x16 (&acc)[D / 32],
                                                   float mul, int accumulate, int lane,
                                                   float* st) {
  const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      st[crow(r, h) * D + ((dt * 32 + l32) ^ (h << 5))] = acc[dt][r] * mul;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int LPR = D / 8, RPI = 64 / LPR;  // lanes per row, rows per pass
  const int c = (lane % LPR) * 8;
#pragma unroll
  for (int it = 0; it < 32 / RPI; ++it) {
    const int rr = it * RPI + lane / LPR;
    const float* src = st + rr * D + (c ^ (rr & 4 ? 32 : 0));
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const int64_t row = row0 + rr;
    if (row < nrows) {
      T* p = out + row * ld + c;
      tg_vec16<T> o;
      if (accumulate) o = tg_load16(p);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o.v[e] = (T)(v[e] + (accumulate ? (float)o.v[e] : 0.f));
      tg_store16(p, o);
    }
  }
}

// ---------------------------------------------------------------- backward tiles
// The backward kernels stage Q/dO (dK/dV kernel) or K/V (dQ kernel) tiles in LDS
// row-major, with no padding and the 16-byte chunks of each row XOR-swizzled by the
// row index (conflict-free 16-byte row reads by 32 consecutive rows).  Tiles are
// copied global -> LDS by the DMA path (global_load_lds, 16 bytes per lane, one
// contiguous KiB per wave instruction, no registers), double-buffered so the next
// tile streams in while the current one is computed.  Operands whose k index runs
// along the rows (P^T dO, dS^T Q, dS K) are read with ds_read_b64_tr_b16, which
// returns a column of 4 consecutive rows per lane: two such reads give an 8-element
// MFMA operand in the k order the C-tile trick needs.
typedef short v4i16 __attribute__((ext_vector_type(4)));
#define TG_LDS __attribute__((address_space(3)))
#define TG_GLB __attribute__((address_space(1)))

template <int D> struct SwzTile {
  static constexpr int CH = D / 8;  // 16-byte chunks per row
  static constexpr int RB = D * 2;  // bytes per row
  // XOR key of row r: 16 consecutive rows get distinct chunk positions (16-byte row
  // reads by 16 lanes hit every bank once) and rows r..r+3 of a transpose read land in
  // different 64-byte bank groups.
  __device__ static int key(int r) {
    if (CH == 8) {
      const int x = (r >> 1) & 7;
      return ((x & 1) << 2) | (x >> 1);
    }
    return ((r & 3) << 2) | ((r >> 2) & 3);
  }
  __device__ static int off(int r, int c) { return r * RB + ((c ^ key(r)) << 4); }
};

// Async copy of rows [row0, row0+R) (rows rs elements apart, D contiguous elements
// each) into a swizzled tile.  Rows past nrows copy row nrows-1; the kernels make
// those rows contribute nothing.  A wave issues NI/4 instructions; DmaPlan holds each
// one's byte offset within a full tile for this lane, and a raw buffer load takes it
// as the per-lane offset against the tile's origin, so a full tile costs no vector
// ALU work (the clamp of a partial last tile recomputes the offsets).
template <typename T, int D, int R>
struct DmaPlan {
  static constexpr int CH = D / 8, NI = R * CH / 64, NW = kThreads / 64, NPW = NI / NW;
  static_assert(NI % NW == 0, "tile must split evenly over the waves");
  uint32_t off[NPW];
  int rs;
  __device__ void init(int lane, int wave, int rs_) {
    rs = rs_;
#pragma unroll
    for (int k = 0; k < NPW; ++k) {
      const int u = (wave + k * NW) * 64 + lane;
      const int r = u / CH, c = (u % CH) ^ SwzTile<D>::key(r);
      off[k] = (uint32_t)((r * rs + c * 8) * (int)sizeof(T));
    }
  }
  __device__ __forceinline__ static void dma(const T* base, uint32_t o, char* l) {
    // the buffer-resource type is compiled in the device pass only (the host pass of
    // this compiler drops launch stubs of kernel instantiations whose bodies hold it)
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(base), (short)0, 0x7fffffff, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (TG_LDS void*)l, 16, o, 0, 0, 0);
#endif
  }
  // copy() issues this wave's instructions k0 <= k < k1 (all by default), so a caller
  // can spread a tile's copy over its compute.
  __device__ __forceinline__ void copy(const T* __restrict__ g, int64_t row0, int64_t nrows,
                                       char* lds, int k0 = 0, int k1 = NPW) const {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const T* base = g + row0 * rs;
    if (row0 + R <= nrows) {  // uniform
#pragma unroll
      for (int k = 0; k < NPW; ++k)
        if (k >= k0 && k < k1) dma(base, off[k], lds + (wave + k * NW) * 1024);
    } else {
#pragma unroll
      for (int k = 0; k < NPW; ++k) {
        if (k < k0 || k >= k1) continue;
        const int u = (wave + k * NW) * 64 + lane;
        const int r = u / CH, c = (u % CH) ^ SwzTile<D>::key(r);
        const int64_t rr = (row0 + r < nrows ? row0 + r : nrows - 1) - row0;
        dma(base, (uint32_t)((rr * rs + c * 8) * (int64_t)sizeof(T)),
            lds + (wave + k * NW) * 1024);
      }
    }
  }
};

// Wait for this wave's outstanding DMA and global loads; a barrier then makes every
// wave's part of the tile visible.
__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type lds_a(const char* p) {
  return *reinterpret_cast<const typename Vec8<T>::type*>(p);
}
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type lds_tr(const char* p0, const char* p1) {
  union {
    v4i16 h[2];
    typename Vec8<T>::type v;
  } u;
  u.h[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TG_LDS v4i16*)p0);
  u.h[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TG_LDS v4i16*)p1);
  return u.v;
}

// Per-lane byte offsets within a 32-row swizzled sub-tile.
//   a[ks]: 16-byte row read, row l32, chunk 2ks + h (A operand, k = d).
//   t[j][dt]: transposed read j (rows 4h + s/4 + 8j, s = lane % 16; the caller adds
//             16 rows per k-step) at column dt*32 + 16*((lane/16) % 2) + 4*(s % 4), so
//             the lane receives column dt*32 + lane%32 of rows 4h + 8j + 0..3.
template <int D>
struct LaneOffs {
  int a[D / 16];
  int t[2][D / 32];
  __device__ void init(int lane) {
    const int l32 = lane & 31, h = lane >> 5, s = lane & 15, nh = (lane >> 4) & 1;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) a[ks] = SwzTile<D>::off(l32, 2 * ks + h);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const int row = 4 * h + (s >> 2) + 8 * j;
        const int col = dt * 32 + 16 * nh + 4 * (s & 3);
        t[j][dt] = SwzTile<D>::off(row, col >> 3) + (col & 7) * 2;
      }
  }
};

// Hand-ordered variant of dkdv_sub for one key group.  The compiler, at one wave per
// SIMD and ~400 live registers, issues each LDS fragment read right before the MFMA
// that consumes it and waits for it there, so every MFMA pays a full LDS latency.
// Here sched_barrier fences fix the order: fragment reads run PF ahead of their
// MFMAs, the exp of S is spread over the dP MFMAs, dS over the dV MFMAs, and the
// transpose reads of each phase are issued during the previous one.
#define TG_SB() __builtin_amdgcn_sched_barrier(0)
template <typename T, int D, bool DIAG>
__device__ __forceinline__ void dkdv_sub_pipe(const char* qs, const char* dos,
                                              const float* lse, const float* dvs, int h,
                                              const LaneOffs<D>& o,
                                              const typename Vec8<T>::type (&kf)[D / 16],
                                              const typename Vec8<T>::type (&vf)[D / 16],
                                              f32x16 (&dk)[D / 32], f32x16 (&dv)[D / 32],
                                              float sl2, float scale, int mb) {
  using V8 = typename Vec8<T>::type;
  constexpr int DK = D / 16, DT = D / 32, RB = D * 2, PF = 4;
  constexpr int NB = 2 * DT;          // MFMAs of the dV (and of the dK) phase
  constexpr int EA = 16 / DK;         // exp elements per dP MFMA
  constexpr int EB = 16 / NB;         // dS elements per dV MFMA
  // transpose operand n of a phase: sg = n / DT, dt = n % DT
  auto tr = [&](const char* base, int n) {
    const char* b = base + (n / DT) * 16 * RB;
    return lds_tr<T>(b + o.t[0][n % DT], b + o.t[1][n % DT]);
  };
  V8 qa[DK], da[DK], bv[NB], bk[NB];
#pragma unroll
  for (int i = 0; i < PF; ++i) qa[i] = lds_a<T>(qs + o.a[i]);
  // lse and dvs hold log2e*lse and D of the query rows: P = exp2(S*scale*log2e - la)
  // and dS/scale = P * (dP - D) (dK takes the factor scale when it is stored).
  float la[16], db[16];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 a = *reinterpret_cast<const float4*>(lse + 8 * g + 4 * h);
    const float4 b = *reinterpret_cast<const float4*>(dvs + 8 * g + 4 * h);
    la[4 * g] = a.x; la[4 * g + 1] = a.y; la[4 * g + 2] = a.z; la[4 * g + 3] = a.w;
    db[4 * g] = b.x; db[4 * g + 1] = b.y; db[4 * g + 2] = b.z; db[4 * g + 3] = b.w;
  }
  f32x16 sa, dpa;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    sa[r] = 0.f;
    dpa[r] = 0.f;
  }
  TG_SB();
  // phase A: S = Q K^T while the Q then dO fragment reads run PF ahead
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    sa = mfma(qa[ks], kf[ks], sa);
    const int n = ks + PF;
    if (n < DK) qa[n] = lds_a<T>(qs + o.a[n]);
    else da[n - DK] = lds_a<T>(dos + o.a[n - DK]);
    TG_SB();
  }
  // phase A': dP = dO V^T; exp of S spread behind it; dO^T transpose reads start
  float p[16];
  auto expo = [&](int r) {
    float pv = fexp2(fmaf(sa[r], sl2, -la[r]));
    if (DIAG) pv = (mb > 8 * (r >> 2) + (r & 3)) ? 0.f : pv;
    p[r] = pv;
  };
  int nv = 0;
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    dpa = mfma(da[ks], vf[ks], dpa);
    const int n = ks + PF;
    if (n < DK) da[n] = lds_a<T>(dos + o.a[n]);
    else if (nv < NB) { bv[nv] = tr(dos, nv); ++nv; }
    if (ks > 0)
#pragma unroll
      for (int e = 0; e < EA; ++e) expo((ks - 1) * EA + e);
    TG_SB();
  }
#pragma unroll
  for (int e = 0; e < EA; ++e) expo((DK - 1) * EA + e);
  V8 pa[2] = {pack8<T>(&p[0]), pack8<T>(&p[8])};
  TG_SB();
  // phase B: dV += P^T dO; dS spread behind it; remaining dO^T then Q^T reads
  float ds[16];
  int nk = 0;
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    while (nv <= n) { bv[nv] = tr(dos, nv); ++nv; }
    dv[n % DT] = mfma(pa[n / DT], bv[n], dv[n % DT]);
    if (nv < NB) { bv[nv] = tr(dos, nv); ++nv; }
    else if (nk < NB) { bk[nk] = tr(qs, nk); ++nk; }
    if (n > 0)
#pragma unroll
      for (int e = 0; e < EB; ++e) {
        const int r = (n - 1) * EB + e;
        ds[r] = p[r] * (dpa[r] - db[r]);
      }
    TG_SB();
  }
#pragma unroll
  for (int e = 0; e < EB; ++e) {
    const int r = (NB - 1) * EB + e;
    ds[r] = p[r] * (dpa[r] - db[r]);
  }
  V8 dsa[2] = {pack8<T>(&ds[0]), pack8<T>(&ds[8])};
  TG_SB();
  // phase C: dK += dS^T Q
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    while (nk <= n) { bk[nk] = tr(qs, nk); ++nk; }
    dk[n % DT] = mfma(dsa[n / DT], bk[n], dk[n % DT]);
    if (nk < NB) { bk[nk] = tr(qs, nk); ++nk; }
    TG_SB();
  }
}

// The BM/32 sub-tiles of one staged query tile; kq = first key of this wave minus the
// tile's first query.  The wave's keys are kq .. kq + 31.
// issue(t) runs before sub-tile t whether or not the sub-tile is skipped (the caller
// spreads the next tile's DMA over the first sub-tiles with it).
template <typename T, int D, int BM, typename F>
__device__ __forceinline__ void dkdv_tile(const char* qs, const char* dos, const float* lse,
                                          const float* dvs, int kq, int causal, int h, int l32,
                                          const LaneOffs<D>& o,
                                          const typename Vec8<T>::type (&kf)[D / 16],
                                          const typename Vec8<T>::type (&vf)[D / 16],
                                          f32x16 (&dk)[D / 32], f32x16 (&dv)[D / 32],
                                          float sl2, float scale, F&& issue) {
  constexpr int RB = D * 2;
#pragma unroll
  for (int t = 0; t < BM / 32; ++t) {
    issue(t);
    // causal: a 32-query sub-tile wholly before this wave's keys contributes nothing
    if (causal && t * 32 + 31 < kq) continue;
    const char* q = qs + t * 32 * RB;
    const char* d = dos + t * 32 * RB;
    if (causal && kq + 31 > t * 32)
      dkdv_sub_pipe<T, D, true>(q, d, lse + t * 32, dvs + t * 32, h, o, kf, vf, dk, dv, sl2,
                                scale, kq + l32 - t * 32 - 4 * h);
    else
      dkdv_sub_pipe<T, D, false>(q, d, lse + t * 32, dvs + t * 32, h, o, kf, vf, dk, dv, sl2,
                                 scale, 0);
  }
}

// dK, dV.  grid = (ceil(Sk/128), B*H); one workgroup = 128 keys (4 waves x 32 keys,
// K/V fragments in registers), looping over query tiles of BM rows double-buffered
// in LDS (stage buffers are separate arrays so the compiler can tell the tile being
// read from the one being written by the DMA).
template <typename T, int D, int BM, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void k_fa_bwd_dkdv(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Dv,
    T* __restrict__ dK, T* __restrict__ dV, int64_t Sq, int64_t Sk, float scale, int causal,
    int accumulate, FaLay lay) {
  constexpr int DK = D / 16, DT = D / 32, TB = BM * D * 2;
  __shared__ __attribute__((aligned(1024))) char q0s[TB];
  __shared__ __attribute__((aligned(1024))) char do0s[TB];
  __shared__ __attribute__((aligned(1024))) char q1s[TB];
  __shared__ __attribute__((aligned(1024))) char do1s[TB];
  __shared__ __attribute__((aligned(16))) float lse0[BM], dvs0[BM], lse1[BM], dvs1[BM];
  int64_t tile, bh;
  fa_block(tile, bh, lay.G);
  Q += lay.ha(bh, Sq, D);
  dO += lay.ho(bh, Sq, D);
  K += lay.ha(bh, Sk, D);
  V += lay.ha(bh, Sk, D);
  dK += lay.ha(bh, Sk, D);
  dV += lay.ha(bh, Sk, D);
  LSE += bh * Sq;
  Dv += bh * Sq;
  const int rs = lay.rsa, ro = lay.rso;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t kblk = tile * 128;
  const int64_t kw = kblk + wave * 32;  // first key of this wave
  const float sl2 = scale * kLog2e;
  // Lane l32 holds key kw + l32 (C-tile column).  A key past Sk reads a clamped row:
  // it only feeds dK/dV rows of that key, which are never stored.
  typename Vec8<T>::type kf[DK], vf[DK];
  {
    const int64_t key = kw + l32;
    const int64_t kc = key < Sk ? key : Sk - 1;
#pragma unroll
    for (int ks = 0; ks < DK; ++ks) {
      kf[ks] = ld8(K + kc * rs + ks * 16 + h * 8);
      vf[ks] = ld8(V + kc * rs + ks * 16 + h * 8);
    }
    // At d = 128 the kernel holds more than the 256 vector registers: K and V, used only
    // as MFMA operands, are placed in accumulation registers (an empty asm whose "a"
    // constraint emits no instruction), leaving the vector registers to S, dP and the
    // values the VALU works on.
    if (D == 128) {
#pragma unroll
      for (int ks = 0; ks < DK; ++ks) asm volatile("" : "+a"(kf[ks]), "+a"(vf[ks]));
    }
  }
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dk[dt][r] = 0.f;
      dv[dt][r] = 0.f;
    }
  LaneOffs<D> o;
  o.init(lane);
  DmaPlan<T, D, BM> plan, plano;  // Q and dO tiles
  plan.init(lane, wave, rs);
  plano.init(lane, wave, ro);
  // causal: queries below the first key of this block contribute nothing
  const int64_t qstart = causal ? (kblk / BM) * BM : 0;
  // log2e*lse and D of one tile's rows (+inf / 0 past Sq, so P = 0 for padded rows).
  // The
  // two global loads are issued before the tile's DMA and converted only when stored
  // to LDS after the current tile's compute: vector-memory loads retire in issue order,
  // so a use right behind the DMA would wait for the whole DMA.
  float lv = 0.f, dd = 0.f;
  bool lok = false;
  auto lsed = [&](int64_t q0) {
    const int64_t qq = q0 + (threadIdx.x % BM);
    const int64_t qqc = qq < Sq ? qq : Sq - 1;  // load unconditionally, select after
    lv = LSE[qqc];
    dd = Dv[qqc];
    lok = qq < Sq;
  };
  auto put = [&](float* lse_s, float* dvs_s) {
    if (threadIdx.x < BM) {
      lse_s[threadIdx.x] = lok ? lv * kLog2e : INFINITY;
      dvs_s[threadIdx.x] = lok ? dd : 0.f;
    }
  };
  if (qstart < Sq) {
    lsed(qstart);
    plan.copy(Q, qstart, Sq, q0s);
    plano.copy(dO, qstart, Sq, do0s);
    put(lse0, dvs0);
  }
  // The next tile's copy is issued in two halves, before the first two sub-tiles of
  // the current one: issued all at once right after the barrier, the four waves'
  // copies queue up behind each other in the address unit while no MFMA runs.
  constexpr int NPW = DmaPlan<T, D, BM>::NPW;
  auto stage = [&](int64_t qn, char* qd, char* dd) {
    return [&plan, &plano, &Q, &dO, qn, qd, dd, Sq](int t) {
      if (t < 2 && qn < Sq) {
        plan.copy(Q, qn, Sq, qd, t * NPW / 2, (t + 1) * NPW / 2);
        plano.copy(dO, qn, Sq, dd, t * NPW / 2, (t + 1) * NPW / 2);
      }
    };
  };
  for (int64_t q0 = qstart; q0 < Sq; q0 += 2 * BM) {
    // stage 0 holds tile q0; stage 1 is free (its last readers passed the barrier)
    dma_wait();
    __syncthreads();
    const bool more1 = q0 + BM < Sq;
    if (more1) lsed(q0 + BM);
    dkdv_tile<T, D, BM>(q0s, do0s, lse0, dvs0, (int)(kw - q0), causal, h, l32, o, kf, vf, dk,
                        dv, sl2, scale, stage(q0 + BM, q1s, do1s));
    if (!more1) break;
    put(lse1, dvs1);
    // stage 1 holds tile q0 + BM
    dma_wait();
    __syncthreads();
    const bool more2 = q0 + 2 * BM < Sq;
    if (more2) lsed(q0 + 2 * BM);
    dkdv_tile<T, D, BM>(q1s, do1s, lse1, dvs1, (int)(kw - q0 - BM), causal, h, l32, o, kf, vf,
                        dk, dv, sl2, scale, stage(q0 + 2 * BM, q0s, do0s));
    if (!more2) break;
    put(lse0, dvs0);
  }
  // C tiles (rows = keys of this wave, cols = d) staged through the first stage's
  // buffers, 32 x D floats per wave, once every wave is done reading them
  static_assert(2 * 32 * D * 4 <= TB, "two waves' staging per stage buffer");
  __syncthreads();
  float* st = reinterpret_cast<float*>(wave < 2 ? q0s : do0s) + (wave & 1) * 32 * D;
  store_tiles_staged<T, D>(dK, rs, kw, Sk, dk, scale, accumulate, lane, st);  // dS's scale
  store_tiles_staged<T, D>(dV, rs, kw, Sk, dv, 1.f, accumulate, lane, st);
}

// One 32-key x 32-query sub-tile of the dQ kernel for one wave (lane = query):
//   ks/vs: the sub-tile's first row in the K / V tiles.
//   MASK: keys are masked when 8*(r/4) + r%4 > thr for accumulator register r, where
//   thr folds the causal limit (query of this lane - first key of the sub-tile - 4h)
//   and the end of the keys (keys - first key of the sub-tile - 4h - 1).
// Hand-ordered (same scheme as dkdv_sub_pipe): K then V fragment reads run PF
// ahead of their MFMAs, exp(S) is spread over the dP MFMAs, the dS of the second half
// is computed behind the first half's dQ MFMAs, and K^T transpose reads are issued
// during the dP phase.
template <typename T, int D, bool MASK>
__device__ __forceinline__ void dq_sub_pipe(const char* ks, const char* vs,
                                            const LaneOffs<D>& o,
                                            const typename Vec8<T>::type (&qf)[D / 16],
                                            const typename Vec8<T>::type (&of)[D / 16],
                                            f32x16 (&acc)[D / 32], float sl2, float scale,
                                            float lq, float dqs, int thr) {
  using V8 = typename Vec8<T>::type;
  constexpr int DK = D / 16, DT = D / 32, RB = D * 2, PF = 4;
  constexpr int NB = 2 * DT;
  constexpr int EA = 16 / DK;
  auto tr = [&](int n) {
    const char* b = ks + (n / DT) * 16 * RB;
    return lds_tr<T>(b + o.t[0][n % DT], b + o.t[1][n % DT]);
  };
  V8 ka[DK], va[DK], bk[NB];
#pragma unroll
  for (int i = 0; i < PF; ++i) ka[i] = lds_a<T>(ks + o.a[i]);
  f32x16 sa, dpa;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    sa[r] = 0.f;
    dpa[r] = 0.f;
  }
  TG_SB();
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    sa = mfma(ka[k], qf[k], sa);
    const int n = k + PF;
    if (n < DK) ka[n] = lds_a<T>(ks + o.a[n]);
    else va[n - DK] = lds_a<T>(vs + o.a[n - DK]);
    TG_SB();
  }
  float p[16];
  auto expo = [&](int r) {
    float pv = fexp2(fmaf(sa[r], sl2, -lq));
    if (MASK) pv = (8 * (r >> 2) + (r & 3) > thr) ? 0.f : pv;
    p[r] = pv;
  };
  int nk = 0;
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    dpa = mfma(va[k], of[k], dpa);
    const int n = k + PF;
    if (n < DK) va[n] = lds_a<T>(vs + o.a[n]);
    else if (nk < NB) { bk[nk] = tr(nk); ++nk; }
    if (k > 0)
#pragma unroll
      for (int e = 0; e < EA; ++e) expo((k - 1) * EA + e);
    TG_SB();
  }
#pragma unroll
  for (int e = 0; e < EA; ++e) expo((DK - 1) * EA + e);
  float ds[16];
#pragma unroll
  for (int r = 0; r < 8; ++r) ds[r] = p[r] * fmaf(dpa[r], scale, -dqs);
  const V8 d0 = pack8<T>(&ds[0]);
  TG_SB();
  constexpr int EB = 8 / DT;
  V8 d1;
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    while (nk <= n) { bk[nk] = tr(nk); ++nk; }
    acc[n % DT] = mfma(n < DT ? d0 : d1, bk[n], acc[n % DT]);
    if (nk < NB) { bk[nk] = tr(nk); ++nk; }
    if (n < DT) {
#pragma unroll
      for (int e = 0; e < EB; ++e) {
        const int r = 8 + n * EB + e;
        ds[r] = p[r] * fmaf(dpa[r], scale, -dqs);
      }
      if (n == DT - 1) d1 = pack8<T>(&ds[8]);
    }
    TG_SB();
  }
}

// The BN/32 sub-tiles of one staged key tile starting at key k0.
template <typename T, int D, int BN>
__device__ __forceinline__ void dq_tile(const char* ks, const char* vs, int64_t k0, int64_t Sk,
                                        int qk, int causal, int h, int l32, const LaneOffs<D>& o,
                                        const typename Vec8<T>::type (&qf)[D / 16],
                                        const typename Vec8<T>::type (&of)[D / 16],
                                        f32x16 (&acc)[D / 32], float sl2, float scale, float lq,
                                        float dqs) {
  constexpr int RB = D * 2;
#pragma unroll
  for (int kt = 0; kt < BN / 32; ++kt) {
    const int64_t kb0 = k0 + kt * 32;
    if (kb0 >= Sk) break;
    // causal: a 32-key sub-tile wholly after this wave's queries contributes nothing
    if (causal && kt * 32 > qk + 31) continue;
    const bool diag = causal && kt * 32 + 31 > qk;
    const bool edge = kb0 + 32 > Sk;
    const char* k = ks + kt * 32 * RB;
    const char* v = vs + kt * 32 * RB;
    if (diag || edge) {
      int thr = 1 << 30;
      if (diag) thr = qk + l32 - kt * 32 - 4 * h;
      if (edge) {
        const int kb = (int)(Sk - kb0) - 4 * h - 1;
        thr = kb < thr ? kb : thr;
      }
      dq_sub_pipe<T, D, true>(k, v, o, qf, of, acc, sl2, scale, lq, dqs, thr);
    } else {
      dq_sub_pipe<T, D, false>(k, v, o, qf, of, acc, sl2, scale, lq, dqs, 0);
    }
  }
}

// dQ.  grid = (ceil(Sq/128), B*H); one workgroup = 128 queries (4 waves x 32, Q/dO
// fragments in registers), looping over key tiles of BN rows double-buffered in LDS.
template <typename T, int D, int BN, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void k_fa_bwd_dq(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ O, const T* __restrict__ dO, const float* __restrict__ LSE,
    float* __restrict__ Dv, T* __restrict__ dQ, int64_t Sq, int64_t Sk, float scale,
    int causal, int accumulate, FaLay lay) {
  constexpr int DK = D / 16, DT = D / 32, TB = BN * D * 2;
  __shared__ __attribute__((aligned(1024))) char k0s[TB];
  __shared__ __attribute__((aligned(1024))) char v0s[TB];
  __shared__ __attribute__((aligned(1024))) char k1s[TB];
  __shared__ __attribute__((aligned(1024))) char v1s[TB];
  int64_t tile, bh;
  fa_block(tile, bh, lay.G);
  Q += lay.ha(bh, Sq, D);
  O += lay.ho(bh, Sq, D);
  dO += lay.ho(bh, Sq, D);
  dQ += lay.ha(bh, Sq, D);
  K += lay.ha(bh, Sk, D);
  V += lay.ha(bh, Sk, D);
  LSE += bh * Sq;
  Dv += bh * Sq;
  const int rs = lay.rsa, ro = lay.rso;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  // causal: the last query blocks carry the most keys, so they are dispatched first
  const int64_t qb = causal ? (int64_t)gridDim.x - 1 - tile : tile;
  const int64_t qblk = qb * 128;
  const int64_t q = qblk + wave * 32 + l32;
  const float sl2 = scale * kLog2e;
  // A query lane past Sq reads a clamped row; its dQ row is never stored.
  const int64_t qc = q < Sq ? q : Sq - 1;
  typename Vec8<T>::type qf[DK], of[DK];
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    qf[ks] = ld8(Q + qc * rs + ks * 16 + h * 8);
    of[ks] = ld8(dO + qc * ro + ks * 16 + h * 8);
  }
  const float lq = LSE[qc] * kLog2e;
  // D = rowsum(dO * O) of this lane's query: the two lane halves hold the two halves of
  // the head dimension.  Stored for the dK/dV kernel, which runs after this one.
  float dsum = 0.f;
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    const typename Vec8<T>::type ov = ld8(O + qc * ro + ks * 16 + h * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) dsum += (float)ov[e] * (float)of[ks][e];
  }
  dsum += __shfl_xor(dsum, 32, 64);
  if (h == 0 && q < Sq) Dv[q] = dsum;
  const float dqs = dsum * scale;
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
  LaneOffs<D> o;
  o.init(lane);
  DmaPlan<T, D, BN> plan;
  plan.init(lane, wave, rs);
  int64_t kend = Sk;
  if (causal) kend = (qblk + 128 < Sk) ? qblk + 128 : Sk;
  if (kend > 0) {
    plan.copy(K, 0, Sk, k0s);
    plan.copy(V, 0, Sk, v0s);
  }
  for (int64_t k0 = 0; k0 < kend; k0 += 2 * BN) {
    dma_wait();
    __syncthreads();
    const bool more1 = k0 + BN < kend;
    if (more1) {
      plan.copy(K, k0 + BN, Sk, k1s);
      plan.copy(V, k0 + BN, Sk, v1s);
    }
    dq_tile<T, D, BN>(k0s, v0s, k0, Sk, (int)(qblk - k0) + wave * 32, causal, h, l32, o, qf, of,
                      acc, sl2, scale, lq, dqs);
    if (!more1) break;
    dma_wait();
    __syncthreads();
    const bool more2 = k0 + 2 * BN < kend;
    if (more2) {
      plan.copy(K, k0 + 2 * BN, Sk, k0s);
      plan.copy(V, k0 + 2 * BN, Sk, v0s);
    }
    dq_tile<T, D, BN>(k1s, v1s, k0 + BN, Sk, (int)(qblk - k0 - BN) + wave * 32, causal, h, l32,
                      o, qf, of, acc, sl2, scale, lq, dqs);
    if (!more2) break;
  }
  // C tiles (rows = queries of this wave, cols = d) staged through the stage buffers,
  // one 32 x D float region per wave, once every wave is done reading them
  static_assert(32 * D * 4 <= TB, "one wave's staging per stage buffer");
  __syncthreads();
  char* const stb = wave == 0 ? k0s : wave == 1 ? v0s : wave == 2 ? k1s : v1s;
  store_tiles_staged<T, D>(dQ, rs, qblk + wave * 32, Sq, acc, 1.f, accumulate, lane,
                           reinterpret_cast<float*>(stb));
}

// ---------------------------------------------------------------- forward, DMA-staged
// One 32-key sub-tile of the forward for one wave (lane = query), in two halves:
// fwd_s forms S^T = K Q^T (keys on the accumulator rows); fwd_pv runs the online
// softmax per lane and O^T += V^T P^T with V^T read by transpose reads and P^T taken
// straight from the accumulator registers.  The caller issues fwd_s of sub-tile j + 1
// before fwd_pv of sub-tile j, so the softmax's vector ALU work overlaps those MFMAs.
// O^T is only rescaled when some lane's running maximum rose by more than kLazy (log2
// units): P is then at most 2^kLazy against the stale maximum, O and l use the same
// maximum, and the result is exact.
constexpr float kLazy = 8.f;
template <typename T, int D>
__device__ __forceinline__ f32x16 fwd_s(const char* ks, const LaneOffs<D>& o,
                                        const typename Vec8<T>::type (&qf)[D / 16]) {
  using V8 = typename Vec8<T>::type;
  constexpr int DK = D / 16, PF = 4;
  V8 ka[DK];
#pragma unroll
  for (int i = 0; i < PF; ++i) ka[i] = lds_a<T>(ks + o.a[i]);
  f32x16 sa;
#pragma unroll
  for (int r = 0; r < 16; ++r) sa[r] = 0.f;
  TG_SB();
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    sa = mfma(ka[k], qf[k], sa);
    if (k + PF < DK) ka[k + PF] = lds_a<T>(ks + o.a[k + PF]);
    TG_SB();
  }
  return sa;
}

// Running maximum m starts at kMInit, finite, so exp2(x - m) needs no guard: until a
// lane sees a finite score, m stays kMInit and every (masked, -inf) score gives 0; the
// first finite maximum is more than kLazy above kMInit and replaces it.
constexpr float kMInit = -1e30f;

// max / sum of x over lanes l and l ^ 32, in every lane, with one v_permlane32_swap
// (x swapped with itself: one result holds lane l's value, the other lane l ^ 32's)
// instead of an LDS permute.
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return a > b ? a : b;
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <typename T, int D, bool MASK>
__device__ __forceinline__ void fwd_pv(const f32x16& sa, const char* vs, const LaneOffs<D>& o,
                                       f32x16 (&acc)[D / 32], float sl2, float& m, float& l,
                                       int thr) {
  using V8 = typename Vec8<T>::type;
  constexpr int DT = D / 32, RB = D * 2, NB = 2 * DT;
  V8 bt[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    const char* b = vs + (n / DT) * 16 * RB;
    bt[n] = lds_tr<T>(b + o.t[0][n % DT], b + o.t[1][n % DT]);
  }
  // raw scores (masked keys at -inf); their maximum is scaled once (sl2 > 0, so the
  // maximum of the scaled scores is the scaled maximum), and each exponent argument is
  // one fused multiply-add
  float x[16];
  float mloc = -INFINITY;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float v = sa[r];
    if (MASK) v = (8 * (r >> 2) + (r & 3) > thr) ? -INFINITY : v;
    x[r] = v;
    mloc = fmaxf(mloc, v);
  }
  mloc = xhalf_max(mloc) * sl2;
  const bool grow = mloc > m + kLazy;
  if (__any(grow)) {
    const float mn = fmaxf(m, mloc);
    const float alpha = fexp2(m - mn);
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
    m = mn;
  }
  float p[16], ls = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float e = fexp2(fmaf(x[r], sl2, -m));
    p[r] = e;
    ls += e;
  }
  l += xhalf_sum(ls);
#pragma unroll
  for (int sg = 0; sg < 2; ++sg) {
    const V8 pb = pack8<T>(&p[8 * sg]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma(bt[sg * DT + dt], pb, acc[dt]);
  }
}

// Forward with DMA-staged K/V tiles.  grid = (ceil(Sq/128), B*H); one workgroup = 128
// queries (4 waves x 32, Q fragments in registers) looping over key tiles of BN rows
// double-buffered in swizzled LDS.  Writes O and the row log-sum-exp (natural log).
template <typename T, int D, int BN, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void k_fa_fwd2(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, T* __restrict__ O,
    float* __restrict__ LSE, int64_t Sq, int64_t Sk, float scale, int causal, FaLay lay) {
  constexpr int DK = D / 16, DT = D / 32, TB = BN * D * 2, RB = D * 2;
  __shared__ __attribute__((aligned(1024))) char k0s[TB];
  __shared__ __attribute__((aligned(1024))) char v0s[TB];
  __shared__ __attribute__((aligned(1024))) char k1s[TB];
  __shared__ __attribute__((aligned(1024))) char v1s[TB];
  int64_t tile, bh;
  fa_block(tile, bh, lay.G);
  Q += lay.ha(bh, Sq, D);
  O += lay.ho(bh, Sq, D);
  K += lay.ha(bh, Sk, D);
  V += lay.ha(bh, Sk, D);
  LSE += bh * Sq;
  const int rs = lay.rsa, ro = lay.rso;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  // causal: the last query blocks carry the most keys, so they are dispatched first
  const int64_t qb = causal ? (int64_t)gridDim.x - 1 - tile : tile;
  const int64_t qblk = qb * 128;
  const int64_t q = qblk + wave * 32 + l32;
  const float sl2 = scale * kLog2e;
  // A query lane past Sq reads a clamped row; its output row is never stored.
  const int64_t qc = q < Sq ? q : Sq - 1;
  typename Vec8<T>::type qf[DK];
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) qf[ks] = ld8(Q + qc * rs + ks * 16 + h * 8);
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
  float m = kMInit, l = 0.f;
  LaneOffs<D> o;
  o.init(lane);
  DmaPlan<T, D, BN> plan;
  plan.init(lane, wave, rs);
  int64_t kend = Sk;
  if (causal) kend = (qblk + 128 < Sk) ? qblk + 128 : Sk;
  // the sub-tiles of one staged key tile (first key k0); qk = first query of this wave
  // minus k0
  auto tile_fn = [&](const char* ks_, const char* vs_, int64_t k0) {
    const int qk = (int)(qblk - k0) + wave * 32;
    // active sub-tiles: a prefix [0, na) (keys past Sk, or wholly after this wave's
    // queries under causal masking, are skipped)
    int na = BN / 32;
    const int64_t nk = (Sk - k0 + 31) / 32;
    if (nk < na) na = (int)nk;
    if (causal) {
      const int nc = qk + 31 >= 0 ? (qk + 31) / 32 + 1 : 0;
      if (nc < na) na = nc;
    }
    if (na <= 0) return;
    f32x16 sa = fwd_s<T, D>(ks_, o, qf);
#pragma unroll
    for (int kt = 0; kt < BN / 32; ++kt) {
      if (kt >= na) break;
      f32x16 sn;
      if (kt + 1 < na) sn = fwd_s<T, D>(ks_ + (kt + 1) * 32 * RB, o, qf);
      const int64_t kb0 = k0 + kt * 32;
      const bool diag = causal && kt * 32 + 31 > qk;
      const bool edge = kb0 + 32 > Sk;
      const char* vv = vs_ + kt * 32 * RB;
      if (diag || edge) {
        int thr = 1 << 30;
        if (diag) thr = qk + l32 - kt * 32 - 4 * h;
        if (edge) {
          const int kb = (int)(Sk - kb0) - 4 * h - 1;
          thr = kb < thr ? kb : thr;
        }
        fwd_pv<T, D, true>(sa, vv, o, acc, sl2, m, l, thr);
      } else {
        fwd_pv<T, D, false>(sa, vv, o, acc, sl2, m, l, 0);
      }
      if (kt + 1 < na) sa = sn;
    }
  };
  if (kend > 0) {
    plan.copy(K, 0, Sk, k0s);
    plan.copy(V, 0, Sk, v0s);
  }
  for (int64_t k0 = 0; k0 < kend; k0 += 2 * BN) {
    dma_wait();
    __syncthreads();
    const bool more1 = k0 + BN < kend;
    if (more1) {
      plan.copy(K, k0 + BN, Sk, k1s);
      plan.copy(V, k0 + BN, Sk, v1s);
    }
    tile_fn(k0s, v0s, k0);
    if (!more1) break;
    dma_wait();
    __syncthreads();
    const bool more2 = k0 + 2 * BN < kend;
    if (more2) {
      plan.copy(K, k0 + 2 * BN, Sk, k0s);
      plan.copy(V, k0 + 2 * BN, Sk, v0s);
    }
    tile_fn(k1s, v1s, k0 + BN);
    if (!more2) break;
  }
  if (q < Sq) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        T w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (T)(acc[dt][g * 4 + i] * inv);
        *reinterpret_cast<uint2*>(O + q * ro + dt * 32 + g * 8 + h * 4) =
            *reinterpret_cast<const uint2*>(w);
      }
    if (h == 0) LSE[q] = l > 0.f ? (m + log2f(l)) / kLog2e : -INFINITY;
  }
}

template <int D> struct FwdCfg;
template <> struct FwdCfg<64> { static constexpr int BN = 64, OCC = 3; };
template <> struct FwdCfg<128> { static constexpr int BN = 64, OCC = 2; };

template <typename T, int D>
int fwd_t(const void* q, const void* k, const void* v, void* o, float* lse, int64_t BH,
          int64_t Sq, int64_t Sk, float scale, int causal, FaLay lay, hipStream_t s) {
  dim3 grid((unsigned)((Sq + 127) / 128), (unsigned)BH);
  k_fa_fwd2<T, D, FwdCfg<D>::BN, FwdCfg<D>::OCC><<<grid, kThreads, 0, s>>>(
      (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, Sq, Sk, scale, causal, lay);
  return tg_check_launch("tg_flash_attn_fwd");
}

// Backward tile shapes per head dim: staged query rows of the dK/dV kernel, staged
// key rows of the dQ kernel, and the workgroups per CU each is compiled for.
template <int D> struct BwdCfg;
template <> struct BwdCfg<64> {
  static constexpr int BM = 128, OCC_KV = 2, BN = 64, OCC_Q = 3;
};
template <> struct BwdCfg<128> {
  static constexpr int BM = 128, OCC_KV = 1, BN = 64, OCC_Q = 2;
};

template <typename T, int D>
int bwd_t(const void* q, const void* k, const void* v, const void* o, const void* dout,
          const float* lse, void* dq, void* dk, void* dv, int64_t BH, int64_t Sq, int64_t Sk,
          float scale, int causal, int acc, float* dvec, FaLay lay, hipStream_t s) {
  using C = BwdCfg<D>;
  // dQ first: it also forms D = rowsum(dO * O) per query, which the dK/dV kernel reads.
  dim3 gq((unsigned)((Sq + 127) / 128), (unsigned)BH);
  k_fa_bwd_dq<T, D, C::BN, C::OCC_Q><<<gq, kThreads, 0, s>>>((const T*)q, (const T*)k, (const T*)v,
                                            (const T*)o, (const T*)dout, lse, dvec, (T*)dq, Sq,
                                            Sk, scale, causal, acc, lay);
  dim3 gkv((unsigned)((Sk + 127) / 128), (unsigned)BH);
  k_fa_bwd_dkdv<T, D, C::BM, C::OCC_KV><<<gkv, kThreads, 0, s>>>((const T*)q, (const T*)k, (const T*)v,
                                               (const T*)dout, lse, dvec, (T*)dk, (T*)dv, Sq, Sk,
                                               scale, causal, acc, lay);
  return tg_check_launch("tg_flash_attn_bwd");
}

// ============================================================ generic head dims / fp32
// Any head dim D <= 256 and fp32 as well as fp16/bf16 inputs: the same algorithm as
// the kernels above on the fp32 matrix cores (v_mfma_f32_32x32x2_f32), so fp32
// attention keeps fp32 precision.  D is padded with zeros to DP, a multiple of 32,
// inside the kernels; loads and stores are element-wise (no alignment requirement).
//
// 32x32x2 MFMA: A lane (row i = lane%32, k = lane/32) supplies one element, B lane
// (col j = lane%32, k = lane/32) one element, C as above.  A contraction over the head
// dim takes DP/2 steps; in step s lane half h supplies head-dim index
// kap(s, h) = 8*(s/4) + 4h + s%4, so a lane's operand for four steps is one 16-byte
// read of 4 adjacent elements.  A contraction over 32 keys (or queries) held in a C
// tile takes 16 steps; in step s lane half h supplies row crow(s, h), i.e. its own
// accumulator register s, and the other operand is read at that row.
typedef float gf32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ float gld(const T* p, int64_t i) { return (float)p[i]; }

// Row `row` of a [*, D] operand, head-dim indices kap(s, h) for s < DP/2, into
// registers (zero past D or for an invalid row).
template <typename T, int DP>
__device__ __forceinline__ void load_kap(const T* __restrict__ g, int64_t row, int rs, int D,
                                         bool valid, int h, float (&r)[DP / 2]) {
#pragma unroll
  for (int t = 0; t < DP / 8; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 8 * t + 4 * h + e;
      r[4 * t + e] = (valid && d < D) ? gld(g, row * rs + d) : 0.f;
    }
}

// Stage rows [row0, row0+32) x DP of a [nrows, D] operand into LDS (row stride LD),
// zero past nrows or D.  All 256 threads of the workgroup take part.
template <typename T, int DP>
__device__ __forceinline__ void stage32(const T* __restrict__ g, int64_t row0, int64_t nrows,
                                        int rs, int D, float* s) {
  constexpr int LD = DP + 4;
  for (int e = threadIdx.x; e < 32 * DP; e += kThreads) {
    const int r = e / DP, d = e - r * DP;
    const int64_t row = row0 + r;
    s[r * LD + d] = (row < nrows && d < D) ? gld(g, row * rs + d) : 0.f;
  }
}

// S^T (or S) tile: sum over the head dim of A rows (LDS, row = lane%32) against the
// B operand registers b (kap order).
template <int DP>
__device__ __forceinline__ f32x16 gen_dot(const float* As, int l32, int h, const float (&b)[DP / 2]) {
  constexpr int LD = DP + 4;
  f32x16 c;
#pragma unroll
  for (int r = 0; r < 16; ++r) c[r] = 0.f;
#pragma unroll
  for (int t = 0; t < DP / 8; ++t) {
    const gf32x4 a = *reinterpret_cast<const gf32x4*>(As + l32 * LD + 8 * t + 4 * h);
#pragma unroll
    for (int e = 0; e < 4; ++e) c = mfma2(a[e], b[4 * t + e], c);
  }
  return c;
}

// acc[db] += X^T[d][row] * P[row][col] over the 32 rows of a C tile P (registers p):
// A operand X read from LDS at rows crow(s, h), head-dim columns d0 + 32*db + lane%32.
template <int DP, int NDB>
__device__ __forceinline__ void gen_acc(f32x16 (&acc)[NDB], const float* Xs, int d0, int l32,
                                        int h, const f32x16& p) {
  constexpr int LD = DP + 4;
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const float* row = Xs + crow(s, h) * LD + d0 + l32;
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] = mfma2(row[32 * db], p[s], acc[db]);
  }
}

// Forward.  grid = (ceil(Sq/128), B*H); one workgroup = 128 queries (4 waves x 32,
// lane = query, Q in registers), key tiles of 32 staged in LDS.
template <typename T, int DP>
__global__ __launch_bounds__(kThreads) void k_fa_fwd_gen(const T* __restrict__ Q,
                                                         const T* __restrict__ K,
                                                         const T* __restrict__ V,
                                                         T* __restrict__ O, float* __restrict__ LSE,
                                                         int64_t Sq, int64_t Sk, int D,
                                                         float scale, int causal, FaLay lay) {
  constexpr int NS = DP / 2, NDB = DP / 32, LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float Ks[32 * LD];
  __shared__ __attribute__((aligned(16))) float Vs[32 * LD];
  int64_t tile, bh;
  fa_block(tile, bh, lay.G);
  Q += lay.ha(bh, Sq, D);
  O += lay.ho(bh, Sq, D);
  K += lay.ha(bh, Sk, D);
  V += lay.ha(bh, Sk, D);
  LSE += bh * Sq;
  const int rs = lay.rsa, ro = lay.rso;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t qb = causal ? (int64_t)gridDim.x - 1 - tile : tile;
  const int64_t q = qb * 128 + wave * 32 + l32;
  float qr[NS];
  load_kap<T, DP>(Q, q, rs, D, q < Sq, h, qr);
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  const float sl2 = scale * kLog2e;
  float m = -INFINITY, l = 0.f;
  const int64_t kend = causal ? (qb * 128 + 128 < Sk ? qb * 128 + 128 : Sk) : Sk;
  for (int64_t k0 = 0; k0 < kend; k0 += 32) {
    __syncthreads();
    stage32<T, DP>(K, k0, Sk, rs, D, Ks);
    stage32<T, DP>(V, k0, Sk, rs, D, Vs);
    __syncthreads();
    f32x16 s = gen_dot<DP>(Ks, l32, h, qr);
    float smax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t key = k0 + crow(r, h);
      const bool ok = key < Sk && (!causal || key <= q);
      s[r] = ok ? s[r] * sl2 : -INFINITY;
      smax = fmaxf(smax, s[r]);
    }
    smax = fmaxf(smax, __shfl_xor(smax, 32, 64));
    const float mn = fmaxf(m, smax);
    // every key so far masked for this query: p = 0 and nothing is rescaled (no branch,
    // so the whole wavefront reaches the MFMAs)
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float alpha = fexp2(m - mref);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = fexp2(s[r] - mref);
      ps += s[r];
    }
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
    gen_acc<DP, NDB>(acc, Vs, 0, l32, h, s);
  }
  l += __shfl_xor(l, 32, 64);
  if (q < Sq) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = 32 * db + crow(r, h);
        if (d < D) O[q * ro + d] = (T)(acc[db][r] * inv);
      }
    if (h == 0) LSE[q] = l > 0.f ? (m + log2f(l)) / kLog2e : -INFINITY;
  }
}

// dQ (and D = rowsum(dO * O)).  grid = (ceil(Sq/128), B*H, DP/DO); lane = query, Q and
// dO in registers, key tiles of 32 in LDS; the workgroup writes head-dim columns
// [z*DO, z*DO + DO) of dQ (S and dP are recomputed per column range).
template <typename T, int DP, int DO>
__global__ __launch_bounds__(kThreads) void k_fa_bwd_dq_gen(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ O, const T* __restrict__ dO, const float* __restrict__ LSE,
    float* __restrict__ Dv, T* __restrict__ dQ, int64_t Sq, int64_t Sk, int D, float scale,
    int causal, int accumulate, FaLay lay) {
  constexpr int NS = DP / 2, NDB = DO / 32, LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float Ks[32 * LD];
  __shared__ __attribute__((aligned(16))) float Vs[32 * LD];
  int64_t tile, bh;
  fa_block(tile, bh, lay.G);
  Q += lay.ha(bh, Sq, D);
  O += lay.ho(bh, Sq, D);
  dO += lay.ho(bh, Sq, D);
  dQ += lay.ha(bh, Sq, D);
  K += lay.ha(bh, Sk, D);
  V += lay.ha(bh, Sk, D);
  LSE += bh * Sq;
  Dv += bh * Sq;
  const int rs = lay.rsa, ro = lay.rso;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int d0 = blockIdx.z * DO;
  const int64_t qb = causal ? (int64_t)gridDim.x - 1 - tile : tile;
  const int64_t q = qb * 128 + wave * 32 + l32;
  const bool qv = q < Sq;
  float qr[NS], dor[NS];
  load_kap<T, DP>(Q, q, rs, D, qv, h, qr);
  load_kap<T, DP>(dO, q, ro, D, qv, h, dor);
  float dsum = 0.f;
#pragma unroll
  for (int t = 0; t < DP / 8; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 8 * t + 4 * h + e;
      if (qv && d < D) dsum += gld(O, q * ro + d) * dor[4 * t + e];
    }
  dsum += __shfl_xor(dsum, 32, 64);
  if (qv && h == 0 && blockIdx.z == 0) Dv[q] = dsum;
  const float lq = qv ? LSE[q] * kLog2e : 0.f;
  const float sl2 = scale * kLog2e;
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  const int64_t kend = causal ? (qb * 128 + 128 < Sk ? qb * 128 + 128 : Sk) : Sk;
  for (int64_t k0 = 0; k0 < kend; k0 += 32) {
    __syncthreads();
    stage32<T, DP>(K, k0, Sk, rs, D, Ks);
    stage32<T, DP>(V, k0, Sk, rs, D, Vs);
    __syncthreads();
    f32x16 p = gen_dot<DP>(Ks, l32, h, qr);
    const f32x16 dp = gen_dot<DP>(Vs, l32, h, dor);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t key = k0 + crow(r, h);
      const bool ok = qv && key < Sk && (!causal || key <= q);
      const float pr = ok ? fexp2(p[r] * sl2 - lq) : 0.f;
      p[r] = pr * (dp[r] - dsum) * scale;  // dS^T
    }
    gen_acc<DP, NDB>(acc, Ks, d0, l32, h, p);
  }
  if (qv) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = d0 + 32 * db + crow(r, h);
        if (d < D) {
          const int64_t i = q * rs + d;
          dQ[i] = (T)(acc[db][r] + (accumulate ? (float)dQ[i] : 0.f));
        }
      }
  }
}

// dK, dV.  grid = (ceil(Sk/128), B*H, DP/DO); lane = key, K and V in registers, query
// tiles of 32 (Q, dO, their LSE and D) in LDS; the workgroup writes head-dim columns
// [z*DO, z*DO + DO) of dK and dV.
template <typename T, int DP, int DO>
__global__ __launch_bounds__(kThreads) void k_fa_bwd_dkdv_gen(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Dv,
    T* __restrict__ dK, T* __restrict__ dV, int64_t Sq, int64_t Sk, int D, float scale,
    int causal, int accumulate, FaLay lay) {
  constexpr int NS = DP / 2, NDB = DO / 32, LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float Qs[32 * LD];
  __shared__ __attribute__((aligned(16))) float dOs[32 * LD];
  __shared__ float ls[32], ds[32];
  int64_t tile, bh;
  fa_block(tile, bh, lay.G);
  Q += lay.ha(bh, Sq, D);
  dO += lay.ho(bh, Sq, D);
  K += lay.ha(bh, Sk, D);
  V += lay.ha(bh, Sk, D);
  dK += lay.ha(bh, Sk, D);
  dV += lay.ha(bh, Sk, D);
  LSE += bh * Sq;
  Dv += bh * Sq;
  const int rs = lay.rsa, ro = lay.rso;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int d0 = blockIdx.z * DO;
  // causal: the first key blocks see the most queries, so they are dispatched first
  const int64_t kb = tile;
  const int64_t key = kb * 128 + wave * 32 + l32;
  const bool kv = key < Sk;
  float kr[NS], vr[NS];
  load_kap<T, DP>(K, key, rs, D, kv, h, kr);
  load_kap<T, DP>(V, key, rs, D, kv, h, vr);
  const float sl2 = scale * kLog2e;
  f32x16 ak[NDB], av[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) ak[db][r] = av[db][r] = 0.f;
  const int64_t qstart = causal ? kb * 128 : 0;
  for (int64_t q0 = qstart; q0 < Sq; q0 += 32) {
    __syncthreads();
    stage32<T, DP>(Q, q0, Sq, rs, D, Qs);
    stage32<T, DP>(dO, q0, Sq, ro, D, dOs);
    if (threadIdx.x < 32) {
      const int64_t qq = q0 + threadIdx.x;
      ls[threadIdx.x] = qq < Sq ? LSE[qq] * kLog2e : 0.f;
      ds[threadIdx.x] = qq < Sq ? Dv[qq] : 0.f;
    }
    __syncthreads();
    f32x16 p = gen_dot<DP>(Qs, l32, h, kr);
    const f32x16 dp = gen_dot<DP>(dOs, l32, h, vr);
    f32x16 dsv;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = crow(r, h);
      const int64_t qq = q0 + qi;
      const bool ok = kv && qq < Sq && (!causal || key <= qq);
      p[r] = ok ? fexp2(p[r] * sl2 - ls[qi]) : 0.f;
      dsv[r] = p[r] * (dp[r] - ds[qi]) * scale;
    }
    gen_acc<DP, NDB>(av, dOs, d0, l32, h, p);
    gen_acc<DP, NDB>(ak, Qs, d0, l32, h, dsv);
  }
  if (kv) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = d0 + 32 * db + crow(r, h);
        if (d < D) {
          const int64_t i = key * rs + d;
          dK[i] = (T)(ak[db][r] + (accumulate ? (float)dK[i] : 0.f));
          dV[i] = (T)(av[db][r] + (accumulate ? (float)dV[i] : 0.f));
        }
      }
  }
}

// Output head-dim columns per workgroup of the generic backward: all of DP up to 128,
// else half of it (the registers of a wave then hold K, V (or Q, dO) for the whole
// head dim plus accumulators for half of it).
template <int DP> struct GenSplit {
  static constexpr int DO = DP <= 128 ? DP : DP / 2;
  static_assert(DP % DO == 0 && DO % 32 == 0, "head-dim split");
};

template <typename T, int DP>
int fwd_gen_t(const void* q, const void* k, const void* v, void* o, float* lse, int64_t BH,
              int64_t Sq, int64_t Sk, int D, float scale, int causal, FaLay lay, hipStream_t s) {
  dim3 grid((unsigned)((Sq + 127) / 128), (unsigned)BH);
  k_fa_fwd_gen<T, DP><<<grid, kThreads, 0, s>>>((const T*)q, (const T*)k, (const T*)v, (T*)o, lse,
                                                Sq, Sk, D, scale, causal, lay);
  return tg_check_launch("tg_flash_attn_fwd");
}

template <typename T, int DP>
int bwd_gen_t(const void* q, const void* k, const void* v, const void* o, const void* dout,
              const float* lse, void* dq, void* dk, void* dv, int64_t BH, int64_t Sq, int64_t Sk,
              int D, float scale, int causal, int acc, float* dvec, FaLay lay, hipStream_t s) {
  constexpr int DO = GenSplit<DP>::DO;
  dim3 gq((unsigned)((Sq + 127) / 128), (unsigned)BH, DP / DO);
  k_fa_bwd_dq_gen<T, DP, DO><<<gq, kThreads, 0, s>>>(
      (const T*)q, (const T*)k, (const T*)v, (const T*)o, (const T*)dout, lse, dvec, (T*)dq, Sq,
      Sk, D, scale, causal, acc, lay);
  dim3 gkv((unsigned)((Sk + 127) / 128), (unsigned)BH, DP / DO);
  k_fa_bwd_dkdv_gen<T, DP, DO><<<gkv, kThreads, 0, s>>>(
      (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, dvec, (T*)dk, (T*)dv, Sq, Sk, D,
      scale, causal, acc, lay);
  return tg_check_launch("tg_flash_attn_bwd");
}

// Padded head dims of the generic path.
#define TG_GEN_DP(X) X(32) X(64) X(96) X(128) X(192) X(256)

int gen_dp(int64_t D) {
  if (D <= 32) return 32;
  if (D <= 64) return 64;
  if (D <= 96) return 96;
  if (D <= 128) return 128;
  if (D <= 192) return 192;
  return 256;
}

template <typename T>
int fwd_gen(const void* q, const void* k, const void* v, void* o, float* lse, int64_t BH,
            int64_t Sq, int64_t Sk, int D, float scale, int causal, FaLay lay, hipStream_t s) {
  switch (gen_dp(D)) {
#define C(DP) \
  case DP: return fwd_gen_t<T, DP>(q, k, v, o, lse, BH, Sq, Sk, D, scale, causal, lay, s);
    TG_GEN_DP(C)
#undef C
  }
  return TG_ERR_UNSUPPORTED;
}

template <typename T>
int bwd_gen(const void* q, const void* k, const void* v, const void* o, const void* dout,
            const float* lse, void* dq, void* dk, void* dv, int64_t BH, int64_t Sq, int64_t Sk,
            int D, float scale, int causal, int acc, float* dvec, FaLay lay, hipStream_t s) {
  switch (gen_dp(D)) {
#define C(DP)                                                                                  \
  case DP: return bwd_gen_t<T, DP>(q, k, v, o, dout, lse, dq, dk, dv, BH, Sq, Sk, D, scale,   \
                                   causal, acc, dvec, lay, s);
    TG_GEN_DP(C)
#undef C
  }
  return TG_ERR_UNSUPPORTED;
}

int check_fa(int dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
             const char* who) {
  TG_REQUIRE(dtype == TG_F16 || dtype == TG_BF16 || dtype == TG_F32,
             "%s: dtype must be fp32, fp16 or bf16", who);
  TG_REQUIRE(D >= 1 && D <= 256, "%s: head dim %lld not supported (1..256)", who, (long long)D);
  TG_REQUIRE(B > 0 && H > 0 && Sq > 0 && Sk > 0, "%s: empty or negative shape", who);
  TG_REQUIRE(H <= 65535, "%s: H = %lld exceeds 65535", who, (long long)H);
  return TG_OK;
}

}  // namespace

namespace {
// Heads per dispatch group (fa_block): 1 without masking, up to 8 under causal masking;
// a divisor of the heads each XCD receives.
int fa_group(int64_t BH, int causal, int fwd) {
  const int64_t hx = BH % 8 == 0 ? BH / 8 : BH;
  // measured at B*H = 128: causal bwd d128 0.72 -> 0.64 ms with groups of 8 (16: no
  // better); the causal forward gains from 16 (all of an XCD's heads at B*H = 128:
  // S = 1024 d64 38.5 -> 36.3 us, S = 2048 124 -> 115 us)
  int g = causal ? (fwd ? 16 : 8) : 1;
  while (g > 1 && hx % g) g >>= 1;
  return g;
}

// Backward dispatch order.  Under causal masking the work of a tile falls with its
// position in the grid (the heaviest first), and the hardware fills each CU with
// workgroups k, k + 256, k + 512, ... of the launch (round-robin over the XCDs first).
// With all heads tile-major (G = 0: no head groups, no XCD bands) those co-resident
// workgroups are a heavy, a medium and a light one; the XCDs still own fixed heads
// (head = index mod B*H, every 8th to one XCD).  Used where an XCD's share of the
// streamed operands fits its 4 MiB L2: measured at B*H = 128, d 64, causal: S = 1024
// 103 -> 96 us (dK/dV + dQ), S = 2048 even, S = 4096 1 % slower.
int fa_group_bwd(int64_t BH, int causal, int64_t S, int64_t D) {
  if (causal && BH % 8 == 0 && (BH / 8) * S * D * 4 <= (int64_t{4} << 20)) return 0;
  return fa_group(BH, causal, 0);
}

// The tuned fp16/bf16 kernels serve head dims 64 and 128 with 16-byte aligned operands;
// everything else runs on the generic fp32-MFMA kernels.
bool fa_fast(int dtype, int64_t D, std::initializer_list<const void*> ptrs) {
  if (dtype == TG_F32 || (D != 64 && D != 128)) return false;
  for (const void* p : ptrs)
    if (!tg_aligned16(p)) return false;
  return true;
}

// Batches per launch: the grid's y dimension (B*H heads) is limited to 65535.
int64_t fa_batch_chunk(int64_t B, int64_t H) {
  const int64_t nb = 65535 / H;
  return nb < B ? nb : B;
}

const char* off(const void* p, int64_t elems, int esz) {
  return (const char*)p + elems * esz;
}

// Layouts: 0 = [B, H, S, D], 1 = [B, S, H, D] (separate tensors), 2 = Q, K and V (and
// dQ, dK, dV) interleaved in one [B, S, 3, H, D] buffer, O and dO [B, S, H, D].
int check_layout(int layout, int64_t Sq, int64_t Sk, const char* who) {
  TG_REQUIRE(layout == 0 || layout == 1 || layout == 2,
             "%s: layout must be 0 (BHSD), 1 (BSHD) or 2 (packed QKV)", who);
  TG_REQUIRE(layout != 2 || Sq == Sk, "%s: packed QKV needs Sq == Sk", who);
  return TG_OK;
}

FaLay fa_lay(int layout, int64_t H, int64_t D, int G) {
  const int hd = (int)(H * D);
  return FaLay{H, layout != 0, G, layout == 0 ? (int)D : layout == 1 ? hd : 3 * hd,
               layout == 0 ? (int)D : hd};
}

// Element offset of batch b0 in a Q/K/V-family tensor of S rows.
int64_t fa_in_off(int layout, int64_t b0, int64_t H, int64_t S, int64_t D) {
  return (layout == 2 ? 3 : 1) * b0 * H * S * D;
}

int fa_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
           int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D, float scale, int causal,
           int layout, void* stream, const char* who) {
  int st = check_fa(dtype, B, H, Sq, Sk, D, who);
  if (st) return st;
  st = check_layout(layout, Sq, Sk, who);
  if (st) return st;
  TG_REQUIRE(q && k && v && o && lse, "%s: null pointer", who);
  hipStream_t s = tg_stream(stream);
  const bool fast = fa_fast(dtype, D, {q, k, v, o});
  const int es = tg_dtype_size(dtype);
  const int64_t nb = fa_batch_chunk(B, H);
  for (int64_t b0 = 0; b0 < B; b0 += nb) {
    const int64_t bn = B - b0 < nb ? B - b0 : nb, BH = bn * H;
    const int64_t qo = fa_in_off(layout, b0, H, Sq, D), ko = fa_in_off(layout, b0, H, Sk, D);
    const void *qc = off(q, qo, es), *kc = off(k, ko, es), *vc = off(v, ko, es);
    void* oc = (void*)off(o, b0 * H * Sq * D, es);
    float* lc = lse + b0 * H * Sq;
    const FaLay lay = fa_lay(layout, H, D, fa_group(BH, causal, 1));
    const int Di = (int)D;
    if (fast) {
      if (dtype == TG_F16)
        st = D == 64 ? fwd_t<tg_half, 64>(qc, kc, vc, oc, lc, BH, Sq, Sk, scale, causal, lay, s)
                     : fwd_t<tg_half, 128>(qc, kc, vc, oc, lc, BH, Sq, Sk, scale, causal, lay, s);
      else
        st = D == 64 ? fwd_t<tg_bf16, 64>(qc, kc, vc, oc, lc, BH, Sq, Sk, scale, causal, lay, s)
                     : fwd_t<tg_bf16, 128>(qc, kc, vc, oc, lc, BH, Sq, Sk, scale, causal, lay, s);
    } else if (dtype == TG_F32) {
      st = fwd_gen<float>(qc, kc, vc, oc, lc, BH, Sq, Sk, Di, scale, causal, lay, s);
    } else if (dtype == TG_F16) {
      st = fwd_gen<tg_half>(qc, kc, vc, oc, lc, BH, Sq, Sk, Di, scale, causal, lay, s);
    } else {
      st = fwd_gen<tg_bf16>(qc, kc, vc, oc, lc, BH, Sq, Sk, Di, scale, causal, lay, s);
    }
    if (st) return st;
  }
  return TG_OK;
}

int fa_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
           const void* dout, const float* lse, void* dq, void* dk, void* dv, int64_t B,
           int64_t H, int64_t Sq, int64_t Sk, int64_t D, float scale, int causal, int accumulate,
           int layout, void* workspace, size_t workspace_bytes, void* stream, const char* who) {
  int st = check_fa(dtype, B, H, Sq, Sk, D, who);
  if (st) return st;
  st = check_layout(layout, Sq, Sk, who);
  if (st) return st;
  TG_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv, "%s: null pointer", who);
  const size_t need = (size_t)(B * H * Sq) * sizeof(float);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("%s: workspace of %zu bytes needed", who, need);
    return TG_ERR_WORKSPACE;
  }
  hipStream_t s = tg_stream(stream);
  const bool fast = fa_fast(dtype, D, {q, k, v, o, dout, dq, dk, dv});
  const int es = tg_dtype_size(dtype);
  const int64_t nb = fa_batch_chunk(B, H);
  for (int64_t b0 = 0; b0 < B; b0 += nb) {
    const int64_t bn = B - b0 < nb ? B - b0 : nb, BH = bn * H;
    const int64_t qo = fa_in_off(layout, b0, H, Sq, D), ko = fa_in_off(layout, b0, H, Sk, D);
    const int64_t oo = b0 * H * Sq * D;
    const void *qc = off(q, qo, es), *kc = off(k, ko, es), *vc = off(v, ko, es);
    const void *oc = off(o, oo, es), *gc = off(dout, oo, es);
    void* dqc = (void*)off(dq, qo, es);
    void* dkc = (void*)off(dk, ko, es);
    void* dvc = (void*)off(dv, ko, es);
    const float* lc = lse + b0 * H * Sq;
    float* dvec = (float*)workspace + b0 * H * Sq;
    const FaLay lay = fa_lay(layout, H, D, fa_group_bwd(BH, causal, Sq > Sk ? Sq : Sk, D));
    const int Di = (int)D;
    if (fast) {
      if (dtype == TG_F16)
        st = D == 64 ? bwd_t<tg_half, 64>(qc, kc, vc, oc, gc, lc, dqc, dkc, dvc, BH, Sq, Sk,
                                          scale, causal, accumulate, dvec, lay, s)
                     : bwd_t<tg_half, 128>(qc, kc, vc, oc, gc, lc, dqc, dkc, dvc, BH, Sq, Sk,
                                           scale, causal, accumulate, dvec, lay, s);
      else
        st = D == 64 ? bwd_t<tg_bf16, 64>(qc, kc, vc, oc, gc, lc, dqc, dkc, dvc, BH, Sq, Sk,
                                          scale, causal, accumulate, dvec, lay, s)
                     : bwd_t<tg_bf16, 128>(qc, kc, vc, oc, gc, lc, dqc, dkc, dvc, BH, Sq, Sk,
                                           scale, causal, accumulate, dvec, lay, s);
    } else if (dtype == TG_F32) {
      st = bwd_gen<float>(qc, kc, vc, oc, gc, lc, dqc, dkc, dvc, BH, Sq, Sk, Di, scale, causal,
                          accumulate, dvec, lay, s);
    } else if (dtype == TG_F16) {
      st = bwd_gen<tg_half>(qc, kc, vc, oc, gc, lc, dqc, dkc, dvc, BH, Sq, Sk, Di, scale, causal,
                            accumulate, dvec, lay, s);
    } else {
      st = bwd_gen<tg_bf16>(qc, kc, vc, oc, gc, lc, dqc, dkc, dvc, BH, Sq, Sk, Di, scale, causal,
                            accumulate, dvec, lay, s);
    }
    if (st) return st;
  }
  return TG_OK;
}
}  // namespace

TG_EXPORT int tg_flash_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o,
                                float* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                                int64_t D, float scale, int causal, void* stream) {
  return fa_fwd(dtype, q, k, v, o, lse, B, H, Sq, Sk, D, scale, causal, 0, stream,
                "tg_flash_attn_fwd");
}

TG_EXPORT int tg_flash_attn_fwd_layout(int dtype, const void* q, const void* k, const void* v,
                                       void* o, float* lse, int64_t B, int64_t H, int64_t Sq,
                                       int64_t Sk, int64_t D, float scale, int causal, int layout,
                                       void* stream) {
  TG_REQUIRE(layout == 0 || layout == 1,
             "tg_flash_attn_fwd_layout: layout must be 0 (BHSD) or 1 (BSHD)");
  return fa_fwd(dtype, q, k, v, o, lse, B, H, Sq, Sk, D, scale, causal, layout, stream,
                "tg_flash_attn_fwd_layout");
}

TG_EXPORT size_t tg_flash_attn_bwd_workspace(int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                                             int64_t D) {
  (void)Sk;
  (void)D;
  if (B <= 0 || H <= 0 || Sq <= 0) return 0;
  return (size_t)(B * H * Sq) * sizeof(float);
}

TG_EXPORT int tg_flash_attn_bwd(int dtype, const void* q, const void* k, const void* v,
                                const void* o, const void* dout, const float* lse, void* dq,
                                void* dk, void* dv, int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                                int64_t D, float scale, int causal, int accumulate,
                                void* workspace, size_t workspace_bytes, void* stream) {
  return fa_bwd(dtype, q, k, v, o, dout, lse, dq, dk, dv, B, H, Sq, Sk, D, scale, causal,
                accumulate, 0, workspace, workspace_bytes, stream, "tg_flash_attn_bwd");
}

TG_EXPORT int tg_flash_attn_bwd_layout(int dtype, const void* q, const void* k, const void* v,
                                       const void* o, const void* dout, const float* lse,
                                       void* dq, void* dk, void* dv, int64_t B, int64_t H,
                                       int64_t Sq, int64_t Sk, int64_t D, float scale, int causal,
                                       int accumulate, int layout, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  TG_REQUIRE(layout == 0 || layout == 1,
             "tg_flash_attn_bwd_layout: layout must be 0 (BHSD) or 1 (BSHD)");
  return fa_bwd(dtype, q, k, v, o, dout, lse, dq, dk, dv, B, H, Sq, Sk, D, scale, causal,
                accumulate, layout, workspace, workspace_bytes, stream,
                "tg_flash_attn_bwd_layout");
}

TG_EXPORT int tg_flash_attn_fwd_qkv(int dtype, const void* qkv, void* o, float* lse, int64_t B,
                                    int64_t H, int64_t S, int64_t D, float scale, int causal,
                                    void* stream) {
  TG_REQUIRE(qkv, "tg_flash_attn_fwd_qkv: null pointer");
  const int es = tg_dtype_size(dtype);
  return fa_fwd(dtype, qkv, off(qkv, H * D, es), off(qkv, 2 * H * D, es), o, lse, B, H, S, S,
                D, scale, causal, 2, stream, "tg_flash_attn_fwd_qkv");
}

TG_EXPORT int tg_flash_attn_bwd_qkv(int dtype, const void* qkv, const void* o, const void* dout,
                                    const float* lse, void* dqkv, int64_t B, int64_t H, int64_t S,
                                    int64_t D, float scale, int causal, int accumulate,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  TG_REQUIRE(qkv && dqkv, "tg_flash_attn_bwd_qkv: null pointer");
  const int es = tg_dtype_size(dtype);
  return fa_bwd(dtype, qkv, off(qkv, H * D, es), off(qkv, 2 * H * D, es), o, dout, lse, dqkv,
                (void*)off(dqkv, H * D, es), (void*)off(dqkv, 2 * H * D, es), B, H, S, S, D,
                scale, causal, accumulate, 2, workspace, workspace_bytes, stream,
                "tg_flash_attn_bwd_qkv");
}
