// FlashAttention forward and backward for gfx950 (fp16 / bf16, head dim 64 or 128),
// reference: flash_attention (_core.py:1686-1870).
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
// That other operand is staged in LDS "4-row interleaved" ([row/4][d][row%4]) so
// each lane fetches its two 4-row groups with two 8-byte reads.
//
// Forward: one workgroup = 128 queries (4 waves x 32), K/V tiles of 64 keys.
//   S^T = K Q^T (lane = query), online softmax per lane, O^T += V^T P^T.
// Backward (no atomics, two kernels):
//   k_fa_bwd_dkdv: one workgroup = 128 keys (4 waves x 32 keys), loop over query
//     tiles of 64: S = Q K^T (lane = key), P = exp(S*scale - lse), dP = dO V^T,
//     dS = P*(dP - D)*scale, dV += P^T dO, dK += dS^T Q.
//   k_fa_bwd_dq: one workgroup = 128 queries, loop over key tiles of 64:
//     S^T = K Q^T (lane = query), dP^T = V dO^T, dQ += dS K.
//   D = rowsum(dO * O) comes from k_fa_bwd_prep.
#include "tg_common.h"

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

// Two 4-element groups from an interleaved tile il[rows/4][D][4]: groups g1, g2 at column d.
template <typename T, int D>
__device__ __forceinline__ typename Vec8<T>::type ld_il(const T* il, int g1, int g2, int d) {
  union {
    uint4 u;
    typename Vec8<T>::type v;
  } r;
  const uint2 a = *reinterpret_cast<const uint2*>(il + ((g1 * D) + d) * 4);
  const uint2 b = *reinterpret_cast<const uint2*>(il + ((g2 * D) + d) * 4);
  r.u = make_uint4(a.x, a.y, b.x, b.y);
  return r.v;
}

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type pack8(const float* v) {
  typename Vec8<T>::type r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (T)v[e];
  return r;
}

// Stage ROWS x D rows [row0, row0+ROWS) of a [nrows, D] matrix into LDS, row-major
// (rm, row stride D+8) and/or 4-row interleaved (il).  Rows past nrows are zero.
template <typename T, int ROWS, int D, bool RM, bool IL>
__device__ __forceinline__ void stage(const T* __restrict__ g, int64_t row0, int64_t nrows,
                                      T* rm, T* il) {
  constexpr int DG = D / 8;
  constexpr int UNITS = (ROWS / 4) * DG;
  for (int u = threadIdx.x; u < UNITS; u += kThreads) {
    const int rg = u / DG, dg = u % DG;
    uint4 v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = row0 + rg * 4 + r;
      v[r] = row < nrows ? *reinterpret_cast<const uint4*>(g + row * D + dg * 8)
                         : make_uint4(0, 0, 0, 0);
    }
    if (RM) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<uint4*>(rm + (rg * 4 + r) * (D + 8) + dg * 8) = v[r];
    }
    if (IL) {
      const T* e0 = reinterpret_cast<const T*>(&v[0]);
      const T* e1 = reinterpret_cast<const T*>(&v[1]);
      const T* e2 = reinterpret_cast<const T*>(&v[2]);
      const T* e3 = reinterpret_cast<const T*>(&v[3]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        T q4[4] = {e0[j], e1[j], e2[j], e3[j]};
        *reinterpret_cast<uint2*>(il + ((rg * D) + dg * 8 + j) * 4) =
            *reinterpret_cast<const uint2*>(q4);
      }
    }
  }
}

// Workgroup -> (tile, head) mapping.  Dispatch i lands on XCD i % 8; remap the
// launch index so XCD x gets the contiguous range [x*T/8, (x+1)*T/8) of the
// head-major tile order, i.e. whole heads, so causal work (which varies along the
// tile axis) is spread evenly over the XCDs.  Returns (tile, head).
__device__ __forceinline__ void fa_block(int64_t& tile, int64_t& head) {
  const int64_t gx = gridDim.x, T = gx * gridDim.y;
  int64_t lin = (int64_t)blockIdx.y * gx + blockIdx.x;
  if (T % 8 == 0) lin = (lin % 8) * (T / 8) + lin / 8;
  head = lin / gx;
  tile = lin % gx;
}

// Row index (within a 32-row C tile) of accumulator register r for lane half h.
__device__ __forceinline__ int crow(int r, int h) { return ((r >> 2) << 3) + (h << 2) + (r & 3); }

// ============================================================================ forward
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_fa_fwd(const T* __restrict__ Q,
                                                     const T* __restrict__ K,
                                                     const T* __restrict__ V, T* __restrict__ O,
                                                     float* __restrict__ LSE, int64_t Sq,
                                                     int64_t Sk, float scale, int causal) {
  constexpr int BN = 128, DK = D / 16, DT = D / 32;
  __shared__ __attribute__((aligned(16))) T Ks[BN * (D + 8)];
  __shared__ __attribute__((aligned(16))) T Vi[BN * D];
  int64_t tile, bh;
  fa_block(tile, bh);
  Q += bh * Sq * D;
  K += bh * Sk * D;
  V += bh * Sk * D;
  O += bh * Sq * D;
  LSE += bh * Sq;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  // causal: the last query blocks carry the most keys, so they are dispatched first
  const int64_t qb = causal ? (int64_t)gridDim.x - 1 - tile : tile;
  const int64_t qblk = qb * 128;
  const int64_t q = qblk + wave * 32 + l32;
  const float sl2 = scale * kLog2e;

  typename Vec8<T>::type qf[DK];
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    if (q < Sq) {
      qf[ks] = ld8(Q + q * D + ks * 16 + h * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = (T)0.f;
    }
  }
  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m = -INFINITY, l = 0.f;

  int64_t kend = Sk;
  if (causal) kend = (qblk + 128 < Sk) ? qblk + 128 : Sk;
  for (int64_t k0 = 0; k0 < kend; k0 += BN) {
    __syncthreads();
    stage<T, BN, D, true, false>(K, k0, Sk, Ks, nullptr);
    stage<T, BN, D, false, true>(V, k0, Sk, nullptr, Vi);
    __syncthreads();
#pragma unroll 1
    for (int kt = 0; kt < BN / 32; ++kt) {
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < DK; ++ks)
        s = mfma(ld8(Ks + (kt * 32 + l32) * (D + 8) + ks * 16 + h * 8), qf[ks], s);
      // masks are only needed where the sub-tile crosses Sk or the causal diagonal
      const bool edge = (k0 + kt * 32 + 32 > Sk) ||
                        (causal && k0 + kt * 32 + 31 > qblk + wave * 32);
      float mloc = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[r] * sl2;
        if (edge) {
          const int64_t key = k0 + kt * 32 + crow(r, h);
          if (key >= Sk || (causal && key > q)) x = -INFINITY;
        }
        s[r] = x;
        mloc = fmaxf(mloc, x);
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
      const float mnew = fmaxf(m, mloc);
      const float alpha = (mnew == -INFINITY) ? 1.f : fexp2(m - mnew);
      float lsum = 0.f;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = (mnew == -INFINITY) ? 0.f : fexp2(s[r] - mnew);
        p[r] = e;
        lsum += e;
      }
      lsum += __shfl_xor(lsum, 32, 64);
      l = l * alpha + lsum;
      m = mnew;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
#pragma unroll
      for (int sg = 0; sg < 2; ++sg) {
        const typename Vec8<T>::type pb = pack8<T>(&p[8 * sg]);
        const int g1 = (kt * 32 + 16 * sg + 4 * h) >> 2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          o[dt] = mfma(ld_il<T, D>(Vi, g1, g1 + 2, dt * 32 + l32), pb, o[dt]);
      }
    }
  }
  if (q < Sq) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        T w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (T)(o[dt][g * 4 + i] * inv);
        *reinterpret_cast<uint2*>(O + q * D + dt * 32 + g * 8 + h * 4) =
            *reinterpret_cast<const uint2*>(w);
      }
    if (h == 0) LSE[q] = (m + log2f(l)) / kLog2e;
  }
}

// ============================================================================ backward
// D[q] = sum_d dO[q][d] * O[q][d] (fp32); 16 lanes per row.
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_fa_bwd_prep(const T* __restrict__ O,
                                                          const T* __restrict__ dO,
                                                          float* __restrict__ Dv, int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 16) + threadIdx.x / 16;
  const int sub = threadIdx.x & 15;
  float acc = 0.f;
  if (row < rows) {
    for (int d = sub * 8; d < D; d += 128) {
      const typename Vec8<T>::type a = ld8(O + row * D + d);
      const typename Vec8<T>::type b = ld8(dO + row * D + d);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)a[e] * (float)b[e];
    }
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (row < rows && sub == 0) Dv[row] = acc;
}

template <typename T>
__device__ __forceinline__ void store_c_tile(T* __restrict__ out, int64_t ld, int64_t row0,
                                             int64_t nrows, int col, const f32x16& acc, float mul,
                                             bool accumulate, int h) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = row0 + crow(r, h);
    if (row < nrows) {
      T* p = out + row * ld + col;
      float v = acc[r] * mul;
      if (accumulate) v += (float)*p;
      *p = (T)v;
    }
  }
}

// dK, dV.  grid = (ceil(Sk/128), B*H).  Query tiles of 128 staged per step; the four
// 32-query sub-tiles are processed one after another to keep P/dS in 32 registers.
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_fa_bwd_dkdv(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Dv,
    T* __restrict__ dK, T* __restrict__ dV, int64_t Sq, int64_t Sk, float scale, int causal,
    int accumulate) {
  constexpr int BM = 128, DK = D / 16, DT = D / 32;
  __shared__ __attribute__((aligned(16))) T Qs[BM * (D + 8)];
  __shared__ __attribute__((aligned(16))) T Qi[BM * D];
  __shared__ __attribute__((aligned(16))) T dOs[BM * (D + 8)];
  __shared__ __attribute__((aligned(16))) T dOi[BM * D];
  __shared__ __attribute__((aligned(16))) float lse2[BM];
  __shared__ __attribute__((aligned(16))) float dvec[BM];
  int64_t tile, bh;
  fa_block(tile, bh);
  Q += bh * Sq * D;
  dO += bh * Sq * D;
  K += bh * Sk * D;
  V += bh * Sk * D;
  dK += bh * Sk * D;
  dV += bh * Sk * D;
  LSE += bh * Sq;
  Dv += bh * Sq;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t kblk = tile * 128;
  const int64_t key = kblk + wave * 32 + l32;  // this lane's key (C-tile column)
  const float sl2 = scale * kLog2e;

  typename Vec8<T>::type kf[DK], vf[DK];
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    if (key < Sk) {
      kf[ks] = ld8(K + key * D + ks * 16 + h * 8);
      vf[ks] = ld8(V + key * D + ks * 16 + h * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kf[ks][e] = (T)0.f;
        vf[ks][e] = (T)0.f;
      }
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
  // causal: queries below the first key of this block contribute nothing
  int64_t qstart = 0;
  if (causal) qstart = (kblk / BM) * BM;
  for (int64_t q0 = qstart; q0 < Sq; q0 += BM) {
    __syncthreads();
    stage<T, BM, D, true, true>(Q, q0, Sq, Qs, Qi);
    stage<T, BM, D, true, true>(dO, q0, Sq, dOs, dOi);
    if (threadIdx.x < BM) {
      const int64_t qq = q0 + threadIdx.x;
      lse2[threadIdx.x] = qq < Sq ? LSE[qq] * kLog2e : 0.f;
      dvec[threadIdx.x] = qq < Sq ? Dv[qq] : 0.f;
    }
    __syncthreads();
#pragma unroll 1
    for (int t = 0; t < BM / 32; ++t) {
      // causal: a 32-query sub-tile wholly before this wave's keys contributes nothing
      if (causal && q0 + t * 32 + 31 < kblk + wave * 32) continue;
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = 0.f;
        dp[r] = 0.f;
      }
#pragma unroll
      for (int ks = 0; ks < DK; ++ks) {
        s = mfma(ld8(Qs + (t * 32 + l32) * (D + 8) + ks * 16 + h * 8), kf[ks], s);
        dp = mfma(ld8(dOs + (t * 32 + l32) * (D + 8) + ks * 16 + h * 8), vf[ks], dp);
      }
      // Padded query rows are zero in Qs/dOs with lse = D = 0, so they add nothing to
      // dV (dO row 0) or dK (dS = P*(0-0) = 0); padded keys only feed dK/dV rows that
      // are never stored.  Only the causal diagonal needs a mask.
      const bool diag = causal && (kblk + wave * 32 + 31 > q0 + t * 32);
      float lv[16], dvv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 a = *reinterpret_cast<const float4*>(lse2 + t * 32 + 8 * g + 4 * h);
        const float4 b = *reinterpret_cast<const float4*>(dvec + t * 32 + 8 * g + 4 * h);
        lv[4 * g] = a.x; lv[4 * g + 1] = a.y; lv[4 * g + 2] = a.z; lv[4 * g + 3] = a.w;
        dvv[4 * g] = b.x; dvv[4 * g + 1] = b.y; dvv[4 * g + 2] = b.z; dvv[4 * g + 3] = b.w;
      }
      float p[16], ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fexp2(fmaf(s[r], sl2, -lv[r]));
        if (diag && key > q0 + t * 32 + crow(r, h)) pv = 0.f;
        p[r] = pv;
        ds[r] = pv * (dp[r] - dvv[r]) * scale;
      }
#pragma unroll
      for (int sg = 0; sg < 2; ++sg) {
        const typename Vec8<T>::type pa = pack8<T>(&p[8 * sg]);
        const typename Vec8<T>::type da = pack8<T>(&ds[8 * sg]);
        const int g1 = (t * 32 + 16 * sg + 4 * h) >> 2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          dv[dt] = mfma(pa, ld_il<T, D>(dOi, g1, g1 + 2, dt * 32 + l32), dv[dt]);
          dk[dt] = mfma(da, ld_il<T, D>(Qi, g1, g1 + 2, dt * 32 + l32), dk[dt]);
        }
      }
    }
  }
  // C tiles: rows = keys of this wave, cols = d
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    store_c_tile<T>(dK, D, kblk + wave * 32, Sk, dt * 32 + l32, dk[dt], 1.f, accumulate, h);
    store_c_tile<T>(dV, D, kblk + wave * 32, Sk, dt * 32 + l32, dv[dt], 1.f, accumulate, h);
  }
}

// dQ.  grid = (ceil(Sq/128), B*H).
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_fa_bwd_dq(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    const T* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Dv,
    T* __restrict__ dQ, int64_t Sq, int64_t Sk, float scale, int causal, int accumulate) {
  constexpr int BN = 128, DK = D / 16, DT = D / 32;
  __shared__ __attribute__((aligned(16))) T Ks[BN * (D + 8)];
  __shared__ __attribute__((aligned(16))) T Ki[BN * D];
  __shared__ __attribute__((aligned(16))) T Vs[BN * (D + 8)];
  int64_t tile, bh;
  fa_block(tile, bh);
  Q += bh * Sq * D;
  dO += bh * Sq * D;
  dQ += bh * Sq * D;
  K += bh * Sk * D;
  V += bh * Sk * D;
  LSE += bh * Sq;
  Dv += bh * Sq;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  // causal: the last query blocks carry the most keys, so they are dispatched first
  const int64_t qb = causal ? (int64_t)gridDim.x - 1 - tile : tile;
  const int64_t qblk = qb * 128;
  const int64_t q = qblk + wave * 32 + l32;
  const float sl2 = scale * kLog2e;
  typename Vec8<T>::type qf[DK], of[DK];
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    if (q < Sq) {
      qf[ks] = ld8(Q + q * D + ks * 16 + h * 8);
      of[ks] = ld8(dO + q * D + ks * 16 + h * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qf[ks][e] = (T)0.f;
        of[ks][e] = (T)0.f;
      }
    }
  }
  const float lq = q < Sq ? LSE[q] * kLog2e : 0.f;
  const float dq_d = q < Sq ? Dv[q] : 0.f;
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
  int64_t kend = Sk;
  if (causal) kend = (qblk + 128 < Sk) ? qblk + 128 : Sk;
  for (int64_t k0 = 0; k0 < kend; k0 += BN) {
    __syncthreads();
    stage<T, BN, D, true, true>(K, k0, Sk, Ks, Ki);
    stage<T, BN, D, true, false>(V, k0, Sk, Vs, nullptr);
    __syncthreads();
#pragma unroll 1
    for (int kt = 0; kt < BN / 32; ++kt) {
      // causal: a 32-key sub-tile wholly after this wave's queries contributes nothing
      if (causal && k0 + kt * 32 > qblk + wave * 32 + 31) continue;
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = 0.f;
        dp[r] = 0.f;
      }
#pragma unroll
      for (int ks = 0; ks < DK; ++ks) {
        s = mfma(ld8(Ks + (kt * 32 + l32) * (D + 8) + ks * 16 + h * 8), qf[ks], s);
        dp = mfma(ld8(Vs + (kt * 32 + l32) * (D + 8) + ks * 16 + h * 8), of[ks], dp);
      }
      // Padded keys are zero rows of K/V, so they add nothing to dQ (dS * 0); only the
      // causal diagonal needs a mask.
      const bool diag = causal && (k0 + kt * 32 + 31 > qblk + wave * 32);
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fexp2(fmaf(s[r], sl2, -lq));
        if (diag && k0 + kt * 32 + crow(r, h) > q) pv = 0.f;
        ds[r] = pv * (dp[r] - dq_d) * scale;
      }
#pragma unroll
      for (int sg = 0; sg < 2; ++sg) {
        const typename Vec8<T>::type da = pack8<T>(&ds[8 * sg]);
        const int g1 = (kt * 32 + 16 * sg + 4 * h) >> 2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          acc[dt] = mfma(da, ld_il<T, D>(Ki, g1, g1 + 2, dt * 32 + l32), acc[dt]);
      }
    }
  }
  // C tiles: rows = queries of this wave, cols = d
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    store_c_tile<T>(dQ, D, qblk + wave * 32, Sq, dt * 32 + l32, acc[dt], 1.f, accumulate, h);
}

template <typename T, int D>
int fwd_t(const void* q, const void* k, const void* v, void* o, float* lse, int64_t BH,
          int64_t Sq, int64_t Sk, float scale, int causal, hipStream_t s) {
  dim3 grid((unsigned)((Sq + 127) / 128), (unsigned)BH);
  k_fa_fwd<T, D><<<grid, kThreads, 0, s>>>((const T*)q, (const T*)k, (const T*)v, (T*)o, lse, Sq,
                                           Sk, scale, causal);
  return tg_check_launch("tg_flash_attn_fwd");
}

template <typename T, int D>
int bwd_t(const void* q, const void* k, const void* v, const void* o, const void* dout,
          const float* lse, void* dq, void* dk, void* dv, int64_t BH, int64_t Sq, int64_t Sk,
          float scale, int causal, int acc, float* dvec, hipStream_t s) {
  const int64_t rows = BH * Sq;
  k_fa_bwd_prep<T, D><<<(unsigned)((rows + 15) / 16), kThreads, 0, s>>>(
      (const T*)o, (const T*)dout, dvec, rows);
  dim3 gkv((unsigned)((Sk + 127) / 128), (unsigned)BH);
  k_fa_bwd_dkdv<T, D><<<gkv, kThreads, 0, s>>>((const T*)q, (const T*)k, (const T*)v,
                                               (const T*)dout, lse, dvec, (T*)dk, (T*)dv, Sq, Sk,
                                               scale, causal, acc);
  dim3 gq((unsigned)((Sq + 127) / 128), (unsigned)BH);
  k_fa_bwd_dq<T, D><<<gq, kThreads, 0, s>>>((const T*)q, (const T*)k, (const T*)v,
                                            (const T*)dout, lse, dvec, (T*)dq, Sq, Sk, scale,
                                            causal, acc);
  return tg_check_launch("tg_flash_attn_bwd");
}

int check_fa(int dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
             const char* who) {
  TG_REQUIRE(dtype == TG_F16 || dtype == TG_BF16, "%s: dtype must be fp16 or bf16", who);
  TG_REQUIRE(D == 64 || D == 128, "%s: head dim %lld not supported (64, 128)", who,
             (long long)D);
  TG_REQUIRE(B > 0 && H > 0 && Sq > 0 && Sk > 0, "%s: empty or negative shape", who);
  TG_REQUIRE(B * H <= 65535, "%s: B*H = %lld exceeds 65535", who, (long long)(B * H));
  return TG_OK;
}

}  // namespace

TG_EXPORT int tg_flash_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o,
                                float* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                                int64_t D, float scale, int causal, void* stream) {
  int st = check_fa(dtype, B, H, Sq, Sk, D, "tg_flash_attn_fwd");
  if (st) return st;
  TG_REQUIRE(q && k && v && o && lse, "tg_flash_attn_fwd: null pointer");
  TG_REQUIRE(tg_aligned16(q) && tg_aligned16(k) && tg_aligned16(v) && tg_aligned16(o),
             "tg_flash_attn_fwd: operands must be 16-byte aligned");
  hipStream_t s = tg_stream(stream);
  const int64_t BH = B * H;
  if (dtype == TG_F16)
    return D == 64 ? fwd_t<tg_half, 64>(q, k, v, o, lse, BH, Sq, Sk, scale, causal, s)
                   : fwd_t<tg_half, 128>(q, k, v, o, lse, BH, Sq, Sk, scale, causal, s);
  return D == 64 ? fwd_t<tg_bf16, 64>(q, k, v, o, lse, BH, Sq, Sk, scale, causal, s)
                 : fwd_t<tg_bf16, 128>(q, k, v, o, lse, BH, Sq, Sk, scale, causal, s);
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
  int st = check_fa(dtype, B, H, Sq, Sk, D, "tg_flash_attn_bwd");
  if (st) return st;
  TG_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv, "tg_flash_attn_bwd: null pointer");
  TG_REQUIRE(tg_aligned16(q) && tg_aligned16(k) && tg_aligned16(v) && tg_aligned16(o) &&
                 tg_aligned16(dout),
             "tg_flash_attn_bwd: operands must be 16-byte aligned");
  const size_t need = tg_flash_attn_bwd_workspace(B, H, Sq, Sk, D);
  if (!workspace || workspace_bytes < need) {
    tg_set_error("tg_flash_attn_bwd: workspace of %zu bytes needed", need);
    return TG_ERR_WORKSPACE;
  }
  hipStream_t s = tg_stream(stream);
  const int64_t BH = B * H;
  float* dvec = (float*)workspace;
  if (dtype == TG_F16)
    return D == 64 ? bwd_t<tg_half, 64>(q, k, v, o, dout, lse, dq, dk, dv, BH, Sq, Sk, scale,
                                        causal, accumulate, dvec, s)
                   : bwd_t<tg_half, 128>(q, k, v, o, dout, lse, dq, dk, dv, BH, Sq, Sk, scale,
                                         causal, accumulate, dvec, s);
  return D == 64 ? bwd_t<tg_bf16, 64>(q, k, v, o, dout, lse, dq, dk, dv, BH, Sq, Sk, scale,
                                      causal, accumulate, dvec, s)
                 : bwd_t<tg_bf16, 128>(q, k, v, o, dout, lse, dq, dk, dv, BH, Sq, Sk, scale,
                                       causal, accumulate, dvec, s);
}
