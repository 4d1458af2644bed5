// Batched row-major GEMM on CDNA4 matrix cores:
//   C[b] = alpha * op(A[b]) @ op(B[b]) + beta * C[b]
// serving the matmul forward and its backward dA = dC @ B^T, dB = A^T @ dC
// (reference: Tensor.__matmul__ and its closure, _core.py:999-1068).
//
// Block tile 128x128xBK, 256 threads = 4 wavefronts in a 2x2 grid, each wave a
// 64x64 sub-tile = 2x2 MFMA 32x32 tiles:
//   fp16 / bf16: v_mfma_f32_32x32x16_{f16,bf16}, BK = 32
//   fp32:        v_mfma_f32_32x32x2_f32,        BK = 16
// Both operands are staged through LDS in k-contiguous layout (As[m][k], Bs[n][k]);
// an operand whose global layout is contiguous along m/n is transposed while it is
// written to LDS.  The next k-tile is fetched into registers while the current one
// is multiplied.  Accumulation is fp32; the epilogue applies alpha/beta and converts.
#include "tg_common.h"

#include <algorithm>
#include <vector>

namespace {

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <typename T> struct Vec8;
template <> struct Vec8<tg_half> { typedef _Float16 type __attribute__((ext_vector_type(8))); };
template <> struct Vec8<tg_bf16> { typedef __bf16 type __attribute__((ext_vector_type(8))); };

__device__ __forceinline__ void mfma_v(const Vec8<tg_half>::type& a, const Vec8<tg_half>::type& b,
                                       f32x16& c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void mfma_v(const Vec8<tg_bf16>::type& a, const Vec8<tg_bf16>::type& b,
                                       f32x16& c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <typename T> struct Mfma;
template <> struct Mfma<tg_half> {
  static constexpr int BK = 32;   // k per tile
  static constexpr int EPL = 8;   // elements a lane feeds one instruction
  __device__ static void run(const tg_half* a, const tg_half* b, f32x16& c) {
    f16x8 av, bv;
#pragma unroll
    for (int e = 0; e < 8; ++e) { av[e] = a[e]; bv[e] = b[e]; }
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, c, 0, 0, 0);
  }
};
template <> struct Mfma<tg_bf16> {
  static constexpr int BK = 32;
  static constexpr int EPL = 8;
  __device__ static void run(const tg_bf16* a, const tg_bf16* b, f32x16& c) {
    bf16x8 av, bv;
#pragma unroll
    for (int e = 0; e < 8; ++e) { av[e] = a[e]; bv[e] = b[e]; }
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
  }
};
template <> struct Mfma<float> {
  static constexpr int BK = 16;
  static constexpr int EPL = 1;
  __device__ static void run(const float* a, const float* b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
  }
};

// Global -> register -> LDS staging of one operand tile (ROWS x BK), where "rows"
// are m (for A) or n (for B).  KC: the operand is contiguous along k in memory.
template <typename T, bool KC, bool VEC>
struct TileLoader {
  static constexpr int BK = Mfma<T>::BK;
  static constexpr int VE = 16 / sizeof(T);                 // elements per 16B vector
  static constexpr int NV = (128 * BK) / (VE * kThreads);   // vectors per thread (2)
  static constexpr int NS = (128 * BK) / kThreads;          // scalars per thread
  static constexpr int LDK = BK + 16 / (int)sizeof(T);      // padded LDS row (k) stride
  T reg[VEC ? NV * VE : NS];

  // rows_total: M or N extent; ld: leading dimension of the stored matrix.
  __device__ void load(const T* __restrict__ base, int64_t ld, int64_t rows_total, int64_t K,
                       int64_t row0, int64_t k0) {
    const int t = threadIdx.x;
    if (VEC) {
#pragma unroll
      for (int r = 0; r < NV; ++r) {
        const int v = t + r * kThreads;
        int64_t row, k;
        if (KC) {
          row = row0 + v / (BK / VE);
          k = k0 + (v % (BK / VE)) * VE;
        } else {
          k = k0 + v / (128 / VE);
          row = row0 + (v % (128 / VE)) * VE;
        }
        uint4 u = make_uint4(0, 0, 0, 0);
        if (KC) {
          if (row < rows_total && k + VE <= K)
            u = *reinterpret_cast<const uint4*>(base + row * ld + k);
          else if (row < rows_total && k < K) {
            T tmp[VE];
#pragma unroll
            for (int e = 0; e < VE; ++e) tmp[e] = (k + e < K) ? base[row * ld + k + e] : T(0);
            u = *reinterpret_cast<uint4*>(tmp);
          }
        } else {
          if (k < K && row + VE <= rows_total)
            u = *reinterpret_cast<const uint4*>(base + k * ld + row);
          else if (k < K && row < rows_total) {
            T tmp[VE];
#pragma unroll
            for (int e = 0; e < VE; ++e)
              tmp[e] = (row + e < rows_total) ? base[k * ld + row + e] : T(0);
            u = *reinterpret_cast<uint4*>(tmp);
          }
        }
        *reinterpret_cast<uint4*>(&reg[r * VE]) = u;
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int e = t + s * kThreads;
        int64_t row, k;
        if (KC) {
          row = row0 + e / BK;
          k = k0 + e % BK;
        } else {
          k = k0 + e / 128;
          row = row0 + e % 128;
        }
        reg[s] = (row < rows_total && k < K) ? (KC ? base[row * ld + k] : base[k * ld + row]) : T(0);
      }
    }
  }

  __device__ void store(T* __restrict__ lds) const {
    const int t = threadIdx.x;
    if (VEC) {
#pragma unroll
      for (int r = 0; r < NV; ++r) {
        const int v = t + r * kThreads;
        if (KC) {
          const int row = v / (BK / VE), k = (v % (BK / VE)) * VE;
          *reinterpret_cast<uint4*>(lds + row * LDK + k) =
              *reinterpret_cast<const uint4*>(&reg[r * VE]);
        } else {
          const int k = v / (128 / VE), row = (v % (128 / VE)) * VE;
#pragma unroll
          for (int e = 0; e < VE; ++e) lds[(row + e) * LDK + k] = reg[r * VE + e];
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int e = t + s * kThreads;
        int row, k;
        if (KC) {
          row = e / BK;
          k = e % BK;
        } else {
          k = e / 128;
          row = e % 128;
        }
        lds[row * LDK + k] = reg[s];
      }
    }
  }
};

template <typename T, typename TC, bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(kThreads) void k_gemm(int64_t M, int64_t N, int64_t K, float alpha,
                                                   const T* __restrict__ A, int64_t lda,
                                                   int64_t sa, const T* __restrict__ B,
                                                   int64_t ldb, int64_t sb, float beta,
                                                   TC* __restrict__ C, int64_t ldc, int64_t sc,
    const float* __restrict__ bias) {
  constexpr int BK = Mfma<T>::BK;
  constexpr int EPL = Mfma<T>::EPL;
  constexpr int KPL = BK / 2;  // k elements per lane per tile (lane half h owns k in [h*KPL, h*KPL+KPL))
  using LA = TileLoader<T, !TA, VEC>;
  using LB = TileLoader<T, TB, VEC>;
  constexpr int LDK = LA::LDK;
  __shared__ __attribute__((aligned(16))) T As[BM * LDK];
  __shared__ __attribute__((aligned(16))) T Bs[BN * LDK];

  const int64_t bz = blockIdx.z;
  A += bz * sa;
  B += bz * sb;
  C += bz * sc;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int lr = lane & 31, lh = lane >> 5;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  LA la;
  LB lb;
  la.load(A, lda, M, K, m0, 0);
  lb.load(B, ldb, N, K, n0, 0);
  for (int64_t k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();
    la.store(As);
    lb.store(Bs);
    __syncthreads();
    if (k0 + BK < K) {
      la.load(A, lda, M, K, m0, k0 + BK);
      lb.load(B, ldb, N, K, n0, k0 + BK);
    }
    T af[2][KPL], bf[2][KPL];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const T* pa = As + (wm + i * 32 + lr) * LDK + lh * KPL;
      const T* pb = Bs + (wn + i * 32 + lr) * LDK + lh * KPL;
#pragma unroll
      for (int e = 0; e < KPL; e += 16 / (int)sizeof(T)) {
        *reinterpret_cast<uint4*>(&af[i][e]) = *reinterpret_cast<const uint4*>(pa + e);
        *reinterpret_cast<uint4*>(&bf[i][e]) = *reinterpret_cast<const uint4*>(pb + e);
      }
    }
#pragma unroll
    for (int s = 0; s < KPL / EPL; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) Mfma<T>::run(&af[i][s * EPL], &bf[j][s * EPL], acc[i][j]);
  }

  // Epilogue: acc[i][j][r], r = g*4 + q  ->  row = 8g + 4*lh + q, col = lr (32x32 tile).
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn + j * 32 + lr;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
        if (row < M) {
          float v = alpha * acc[i][j][r];
          if (bias) v += bias[col];
          TC* pc = C + row * ldc + col;
          if (beta != 0.f) v += beta * tg_to_float(*pc);
          *pc = tg_from_float<TC>(v);
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Small fp32 outputs (the generic kernel's 128 x 128 tiles leave most CUs idle and, for
// a few rows, compute mostly padding): one 32 x 32 output tile per workgroup, its four
// wavefronts each taking a quarter of K with the fp32 MFMA's fragments read straight
// from global memory (no operand is shared between wavefronts), then the four partial
// tiles added in LDS in a fixed order (deterministic).  Of every 8 k, lane half h
// multiplies k + 4h .. k + 4h + 3 in four MFMAs (the same pairing for A and B).
template <typename TC, bool TA, bool TB>
__global__ __launch_bounds__(kThreads) void k_gemm_f32_small(
    int64_t M, int64_t N, int64_t K, float alpha, const float* __restrict__ A, int64_t lda,
    int64_t sa, const float* __restrict__ B, int64_t ldb, int64_t sb, float beta,
    TC* __restrict__ C, int64_t ldc, int64_t sc, const float* __restrict__ bias) {
  const int64_t bz = blockIdx.z;
  A += bz * sa;
  B += bz * sb;
  C += bz * sc;
  const int64_t m0 = (int64_t)blockIdx.y * 32, n0 = (int64_t)blockIdx.x * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t row = m0 + l32, col = n0 + l32;
  const int64_t per = ((K + 31) / 32) * 8;  // k per wavefront, a multiple of 8
  const int64_t kb = wave * per;
  const int64_t ke = kb + per < K ? kb + per : K;
  const bool rok = row < M, cok = col < N;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll 4
  for (int64_t k0 = kb; k0 < ke; k0 += 8) {
    float a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k = k0 + 4 * h + j;
      const bool kok = k < ke;
      a[j] = (rok && kok) ? (TA ? A[k * lda + row] : A[row * lda + k]) : 0.f;
      b[j] = (cok && kok) ? (TB ? B[col * ldb + k] : B[k * ldb + col]) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], acc, 0, 0, 0);
  }
  __shared__ float red[3][16][64];
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave - 1][r][lane] = acc[r];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float v = ((acc[r] + red[0][r][lane]) + red[1][r][lane]) + red[2][r][lane];
    const int64_t i = m0 + (r >> 2) * 8 + h * 4 + (r & 3);
    if (i < M && cok) {
      float o = alpha * v;
      if (bias) o += bias[col];
      TC* pc = C + i * ldc + col;
      if (beta != 0.f) o += beta * tg_to_float(*pc);
      *pc = tg_from_float<TC>(o);
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined kernel for fp16/bf16: block tile 128 x BN x 64 (BN = 128 or 64),
// 4 wavefronts in a 2 x 2 grid, each owning a 64 x BN/2 sub-tile of MFMA 32x32
// tiles; LDS double-buffered so the next k-tile's global loads overlap the
// current MFMAs, one barrier per k-tile.  BN is chosen so the grid holds at least
// two blocks per CU where the problem allows it.
// LDS layout per operand:
//   contiguous along k in memory  -> row-major [row][BK+8]: one 16-byte read per
//                                    8-element fragment;
//   contiguous along m/n          -> 4-k interleaved [k/4][row][4]: staged with
//                                    8-byte writes, read as two 8-byte halves.
// Tiles are assigned XCD-aware: dispatch i runs on XCD i % 8, so the launch index
// is remapped to give each XCD a contiguous band of tiles (shared A rows in its L2).
constexpr int V2_BM = 128, V2_BK = 64;

template <typename T, bool KC, int ROWS>
struct StageV2 {
  static constexpr int NVEC = KC ? (ROWS * V2_BK) / (8 * kThreads) : 4;
  static constexpr int UNITS = (V2_BK / 4) * (ROWS / 8);
  static constexpr int RM_LD = V2_BK + 8;
  static constexpr int LDS_ELEMS = KC ? ROWS * RM_LD : ROWS * V2_BK;
  uint4 r[NVEC];

  __device__ void load(const T* __restrict__ g, int64_t ld, int64_t rows_total, int64_t K,
                       int64_t row0, int64_t k0) {
    const int t = threadIdx.x;
    if (KC) {
#pragma unroll
      for (int i = 0; i < NVEC; ++i) {
        const int v = t + i * kThreads;
        const int64_t row = row0 + v / (V2_BK / 8);
        const int64_t k = k0 + (v % (V2_BK / 8)) * 8;
        r[i] = (row < rows_total && k < K) ? *reinterpret_cast<const uint4*>(g + row * ld + k)
                                           : make_uint4(0, 0, 0, 0);
      }
    } else {
      if (t >= UNITS) return;
      const int kg = t / (ROWS / 8), rg = t % (ROWS / 8);
      const int64_t row = row0 + rg * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t k = k0 + kg * 4 + i;
        r[i] = (k < K && row < rows_total) ? *reinterpret_cast<const uint4*>(g + k * ld + row)
                                           : make_uint4(0, 0, 0, 0);
      }
    }
  }

  __device__ void store(T* lds) const {
    const int t = threadIdx.x;
    if (KC) {
#pragma unroll
      for (int i = 0; i < NVEC; ++i) {
        const int v = t + i * kThreads;
        const int row = v / (V2_BK / 8), k = (v % (V2_BK / 8)) * 8;
        *reinterpret_cast<uint4*>(lds + row * RM_LD + k) = r[i];
      }
    } else {
      if (t >= UNITS) return;
      const int kg = t / (ROWS / 8), rg = t % (ROWS / 8);
      const T* e0 = reinterpret_cast<const T*>(&r[0]);
      const T* e1 = reinterpret_cast<const T*>(&r[1]);
      const T* e2 = reinterpret_cast<const T*>(&r[2]);
      const T* e3 = reinterpret_cast<const T*>(&r[3]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        T q4[4] = {e0[j], e1[j], e2[j], e3[j]};
        *reinterpret_cast<uint2*>(lds + (kg * ROWS + rg * 8 + j) * 4) =
            *reinterpret_cast<const uint2*>(q4);
      }
    }
  }

  // 8-element fragment for `row` (tile-local) and k = ks*16 + h*8 + e.
  __device__ __forceinline__ typename Vec8<T>::type frag(const T* lds, int row, int ks,
                                                         int h) const {
    union {
      uint4 u;
      typename Vec8<T>::type v;
    } r;
    if (KC) {
      r.u = *reinterpret_cast<const uint4*>(lds + row * RM_LD + ks * 16 + h * 8);
    } else {
      const int g = ks * 4 + h * 2;
      const uint2 a = *reinterpret_cast<const uint2*>(lds + (g * ROWS + row) * 4);
      const uint2 b = *reinterpret_cast<const uint2*>(lds + ((g + 1) * ROWS + row) * 4);
      r.u = make_uint4(a.x, a.y, b.x, b.y);
    }
    return r.v;
  }
};

template <typename T, typename TC, bool TA, bool TB, int BNv>
__global__ __launch_bounds__(kThreads) void k_gemm_v2(int64_t M, int64_t N, int64_t K, float alpha,
                                                      const T* __restrict__ A, int64_t lda,
                                                      int64_t sa, const T* __restrict__ B,
                                                      int64_t ldb, int64_t sb, float beta,
                                                      TC* __restrict__ C, int64_t ldc, int64_t sc,
    const float* __restrict__ bias) {
  constexpr int NTW = BNv / 64;  // 32-wide MFMA tiles per wave along n
  using SA = StageV2<T, !TA, V2_BM>;
  using SB = StageV2<T, TB, BNv>;
  __shared__ __attribute__((aligned(16))) T As[2][SA::LDS_ELEMS];
  __shared__ __attribute__((aligned(16))) T Bs[2][SB::LDS_ELEMS];

  const int64_t gx = gridDim.x, gy = gridDim.y;
  const int64_t T_ = gx * gy;
  int64_t lin = (int64_t)blockIdx.y * gx + blockIdx.x;
  if (T_ % 8 == 0) lin = (lin % 8) * (T_ / 8) + lin / 8;
  const int64_t tm = lin / gx, tn = lin % gx;
  const int64_t bz = blockIdx.z;
  A += bz * sa;
  B += bz * sb;
  C += bz * sc;
  const int64_t m0 = tm * V2_BM, n0 = tn * BNv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * (BNv / 2);
  const int lr = lane & 31, lh = lane >> 5;

  f32x16 acc[2][NTW];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  SA sa_;
  SB sb_;
  sa_.load(A, lda, M, K, m0, 0);
  sb_.load(B, ldb, N, K, n0, 0);
  sa_.store(As[0]);
  sb_.store(Bs[0]);
  __syncthreads();
  int cur = 0;
  for (int64_t k0 = 0; k0 < K; k0 += V2_BK) {
    const bool more = k0 + V2_BK < K;
    if (more) {
      sa_.load(A, lda, M, K, m0, k0 + V2_BK);
      sb_.load(B, ldb, N, K, n0, k0 + V2_BK);
    }
#pragma unroll
    for (int ks = 0; ks < V2_BK / 16; ++ks) {
      typename Vec8<T>::type af[2], bfr[NTW];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = sa_.frag(As[cur], wm + i * 32 + lr, ks, lh);
#pragma unroll
      for (int j = 0; j < NTW; ++j) bfr[j] = sb_.frag(Bs[cur], wn + j * 32 + lr, ks, lh);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) mfma_v(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      sa_.store(As[cur ^ 1]);
      sb_.store(Bs[cur ^ 1]);
    }
    __syncthreads();
    cur ^= 1;
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const int64_t col = n0 + wn + j * 32 + lr;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
        if (row < M) {
          float v = alpha * acc[i][j][r];
          if (bias) v += bias[col];
          TC* pc = C + row * ldc + col;
          if (beta != 0.f) v += beta * tg_to_float(*pc);
          *pc = tg_from_float<TC>(v);
        }
      }
    }
}


// ---------------------------------------------------------------------------- v3
// fp16/bf16 GEMM with DMA-staged operands: 128x128 block tile, k-tiles of 64, four
// waves in a 2x2 grid each owning 64x64 of C (2x2 MFMA 32x32x16 tiles).  Both
// operand tiles are copied global -> LDS with global_load_lds (16 bytes per lane,
// one contiguous KiB per wave instruction), double-buffered so the next k-tile
// streams in while the current one is multiplied; no VGPRs and no LDS store
// instructions are spent on staging.  Tiles keep the operand's global orientation:
//   k-contiguous operand (A, or B^T): [128 rows][64 k], fragments are 16-byte row
//     reads (lane = row, 8 consecutive k);
//   m/n-contiguous operand (A^T, or B): [64 k][128 cols], fragments are two
//     ds_read_b64_tr_b16 reads (lane = column, 4 consecutive k each).
// Rows are unpadded with the 16-byte chunks XOR-swizzled by the row index, so both
// read kinds are free of LDS bank conflicts.  Requires K % 64 == 0 and 16-byte
// aligned operands; rows/columns past M or N read clamped addresses and only feed
// C entries that are never stored.
typedef short v4i16_g __attribute__((ext_vector_type(4)));
#define TG_LDS_G __attribute__((address_space(3)))
#define TG_GLB_G __attribute__((address_space(1)))

constexpr int V3_BK = 64;
// 256x256 blocks once there are kHugeTiles/4 of them per CU.
constexpr int kHugeTiles = 4;
// 256x128 blocks: 4x2 waves of 64x64.
constexpr int kBigWGM = 4, kBigWGN = 2, kBigSM = 2, kBigSN = 2;

// XOR key of row r (CH 16-byte chunks per row): 16 consecutive rows get distinct
// chunk positions and rows r..r+3 of a transpose read land in different 64-byte bank
// groups, so both read kinds are conflict-free.
template <int CH> __device__ __forceinline__ int v3_key(int r) {
  if (CH == 8) {
    const int x = (r >> 1) & 7;
    return ((x & 1) << 2) | (x >> 1);
  }
  return ((r & 3) << 2) | ((r >> 2) & 3);
}
template <int CH> __device__ __forceinline__ int v3_off(int r, int c) {
  return r * CH * 16 + ((c ^ v3_key<CH>(r)) << 4);
}

// DMA of R x CW tiles (CW elements per row) of a matrix with leading dimension ld, by
// NW waves.  One operand's tiles all start at the same row (KROWS false: rows are
// m or n, fixed per block; the column is k) or at the same column (KROWS true: rows
// are k, the column is m or n).  The clamp of rows or columns past the matrix edge
// therefore depends only on the block, so each lane's byte offset within a tile is
// computed once; a tile then costs one uniform pointer per wave instruction.  The
// k extent needs no clamp (K % 64 == 0).
template <typename T, int R, int CW, int NW, bool KROWS>
struct V3Dma {
  static constexpr int CH = CW / 8, NI = R * CH / 64, NPW = NI / NW;
  static_assert(NI % NW == 0, "tile must split evenly over the waves");
  uint32_t off[NPW];
  // base0: first row (KROWS false) or first column (KROWS true) of the block; nlim:
  // rows (resp. columns) of the matrix.
  __device__ void init(int64_t ld, int64_t base0, int64_t nlim) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < NPW; ++k) {
      const int u = (wave + k * NW) * 64 + lane;
      const int r = u / CH, c = (u % CH) ^ v3_key<CH>(r);
      int64_t e;
      if (!KROWS) {
        int64_t row = base0 + r;
        row = row < nlim ? row : nlim - 1;
        e = (row - base0) * ld + c * 8;
      } else {
        int64_t col = base0 + c * 8;
        col = col + 8 <= nlim ? col : nlim - 8;
        e = r * ld + (col - base0);
      }
      off[k] = (uint32_t)(e * (int64_t)sizeof(T));
    }
  }
  // Copy the tile whose origin is soff bytes past base (both uniform): a raw buffer
  // load into LDS takes the lane offset in a VGPR and the tile offset in an SGPR, so
  // the copy costs no vector ALU work.  The resource spans [base, base + 2 GiB) (word
  // 3: 32-bit untyped access, no swizzle; the gfx9 raw-buffer format).
  __device__ __forceinline__ void copy(const T* base, uint32_t soff, char* lds) const {
    // The buffer-resource type is compiled in the device pass only: the host pass of
    // this compiler drops the launch stubs of kernel instantiations whose bodies hold it.
#if defined(__HIP_DEVICE_COMPILE__)
    const int wave = threadIdx.x >> 6;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(base), (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int k = 0; k < NPW; ++k)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (TG_LDS_G void*)(lds + (wave + k * NW) * 1024),
                                               16, off[k], soff, 0, 0);
#endif
  }
  // Instruction k of copy() alone, so a caller can spread a tile's copy over its MFMAs.
  __device__ __forceinline__ void copy1(const T* base, uint32_t soff, char* lds, int k) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const int wave = threadIdx.x >> 6;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(base), (short)0, 0x7fffffff, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (TG_LDS_G void*)(lds + (wave + k * NW) * 1024),
                                             16, off[k], soff, 0, 0);
#endif
  }
};

// Fragment reader for one operand tile of EXT rows (m or n) and 64 k.
//   KC: [EXT rows][64 k], 128-byte rows; else [64 k][EXT], EXT*2-byte rows.
// S slabs of 32 rows/columns per wave, starting at the wave's offset wbase.
template <typename T, bool KC, int EXT, int S>
struct V3Frag {
  static constexpr int CHM = EXT / 8;  // chunks per row of the m/n-contiguous layout
  int off[KC ? 4 : 2 * S];
  __device__ void init(int lane, int wbase) {
    const int l32 = lane & 31, h = lane >> 5;
    if (KC) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) off[ks] = v3_off<8>(l32, 2 * ks + h) - l32 * 128;
    } else {
      const int s = lane & 15, nh = (lane >> 4) & 1;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < S; ++i) {
          const int row = 8 * h + 4 * j + (s >> 2);
          const int col = wbase + 32 * i + 16 * nh + 4 * (s & 3);
          off[j * S + i] = v3_off<CHM>(row, col >> 3) + (col & 7) * 2;
        }
    }
  }
  // 8 k-elements k = ks*16 + 8h + e of row/column wbase + 32 i + l32.
  __device__ __forceinline__ typename Vec8<T>::type get(const char* tile, int wbase, int i,
                                                        int ks, int l32) const {
    if (KC) {
      const int row = wbase + 32 * i + l32;  // swizzle key = row bits 1-3 = l32's
      return *reinterpret_cast<const typename Vec8<T>::type*>(tile + row * 128 + off[ks]);
    } else {
      union {
        v4i16_g h[2];
        typename Vec8<T>::type v;
      } u;
      const char* b = tile + ks * 16 * EXT * 2;
      u.h[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TG_LDS_G v4i16_g*)(b + off[i]));
      u.h[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TG_LDS_G v4i16_g*)(b + off[S + i]));
      return u.v;
    }
  }
};

// Sum of the 8 k-elements of a B fragment, added to acc in fp32 (v_dot2 with ones:
// the products are exact, so each step is one fp32 addition of a pair).
__device__ __forceinline__ float frag_sum(const Vec8<tg_half>::type& v, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 one = {(_Float16)1, (_Float16)1};
#pragma unroll
  for (int e = 0; e < 8; e += 2) acc = __builtin_amdgcn_fdot2(h2{v[e], v[e + 1]}, one, acc, false);
  return acc;
}
__device__ __forceinline__ float frag_sum(const Vec8<tg_bf16>::type& v, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
  for (int e = 0; e < 8; e += 2)
    acc = __builtin_amdgcn_fdot2_f32_bf16(b2{v[e], v[e + 1]}, one, acc, false);
  return acc;
}

// Block = WGM x WGN waves, each owning (SM*32) x (SN*32) of C.
// BSUM: the column sums of op(B) over this launch's K range are written too, as fp32
// bsum[batch][N] (the bias gradient of a Linear layer next to its weight gradient
// dW = X^T dY, where op(B) = dY).  Every wave adds up the B fragments it multiplies
// (one v_dot2 per pair of elements, beside the MFMAs); the waves of the first block
// row that hold rows 0.. of C, which between them see every k of every column once,
// store theirs.
// One block's C tile of a DMA-staged GEMM (A, B, C already at their batch entry).
// BSUM: the blocks of the first tile row also sum B's columns over the whole K range
// and store the sums to bsum (fp32) or, with bsum null, to dbo (dtype dbt, added to
// its contents when dbacc; dbo null: nowhere).
// EPI (epilogue fused on the stored values, which are first rounded to TC exactly as a
// plain GEMM stores them, so each fused result equals the separate kernel's bit for bit):
//   EPI_NONE      C (+)= alpha*AB (+ bias)
//   EPI_GELU_BWD  C (+)= round(alpha*AB) * gelu'(X)   (X: the GELU input, [M, N], ldx)
//   EPI_GELU_FWD  C = round(alpha*AB + bias), X = round(gelu(C))  (X written)
//   EPI_RESIDUAL  C = round(alpha*AB + bias) + X      (X: the residual, read)
enum { EPI_NONE = 0, EPI_GELU_BWD = 1, EPI_GELU_FWD = 2, EPI_RESIDUAL = 3 };
// v = the product rounded to TC; c = the old C value (added when beta != 0).  GELU
// backward accumulates with one explicit FMA, as tg_gelu_bwd's accumulate mode does.
template <int EPI>
__device__ __forceinline__ float epi_val(float v, float x, float beta, float c) {
  if (EPI == EPI_GELU_BWD) {
    const float g = tg_gelu_grad(x);
    return tg_f32(beta != 0.f ? fmaf(v, g, beta * c) : v * g);
  }
  if (EPI == EPI_RESIDUAL) return v + x;
  return v;
}

// EXT: the caller names the tile (row tile xtm, column tile xtn); otherwise it follows
// from the block index, XCD-banded.
template <typename T, typename TC, bool TA, bool TB, int WGM, int WGN, int SM, int SN, int OCC,
          bool BSUM, int EPI = EPI_NONE, bool EXT = false>
__device__ __forceinline__ void v3_tile(
    int64_t M, int64_t N, int64_t K, float alpha, const T* __restrict__ A, int64_t lda,
    const T* __restrict__ B, int64_t ldb, float beta, TC* __restrict__ C, int64_t ldc,
    const float* __restrict__ bias, float* __restrict__ bsum, void* dbo, int dbt, bool dbacc,
    TC* __restrict__ X = nullptr, int64_t ldx = 0, int64_t xtm = 0, int64_t xtn = 0) {
  constexpr int NW = WGM * WGN, TBM = WGM * SM * 32, TBN = WGN * SN * 32;
  constexpr int ATILE = TBM * V3_BK * 2, BTILE = TBN * V3_BK * 2;
  __shared__ __attribute__((aligned(1024))) char a0[ATILE];
  __shared__ __attribute__((aligned(1024))) char b0[BTILE];
  __shared__ __attribute__((aligned(1024))) char a1[ATILE];
  __shared__ __attribute__((aligned(1024))) char b1[BTILE];
  constexpr bool AKC = !TA, BKC = TB;
  int64_t tm = xtm, tn = xtn;
  if constexpr (!EXT) {
    const int64_t gx = gridDim.x, gy = gridDim.y;
    const int64_t T_ = gx * gy;
    int64_t lin = (int64_t)blockIdx.y * gx + blockIdx.x;
    if (T_ % 8 == 0) lin = (lin % 8) * (T_ / 8) + lin / 8;  // XCD-contiguous bands
    tm = lin / gx;
    tn = lin % gx;
  }
  const int64_t m0 = tm * TBM, n0 = tn * TBN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave / WGN) * SM * 32, wn = (wave % WGN) * SN * 32;
  const int l32 = lane & 31, lh = lane >> 5;
  V3Frag<T, AKC, TBM, SM> fa;
  V3Frag<T, BKC, TBN, SN> fb;
  fa.init(lane, wm);
  fb.init(lane, wn);
  f32x16 acc[SM][SN];
#pragma unroll
  for (int i = 0; i < SM; ++i)
#pragma unroll
    for (int j = 0; j < SN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float bsums[SN];  // BSUM: this lane's partial column sums (8 k per fragment and k-step)
#pragma unroll
  for (int j = 0; j < SN; ++j) bsums[j] = 0.f;
  // A is [M][K] (lda) or, transposed, [K][M]; B is [K][N] or, transposed, [N][K].
  // Tile origins: k-contiguous operands start at (row m0|n0, column k0), the others
  // at (row k0, column m0|n0); the clamps at the M / N edge are per block.
  V3Dma<T, AKC ? TBM : 64, AKC ? 64 : TBM, NW, !AKC> da;
  V3Dma<T, BKC ? TBN : 64, BKC ? 64 : TBN, NW, !BKC> db;
  da.init(lda, m0, M);
  db.init(ldb, n0, N);
  const T* a_org = A + (AKC ? m0 * lda : m0);
  const T* b_org = B + (BKC ? n0 * ldb : n0);
  auto dma = [&](int64_t k0, char* as, char* bs) {
    da.copy(a_org, (uint32_t)((AKC ? k0 : k0 * lda) * (int64_t)sizeof(T)), as);
    db.copy(b_org, (uint32_t)((BKC ? k0 : k0 * ldb) * (int64_t)sizeof(T)), bs);
  };
  // The next tile's copy, instruction q of ANPW + BNPW (A's first), issued between the
  // MFMAs of the current tile by the pipelined path below (has_next false: nothing).
  constexpr int ANPW = decltype(da)::NPW, BNPW = decltype(db)::NPW;
  auto dma1 = [&](int64_t k0, char* as, char* bs, int q) {
    if (q < ANPW) da.copy1(a_org, (uint32_t)((AKC ? k0 : k0 * lda) * (int64_t)sizeof(T)), as, q);
    else db.copy1(b_org, (uint32_t)((BKC ? k0 : k0 * ldb) * (int64_t)sizeof(T)), bs, q - ANPW);
  };
  auto mul = [&](const char* as, const char* bs, bool has_next, int64_t kn, char* an, char* bn) {
    if constexpr (OCC == 1) {
      // One wave per SIMD: software pipeline.  The fragment reads of k-step ks+1 are
      // issued between the MFMAs of k-step ks (sched_barrier keeps the order), so only
      // the first k-step of a tile waits on LDS latency.  The next tile's DMA goes out
      // one instruction per two MFMAs over the first half of the tile: issued all at
      // once after the barrier, the waves' copies queue in the address unit while no
      // MFMA runs.
      constexpr int NQ = ANPW + BNPW, NMF = (V3_BK / 16) * SM * SN;
      constexpr int QSTEP = NQ * 2 <= NMF / 2 ? 2 : 1;
      int q = 0;
      typename Vec8<T>::type fr[2][SM + SN];
      auto rd = [&](int buf, int ks, int n) {
        if (n < SM) fr[buf][n] = fa.get(as, wm, n, ks, l32);
        else fr[buf][n] = fb.get(bs, wn, n - SM, ks, l32);
      };
#pragma unroll
      for (int n = 0; n < SM + SN; ++n) rd(0, 0, n);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < V3_BK / 16; ++ks) {
        const int cur = ks & 1;
        int nr = 0;
        if constexpr (BSUM) {
#pragma unroll
          for (int j = 0; j < SN; ++j) bsums[j] = frag_sum(fr[cur][SM + j], bsums[j]);
        }
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
          for (int j = 0; j < SN; ++j) {
            mfma_v(fr[cur][i], fr[cur][SM + j], acc[i][j]);
            if (ks + 1 < V3_BK / 16 && nr < SM + SN && (i * SN + j) % 2 == 1) {
              rd(cur ^ 1, ks + 1, nr);
              ++nr;
            }
            const int mf = (ks * SM + i) * SN + j;
            if (has_next && mf % QSTEP == QSTEP - 1 && mf / QSTEP < NQ) dma1(kn, an, bn, mf / QSTEP);
            __builtin_amdgcn_sched_barrier(0);
          }
        if (ks + 1 < V3_BK / 16)
#pragma unroll
          for (; nr < SM + SN; ++nr) rd(cur ^ 1, ks + 1, nr);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      if (has_next) dma(kn, an, bn);
#pragma unroll
      for (int ks = 0; ks < V3_BK / 16; ++ks) {
        typename Vec8<T>::type af[SM], bf[SN];
#pragma unroll
        for (int i = 0; i < SM; ++i) af[i] = fa.get(as, wm, i, ks, l32);
#pragma unroll
        for (int j = 0; j < SN; ++j) bf[j] = fb.get(bs, wn, j, ks, l32);
        if constexpr (BSUM) {
#pragma unroll
          for (int j = 0; j < SN; ++j) bsums[j] = frag_sum(bf[j], bsums[j]);
        }
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
          for (int j = 0; j < SN; ++j) mfma_v(af[i], bf[j], acc[i][j]);
      }
    }
  };
  if (K > 0) dma(0, a0, b0);
  for (int64_t k0 = 0; k0 < K; k0 += 2 * V3_BK) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const bool more1 = k0 + V3_BK < K;
    mul(a0, b0, more1, k0 + V3_BK, a1, b1);
    if (!more1) break;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const bool more2 = k0 + 2 * V3_BK < K;
    mul(a1, b1, more2, k0 + 2 * V3_BK, a0, b0);
    if (!more2) break;
  }
  if constexpr (BSUM) {
    if (tm == 0 && wm == 0) {
      // lanes l32 and l32 + 32 hold the two 8-element k halves of column l32
#pragma unroll
      for (int j = 0; j < SN; ++j) {
        const float v = bsums[j] + __shfl_xor(bsums[j], 32);
        const int64_t col = n0 + wn + j * 32 + l32;
        if (lh == 0 && col < N) {
          if (bsum) bsum[col] = v;
          else if (dbo == nullptr) {
          } else if (dbt == TG_F32) {
            float* d = static_cast<float*>(dbo) + col;
            *d = v + (dbacc ? *d : 0.f);
          } else {
            T* d = static_cast<T*>(dbo) + col;
            *d = tg_from_float<T>(v + (dbacc ? tg_to_float(*d) : 0.f));
          }
        }
      }
    }
  }
  if (m0 + TBM <= M && n0 + TBN <= N) {
    // Full tile: each wave stages one slab of HR rows (32, or 16 when two 32-row
    // slabs per stage array do not fit) of its C tile at a time in its own LDS region
    // (the operand stages are free once every wave has passed the barrier) and writes
    // it back as 16-byte row-contiguous stores.  Row padding puts the two lane halves'
    // stores (4 rows apart) in disjoint banks.
    constexpr int SC = SN * 32;                                          // slab columns
    constexpr int RS = SC * (int)sizeof(TC) + (sizeof(TC) == 4 ? 32 : 16);  // row bytes
    constexpr int NSL = (NW + 3) / 4;                    // slabs per stage array
    constexpr int MINT = ATILE < BTILE ? ATILE : BTILE;
    constexpr int HR = NSL * 32 * RS <= MINT ? 32 : 16;
    static_assert(NSL * HR * RS <= MINT, "slab staging exceeds a stage array");
    constexpr int CPR = SC * (int)sizeof(TC) / 16;                       // chunks per row
    __syncthreads();
    const int st = wave & 3;  // wave w stages in array w % 4, slab w / 4
    char* slab = (st == 0 ? a0 : st == 1 ? b0 : st == 2 ? a1 : b1) + (wave >> 2) * HR * RS;
    float bv[SN];  // bias of this lane's column in each 32-column tile
#pragma unroll
    for (int j = 0; j < SN; ++j) bv[j] = bias ? bias[n0 + wn + j * 32 + l32] : 0.f;
    constexpr int NQ = HR * CPR / 64;  // 16-byte chunks per lane and slab
#pragma unroll
    for (int i = 0; i < SM; ++i) {
#pragma unroll
      for (int half = 0; half < 32 / HR; ++half) {
        // the epilogue operand's chunks of this slab, all loads issued before the slab
        // is staged, so their latency overlaps the staging instead of each store
        uint4 xq[EPI == EPI_GELU_BWD || EPI == EPI_RESIDUAL ? NQ : 1];
        if constexpr (EPI == EPI_GELU_BWD || EPI == EPI_RESIDUAL) {
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            const int u = q * 64 + lane, row = u / CPR, ch = u % CPR;
            xq[q] = *reinterpret_cast<const uint4*>(
                X + (m0 + wm + i * 32 + half * HR + row) * ldx + n0 + wn +
                ch * (16 / (int)sizeof(TC)));
          }
        }
        // accumulator registers r in [half*16*HR/32, ...): rows half*HR .. half*HR+HR-1
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
          for (int rr = 0; rr < HR / 2; ++rr) {
            const int r = half * (HR / 2) + rr;
            const int row = (r >> 2) * 8 + lh * 4 + (r & 3) - half * HR;
            *reinterpret_cast<TC*>(slab + row * RS + (j * 32 + l32) * (int)sizeof(TC)) =
                tg_from_float<TC>(alpha * acc[i][j][r] + bv[j]);
          }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's slab is written
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const int u = q * 64 + lane, row = u / CPR, ch = u % CPR;
          const uint4 v = *reinterpret_cast<const uint4*>(slab + row * RS + ch * 16);
          const int64_t grow = m0 + wm + i * 32 + half * HR + row;
          const int64_t gcol = n0 + wn + ch * (16 / (int)sizeof(TC));
          TC* pc = C + grow * ldc + gcol;
          if constexpr (EPI != EPI_NONE) {
            tg_vec16<TC> o;
            *reinterpret_cast<uint4*>(&o) = v;
            if constexpr (EPI == EPI_GELU_FWD) {
              *reinterpret_cast<uint4*>(pc) = v;
              tg_vec16<TC> a;
#pragma unroll
              for (int e = 0; e < tg_vec16<TC>::N; ++e)
                a.v[e] = tg_from_float<TC>(tg_gelu_fwd(tg_to_float(o.v[e])));
              tg_store16(X + grow * ldx + gcol, a);
            } else {
              tg_vec16<TC> xv;
              *reinterpret_cast<uint4*>(&xv) = xq[q];
              tg_vec16<TC> c;
              if (beta != 0.f) c = tg_load16(pc);
#pragma unroll
              for (int e = 0; e < tg_vec16<TC>::N; ++e) {
                o.v[e] = tg_from_float<TC>(epi_val<EPI>(tg_to_float(o.v[e]), tg_to_float(xv.v[e]),
                                                        beta, beta != 0.f ? tg_to_float(c.v[e]) : 0.f));
              }
              tg_store16(pc, o);
            }
          } else if (beta != 0.f) {
            tg_vec16<TC> o, c = tg_load16(pc);
            *reinterpret_cast<uint4*>(&o) = v;
#pragma unroll
            for (int e = 0; e < tg_vec16<TC>::N; ++e)
              o.v[e] = tg_from_float<TC>(tg_to_float(o.v[e]) + beta * tg_to_float(c.v[e]));
            tg_store16(pc, o);
          } else {
            *reinterpret_cast<uint4*>(pc) = v;
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < SM; ++i)
#pragma unroll
    for (int j = 0; j < SN; ++j) {
      const int64_t col = n0 + wn + j * 32 + l32;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
        if (row < M) {
          float v = alpha * acc[i][j][r];
          if (bias) v += bias[col];
          TC* pc = C + row * ldc + col;
          if constexpr (EPI == EPI_GELU_FWD) {
            const TC h = tg_from_float<TC>(v);
            *pc = h;
            X[row * ldx + col] = tg_from_float<TC>(tg_gelu_fwd(tg_to_float(h)));
            continue;
          } else if constexpr (EPI != EPI_NONE) {
            *pc = tg_from_float<TC>(epi_val<EPI>(tg_to_float(tg_from_float<TC>(v)),
                                                 tg_to_float(X[row * ldx + col]), beta,
                                                 beta != 0.f ? tg_to_float(*pc) : 0.f));
            continue;
          }
          if (beta != 0.f) v += beta * tg_to_float(*pc);
          *pc = tg_from_float<TC>(v);
        }
      }
    }
}

template <typename T, typename TC, bool TA, bool TB, int WGM, int WGN, int SM, int SN, int OCC,
          bool BSUM = false>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void k_gemm_v3(
    int64_t M, int64_t N, int64_t K, float alpha, const T* __restrict__ A, int64_t lda,
    int64_t sa, const T* __restrict__ B, int64_t ldb, int64_t sb, float beta,
    TC* __restrict__ C, int64_t ldc, int64_t sc,
    const float* __restrict__ bias, float* __restrict__ bsum) {
  const int64_t bz = blockIdx.z;
  v3_tile<T, TC, TA, TB, WGM, WGN, SM, SN, OCC, BSUM>(
      M, N, K, alpha, A + bz * sa, lda, B + bz * sb, ldb, beta, C + bz * sc, ldc, bias,
      BSUM ? bsum + bz * N : nullptr, nullptr, 0, false);
}

// k_gemm_v3 (one batch entry) with a fused epilogue operand X (EPI_* above).
// (alpha stays a run-time argument, 1 in every call, so the stored product is formed by
// the same instructions as k_gemm_v3's: a constant 1 would let the compiler replace
// the single-rounding fp32->fp16 multiply-add of alpha*acc + bias by an add and a
// conversion, which round twice)
template <typename T, bool TA, bool TB, int WGM, int WGN, int SM, int SN, int OCC, int EPI>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void k_gemm_v3e(
    int64_t M, int64_t N, int64_t K, float alpha, const T* __restrict__ A, int64_t lda,
    const T* __restrict__ B, int64_t ldb, float beta, T* __restrict__ C, int64_t ldc,
    const float* __restrict__ bias, T* __restrict__ X, int64_t ldx) {
  v3_tile<T, T, TA, TB, WGM, WGN, SM, SN, OCC, false, EPI>(
      M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias, nullptr, nullptr, 0, false, X, ldx);
}

// A group of GEMMs C_g (+)= A_g^T B_g (weight gradients of several layers) with their
// own operands, a common M and K and each its own N and row strides of B_g and C_g,
// passed by value.  The members' output tiles form one list: member g owns
// tiles [tiles[g], tiles[g+1]), row-major over its tile grid.
constexpr int kGroupMax = 32;
template <typename T, typename TC>
struct V3Group {
  const T* A[kGroupMax];
  const T* B[kGroupMax];
  TC* C[kGroupMax];
  void* db[kGroupMax];  // null: no column sums for this member
  int64_t N[kGroupMax], ldb[kGroupMax], ldc[kGroupMax];
  float beta[kGroupMax];
  int tiles[kGroupMax + 1];
  int n;
  unsigned dbacc;       // bit g: add member g's column sums to db's contents
};

template <typename T, typename TC, int WGM, int WGN, int SM, int SN, bool BSUM>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void k_gemm_v3g(
    int64_t M, int64_t K, int64_t lda, const V3Group<T, TC> g, int dbt) {
  constexpr int TBN = WGN * SN * 32;
  // XCD-contiguous bands over the whole list (consecutive tiles share operand rows)
  const int T_ = g.tiles[g.n];
  int lin = (int)blockIdx.x;
  if (T_ % 8 == 0) lin = (lin % 8) * (T_ / 8) + lin / 8;
  int bz = 0;
  while (bz + 1 < g.n && g.tiles[bz + 1] <= lin) ++bz;
  const int loc = lin - g.tiles[bz];
  const int64_t N = g.N[bz], gx = (N + TBN - 1) / TBN;
  // (one v3_tile instance per kernel: each holds its own static LDS stages)
  v3_tile<T, TC, true, false, WGM, WGN, SM, SN, 1, BSUM, EPI_NONE, true>(
      M, N, K, 1.f, g.A[bz], lda, g.B[bz], g.ldb[bz], g.beta[bz], g.C[bz], g.ldc[bz], nullptr,
      nullptr,
      g.db[bz], dbt, (g.dbacc >> bz) & 1u, nullptr, 0, loc / gx, loc % gx);
}

// Block shapes of the DMA-staged kernel (waves of 64 x 64 of C): 4 x 2 waves
// (256 x 128, one block per CU, two waves per SIMD) when the problem has at least
// one such tile per CU, else 2 x 2 waves (128 x 128, two blocks per CU).

// Whether a 16-bit GEMM runs on the DMA-staged kernel (k_gemm_v3).
bool v3_ok(int elem, int ta, int tb, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
           int64_t sa, const void* B, int64_t ldb, int64_t sb) {
  const int VE = 16 / elem;
  const bool vec = tg_aligned16(A) && tg_aligned16(B) && lda % VE == 0 && ldb % VE == 0 &&
                   sa % VE == 0 && sb % VE == 0;
  // The DMA addresses each operand through a 2 GiB buffer window that starts at the
  // block's origin: a k-contiguous operand (A, or B given as [N, K]) spans at most 256
  // of its rows plus K elements from there, an m/n-contiguous one all K of its rows.
  const int64_t a_span = (ta ? K * lda : 256 * lda + K) * (int64_t)elem;
  const int64_t b_span = (tb ? 256 * ldb + K : K * ldb) * (int64_t)elem;
  return elem == 2 && vec && M >= 64 && N >= 64 && K >= 64 && M % 8 == 0 && N % 8 == 0 &&
         K % V3_BK == 0 && a_span < (int64_t{1} << 31) && b_span < (int64_t{1} << 31);
}

// bsum (non-null only where v3_ok holds, with ta = 1, tb = 0): also write the column
// sums of B over each batch entry's K range to bsum[batch][N].
template <typename T, typename TC>
int launch(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const void* A,
           int64_t lda, int64_t sa, const void* B, int64_t ldb, int64_t sb, float beta, void* C,
           int64_t ldc, int64_t sc, int64_t batch, hipStream_t s, const float* bias = nullptr,
           float* bsum = nullptr) {
  constexpr int VE = 16 / sizeof(T);
  const bool vec = tg_aligned16(A) && tg_aligned16(B) && lda % VE == 0 && ldb % VE == 0 &&
                   sa % VE == 0 && sb % VE == 0;
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)batch);
  const T* a = (const T*)A;
  const T* b = (const T*)B;
  TC* c = (TC*)C;
  // v2 stages whole 16-byte vectors along every contiguous dimension: extents must be
  // multiples of 8 so no vector straddles a row end.
  if (bsum && !(ta && !tb && v3_ok((int)sizeof(T), ta, tb, M, N, K, A, lda, sa, B, ldb, sb))) {
    tg_set_error("tg_gemm: fused column sums need the DMA-staged 16-bit kernel");
    return TG_ERR_UNSUPPORTED;
  }
  if constexpr (sizeof(T) == 2) {
  if (v3_ok((int)sizeof(T), ta, tb, M, N, K, A, lda, sa, B, ldb, sb)) {
    // Block shapes (waves x per-wave tile): 4x2 waves of 64x128 (256x256, one block
    // and two waves per SIMD) when the problem has enough such tiles to fill the CUs:
    // fewer global tile bytes per flop than the smaller shapes.  (The same tile as 2x2
    // waves of 128x128, one wave per SIMD, measured 3-8 % slower: nothing overlaps a
    // wave's LDS waits and barrier.)  Else 4x2 waves of 64x64 (256x128), else 2x2
    // waves of 64x64 (128x128, two blocks per CU).
    const int64_t ncu = tg_num_cus();
    const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256) * batch;
    const int64_t t128 = ((M + 255) / 256) * ((N + 127) / 128) * batch;
    const int shape = t256 >= kHugeTiles * ncu / 4 ? 2 : (t128 >= ncu ? 1 : 0);
#define TG_G3_SHAPE(TA_, TB_, WGM, WGN, SM, SN, OCC)                                       \
  do {                                                                                     \
    constexpr int TBM = WGM * SM * 32, TBN = WGN * SN * 32;                                \
    dim3 g3((unsigned)((N + TBN - 1) / TBN), (unsigned)((M + TBM - 1) / TBM), (unsigned)batch); \
    if constexpr (TA_ && !TB_) {                                                           \
      if (bsum) {                                                                          \
        k_gemm_v3<T, TC, TA_, TB_, WGM, WGN, SM, SN, OCC, true><<<g3, 64 * WGM * WGN, 0, s>>>( \
            M, N, K, alpha, a, lda, sa, b, ldb, sb, beta, c, ldc, sc, bias, bsum);          \
        break;                                                                             \
      }                                                                                    \
    }                                                                                      \
    k_gemm_v3<T, TC, TA_, TB_, WGM, WGN, SM, SN, OCC><<<g3, 64 * WGM * WGN, 0, s>>>(        \
        M, N, K, alpha, a, lda, sa, b, ldb, sb, beta, c, ldc, sc, bias, nullptr);           \
  } while (0)
#define TG_G3(TA_, TB_)                                          \
  do {                                                           \
    if (shape == 2) TG_G3_SHAPE(TA_, TB_, 4, 2, 2, 4, 1);        \
    else if (shape == 1) TG_G3_SHAPE(TA_, TB_, kBigWGM, kBigWGN, kBigSM, kBigSN, 1); \
    else TG_G3_SHAPE(TA_, TB_, 2, 2, 2, 2, 2);                   \
  } while (0)
    if (!ta && !tb) TG_G3(false, false);
    else if (!ta && tb) TG_G3(false, true);
    else if (ta && !tb) TG_G3(true, false);
    else TG_G3(true, true);
#undef TG_G3_SHAPE
#undef TG_G3
    return tg_check_launch("tg_gemm");
  }
  if (vec && M >= 128 && N >= 64 && K >= 64 && M % 8 == 0 && N % 8 == 0 && K % 8 == 0) {
    // BN = 128 unless that leaves fewer than two blocks per CU.
    const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
    const bool wide = tiles128 >= 2 * (int64_t)tg_num_cus() && N >= 128;
    const int bn = wide ? 128 : 64;
    dim3 g2((unsigned)((N + bn - 1) / bn), (unsigned)((M + V2_BM - 1) / V2_BM), (unsigned)batch);
#define TG_G2(TA_, TB_)                                                                        \
  do {                                                                                         \
    if (wide)                                                                                  \
      k_gemm_v2<T, TC, TA_, TB_, 128><<<g2, kThreads, 0, s>>>(M, N, K, alpha, a, lda, sa, b,    \
                                                              ldb, sb, beta, c, ldc, sc, bias); \
    else                                                                                       \
      k_gemm_v2<T, TC, TA_, TB_, 64><<<g2, kThreads, 0, s>>>(M, N, K, alpha, a, lda, sa, b, ldb, \
                                                             sb, beta, c, ldc, sc, bias);    \
  } while (0)
    if (!ta && !tb) TG_G2(false, false);
    else if (!ta && tb) TG_G2(false, true);
    else if (ta && !tb) TG_G2(true, false);
    else TG_G2(true, true);
#undef TG_G2
    return tg_check_launch("tg_gemm");
  }
  }
  if constexpr (sizeof(T) == 4) {
    // fewer 128 x 128 tiles than a quarter of the CUs: 32 x 32 tiles, K in four
    if ((int64_t)grid.x * grid.y * grid.z * 4 < (int64_t)tg_num_cus() && K >= 64) {
      dim3 gs((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32), (unsigned)batch);
#define TG_GS(TA_, TB_) \
  k_gemm_f32_small<TC, TA_, TB_><<<gs, kThreads, 0, s>>>(M, N, K, alpha, a, lda, sa, b, ldb, sb, beta, c, ldc, sc, bias)
      if (!ta && !tb) TG_GS(false, false);
      else if (!ta && tb) TG_GS(false, true);
      else if (ta && !tb) TG_GS(true, false);
      else TG_GS(true, true);
#undef TG_GS
      return tg_check_launch("tg_gemm");
    }
  }
#define TG_G(TA_, TB_, V_) \
  k_gemm<T, TC, TA_, TB_, V_><<<grid, kThreads, 0, s>>>(M, N, K, alpha, a, lda, sa, b, ldb, sb, beta, c, ldc, sc, bias)
  if (vec) {
    if (!ta && !tb) TG_G(false, false, true);
    else if (!ta && tb) TG_G(false, true, true);
    else if (ta && !tb) TG_G(true, false, true);
    else TG_G(true, true, true);
  } else {
    if (!ta && !tb) TG_G(false, false, false);
    else if (!ta && tb) TG_G(false, true, false);
    else if (ta && !tb) TG_G(true, false, false);
    else TG_G(true, true, false);
  }
#undef TG_G
  return tg_check_launch("tg_gemm");
}

// The fused-epilogue GEMMs on the DMA-staged kernel: GELU backward as C (+)= ...
// (A [M,K], op(B) = B^T with B [N,K]: a Linear layer's input gradient G W^T), GELU
// forward and residual as C = A B + bias (B [K,N]: a Linear layer's forward).  Other
// layouts or shapes return TG_ERR_UNSUPPORTED (the caller runs the separate kernels).
template <typename T>
int launch_epi(int epi, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
               const void* B, int64_t ldb, float beta, void* C, int64_t ldc, const float* bias,
               void* X, int64_t ldx, hipStream_t s) {
  const int tb = epi == EPI_GELU_BWD;
  const int VE = 16 / (int)sizeof(T);
  if (!v3_ok((int)sizeof(T), 0, tb, M, N, K, A, lda, 0, B, ldb, 0) || !tg_aligned16(C) ||
      !tg_aligned16(X) || ldc % VE || ldx % VE || (epi == EPI_GELU_BWD && bias)) {
    tg_set_error("tg_gemm_epilogue: shape or alignment outside the fused kernel");
    return TG_ERR_UNSUPPORTED;
  }
  const int64_t ncu = tg_num_cus();
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t t128 = ((M + 255) / 256) * ((N + 127) / 128);
  const int shape = t256 >= kHugeTiles * ncu / 4 ? 2 : (t128 >= ncu ? 1 : 0);
  const T* a = (const T*)A;
  const T* b = (const T*)B;
#define TG_GE(TB_, E, WGM, WGN, SM, SN, OCC)                                                   \
  do {                                                                                       \
    constexpr int TBM = WGM * SM * 32, TBN = WGN * SN * 32;                                  \
    dim3 g((unsigned)((N + TBN - 1) / TBN), (unsigned)((M + TBM - 1) / TBM), 1);             \
    k_gemm_v3e<T, false, TB_, WGM, WGN, SM, SN, OCC, E><<<g, 64 * WGM * WGN, 0, s>>>(          \
        M, N, K, 1.f, a, lda, b, ldb, beta, (T*)C, ldc, bias, (T*)X, ldx);                     \
  } while (0)
#define TG_GES(TB_, E)                                                          \
  do {                                                                          \
    if (shape == 2) TG_GE(TB_, E, 4, 2, 2, 4, 1);                              \
    else if (shape == 1) TG_GE(TB_, E, kBigWGM, kBigWGN, kBigSM, kBigSN, 1);  \
    else TG_GE(TB_, E, 2, 2, 2, 2, 2);                                         \
  } while (0)
  if (epi == EPI_GELU_BWD) TG_GES(true, EPI_GELU_BWD);
  else if (epi == EPI_GELU_FWD) TG_GES(false, EPI_GELU_FWD);
  else TG_GES(false, EPI_RESIDUAL);
#undef TG_GES
#undef TG_GE
  return tg_check_launch("tg_gemm_epilogue");
}

}  // namespace

namespace {
int gemm_dispatch(const char* who, int dtype_ab, int dtype_c, int trans_a, int trans_b,
                  int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
                  int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, float beta,
                  void* C, int64_t ldc, int64_t stride_c, int64_t batch, const float* bias,
                  void* stream) {
  TG_REQUIRE(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "%s: negative extent", who);
  if (M == 0 || N == 0 || batch == 0) return TG_OK;
  TG_REQUIRE(C, "%s: null C", who);
  TG_REQUIRE(ldc >= N, "%s: ldc %lld < N %lld", who, (long long)ldc, (long long)N);
  TG_REQUIRE(batch <= 65535, "%s: batch %lld exceeds 65535", who, (long long)batch);
  TG_REQUIRE((M + BM - 1) / BM <= 65535, "%s: M too large", who);
  hipStream_t s = tg_stream(stream);
  if (K == 0) {
    // C = beta*C (+ bias): no product term; reuse the kernel with K = 0 (acc stays zero).
  } else {
    TG_REQUIRE(A && B, "%s: null operand", who);
    TG_REQUIRE(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N), "%s: bad leading dim", who);
  }
  if (dtype_ab == TG_F64 && dtype_c == TG_F64) {
    TG_REQUIRE(!bias, "%s: fp64 takes no fused bias", who);
    TG_REQUIRE((M + 63) / 64 <= 65535, "%s: M too large", who);
    return tg64_gemm(trans_a, trans_b, M, N, K, (double)alpha, (const double*)A, lda, stride_a,
                     (const double*)B, ldb, stride_b, (double)beta, (double*)C, ldc, stride_c,
                     batch, nullptr, s);
  }
#define TG_GEMM_CALL(TA, TC)                                                                  \
  return launch<TA, TC>(trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, \
                        beta, C, ldc, stride_c, batch, s, bias)
  if (dtype_ab == TG_F16) {
    if (dtype_c == TG_F32) TG_GEMM_CALL(tg_half, float);
    if (dtype_c == TG_F16) TG_GEMM_CALL(tg_half, tg_half);
  } else if (dtype_ab == TG_BF16) {
    if (dtype_c == TG_F32) TG_GEMM_CALL(tg_bf16, float);
    if (dtype_c == TG_BF16) TG_GEMM_CALL(tg_bf16, tg_bf16);
  } else if (dtype_ab == TG_F32 && dtype_c == TG_F32) {
    TG_GEMM_CALL(float, float);
  }
#undef TG_GEMM_CALL
  tg_set_error("%s: unsupported dtype combination ab=%d c=%d", who, dtype_ab, dtype_c);
  return TG_ERR_UNSUPPORTED;
}
}  // namespace

namespace {
// Finishing pass of the weight-gradient entry: dW[i] (+)= sum_s parts[s][i] over the
// M*N elements (when K was split), then db[c] (+)= sum_s bparts[s][c].  A thread owns 4
// adjacent elements and adds the S partials in order with 4 rows of loads in flight,
// so the result does not depend on scheduling.
constexpr int kFinBlock = 256;

template <typename TO>
__device__ __forceinline__ void fin_store(void* out, int64_t i, const float a[4], int acc) {
  TO* o = reinterpret_cast<TO*>(out) + i;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = a[j];
    if (acc) v += tg_to_float(o[j]);
    o[j] = tg_from_float<TO>(v);
  }
}

__global__ __launch_bounds__(kFinBlock) void k_wgrad_finish(
    const float* __restrict__ parts, int S, int64_t MN, void* dW, int dtw, int accw,
    const float* __restrict__ bparts, int64_t N, void* db, int dtb, int accb) {
  const int64_t q = (int64_t)blockIdx.x * kFinBlock + threadIdx.x;
  const int64_t qw = MN / 4;
  const float* in;
  int64_t stride, i;
  void* out;
  int dt, acc;
  if (q < qw) {
    in = parts, stride = MN, i = q * 4, out = dW, dt = dtw, acc = accw;
  } else {
    i = (q - qw) * 4;
    if (db == nullptr || i >= N) return;
    in = bparts, stride = N, out = db, dt = dtb, acc = accb;
  }
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  int r = 0;
  for (; r + 4 <= S; r += 4) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4*>(in + (r + u) * stride + i);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[0] += v[u].x;
      a[1] += v[u].y;
      a[2] += v[u].z;
      a[3] += v[u].w;
    }
  }
  for (; r < S; ++r) {
    const float4 v = *reinterpret_cast<const float4*>(in + r * stride + i);
    a[0] += v.x;
    a[1] += v.y;
    a[2] += v.z;
    a[3] += v.w;
  }
  if (dt == TG_F32) fin_store<float>(out, i, a, acc);
  else if (dt == TG_F16) fin_store<tg_half>(out, i, a, acc);
  else fin_store<tg_bf16>(out, i, a, acc);
}

// K split of a weight gradient whose output has too few 128x128 tiles for two per CU
// (qkv/out projections [1024, 1024] and FC weights [1024, 4096] over 8192 tokens), or
// whose K is very long: returns s with K % s == 0 and (K / s) % 64 == 0, or 1.
int64_t wgrad_split(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N % 4 != 0) return 1;  // the finish reads 4-element groups
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  const int64_t cus = tg_num_cus();
  int64_t want;
  if (K >= 16384 && tiles < 4 * cus) want = 2;
  else if (tiles >= 2 * cus || K < 2048) return 1;
  else want = std::min((2 * cus + tiles - 1) / tiles, K / 1024);
  for (int64_t s = want; s > 1; --s)
    if (K % s == 0 && (K / s) % 64 == 0) return s;
  return 1;
}

size_t al256(size_t n) { return (n + 255) & ~size_t{255}; }

struct WgradPlan {
  int64_t split;
  size_t parts, bparts, red;  // byte offsets-to-be: sizes of the three workspace regions
};

WgradPlan wgrad_plan(int dtype_ab, int64_t M, int64_t N, int64_t K, bool has_b) {
  WgradPlan p{1, 0, 0, 0};
  if (dtype_ab != TG_F64) p.split = wgrad_split(M, N, K);
  if (p.split > 1) p.parts = al256((size_t)(p.split * M * N) * sizeof(float));
  if (has_b) {
    p.bparts = al256((size_t)(p.split * N) * sizeof(float));
    p.red = al256(tg_reduce_rows_workspace(K, N));
  }
  return p;
}
}  // namespace

TG_EXPORT size_t tg_gemm_wgrad_workspace(int dtype_ab, int64_t M, int64_t N, int64_t K,
                                         int with_bias) {
  if (N <= 0 || M < 0 || K < 0) return 0;
  const WgradPlan p = wgrad_plan(dtype_ab, M, N, K, with_bias != 0);
  return p.parts + p.bparts + p.red;
}

TG_EXPORT int tg_gemm_wgrad(int dtype_ab, int64_t M, int64_t N, int64_t K, const void* X,
                            int64_t ldx, const void* G, int64_t ldg, int dtype_w, void* dW,
                            int64_t ldw, int acc_w, int dtype_b, void* db, int acc_b,
                            void* workspace, size_t workspace_bytes, void* stream) {
  TG_REQUIRE(M >= 0 && N >= 0 && K >= 0, "tg_gemm_wgrad: negative extent");
  if (M == 0 || N == 0) {
    if (N == 0 || db == nullptr) return TG_OK;
    // no weight, only the bias gradient
    return tg_reduce_rows(dtype_ab, G, dtype_b, db, K, N, acc_b, workspace, workspace_bytes,
                          stream);
  }
  TG_REQUIRE(dW, "tg_gemm_wgrad: null dW");
  TG_REQUIRE(ldw >= N && ldx >= M && ldg >= N, "tg_gemm_wgrad: bad leading dimension");
  TG_REQUIRE(dtype_w == TG_F32 || dtype_w == dtype_ab, "tg_gemm_wgrad: dW dtype %d", dtype_w);
  TG_REQUIRE(!db || dtype_b == TG_F32 || dtype_b == dtype_ab, "tg_gemm_wgrad: db dtype %d",
             dtype_b);
  TG_REQUIRE(dtype_ab != TG_F64 || (dtype_w == TG_F64 && (!db || dtype_b == TG_F64)),
             "tg_gemm_wgrad: fp64 operands take fp64 gradients");
  if (K > 0) TG_REQUIRE(X && G, "tg_gemm_wgrad: null operand");
  WgradPlan p = wgrad_plan(dtype_ab, M, N, K, db != nullptr);
  if (ldw != N) p.split = 1;  // the split finish writes a dense dW
  TG_REQUIRE(workspace_bytes >= p.parts + p.bparts + p.red && (workspace || !p.parts),
             "tg_gemm_wgrad: workspace of %zu bytes, need %zu", workspace_bytes,
             p.parts + p.bparts + p.red);
  char* ws = static_cast<char*>(workspace);
  float* parts = reinterpret_cast<float*>(ws);
  float* bparts = reinterpret_cast<float*>(ws + p.parts);
  void* red = ws + p.parts + p.bparts;
  hipStream_t s = tg_stream(stream);
  const int64_t S = p.split, kc = K / S;
  const float bw = acc_w ? 1.f : 0.f;
  const bool fused = db && K > 0 && (dtype_ab == TG_F16 || dtype_ab == TG_BF16) &&
                     v3_ok(2, 1, 0, M, N, kc, X, ldx, kc * ldx, G, ldg, kc * ldg);
  int rc;
  if (fused) {
#define TG_WG(T)                                                                              \
  if (S > 1)                                                                                  \
    rc = launch<T, float>(1, 0, M, N, kc, 1.f, X, ldx, kc * ldx, G, ldg, kc * ldg, 0.f, parts, \
                          N, M * N, S, s, nullptr, bparts);                                   \
  else if (dtype_w == TG_F32)                                                                 \
    rc = launch<T, float>(1, 0, M, N, K, 1.f, X, ldx, 0, G, ldg, 0, bw, dW, ldw, 0, 1, s,       \
                          nullptr, bparts);                                                   \
  else                                                                                        \
    rc = launch<T, T>(1, 0, M, N, K, 1.f, X, ldx, 0, G, ldg, 0, bw, dW, ldw, 0, 1, s, nullptr, \
                      bparts)
    if (dtype_ab == TG_F16) { TG_WG(tg_half); } else { TG_WG(tg_bf16); }
#undef TG_WG
    if (rc != TG_OK) return rc;
  } else if (S > 1) {
    rc = gemm_dispatch("tg_gemm_wgrad", dtype_ab, TG_F32, 1, 0, M, N, kc, 1.f, X, ldx, kc * ldx,
                       G, ldg, kc * ldg, 0.f, parts, N, M * N, S, nullptr, stream);
    if (rc != TG_OK) return rc;
  } else {
    rc = gemm_dispatch("tg_gemm_wgrad", dtype_ab, dtype_w, 1, 0, M, N, K, 1.f, X, ldx, 0, G, ldg,
                       0, bw, dW, ldw, 0, 1, nullptr, stream);
    if (rc != TG_OK) return rc;
  }
  const int64_t MN = S > 1 ? M * N : 0;
  const int64_t nb = fused ? N : 0;
  if (MN + nb > 0) {
    const int64_t groups = (MN + nb) / 4;
    k_wgrad_finish<<<(unsigned)((groups + kFinBlock - 1) / kFinBlock), kFinBlock, 0, s>>>(
        parts, (int)S, MN, dW, dtype_w, acc_w, bparts, N, fused ? db : nullptr, dtype_b, acc_b);
    rc = tg_check_launch("tg_gemm_wgrad");
    if (rc != TG_OK) return rc;
  }
  if (db && !fused)
    return tg_reduce_rows(dtype_ab, G, dtype_b, db, K, N, acc_b, red, p.red, stream);
  return TG_OK;
}

namespace {
// One launch of k_gemm_v3g over members idx[0..n) (n <= kGroupMax, every member passing
// v3_ok): 256x256 blocks (shape 2) or 256x128 blocks (shape 1), whole K per block.
template <typename T, typename TC>
int wgrad_group_launch(int shape, const int* idx, int n, int64_t M, const int64_t* N,
                       int64_t K, const void* const* X, int64_t ldx, const void* const* G,
                       const int64_t* ldg, void* const* dW, const int64_t* ldw,
                       const int* acc_w, int dtype_b, void* const* db, const int* acc_b,
                       hipStream_t s) {
  V3Group<T, TC> grp{};
  bool any_b = false;
  grp.n = n;
  const int tbn = shape == 2 ? 2 * 4 * 32 : kBigWGN * kBigSN * 32;
  const int tbm = shape == 2 ? 4 * 2 * 32 : kBigWGM * kBigSM * 32;
  const int64_t gy = (M + tbm - 1) / tbm;
  for (int i = 0; i < n; ++i) {
    const int m = idx[i];
    grp.A[i] = static_cast<const T*>(X[m]);
    grp.B[i] = static_cast<const T*>(G[m]);
    grp.C[i] = static_cast<TC*>(dW[m]);
    grp.N[i] = N[m];
    grp.ldb[i] = ldg[m];
    grp.ldc[i] = ldw[m];
    grp.beta[i] = acc_w && acc_w[m] ? 1.f : 0.f;
    grp.db[i] = db ? db[m] : nullptr;
    grp.tiles[i + 1] = grp.tiles[i] + (int)(gy * ((N[m] + tbn - 1) / tbn));
    if (grp.db[i]) {
      any_b = true;
      if (acc_b && acc_b[m]) grp.dbacc |= 1u << i;
    }
  }
#define TG_GG(WGM, WGN, SM, SN)                                                                \
  do {                                                                                         \
    static_assert(WGM * SM * 32 > 0 && WGN * SN * 32 > 0, "tile");                            \
    dim3 g3((unsigned)grp.tiles[n]);                                                           \
    if (any_b)                                                                                 \
      k_gemm_v3g<T, TC, WGM, WGN, SM, SN, true><<<g3, 64 * WGM * WGN, 0, s>>>(M, K, ldx, grp,   \
                                                                            dtype_b);          \
    else                                                                                       \
      k_gemm_v3g<T, TC, WGM, WGN, SM, SN, false><<<g3, 64 * WGM * WGN, 0, s>>>(M, K, ldx, grp,  \
                                                                             dtype_b);         \
  } while (0)
  if (shape == 2) TG_GG(4, 2, 2, 4);
  else TG_GG(kBigWGM, kBigWGN, kBigSM, kBigSN);
#undef TG_GG
  return tg_check_launch("tg_gemm_wgrad_group");
}

size_t wgrad_group_ws(int dtype_ab, int n, int64_t M, const int64_t* N, int64_t K,
                      int with_bias) {
  // members that cannot be grouped run one by one through tg_gemm_wgrad, in stream
  // order over the same workspace
  size_t w = 0;
  for (int i = 0; i < n; ++i) w = std::max(w, tg_gemm_wgrad_workspace(dtype_ab, M, N[i], K, with_bias));
  return w;
}

int wgrad_group_impl(const char* who, int dtype_ab, int n, int64_t M, const int64_t* N,
                     int64_t K, const void* const* X, int64_t ldx, const void* const* G,
                     const int64_t* ldg, int dtype_w, void* const* dW, const int64_t* ldw,
                     const int* acc_w, int dtype_b, void* const* db, const int* acc_b,
                     void* workspace, size_t workspace_bytes, void* stream) {
  TG_REQUIRE(n >= 0 && M >= 0 && K >= 0, "%s: negative extent", who);
  if (n == 0) return TG_OK;
  TG_REQUIRE(X && G && dW && N && ldg && ldw, "%s: null pointer array", who);
  bool with_b = false;
  for (int i = 0; i < n; ++i) {
    TG_REQUIRE(N[i] >= 0, "%s: negative extent", who);
    with_b = with_b || (db && db[i] != nullptr);
  }
  const size_t need = wgrad_group_ws(dtype_ab, n, M, N, K, with_b);
  TG_REQUIRE(workspace_bytes >= need, "%s: workspace of %zu bytes, need %zu", who,
             workspace_bytes, need);
  hipStream_t s = tg_stream(stream);
  const int64_t ncu = tg_num_cus();
  const bool lowp = dtype_ab == TG_F16 || dtype_ab == TG_BF16;
  const bool kinds = lowp && M > 0 && K > 0 && (dtype_w == TG_F32 || dtype_w == dtype_ab) &&
                     (!with_b || dtype_b == TG_F32 || dtype_b == dtype_ab);
  // members the grouped kernel takes, in order; the rest run one by one
  int ok[kGroupMax];
  int g0 = 0;
  std::vector<char> done(n, 0);
  while (kinds && g0 < n) {
    int cnt = 0;
    int64_t t256 = 0, t128 = 0;
    int g = g0;
    for (; g < n && cnt < kGroupMax; ++g) {
      if (!(dW[g] && N[g] > 0 && ldw[g] >= N[g] &&
            v3_ok(2, 1, 0, M, N[g], K, X[g], ldx, 0, G[g], ldg[g], 0)))
        continue;
      ok[cnt++] = g;
      t256 += ((M + 255) / 256) * ((N[g] + 255) / 256);
      t128 += ((M + 255) / 256) * ((N[g] + 127) / 128);
    }
    g0 = g;
    // whole-K blocks only where the members' tiles fill the CUs; else the K split
    const int shape = t256 >= kHugeTiles * ncu / 4 ? 2 : (t128 >= ncu ? 1 : 0);
    if (cnt == 0 || shape == 0 || t128 > INT32_MAX) continue;
    int rc;
#define TG_WGG(T, TC)                                                                     \
  rc = wgrad_group_launch<T, TC>(shape, ok, cnt, M, N, K, X, ldx, G, ldg, dW, ldw, acc_w, \
                                 dtype_b, with_b ? db : nullptr, acc_b, s)
    if (dtype_ab == TG_F16) {
      if (dtype_w == TG_F32) TG_WGG(tg_half, float); else TG_WGG(tg_half, tg_half);
    } else {
      if (dtype_w == TG_F32) TG_WGG(tg_bf16, float); else TG_WGG(tg_bf16, tg_bf16);
    }
#undef TG_WGG
    if (rc != TG_OK) return rc;
    for (int i = 0; i < cnt; ++i) done[ok[i]] = 1;
  }
  for (int g = 0; g < n; ++g) {
    if (done[g]) continue;
    const int rc = tg_gemm_wgrad(dtype_ab, M, N[g], K, X[g], ldx, G[g], ldg[g], dtype_w, dW[g],
                                 ldw[g], acc_w ? acc_w[g] : 0, dtype_b, db ? db[g] : nullptr,
                                 acc_b ? acc_b[g] : 0, workspace, workspace_bytes, stream);
    if (rc != TG_OK) return rc;
  }
  return TG_OK;
}
}  // namespace

TG_EXPORT size_t tg_gemm_wgrad_group_workspace(int dtype_ab, int n, int64_t M, int64_t N,
                                               int64_t K, int with_bias) {
  return n > 0 ? tg_gemm_wgrad_workspace(dtype_ab, M, N, K, with_bias) : 0;
}

TG_EXPORT int tg_gemm_wgrad_group(int dtype_ab, int n, int64_t M, int64_t N, int64_t K,
                                  const void* const* X, int64_t ldx, const void* const* G,
                                  int64_t ldg, int dtype_w, void* const* dW, int64_t ldw,
                                  const int* acc_w, int dtype_b, void* const* db,
                                  const int* acc_b, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  TG_REQUIRE(n >= 0, "tg_gemm_wgrad_group: negative extent");
  const std::vector<int64_t> Ns(n, N), lg(n, ldg), lw(n, ldw);
  return wgrad_group_impl("tg_gemm_wgrad_group", dtype_ab, n, M, Ns.data(), K, X, ldx, G,
                          lg.data(), dtype_w, dW, lw.data(), acc_w, dtype_b, db, acc_b,
                          workspace, workspace_bytes, stream);
}

TG_EXPORT size_t tg_gemm_wgrad_group_n_workspace(int dtype_ab, int n, int64_t M,
                                                 const int64_t* N, int64_t K, int with_bias) {
  return n > 0 && N ? wgrad_group_ws(dtype_ab, n, M, N, K, with_bias) : 0;
}

TG_EXPORT int tg_gemm_wgrad_group_n(int dtype_ab, int n, int64_t M, const int64_t* N, int64_t K,
                                    const void* const* X, int64_t ldx, const void* const* G,
                                    const int64_t* ldg, int dtype_w, void* const* dW,
                                    const int64_t* ldw, const int* acc_w, int dtype_b,
                                    void* const* db, const int* acc_b, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  return wgrad_group_impl("tg_gemm_wgrad_group_n", dtype_ab, n, M, N, K, X, ldx, G, ldg,
                          dtype_w, dW, ldw, acc_w, dtype_b, db, acc_b, workspace,
                          workspace_bytes, stream);
}

TG_EXPORT int tg_gemm(int dtype_ab, int dtype_c, int trans_a, int trans_b, int64_t M, int64_t N,
                      int64_t K, float alpha, const void* A, int64_t lda, int64_t stride_a,
                      const void* B, int64_t ldb, int64_t stride_b, float beta, void* C,
                      int64_t ldc, int64_t stride_c, int64_t batch, void* stream) {
  return gemm_dispatch("tg_gemm", dtype_ab, dtype_c, trans_a, trans_b, M, N, K, alpha, A, lda,
                       stride_a, B, ldb, stride_b, beta, C, ldc, stride_c, batch, nullptr, stream);
}

TG_EXPORT int tg_gemm_bias(int dtype_ab, int dtype_c, int trans_a, int trans_b, int64_t M,
                           int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
                           const void* B, int64_t ldb, const float* bias, void* C, int64_t ldc,
                           void* stream) {
  TG_REQUIRE(bias, "tg_gemm_bias: null bias");
  return gemm_dispatch("tg_gemm_bias", dtype_ab, dtype_c, trans_a, trans_b, M, N, K, alpha, A,
                       lda, 0, B, ldb, 0, 0.f, C, ldc, 0, 1, bias, stream);
}

TG_EXPORT int tg_gemm_epilogue(int dtype, int epi, int64_t M, int64_t N, int64_t K,
                               const void* A, int64_t lda, const void* B, int64_t ldb,
                               const float* bias, void* X, int64_t ldx, float beta, void* C,
                               int64_t ldc, void* stream) {
  TG_REQUIRE(M >= 0 && N >= 0 && K >= 0, "tg_gemm_epilogue: negative extent");
  TG_REQUIRE(epi >= EPI_GELU_BWD && epi <= EPI_RESIDUAL, "tg_gemm_epilogue: unknown epilogue %d",
             epi);
  if (M == 0 || N == 0) return TG_OK;
  TG_REQUIRE(A && B && C && X, "tg_gemm_epilogue: null pointer");
  TG_REQUIRE(ldc >= N && ldx >= N, "tg_gemm_epilogue: ldc / ldx below N");
  TG_REQUIRE(epi == EPI_GELU_BWD || beta == 0.f, "tg_gemm_epilogue: beta only with GELU bwd");
  hipStream_t s = tg_stream(stream);
  if (dtype == TG_F16)
    return launch_epi<tg_half>(epi, M, N, K, A, lda, B, ldb, beta, C, ldc, bias, X, ldx, s);
  if (dtype == TG_BF16)
    return launch_epi<tg_bf16>(epi, M, N, K, A, lda, B, ldb, beta, C, ldc, bias, X, ldx, s);
  tg_set_error("tg_gemm_epilogue: dtype %d has no fused kernel (fp16 / bf16 only)", dtype);
  return TG_ERR_UNSUPPORTED;
}
