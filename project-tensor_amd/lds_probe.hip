// LDS read-rate probe for gfx950 (measurement tooling, not part of libtgbwd).  One
// workgroup per CU fills 64 KiB of LDS, then every wave reads it in a loop with
// conflict-free lane-contiguous addresses (eight reads in flight per wave) and XORs the
// data into registers.  Prints the sustained read rate per CU for ds_read_b128,
// ds_read_b64, ds_read_b64_tr_b16 and ds_read_b32 at 1, 2 and 4 waves per SIMD.
//   hipcc --offload-arch=gfx950 -O3 lds_probe.hip -o lds_probe && ./lds_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
typedef short v4i16 __attribute__((ext_vector_type(4)));
#define LDSP __attribute__((address_space(3)))

template <int KIND>
__global__ void k_lds(int iters, unsigned* out) {
  __shared__ __attribute__((aligned(1024))) char buf[65536];
  for (int i = threadIdx.x; i < 65536 / 4; i += blockDim.x) ((unsigned*)buf)[i] = i * 2654435761u;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned acc0 = 0, acc1 = 0, acc2 = 0, acc3 = 0;
  int base = (wave * 4096) & 0xffff;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int off = (base + u * 1024 + it * 64) & 0xfc00;  // 1 KiB-aligned block
      if (KIND == 0) {  // ds_read_b128, 1 KiB per wave instruction
        const uint4 v = *reinterpret_cast<const uint4*>(buf + off + lane * 16);
        acc0 ^= v.x; acc1 ^= v.y; acc2 ^= v.z; acc3 ^= v.w;
      } else if (KIND == 1) {  // ds_read_b64, 512 B
        const uint2 v = *reinterpret_cast<const uint2*>(buf + off + lane * 8);
        acc0 ^= v.x; acc1 ^= v.y;
      } else if (KIND == 2) {  // ds_read_b64_tr_b16, 512 B
        const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDSP v4i16*)(buf + off + lane * 8));
        acc0 ^= (unsigned)(unsigned short)v[0] | ((unsigned)(unsigned short)v[1] << 16);
        acc1 ^= (unsigned)(unsigned short)v[2] | ((unsigned)(unsigned short)v[3] << 16);
      } else {  // ds_read_b32, 256 B
        const unsigned v = *reinterpret_cast<const unsigned*>(buf + off + lane * 4);
        acc0 ^= v;
      }
    }
  }
  if ((acc0 ^ acc1 ^ acc2 ^ acc3) == 0x12345678u) out[blockIdx.x] = 1;
}

int main() {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return 1;
  const int cus = prop.multiProcessorCount;
  unsigned* out;
  if (hipMalloc(&out, 1 << 20) != hipSuccess) return 1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
  const int iters = 4000;
  const char* names[4] = {"ds_read_b128", "ds_read_b64", "ds_read_b64_tr_b16", "ds_read_b32"};
  const int bytes[4] = {1024, 512, 512, 256};
  printf("CUs %d clock %d kHz\n", cus, prop.clockRate);
  for (int kind = 0; kind < 4; ++kind)
    for (int threads : {256, 512, 1024}) {
      float best = 1e30f;
      for (int rep = 0; rep < 3; ++rep) {
        hipEventRecord(a);
        if (kind == 0) k_lds<0><<<cus, threads>>>(iters, out);
        if (kind == 1) k_lds<1><<<cus, threads>>>(iters, out);
        if (kind == 2) k_lds<2><<<cus, threads>>>(iters, out);
        if (kind == 3) k_lds<3><<<cus, threads>>>(iters, out);
        hipEventRecord(b);
        hipEventSynchronize(b);
        float ms;
        hipEventElapsedTime(&ms, a, b);
        if (ms < best) best = ms;
      }
      if (hipGetLastError() != hipSuccess) return 1;
      const double total = (double)cus * (threads / 64) * iters * 8 * bytes[kind];
      printf("%-20s waves/CU %2d: %.3f ms  %.1f TB/s  %.1f B/clk/CU at 2.4 GHz\n", names[kind],
             threads / 64, best, total / best / 1e9, total / (best * 1e-3) / cus / 2.4e9);
    }
  return 0;
}
