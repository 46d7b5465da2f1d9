// LDS read bandwidth of one gfx950 compute unit, for the prefill kernel's
// ceiling: the MFMA phase reads every K and V^T fragment from LDS (1 KB per
// 32x32x16 MFMA), so at full MFMA rate a CU needs 4 KB per 32 cycles.
// Every lane reads 16 B (ds_read_b128) or 8 B (ds_read_b64_tr_b16) per
// instruction from a 64 KB static LDS array (conflict-free: lane * 16
// within a 1 KB row), 8 waves per CU, all accesses in bounds.
//
// Build and run (from the repository root, on the GPU machine):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature \
//     -Xclang -packed-fp32-ops -I tm-opt_amd/csrc \
//     tm-opt_amd/probes/lds_read_bw.hip -o /tmp/lds_read_bw && /tmp/lds_read_bw
// B/clk/CU is reported against the maximum engine clock (a lower running
// clock makes the true figure higher).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include "common.h"
using namespace tmopt;
constexpr int ITERS = 4096;
template <int MODE>
__global__ __launch_bounds__(256) void k(uint32_t* out) {
  __shared__ __attribute__((aligned(16))) char lds[65536];
  const int t = threadIdx.x;
  for (int i = t; i < 65536 / 4; i += 256) reinterpret_cast<uint32_t*>(lds)[i] = i * 2654435761u;
  __syncthreads();
  const uint32_t base = (uint32_t)(uintptr_t)lds;
  const int lane = t & 63, w = t >> 6;
  uint32_t acc = 0;
  for (int it = 0; it < ITERS; ++it) {
    const uint32_t row = ((it * 4 + w) & 63) * 1024;   // 64 rows of 1 KB
    if constexpr (MODE == 0) {
      u32x4 x = __builtin_bit_cast(u32x4, lds_ld128(base + row + lane * 16));
      acc ^= x[0] ^ x[1] ^ x[2] ^ x[3];
    } else {
      auto x = __builtin_bit_cast(uint2, lds_tr16(base + row + lane * 8));
      acc ^= x.x ^ x.y;
    }
  }
  out[blockIdx.x * 256 + t] = acc;
}
int main() {
  int ncu; hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0);
  int clk; hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, 0);
  const int blocks = ncu * 2;   // 2 blocks (8 waves) per CU
  uint32_t* out; hipMalloc(&out, blocks * 256 * 4);
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  for (int mode = 0; mode < 2; ++mode) {
    for (int rep = 0; rep < 3; ++rep) {
      hipEventRecord(e0);
      if (mode == 0) hipLaunchKernelGGL(k<0>, dim3(blocks), dim3(256), 0, 0, out);
      else hipLaunchKernelGGL(k<1>, dim3(blocks), dim3(256), 0, 0, out);
      hipEventRecord(e1); hipEventSynchronize(e1);
      float ms; hipEventElapsedTime(&ms, e0, e1);
      const double bytes = (double)blocks * 256 * ITERS * (mode == 0 ? 16 : 8);
      printf("%s rep %d: %.3f ms  %.1f TB/s total  %.1f B/clk/CU at %.2f GHz (max clock)\n",
             mode == 0 ? "ds_read_b128      " : "ds_read_b64_tr_b16", rep, ms,
             bytes / (ms * 1e-3) / 1e12, bytes / (ms * 1e-3) / ncu / (clk * 1e3), clk / 1e6);
    }
  }
  printf("CUs %d\n", ncu);
  return hipGetLastError() != hipSuccess;
}
