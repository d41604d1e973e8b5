// Wave-to-SIMD placement probe (gfx950). Not part of the library: launches
// 16 workgroups of 8 waves and prints each wave's HW_ID fields (SIMD, wave
// slot, CU, shader engine), read with s_getreg_b32. The attention kernels
// pair waves w and w + 4 on one SIMD; this shows the hardware places them so.
//
// Build and run (repository root):
//   hipcc --offload-arch=gfx950 -O3 enzyme_amd/probes/wave_simd_probe.hip \
//       -o enzyme_amd/probes/_build/wave_simd_probe
//   enzyme_amd/probes/_build/wave_simd_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
__global__ __launch_bounds__(512) void hwid(unsigned* out) {
  const unsigned v = __builtin_amdgcn_s_getreg(4 | (31 << 11));
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * 8 + (threadIdx.x >> 6)] = v;
}
int main() {
  const int blocks = 16;
  unsigned* d;
  if (hipMalloc(&d, blocks * 8 * 4) != hipSuccess) return 1;
  hipLaunchKernelGGL(hwid, dim3(blocks), dim3(512), 0, 0, d);
  if (hipDeviceSynchronize() != hipSuccess) return 2;
  std::vector<unsigned> h(blocks * 8);
  if (hipMemcpy(h.data(), d, h.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return 3;
  for (int b = 0; b < blocks; ++b) {
    printf("block %2d:", b);
    for (int w = 0; w < 8; ++w) {
      unsigned v = h[b * 8 + w];
      printf("  w%d simd%u wid%u cu%u se%u", w, (v >> 4) & 3, v & 15, (v >> 8) & 15, (v >> 13) & 7);
    }
    printf("\n");
  }
  return 0;
}
