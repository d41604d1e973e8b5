// MFMA / VALU co-issue probe (gfx950). Not part of the library: a standalone
// program that answers whether the matrix cores keep running while vector
// ALU work is issued on the same SIMD, by the same wave or by the other wave
// of the SIMD. One 8-wave workgroup per CU (waves w and w + 4 share a SIMD,
// wave_simd_probe.hip), 2000 iterations per launch:
//   mode 0  all 8 waves: 32 independent v_mfma_f32_32x32x16_bf16 per iteration
//   mode 5  waves 0-3 only: the same MFMAs, waves 4-7 idle
//   mode 1  all 8 waves: 128 dependent-chain v_fma per iteration (8 chains)
//   mode 2  waves 0-3 MFMAs, waves 4-7 the VALU work (same SIMDs)
//   mode 3  all 8 waves: 32 MFMAs with 4 VALU ops after each
//   mode 4  waves 0-3 MFMAs, waves 4-7 32 v_exp_f32 + 32 v_fma
// If mode 2 and mode 4 take about as long as mode 5, a SIMD overlaps one
// wave's MFMAs with the other wave's vector work.
//
// Build and run (repository root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       enzyme_amd/probes/coissue_probe.hip -o enzyme_amd/probes/_build/coissue_probe
//   enzyme_amd/probes/_build/coissue_probe
#include <hip/hip_runtime.h>
#include <cstdio>
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
template <int MODE>
__global__ __launch_bounds__(512) void probe(float* out, int iters) {
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) { a[i] = (__bf16)(0.001f * (tid + i)); b[i] = (__bf16)(0.002f * (tid - i)); }
  floatx16 acc[4];
  for (int c = 0; c < 4; ++c) for (int e = 0; e < 16; ++e) acc[c][e] = 0.f;
  float x[8];
  for (int c = 0; c < 8; ++c) x[c] = 0.01f * (tid + c);
  const float k1 = 0.999f, k2 = 0.001f;
  const bool do_mfma = MODE == 0 || MODE == 3 || ((MODE == 2 || MODE == 4 || MODE == 5) && wave < 4);
  const bool do_valu = MODE == 1 || MODE == 3 || (MODE == 2 && wave >= 4);
  const bool do_exp = MODE == 4 && wave >= 4;
  for (int it = 0; it < iters; ++it) {
    if (do_mfma && !do_valu) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    } else if (do_valu && !do_mfma) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) x[c] = fmaf(x[c], k1, k2);
    } else if (do_valu && do_mfma) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
#pragma unroll
          for (int q = 0; q < 4; ++q) x[(c * 2 + q) & 7] = fmaf(x[(c * 2 + q) & 7], k1, k2);
        }
    } else if (do_exp) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) x[c] = __builtin_amdgcn_exp2f(fmaf(x[c], k1, -k2));
    }
  }
  float s = 0.f;
  for (int c = 0; c < 4; ++c) for (int e = 0; e < 16; ++e) s += acc[c][e];
  for (int c = 0; c < 8; ++c) s += x[c];
  out[blockIdx.x * 512 + tid] = s;
}
template <int MODE>
void run(float* d, int iters, const char* what) {
  for (int w = 0; w < 3; ++w) hipLaunchKernelGGL(probe<MODE>, dim3(256), dim3(512), 0, 0, d, iters);
  hipEvent_t a, b;
  hipEventCreate(&a); hipEventCreate(&b);
  hipEventRecord(a);
  for (int w = 0; w < 5; ++w) hipLaunchKernelGGL(probe<MODE>, dim3(256), dim3(512), 0, 0, d, iters);
  hipEventRecord(b);
  hipEventSynchronize(b);
  float ms = 0.f;
  hipEventElapsedTime(&ms, a, b);
  printf("mode %d %-48s %8.1f us/launch\n", MODE, what, ms * 1e3 / 5);
}
int main() {
  float* d;
  if (hipMalloc(&d, 256 * 512 * 4) != hipSuccess) return 1;
  const int iters = 2000;
  run<0>(d, iters, "all 8 waves: 32 MFMA/iter");
  run<5>(d, iters, "waves 0-3: 32 MFMA/iter, 4-7 idle");
  run<1>(d, iters, "all 8 waves: 128 VALU fma/iter");
  run<2>(d, iters, "waves 0-3 MFMA, waves 4-7 VALU (same SIMDs)");
  run<3>(d, iters, "all 8 waves: 32 MFMA + 128 VALU interleaved");
  run<4>(d, iters, "waves 0-3 MFMA, waves 4-7 32 exp2+32 fma/iter");
  if (hipDeviceSynchronize() != hipSuccess) return 2;
  return 0;
}
