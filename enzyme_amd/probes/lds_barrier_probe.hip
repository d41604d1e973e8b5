// LDS write and workgroup-barrier cost probe (gfx950). Not part of the
// library. One 8-wave workgroup per CU, 10000 rounds per launch; per round:
//   mode 0  s_waitcnt lgkmcnt(0) + s_barrier only
//   mode 1  4 x 16-byte LDS stores per thread (32 KiB per workgroup), wait, barrier
//   mode 2  16 x 4-byte LDS stores per thread (32 KiB), wait, barrier
//   mode 3  as mode 1 without the barrier
// Every store is conflict-free (consecutive threads, consecutive words).
// Reported: ns per round; 32 KiB / round time is the CU's LDS write rate.
//
// Build and run (repository root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       enzyme_amd/probes/lds_barrier_probe.hip -o enzyme_amd/probes/_build/lds_barrier_probe
//   enzyme_amd/probes/_build/lds_barrier_probe
#include <hip/hip_runtime.h>
#include <cstdio>
template <int MODE>
__global__ __launch_bounds__(512) void probe(float* out, int iters) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  float4 v = make_float4(tid, tid + 1, tid + 2, tid + 3);
  float* f = reinterpret_cast<float*>(smem);
  float4* f4 = reinterpret_cast<float4*>(smem);
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE == 1 || MODE == 3) {
#pragma unroll
      for (int i = 0; i < 4; ++i) f4[(it & 1) * 2048 + i * 512 + tid] = v;
    } else if constexpr (MODE == 2) {
#pragma unroll
      for (int i = 0; i < 16; ++i) f[(it & 1) * 8192 + i * 512 + tid] = v.x + i;
    }
    if constexpr (MODE == 3) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    v.x += 1.f;
  }
  out[blockIdx.x * 512 + tid] = v.x + f[tid];
}
template <int MODE>
void run(float* d, int iters, const char* what) {
  const size_t lds = 65536;
  hipFuncSetAttribute(reinterpret_cast<const void*>(probe<MODE>), hipFuncAttributeMaxDynamicSharedMemorySize, 65536);
  for (int w = 0; w < 3; ++w) hipLaunchKernelGGL(probe<MODE>, dim3(256), dim3(512), lds, 0, d, iters);
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  (void)hipEventRecord(a);
  for (int w = 0; w < 5; ++w) hipLaunchKernelGGL(probe<MODE>, dim3(256), dim3(512), lds, 0, d, iters);
  (void)hipEventRecord(b);
  (void)hipEventSynchronize(b);
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, a, b);
  printf("mode %d %-40s %8.2f us/launch  %7.1f ns/iter\n", MODE, what, ms * 1e3 / 5, ms * 1e6 / 5 / iters);
}
int main() {
  float* d;
  if (hipMalloc(&d, 256 * 512 * 4) != hipSuccess) return 1;
  const int iters = 10000;
  run<0>(d, iters, "barrier only");
  run<1>(d, iters, "4 x b128 LDS stores + wait + barrier");
  run<2>(d, iters, "16 x b32 LDS stores + wait + barrier");
  run<3>(d, iters, "4 x b128 LDS stores + wait, no barrier");
  if (hipDeviceSynchronize() != hipSuccess) return 2;
  return 0;
}
