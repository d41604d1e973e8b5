// LDS read throughput probe (gfx950). Not part of the library. One 8-wave
// workgroup per CU, each wave issuing 16 independent ds_read_b128 per
// iteration (20000 iterations), by address pattern:
//   0  linear: lane * 16 + i * 1024
//   1  attention K fragments: row pitch 272 B, (t*32 + lane%32) * 272 + st*32 + h*16
//   2  attention V^T fragments: row pitch 144 B, (dt*32 + lane%32) * 144 + t*64 + k2*32 + h*16
//   3  K fragments with a 256-B pitch and 16-byte chunks XOR-swizzled by row
// (h = lane / 32). Reported: bytes per clock per CU at 2.1 GHz.
//
// Build and run (repository root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       enzyme_amd/probes/lds_read_probe.hip -o enzyme_amd/probes/_build/lds_read_probe
//   enzyme_amd/probes/_build/lds_read_probe
#include <hip/hip_runtime.h>
#include <cstdio>
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <int PAT>
__global__ __launch_bounds__(512) void probe(unsigned* out, int iters) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, r = lane & 31;
  for (int i = tid; i < 65536 / 4; i += 512) reinterpret_cast<unsigned*>(smem)[i] = i;
  __syncthreads();
  u32x4 acc = {0, 0, 0, 0};
  unsigned off[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (PAT == 0) off[i] = lane * 16 + i * 1024;
    if (PAT == 1) { const int t = i >> 3, st = i & 7; off[i] = (t * 32 + r) * 272 + st * 32 + h * 16; }
    if (PAT == 2) { const int dt = i & 3, k2 = (i >> 2) & 1, t = i >> 3; off[i] = (dt * 32 + r) * 144 + t * 64 + k2 * 32 + h * 16; }
    if (PAT == 3) { const int t = i >> 3, st = i & 7, row = t * 32 + r; off[i] = row * 256 + (((st * 2 + h) ^ (row & 15)) * 16); }
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc ^= *reinterpret_cast<const u32x4*>(smem + off[i] + (it & 1) * 16384);
  }
  if (acc.x == 0x12345u) out[blockIdx.x * 512 + tid] = acc.y;
}
template <int PAT>
void run(unsigned* d, const char* what) {
  const int iters = 20000;
  hipFuncSetAttribute(reinterpret_cast<const void*>(probe<PAT>), hipFuncAttributeMaxDynamicSharedMemorySize, 65536);
  hipLaunchKernelGGL(probe<PAT>, dim3(256), dim3(512), 65536, 0, d, iters);
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  (void)hipEventRecord(a);
  hipLaunchKernelGGL(probe<PAT>, dim3(256), dim3(512), 65536, 0, d, iters);
  (void)hipEventRecord(b);
  (void)hipEventSynchronize(b);
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, a, b);
  const double bytes = 8.0 * 16 * 1024 * iters;  // per CU
  printf("pattern %d %-34s %8.1f us  %6.1f B/clk/CU at 2.1 GHz\n", PAT, what, ms * 1e3, bytes / (ms * 1e-3) / 2.1e9);
}
int main() {
  unsigned* d;
  if (hipMalloc(&d, 256 * 512 * 4) != hipSuccess) return 1;
  run<0>(d, "linear");
  run<1>(d, "attention K fragments (pitch 272)");
  run<2>(d, "attention V^T fragments (pitch 144)");
  run<3>(d, "K fragments, 256 B pitch, XOR chunks");
  return hipDeviceSynchronize() != hipSuccess;
}
