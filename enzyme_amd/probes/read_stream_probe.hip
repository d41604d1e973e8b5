// Read-only HBM stream probe (gfx950). Not part of the library: how fast a
// kernel that only reads can pull bytes from HBM, the ceiling of a
// read-dominated workload such as the residual-add + RMSNorm + projection
// (830 MB read, 16 MB written). Each case reads NB bytes once (two buffer sets
// of NB alternate, so nothing is left in the 256 MB Infinity Cache between
// launches) either as one array or as three arrays read at the same offsets
// (three concurrent streams, as that workload reads x, mlp_prev and
// attention_prev), over a grid of G workgroups of T threads, each thread
// holding V 16-byte loads in flight per round, plain or non-temporal loads.
// The XOR of the data is written only on an impossible value, so the loads
// stay live. Reported: time per launch and GB/s.
//
// Second part ("tile"): the same three 16384 x 8192 bf16 arrays read the way a
// split-K GEMM tile reads its A operand: workgroup (split z, M tile mt, N tile
// nt) walks rows mt*BM..+BM-1 over K range z*4096..+4095, RB bytes of each row
// of each array per K step (the N tiles of one M tile read the same rows on
// one XCD, as the GEMM's XCD-aware unit numbering places them), with PD steps
// of loads issued before the first is consumed. RB = 128 is a 64-deep K step.
// A is read with non-temporal loads unless a case says otherwise (plain loads
// let the N tiles of one row block share lines in L2).
//
// Build and run (repository root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       enzyme_amd/probes/read_stream_probe.hip -o enzyme_amd/probes/_build/read_stream_probe
//   enzyme_amd/probes/_build/read_stream_probe [reps [t]]   (t: the tile part only)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define CK(x)                                                                \
  do {                                                                       \
    hipError_t e_ = (x);                                                     \
    if (e_ != hipSuccess) {                                                  \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));    \
      std::exit(1);                                                          \
    }                                                                        \
  } while (0)

namespace {

// NS streams of n16 vectors each (stream s at base + s * n16). Grid-stride
// rounds of G * T * V vectors; every index is checked against n16.
template <int V, int NS, bool NT>
__global__ void read_stream(const u32x4* __restrict__ base, size_t n16, u32x4* __restrict__ sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x * V;
  u32x4 acc = {0, 0, 0, 0};
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x * V + threadIdx.x; i < n16; i += stride) {
    u32x4 t[NS][V];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const size_t idx = min(i + static_cast<size_t>(v) * blockDim.x, n16 - 1);
        const u32x4* p = base + static_cast<size_t>(s) * n16 + idx;
        t[s][v] = NT ? __builtin_nontemporal_load(p) : *p;
      }
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int v = 0; v < V; ++v) acc ^= t[s][v];
  }
  if (acc.x == 0x12345678u && acc.y == 0x9abcdefu && acc.z == 0x3u) sink[blockIdx.x] = acc;
}

int g_reps = 20;

constexpr int kXcds = 8;
constexpr int kM = 16384, kK = 8192, kS = 2;

// Rows of 8192 bf16 (16 KiB, 1024 vectors) in three arrays at a, a + n16, a +
// 2 n16 (n16 = kM * 1024). A K step covers RB bytes (RB / 16 vectors) of each
// of the tile's BM rows; thread t loads vectors v = t + i * T of the step,
// v -> row v / (RB / 16), vector v % (RB / 16). Every index stays inside its
// array: rows < kM (m0 + BM <= kM), columns < 1024 (K range and RB divide it).
// With BN > 0 each step also loads the B block of a GEMM over these rows:
// RB / 2 rows (k) of BN bf16 columns of a 8192 x 512 bf16 w (row-major, 1 KiB
// rows, 64 vectors), columns nt*BN..+BN-1 (NT * BN == 512), k in the
// workgroup's K range; thread t loads vectors u = t + i * T, u -> k row
// u / (BN / 8), vector u % (BN / 8).
template <int BM, int RB, int T, int PD, int BN = 0, bool NTA = true>
__global__ __launch_bounds__(T) void tile_stream(const u32x4* __restrict__ a, const u32x4* __restrict__ w,
                                                 u32x4* __restrict__ sink, int NT) {
  constexpr int VPR = RB / 16;             // vectors per row per step
  constexpr int V = BM * VPR / T;          // vectors per thread per step per array
  constexpr int VB = BN > 0 ? (RB / 2) * (BN / 8) / T : 0;  // B vectors per thread per step
  static_assert(V >= 1 && BM * VPR % T == 0, "tile shape");
  static_assert(BN == 0 || ((RB / 2) * (BN / 8) % T == 0 && VB >= 1), "B block shape");
  const size_t n16 = static_cast<size_t>(kM) * 1024;
  const int MT = kM / BM;
  const int G = kS * MT * NT;
  int unit = blockIdx.x;
  if (G % kXcds == 0) unit = (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds;
  const int z = unit / (MT * NT);
  const int mt = (unit - z * MT * NT) / NT;
  const int nt = unit - z * MT * NT - mt * NT;
  const int m0 = mt * BM;
  const int c0 = z * 512;                  // first vector of the K range (4096 bf16)
  constexpr int nsteps = 512 / VPR;
  u32x4 acc = {0, 0, 0, 0};
  int off[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int v = threadIdx.x + i * T;
    off[i] = (m0 + v / VPR) * 1024 + c0 + v % VPR;
  }
  int boff[VB > 0 ? VB : 1];
#pragma unroll
  for (int i = 0; i < VB; ++i) {
    const int u = threadIdx.x + i * T;
    constexpr int BV = BN > 0 ? BN / 8 : 1;  // B vectors per k row
    boff[i] = (z * 4096 + u / BV) * 64 + nt * BV + u % BV;  // < 8192 * 64
  }
  for (int s = 0; s < nsteps; s += PD) {
    u32x4 t[PD][3][V];
    u32x4 tb[PD][VB > 0 ? VB : 1];
#pragma unroll
    for (int p = 0; p < PD; ++p) {
#pragma unroll
      for (int q = 0; q < 3; ++q)
#pragma unroll
        for (int i = 0; i < V; ++i)
        {
          const u32x4* src = a + q * n16 + off[i] + min(s + p, nsteps - 1) * VPR;
          t[p][q][i] = NTA ? __builtin_nontemporal_load(src) : *src;
        }
#pragma unroll
      for (int i = 0; i < VB; ++i) tb[p][i] = w[boff[i] + min(s + p, nsteps - 1) * (RB / 2) * 64];
    }
#pragma unroll
    for (int p = 0; p < PD; ++p)
#pragma unroll
      for (int i = 0; i < VB; ++i) acc ^= tb[p][i];
#pragma unroll
    for (int p = 0; p < PD; ++p)
#pragma unroll
      for (int q = 0; q < 3; ++q)
#pragma unroll
        for (int i = 0; i < V; ++i) acc ^= t[p][q][i];
  }
  if (acc.x == 0x12345678u && acc.y == 0x9abcdefu && acc.z == 0x3u) sink[blockIdx.x] = acc;
}

template <int BM, int RB, int T, int PD, int BN = 0, bool NTA = true>
void tile_case(const u32x4* const bufs[2], const u32x4* w, u32x4* sink, int NT) {
  const int G = kS * (kM / BM) * NT;
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  for (int r = 0; r < 6; ++r)
    hipLaunchKernelGGL((tile_stream<BM, RB, T, PD, BN, NTA>), dim3(G), dim3(T), 0, 0, bufs[r & 1], w, sink, NT);
  CK(hipGetLastError());
  CK(hipEventRecord(a));
  for (int r = 0; r < g_reps; ++r)
    hipLaunchKernelGGL((tile_stream<BM, RB, T, PD, BN, NTA>), dim3(G), dim3(T), 0, 0, bufs[r & 1], w, sink, NT);
  CK(hipEventRecord(b));
  CK(hipEventSynchronize(b));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, a, b));
  const double us = ms * 1e3 / g_reps;
  const double bytes = 3.0 * kM * kK * 2;
  std::printf("tile  BM %3d  N tiles %d  BN %3d  G %4d  RB %3d  T %4d  PD %d  A %s: %8.2f us  %6.0f GB/s (unique A bytes)\n",
              BM, NT, BN, G, RB, T, PD, NTA ? "nt " : "reg", us, bytes / (us * 1e-6) / 1e9);
  CK(hipEventDestroy(a));
  CK(hipEventDestroy(b));
}

template <int V, int NS, bool NT>
void run_case(const u32x4* const bufs[2], size_t total16, u32x4* sink, int G, int T) {
  const size_t n16 = total16 / NS;
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  for (int w = 0; w < 6; ++w)
    hipLaunchKernelGGL((read_stream<V, NS, NT>), dim3(G), dim3(T), 0, 0, bufs[w & 1], n16, sink);
  CK(hipGetLastError());
  CK(hipEventRecord(a));
  for (int w = 0; w < g_reps; ++w)
    hipLaunchKernelGGL((read_stream<V, NS, NT>), dim3(G), dim3(T), 0, 0, bufs[w & 1], n16, sink);
  CK(hipEventRecord(b));
  CK(hipEventSynchronize(b));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, a, b));
  const double us = ms * 1e3 / g_reps;
  const double bytes = static_cast<double>(n16) * NS * 16.0;
  std::printf("streams %d  G %5d  T %4d  V %d  %s: %8.2f us  %6.0f GB/s\n", NS, G, T, V, NT ? "nt " : "reg", us,
              bytes / (us * 1e-6) / 1e9);
  CK(hipEventDestroy(a));
  CK(hipEventDestroy(b));
}

template <int V, int NS>
void sweep(const u32x4* const bufs[2], size_t total16, u32x4* sink) {
  for (int T : {256, 512, 1024})
    for (int G : {256, 512, 1024, 2048, 4096}) {
      run_case<V, NS, false>(bufs, total16, sink, G, T);
      run_case<V, NS, true>(bufs, total16, sink, G, T);
    }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc > 1) g_reps = std::max(1, std::atoi(argv[1]));
  const bool tiles_only = argc > 2 && argv[2][0] == 't';
  // 830,472,192 bytes: the llama70b residual-add + RMSNorm + projection's
  // reads, rounded to whole vectors of three equal streams.
  const size_t total16 = (830472192ull / 16) / 3 * 3;
  u32x4* bufs[2] = {nullptr, nullptr};
  for (auto& p : bufs) {
    CK(hipMalloc(&p, total16 * 16));
    CK(hipMemset(p, 1, total16 * 16));
  }
  u32x4* sink = nullptr;
  CK(hipMalloc(&sink, 4096 * sizeof(u32x4)));
  const u32x4* const cb[2] = {bufs[0], bufs[1]};
  u32x4* w = nullptr;
  CK(hipMalloc(&w, 8192ull * 512 * 2));
  CK(hipMemset(w, 1, 8192ull * 512 * 2));
  if (!tiles_only) {
    sweep<1, 1>(cb, total16, sink);
    sweep<4, 1>(cb, total16, sink);
    sweep<8, 1>(cb, total16, sink);
    sweep<1, 3>(cb, total16, sink);
    sweep<2, 3>(cb, total16, sink);
    sweep<4, 3>(cb, total16, sink);
  }
  // The three-array tile reads (need 3 * kM * kK * 2 bytes per buffer set).
  static_assert(3ull * kM * kK * 2 <= 830472192ull, "tile arrays fit the buffers");
  tile_case<256, 128, 256, 1>(cb, w, sink, 2);
  tile_case<256, 128, 256, 2>(cb, w, sink, 2);
  tile_case<256, 256, 256, 1>(cb, w, sink, 2);
  tile_case<256, 128, 512, 1>(cb, w, sink, 2);
  tile_case<256, 128, 512, 2>(cb, w, sink, 2);
  tile_case<256, 256, 512, 1>(cb, w, sink, 2);
  tile_case<128, 128, 256, 1>(cb, w, sink, 1);
  tile_case<128, 128, 256, 2>(cb, w, sink, 1);
  tile_case<128, 256, 256, 1>(cb, w, sink, 1);
  tile_case<128, 256, 256, 2>(cb, w, sink, 1);
  tile_case<128, 512, 256, 1>(cb, w, sink, 1);
  tile_case<128, 128, 512, 2>(cb, w, sink, 1);
  tile_case<128, 256, 512, 2>(cb, w, sink, 1);
  tile_case<64, 512, 256, 1>(cb, w, sink, 1);
  tile_case<64, 512, 256, 2>(cb, w, sink, 1);
  tile_case<64, 1024, 256, 1>(cb, w, sink, 1);
  // With the B block of the projection (w: 8192 x 512 bf16, L2-resident).
  tile_case<256, 128, 256, 1, 256>(cb, w, sink, 2);
  tile_case<256, 128, 512, 1, 256>(cb, w, sink, 2);
  tile_case<128, 128, 256, 1, 512>(cb, w, sink, 1);
  tile_case<128, 128, 512, 1, 512>(cb, w, sink, 1);
  tile_case<128, 128, 512, 2, 512>(cb, w, sink, 1);
  tile_case<128, 256, 256, 1, 512>(cb, w, sink, 1);
  // Plain A loads: the N tiles of one row block can share lines in L2.
  tile_case<256, 128, 256, 1, 0, false>(cb, w, sink, 2);
  tile_case<256, 128, 512, 2, 0, false>(cb, w, sink, 2);
  tile_case<128, 128, 256, 1, 0, false>(cb, w, sink, 1);
  tile_case<256, 128, 256, 1, 256, false>(cb, w, sink, 2);
  tile_case<256, 128, 512, 1, 256, false>(cb, w, sink, 2);
  tile_case<128, 128, 512, 1, 512, false>(cb, w, sink, 1);
  for (auto& p : bufs) CK(hipFree(p));
  CK(hipFree(w));
  CK(hipFree(sink));
  return 0;
}
