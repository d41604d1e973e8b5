// Load-stream probe of the skinny split-K GEMM by workgroup width and
// prefetch depth (gfx950). Not part of the library: the A and B tile loads of
// one 1024x512x16384 split-K GEMM launch (same grid, XCD-aware unit numbering
// and 64-deep K steps as gemm.hip), without arithmetic, for 256, 512 and 1024
// threads per workgroup (each thread loading 1/threads of a step's tiles) and
// 1, 2 or 4 K steps of loads in flight, at 128x128 tiles (K range 2048),
// 256x128 (1024) and 256x256 (512). Inputs rotate over ~1 GiB. Reported:
// time per launch and the bytes per clock per CU taken into the CUs.
//
// Build and run (repository root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       enzyme_amd/probes/feed_waves_probe.hip -o enzyme_amd/probes/_build/feed_waves_probe
//   enzyme_amd/probes/_build/feed_waves_probe [reps [first_case last_case]]
// With arguments (for counter runs): reps timed and reps untimed launches per
// case, and only cases first_case..last_case (0-11, in the order printed).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

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

constexpr int kXcds = 8;
constexpr double kClockHz = 2.4e9;
constexpr int kCus = 256;

// ---- l2: re-read an XCD-owned region ---------------------------------------
template <int V>
__global__ void l2_read(const u32x4* __restrict__ src, u32x4* __restrict__ sink, unsigned region16, int iters) {
  const u32x4* base = src + static_cast<size_t>(blockIdx.x % kXcds) * region16;
  const unsigned per_round = blockDim.x * V;
  // Workgroups of one XCD start 64 KiB apart so they do not all ask for the
  // same lines at once.
  const unsigned off = ((blockIdx.x / kXcds) * 4096u) % region16;
  const unsigned rounds = region16 / per_round;
  u32x4 acc = {0, 0, 0, 0};
  for (int it = 0; it < iters; ++it)
    for (unsigned r = 0; r < rounds; ++r) {
      u32x4 t[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        unsigned i = off + r * per_round + v * blockDim.x + threadIdx.x;  // < 2 * region16
        if (i >= region16) i -= region16;
        t[v] = base[i];
      }
#pragma unroll
      for (int v = 0; v < V; ++v) acc ^= t[v];
    }
  if (acc.x == 0x12345678u && acc.y == 0x9abcdefu) sink[blockIdx.x] = acc;
}

template <int V>
void l2_case(const u32x4* src, u32x4* sink, unsigned region16, int threads) {
  const int blocks = kCus, iters = 8, reps = 10;
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  for (int w = 0; w < 3; ++w) hipLaunchKernelGGL(l2_read<V>, dim3(blocks), dim3(threads), 0, 0, src, sink, region16, iters);
  CK(hipGetLastError());
  CK(hipEventRecord(a));
  for (int w = 0; w < reps; ++w) hipLaunchKernelGGL(l2_read<V>, dim3(blocks), dim3(threads), 0, 0, src, sink, region16, iters);
  CK(hipEventRecord(b));
  CK(hipEventSynchronize(b));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, a, b));
  const double bytes = static_cast<double>(blocks) * iters * (region16 / (threads * V)) * threads * V * 16.0 * reps;
  const double s = ms * 1e-3;
  std::printf("l2  threads %4d  loads in flight %2d: %8.1f us/launch  %7.0f GB/s  %5.1f B/clk/CU\n", threads, V,
              ms * 1e3 / reps, bytes / s / 1e9, bytes / s / kClockHz / kCus);
  CK(hipEventDestroy(a));
  CK(hipEventDestroy(b));
}

int run_l2() {
  const unsigned region16 = (1u << 20) / 16;  // 1 MiB per XCD, a quarter of its L2
  u32x4 *src = nullptr, *sink = nullptr;
  CK(hipMalloc(&src, static_cast<size_t>(kXcds) * region16 * 16));
  CK(hipMalloc(&sink, kCus * sizeof(u32x4)));
  CK(hipMemset(src, 1, static_cast<size_t>(kXcds) * region16 * 16));
  for (int threads : {256, 512, 1024}) {
    l2_case<4>(src, sink, region16, threads);
    l2_case<8>(src, sink, region16, threads);
    l2_case<16>(src, sink, region16, threads);
  }
  CK(hipFree(src));
  CK(hipFree(sink));
  return 0;
}


struct Shape {
  int M, N, K, BM, BN, krange, S, MT, NT;
};

// NT threads per workgroup, PD K steps of loads in flight (register ring).
template <int BM, int BN, int NT, int PD>
__global__ __launch_bounds__(NT) void gemm_loads(const unsigned short* __restrict__ A, const unsigned short* __restrict__ B,
                                                 u32x4* __restrict__ sink, Shape sh) {
  constexpr int AV = BM * 64 / 8 / NT;
  constexpr int KR = BN * 64 / 8 / NT;
  static_assert(AV >= 1 && KR >= 1, "shape");
  const int G = sh.S * sh.MT * sh.NT;
  int unit = blockIdx.x;
  if (G % kXcds == 0) unit = (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds;
  const int z = unit / (sh.MT * sh.NT), tile = unit % (sh.MT * sh.NT);
  const int m0 = (tile / sh.NT) * BM, n0 = (tile % sh.NT) * BN, kbeg = z * sh.krange;
  const int tid = threadIdx.x;
  const int nsteps = sh.krange / 64;
  u32x4 acc = {0, 0, 0, 0};
  u32x4 t[PD][AV + KR];
  auto issue = [&](int s, u32x4 (&tt)[AV + KR]) {
    const int k0 = kbeg + min(s, nsteps - 1) * 64;
#pragma unroll
    for (int j = 0; j < AV; ++j) {
      const int v = tid + j * NT, r = v >> 3, kc = (v & 7) * 8;
      tt[j] = *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(m0 + r) * sh.K + k0 + kc);
    }
#pragma unroll
    for (int j = 0; j < KR; ++j) {
      const int v = tid + j * NT, kr = v / (BN / 8), gn = n0 + (v % (BN / 8)) * 8;
      tt[AV + j] = *reinterpret_cast<const u32x4*>(B + static_cast<size_t>(k0 + kr) * sh.N + gn);
    }
  };
#pragma unroll
  for (int p = 0; p < PD; ++p) issue(p, t[p]);
  for (int s = 0; s < nsteps; s += PD) {
#pragma unroll
    for (int p = 0; p < PD; ++p) {
#pragma unroll
      for (int j = 0; j < AV + KR; ++j) acc ^= t[p][j];
      issue(s + p + PD, t[p]);
    }
  }
  if (acc.x == 0x12345678u && acc.y == 0x9abcdefu) sink[blockIdx.x] = acc;
}

int g_reps = 200, g_warm = 300, g_first = 0, g_last = 1 << 30, g_case = 0;

template <int BM, int BN, int NT, int PD>
int gemm_case(const Shape& sh) {
  const int idx = g_case++;
  if (idx < g_first || idx > g_last) return 0;
  const size_t abytes = static_cast<size_t>(sh.M) * sh.K * 2, bbytes = static_cast<size_t>(sh.K) * sh.N * 2;
  const int nsets = static_cast<int>(std::max<size_t>(1, std::min<size_t>(64, ((1ull << 30) + abytes + bbytes - 1) / (abytes + bbytes))));
  std::vector<unsigned short*> as(nsets), bs(nsets);
  for (int i = 0; i < nsets; ++i) {
    CK(hipMalloc(&as[i], abytes));
    CK(hipMalloc(&bs[i], bbytes));
    CK(hipMemset(as[i], 1, abytes));
    CK(hipMemset(bs[i], 1, bbytes));
  }
  u32x4* sink = nullptr;
  const int G = sh.S * sh.MT * sh.NT;
  CK(hipMalloc(&sink, static_cast<size_t>(G) * sizeof(u32x4)));
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  const int warm = g_warm, reps = g_reps;
  for (int w = 0; w < warm; ++w)
    hipLaunchKernelGGL((gemm_loads<BM, BN, NT, PD>), dim3(G), dim3(NT), 0, 0, as[w % nsets], bs[w % nsets], sink, sh);
  CK(hipGetLastError());
  CK(hipEventRecord(a));
  for (int w = 0; w < reps; ++w)
    hipLaunchKernelGGL((gemm_loads<BM, BN, NT, PD>), dim3(G), dim3(NT), 0, 0, as[w % nsets], bs[w % nsets], sink, sh);
  CK(hipEventRecord(b));
  CK(hipEventSynchronize(b));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, a, b));
  const double us = ms * 1e3 / reps;
  const double cu_bytes = static_cast<double>(G) * (static_cast<double>(BM) + BN) * sh.krange * 2.0;
  std::printf("case %d gemm %dx%dx%d tiles %dx%d Krange %d G %d threads %d PD %d: %.2f us  %.1f B/clk/CU\n",
              idx, sh.M, sh.N, sh.K, BM, BN, sh.krange, G, NT, PD, us, cu_bytes / (us * 1e-6) / kClockHz / kCus);
  for (int i = 0; i < nsets; ++i) {
    CK(hipFree(as[i]));
    CK(hipFree(bs[i]));
  }
  CK(hipFree(sink));
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc > 1) g_reps = g_warm = std::max(1, std::atoi(argv[1]));
  if (argc > 3) {
    g_first = std::atoi(argv[2]);
    g_last = std::atoi(argv[3]);
  }
  Shape sh;
  sh.M = 1024; sh.N = 512; sh.K = 16384; sh.BM = 128; sh.BN = 128; sh.krange = 2048;
  sh.MT = sh.M / sh.BM; sh.NT = sh.N / sh.BN; sh.S = sh.K / sh.krange;
  gemm_case<128, 128, 256, 1>(sh);
  gemm_case<128, 128, 256, 2>(sh);
  gemm_case<128, 128, 256, 4>(sh);
  gemm_case<128, 128, 512, 1>(sh);
  gemm_case<128, 128, 512, 2>(sh);
  gemm_case<128, 128, 512, 4>(sh);
  gemm_case<128, 128, 1024, 1>(sh);
  gemm_case<128, 128, 1024, 2>(sh);
  Shape s2 = sh; s2.BM = 256; s2.BN = 128; s2.MT = 4; s2.NT = 4; s2.krange = 1024; s2.S = 16;
  gemm_case<256, 128, 256, 2>(s2);
  gemm_case<256, 128, 512, 2>(s2);
  Shape s3 = sh; s3.BM = 256; s3.BN = 256; s3.MT = 4; s3.NT = 2; s3.krange = 512; s3.S = 32;
  gemm_case<256, 256, 512, 2>(s3);
  gemm_case<256, 256, 1024, 2>(s3);
  return 0;
}
