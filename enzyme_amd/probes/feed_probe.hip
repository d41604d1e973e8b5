// Memory-feed probes for the GEMM kernels (gfx950). Not part of the library:
// a standalone program that measures the two ceilings the split-K GEMM's
// K loop runs against.
//
//   feed_probe l2
//       Every workgroup (256 per launch, dealt round-robin over the 8 XCDs)
//       re-reads a 1 MiB region owned by its XCD, so after the first pass
//       every load hits that XCD's L2. Reported per launch shape (threads per
//       workgroup x 16-byte loads in flight per thread) as bytes per clock per
//       CU at 2.4 GHz: the L2 -> CU feed a K loop could reach on L2 hits.
//
//   feed_probe gemm M N K BM BN KRANGE
//       The load stream of one split-K GEMM launch without its arithmetic:
//       the same grid (K / KRANGE splits x M/BM x N/BN tiles), the same
//       XCD-aware unit numbering as gemm.hip (each XCD a contiguous run of
//       units, split-major), the same 64-deep K steps and the same per-thread
//       16-byte loads of the A tile [BM x 64] and the B tile [64 x BN]. The
//       data are XOR-folded and never stored (unless a sentinel matches), and
//       input sets are rotated over ~1 GiB so the Infinity Cache does not hold
//       them. Reported: time per launch, the CU-side feed in bytes per clock
//       per CU, and the HBM rate of the algorithmic A + B bytes. A kernel
//       whose launch takes about this long is bound by its load stream, not
//       by its arithmetic.
//
// Build and run (repository root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       enzyme_amd/probes/feed_probe.hip -o enzyme_amd/probes/_build/feed_probe
//   enzyme_amd/probes/_build/feed_probe l2
//   enzyme_amd/probes/_build/feed_probe gemm 1024 512 16384 128 128 2048
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

// ---- gemm: the load stream of one split-K GEMM launch ----------------------
struct Shape {
  int M, N, K, BM, BN, krange, S, MT, NT;
};

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_loads(const unsigned short* __restrict__ A, const unsigned short* __restrict__ B,
                                                  u32x4* __restrict__ sink, Shape sh) {
  constexpr int AV = BM * 64 / 8 / 256;  // 16-byte A loads per thread per K step
  constexpr int KR = BN / 32;            // 16-byte B loads per thread per K step
  const int G = sh.S * sh.MT * sh.NT;
  int unit = blockIdx.x;
  if (G % kXcds == 0) unit = (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds;
  const int z = unit / (sh.MT * sh.NT), tile = unit % (sh.MT * sh.NT);
  const int m0 = (tile / sh.NT) * BM, n0 = (tile % sh.NT) * BN, kbeg = z * sh.krange;
  const int tid = threadIdx.x;
  u32x4 acc = {0, 0, 0, 0};
  for (int s = 0; s < sh.krange / 64; ++s) {
    const int k0 = kbeg + s * 64;
    u32x4 t[AV + KR];
#pragma unroll
    for (int j = 0; j < AV; ++j) {
      const int v = tid + j * 256, r = v >> 3, kc = (v & 7) * 8;
      t[j] = *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(m0 + r) * sh.K + k0 + kc);
    }
#pragma unroll
    for (int j = 0; j < KR; ++j) {
      const int v = tid + j * 256, kr = v / (BN / 8), gn = n0 + (v % (BN / 8)) * 8;
      t[AV + j] = *reinterpret_cast<const u32x4*>(B + static_cast<size_t>(k0 + kr) * sh.N + gn);
    }
#pragma unroll
    for (int j = 0; j < AV + KR; ++j) acc ^= t[j];
  }
  if (acc.x == 0x12345678u && acc.y == 0x9abcdefu) sink[blockIdx.x] = acc;
}

template <int BM, int BN>
int gemm_case(const Shape& sh) {
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
  const int warm = 200, reps = 200;  // the warm-up also lets the clocks settle
  for (int w = 0; w < warm; ++w)
    hipLaunchKernelGGL((gemm_loads<BM, BN>), dim3(G), dim3(256), 0, 0, as[w % nsets], bs[w % nsets], sink, sh);
  CK(hipGetLastError());
  CK(hipEventRecord(a));
  for (int w = 0; w < reps; ++w)
    hipLaunchKernelGGL((gemm_loads<BM, BN>), dim3(G), dim3(256), 0, 0, as[w % nsets], bs[w % nsets], sink, sh);
  CK(hipEventRecord(b));
  CK(hipEventSynchronize(b));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, a, b));
  const double us = ms * 1e3 / reps;
  const double cu_bytes = static_cast<double>(G) * (static_cast<double>(BM) + BN) * sh.krange * 2.0;
  std::printf("gemm %dx%dx%d  tiles %dx%d  K range %d  (%d workgroups, %d input sets): %.2f us/launch  "
              "%.1f B/clk/CU into the CUs  A+B at %.0f GB/s\n",
              sh.M, sh.N, sh.K, BM, BN, sh.krange, G, nsets, us, cu_bytes / (us * 1e-6) / kClockHz / kCus,
              static_cast<double>(abytes + bbytes) / (us * 1e-6) / 1e9);
  for (int i = 0; i < nsets; ++i) {
    CK(hipFree(as[i]));
    CK(hipFree(bs[i]));
  }
  CK(hipFree(sink));
  return 0;
}

int run_gemm(int argc, char** argv) {
  if (argc != 8) {
    std::fprintf(stderr, "usage: feed_probe gemm M N K BM BN KRANGE\n");
    return 2;
  }
  Shape sh{};
  sh.M = std::atoi(argv[2]);
  sh.N = std::atoi(argv[3]);
  sh.K = std::atoi(argv[4]);
  sh.BM = std::atoi(argv[5]);
  sh.BN = std::atoi(argv[6]);
  sh.krange = std::atoi(argv[7]);
  // Whole tiles and whole K steps only: every load below stays inside A and B.
  if (sh.M <= 0 || sh.N <= 0 || sh.K <= 0 || sh.krange <= 0 || sh.M % sh.BM || sh.N % sh.BN || sh.K % sh.krange ||
      sh.krange % 64) {
    std::fprintf(stderr, "need M %% BM == N %% BN == K %% KRANGE == KRANGE %% 64 == 0\n");
    return 2;
  }
  sh.S = sh.K / sh.krange;
  sh.MT = sh.M / sh.BM;
  sh.NT = sh.N / sh.BN;
#define FEED_CASE(bm, bn) \
  if (sh.BM == bm && sh.BN == bn) return gemm_case<bm, bn>(sh);
  FEED_CASE(64, 64)
  FEED_CASE(128, 128)
  FEED_CASE(128, 256)
  FEED_CASE(256, 128)
  FEED_CASE(256, 256)
#undef FEED_CASE
  std::fprintf(stderr, "tiles: 64x64, 128x128, 128x256, 256x128 or 256x256\n");
  return 2;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc >= 2 && std::strcmp(argv[1], "l2") == 0) return run_l2();
  if (argc >= 2 && std::strcmp(argv[1], "gemm") == 0) return run_gemm(argc, argv);
  std::fprintf(stderr, "usage: feed_probe l2 | feed_probe gemm M N K BM BN KRANGE\n");
  return 2;
}
