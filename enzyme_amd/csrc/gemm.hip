// bf16 MFMA GEMM family: matmul, matmul_std002, rmsnorm_matmul (sum form),
// rmsnorm_matmul_eps, the two-stage silu_mlp and qkv_cte.
//
//   matmul               C = A @ B                         kernels/matmul/kernel.py:7-8
//   rmsnorm_matmul       C = diag(1/sqrt(sum_k A^2)) (A @ B)  kernels/rmsnorm_matmul/kernel.py:7-16
//   rmsnorm_matmul_eps   C = diag(rsqrt(mean_k A^2 + 1e-6)) (A @ B)
//   silu_mlp             H = silu(X @ W1) * (X @ W2);  C = H @ W3  kernels/silu_mlp/kernel.py:7-14
//   qkv_cte              h = x + mlp_prev + attention_prev;
//                        C = diag(rsqrt(mean_k h^2 + 1e-6)) (h @ W)   kernels/qkv_cte/kernel.py:18-27
// A is [M, K] row-major (K contiguous), B is [K, N] row-major (N contiguous),
// C is [M, N] bf16; accumulation is fp32.
//
// Schedule (hw variant 0): a workgroup of 4 waves (2 x 2) owns a BM x BN
// output tile and a K range of 64*TK. Per 64-deep K step it loads the A tile
// (16-byte vectors along K) and the B tile (16-byte vectors along N) into
// one register set and stores both to the LDS buffer the MFMAs
// (v_mfma_f32_32x32x16_bf16) do not read; LDS is double-buffered. The step
// is a rolling refill: A vector j is stored and at once reloaded for the
// step after next, and the step's MFMAs are cut into slices issued between
// those stores, so the matrix cores run under the staging work (fp32 A:
// exp, hi/lo split) and the load waits; B (both operands for silu_mlp) is
// stored as loaded ([k][n]) and its MFMA fragments come from the
// transposing LDS read (below).
// The RMSNorm row scale needs sum_k A^2: each thread accumulates the squares
// of the A vectors it already holds, so A is read once.
// Split K (K range < K): each workgroup writes its fp32 partial tile (and its
// rows' partial sums of squares) to the workspace; a second, fully parallel
// kernel sums the S partials of every output in split order
// (deterministic), applies the epilogue and writes C.
// Workgroups are numbered so that the ones sharing a K range land on the same
// XCD (blocks are dealt round-robin over the 8 XCDs), keeping that range of A
// and B in one L2.
//
// hw variant 1 keeps PD register sets of global loads in flight (PD = 3 for
// tiles up to 128 x 128, 2 above) in the plain order (all stores, refill,
// then the MFMAs). Both variants stage B as loaded, [k][n], so every B load
// instruction reads whole 128-byte lines (staging B transposed through
// registers reads half lines, and a CU's vector L1 delivers about half the
// useful bytes per cycle on half lines). The MFMA B fragments then come from
// gfx950's transposing LDS read (ds_read_b64_tr_b16): two reads give a lane
// the 8 consecutive k values of its column.
//
// qkv_cte hw variant 3 (qkv_wide_kernel, with its own comment below) is a
// separate schedule: full-width N tiles of 256 or 512 columns, one wave per
// 64 columns, w packed into MFMA operand order by qkv_pack_w_kernel and
// loaded straight into registers.
//
// Tile arguments: TILES_IN_BLOCK_M = BM/64, TILES_IN_BLOCK_N = BN/64 (tiles of
//                 64, 128 or 256; qkv_cte hw variant 3: BN/256), TILES_IN_BLOCK_K
//                 = K range per workgroup / 256 (silu_mlp: TILES_IN_BLOCK_P =
//                 BN/64 of its second GEMM).
// Every tuple the manifest admits is instantiated: silu_mlp narrows its
// stages' tiles to what its two accumulator sets and LDS hold (BM x BN <=
// 128 x 128 per stage, BM <= 128 in stage 2) instead of refusing them.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "registry.hpp"

namespace axon {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int BK = 64;
constexpr int kKUnit = 256;  // TILES_IN_BLOCK_K counts K in units of 256
constexpr int LDK = BK + 8;  // LDS row pitch in elements (144 B; keeps 16 B alignment)

// Row pitch (elements) of the [k][n] B tile: BN + 16 puts the
// four k rows one transposing read touches 8 banks apart.
constexpr int bpitch(int BN) { return BN + 16; }
constexpr int kThreads = 256;
constexpr int kXcds = 8;

// kQkv: A is the sum of three bf16 inputs (A + A2 + A3, added in fp32 as
// loaded), with the kRmsEps row scale taken over that sum.
// kSoftmax: A is replaced by exp(A) as loaded (fp32), and the output row is
// scaled by 1 / sum_k exp(A): softmax without max subtraction, then @ B.
// kColSplit: the plain product with column-split operands (GemmArgs::Bcol,
// Ccol, ncol); a separate instantiation so the other epilogues keep their
// register allocation.
enum Epi { kPlain = 0, kRmsSum = 1, kRmsEps = 2, kSiluMul = 3, kQkv = 4, kSoftmax = 5, kColSplit = 6 };

// Epilogues that scale each output row by a statistic of its A row, summed
// over K as the A tiles are staged (squares for the RMS forms, the values
// themselves for kSoftmax).
template <int EPI>
constexpr bool is_rms() { return EPI == kRmsSum || EPI == kRmsEps || EPI == kQkv || EPI == kSoftmax; }

struct GemmArgs {
  const void* A;        // [M, K] bf16, or fp32 when A_F32
  const bf16* B;        // [K, N]
  const bf16* B2;       // [K, N] second operand (kSiluMul)
  const bf16* A2;       // [M, K] second and third addends of A (kQkv)
  const bf16* A3;
  void* C;              // [M, N] bf16, or fp32 H when kSiluMul
  float* partial;       // [S][M][N] fp32 (x2 for kSiluMul)
  float* rowsq;         // [S][NT][M] fp32
  const float* rscale;  // kPlain: per-row output scale, or null for none
  int M, N, K;
  int kchunk;           // K range per workgroup
  int S, MT, NT;
  float eps;
  int c_f32;            // kPlain: C is fp32 instead of bf16
  // Column-split operands (kColSplit, hw variants 0/1): the logical B [K, N]
  // is [B | Bcol[0] | Bcol[1]] and C [M, N] is [C | Ccol[0] | Ccol[1]], each
  // block ncol columns wide and contiguous on its own (N = 3 ncol, ncol a
  // multiple of BN, so a tile never straddles two).
  const bf16* Bcol[2];
  void* Ccol[2];
  int ncol;
};

__device__ __forceinline__ float silu(float a) { return a / (1.f + __expf(-a)); }

template <int N>
using ic = std::integral_constant<int, N>;

// Prefetch depth 1 (hw variant 0, every epilogue) runs the rolling refill
// with sliced compute (gemm_kernel's step).
template <int PD>
constexpr bool rolling() { return PD == 1; }

// NTH threads per workgroup: 256 (4 waves as 2 x 2 over the tile) or 512
// (hw variant 3 of the plain GEMMs, 2 of the RMSNorm GEMMs): two groups of
// 4 waves on the same 2 x 2 wave tiles, group wk computing the 16-deep
// k-slices 2 wk and 2 wk + 1 of every 64-deep K step. The 8 waves share the
// loads (half per thread) and two waves sit on every SIMD, while the LDS
// fragment reads per step stay those of 4 waves; group 1 adds its
// accumulators into group 0's through LDS once, after the last step.
template <int BM, int BN, int EPI, bool A_F32, int PD, int NTH = kThreads>
__global__ __launch_bounds__(NTH) void gemm_kernel(GemmArgs g) {
  constexpr bool DUAL = EPI == kSiluMul;
  constexpr int KW = NTH / kThreads;       // k-slice groups of 4 waves
  constexpr int WM = BM / 2, WN = BN / 2;  // per-wave tile
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AV = BM * BK / 8 / NTH;  // A vectors per thread (8 k-values each)
  constexpr int KR = BN * BK / 8 / NTH;  // B rows per thread block (k)
  constexpr int NA = A_F32 ? 2 : 1;      // hi/lo planes for an fp32 A
  constexpr int NB = DUAL ? 2 : 1;
  static_assert(KW == 1 || KW == 2, "4 or 8 waves");
  static_assert(AV >= 1 && KR >= 1 && KR <= 8, "tile shape");
  static_assert(KW == 1 || PD > 1, "the 8-wave schedule runs the plain pipeline");

  extern __shared__ __align__(16) unsigned char smem[];
  // B is staged as loaded ([k][n], pitch PB) and read with the transposing
  // LDS read.
  constexpr bool ROLL = rolling<PD>();
  constexpr int PB = bpitch(BN);
  bf16* As = reinterpret_cast<bf16*>(smem);                 // [2][NA][BM][LDK]
  bf16* Bs = As + 2 * NA * BM * LDK;                        // [2][NB][BK][PB]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) & 1, wn = wave & 1;
  const int wk = wave >> 2;  // k-slice group (0 with 4 waves)

  // XCD-aware numbering: blocks b and b+8 run on the same XCD; give each XCD
  // a contiguous run of (split, tile) units in split-major order.
  const int G = g.S * g.MT * g.NT;
  int unit = blockIdx.x;
  if (G % kXcds == 0) unit = (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds;
  const int z = unit / (g.MT * g.NT);
  const int tile = unit - z * g.MT * g.NT;
  const int mt = tile / g.NT, nt = tile - mt * g.NT;
  const int m0 = mt * BM, n0 = nt * BN;
  const int kbeg = z * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  // This tile's B and C blocks (the whole of B and C unless column-split).
  constexpr bool CS = EPI == kColSplit;
  const int csel = CS ? n0 / g.ncol : 0;
  const int ncol0 = CS ? csel * g.ncol : 0;
  const int ldbc = CS ? g.ncol : g.N;
  const bf16* Bw = CS && csel > 0 ? g.Bcol[csel - 1] : g.B;
  void* Cw = CS && csel > 0 ? g.Ccol[csel - 1] : g.C;

  // Global-load assignment.
  // A: vector v = tid + j*NTH -> row v/8, k-chunk v%8.
  // B: vector v = tid + r*NTH -> k row v / (BN/8), column chunk v % (BN/8):
  // whole 128-byte lines per instruction.

  // Global loads are unconditional from clamped (always in-range)
  // addresses, so the compiler issues them back to back and only waits for
  // them when the LDS store needs the data, after the current step's MFMAs;
  // out-of-range elements are zeroed at store time.
  using ARaw = typename std::conditional<A_F32, Vec<float>, Vec<bf16>>::type;
  constexpr int AW = A_F32 ? 2 : (EPI == kQkv ? 3 : 1);  // 16-byte loads per 8 A values
  // PD register sets; set r holds the loads of the K steps t with t % PD == r.
  ARaw a_raw[PD][AV][AW];
  bool a_ok[PD][AV];
  Vec<bf16> b_raw[PD][NB][KR];
  bool b_ok[PD][KR];
  float sq[AV];
#pragma unroll
  for (int j = 0; j < AV; ++j) sq[j] = 0.f;

  const int nsteps = (kend - kbeg + BK - 1) / BK;
  // Loads of steps past this workgroup's K range re-read its last step (L2
  // hits) and are never stored: they keep the pipeline free of branches, so
  // the compiler's memory-counter waits stay exact.
  const int klast = kbeg + max(nsteps - 1, 0) * BK;

  // Loads of A vector j (AW 16-byte loads) and of the whole B block for the
  // K step at k0 into register set P.
  auto load_a = [&](int k0, auto set_tag, int j) {
    constexpr int P = decltype(set_tag)::value;
    const int kl = min(k0, klast);
    {
      const int v = tid + j * NTH;
      const int r = v >> 3, kc = (v & 7) * 8;
      const int gm = m0 + r, gk = k0 + kc;
      a_ok[P][j] = gm < g.M && gk < kend;
      const int64_t off = static_cast<int64_t>(min(gm, g.M - 1)) * g.K + min(kl + kc, g.K - 8);
      if constexpr (A_F32) {
        const float* src = static_cast<const float*>(g.A) + off;
        a_raw[P][j][0] = load_vec(src);
        a_raw[P][j][1] = load_vec(src + 4);
      } else {
        a_raw[P][j][0] = load_vec(static_cast<const bf16*>(g.A) + off);
        if constexpr (EPI == kQkv) {
          a_raw[P][j][1] = load_vec(g.A2 + off);
          a_raw[P][j][2] = load_vec(g.A3 + off);
        }
      }
    }
  };
  auto load_b = [&](int k0, auto set_tag) {
    constexpr int P = decltype(set_tag)::value;
    const int kl = min(k0, klast);
#pragma unroll
    for (int r = 0; r < KR; ++r) {
      const int v = tid + r * NTH;
      const int kr = v / (BN / 8);
      const int gn = n0 + (v % (BN / 8)) * 8;
      const int gk = k0 + kr;
      b_ok[P][r] = gk < kend && gn < g.N;
      const int64_t off = static_cast<int64_t>(min(kl + kr, g.K - 1)) * ldbc + min(gn - ncol0, ldbc - 8);
#pragma unroll
      for (int q = 0; q < NB; ++q) b_raw[P][q][r] = load_vec((q == 0 ? Bw : g.B2) + off);
    }
  };
  auto load_global = [&](int k0, auto set_tag) {
#pragma unroll
    for (int j = 0; j < AV; ++j) load_a(k0, set_tag, j);
    load_b(k0, set_tag);
  };

  // LDS stores of A vector j and of the B block from register set P.
  auto store_a = [&](int buf, auto set_tag, int j) {
    constexpr int P = decltype(set_tag)::value;
    auto& a_raw_p = a_raw[P];
    auto& a_ok_p = a_ok[P];
    {
      const int v = tid + j * NTH;
      const int r = v >> 3, kc = (v & 7) * 8;
      float x[8];
      if constexpr (A_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = a_ok_p[j] ? a_raw_p[j][0].v[e] : 0.f;
          x[4 + e] = a_ok_p[j] ? a_raw_p[j][1].v[e] : 0.f;
        }
        if constexpr (EPI == kSoftmax) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = a_ok_p[j] ? __expf(x[e]) : 0.f;
        }
        Vec<bf16> hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          hi.v[e] = static_cast<bf16>(x[e]);
          lo.v[e] = static_cast<bf16>(x[e] - static_cast<float>(hi.v[e]));
        }
        store_vec(As + ((buf * NA + 0) * BM + r) * LDK + kc, hi);
        store_vec(As + ((buf * NA + 1) * BM + r) * LDK + kc, lo);
      } else if constexpr (EPI == kQkv) {
        // h = (x + mlp_prev) + attention_prev in fp32; its squares feed the
        // row scale before h is rounded to the bf16 MFMA operand.
        Vec<bf16> t;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float h = (to_f32(a_raw_p[j][0].v[e]) + to_f32(a_raw_p[j][1].v[e])) + to_f32(a_raw_p[j][2].v[e]);
          x[e] = a_ok_p[j] ? h : 0.f;
          t.v[e] = static_cast<bf16>(x[e]);
        }
        store_vec(As + ((buf * NA + 0) * BM + r) * LDK + kc, t);
      } else if constexpr (EPI == kSoftmax) {
        // exp in fp32; the row sum takes the unrounded values.
        Vec<bf16> t;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] = a_ok_p[j] ? __expf(to_f32(a_raw_p[j][0].v[e])) : 0.f;
          t.v[e] = static_cast<bf16>(x[e]);
        }
        store_vec(As + ((buf * NA + 0) * BM + r) * LDK + kc, t);
      } else {
        Vec<bf16> t = a_raw_p[j][0];
        if (!a_ok_p[j]) {
#pragma unroll
          for (int e = 0; e < 8; ++e) t.v[e] = static_cast<bf16>(0.f);
        }
        store_vec(As + ((buf * NA + 0) * BM + r) * LDK + kc, t);
        if constexpr (EPI == kRmsSum || EPI == kRmsEps) {
          // Sum of squares straight from the bf16 pairs: v_dot2c_f32_bf16
          // (exact bf16 products, fp32 accumulation), 4 instructions for 8
          // values instead of 8 conversions and 8 FMAs.
          const bf16x2* pr = reinterpret_cast<const bf16x2*>(&t);
#pragma unroll
          for (int q = 0; q < 4; ++q) sq[j] = __builtin_amdgcn_fdot2_f32_bf16(pr[q], pr[q], sq[j], false);
        }
      }
      if constexpr (EPI == kSoftmax) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sq[j] += x[e];
      } else if constexpr (EPI == kQkv || (A_F32 && is_rms<EPI>())) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sq[j] += x[e] * x[e];
      }
    }
  };
  auto store_b = [&](int buf, auto set_tag) {
    constexpr int P = decltype(set_tag)::value;
    auto& b_raw_p = b_raw[P];
    auto& b_ok_p = b_ok[P];
#pragma unroll
    for (int q = 0; q < NB; ++q)
#pragma unroll
      for (int r = 0; r < KR; ++r) {
        // Opaque until here: otherwise the zeroing below is placed right
        // after the load and waits for it PD steps early.
        u32x4 raw = *reinterpret_cast<const u32x4*>(&b_raw_p[q][r]);
        asm volatile("" : "+v"(raw));
        if (!b_ok_p[r]) raw = u32x4{0u, 0u, 0u, 0u};
        const int v = tid + r * NTH;
        *reinterpret_cast<u32x4*>(Bs + ((buf * NB + q) * BK + v / (BN / 8)) * PB + (v % (BN / 8)) * 8) = raw;
      }
  };
  auto store_lds = [&](int buf, auto set_tag) {
#pragma unroll
    for (int j = 0; j < AV; ++j) store_a(buf, set_tag, j);
    store_b(buf, set_tag);
  };

  floatx16 acc[NB][TM][TN];
#pragma unroll
  for (int q = 0; q < NB; ++q)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[q][i][j][e] = 0.f;

  auto compute = [&](int buf) {
#pragma unroll
    for (int k2 = 0; k2 < BK / 16 / KW; ++k2) {
      const int kk = wk * (BK / 16 / KW) + k2;
      const int kof = kk * 16 + (lane >> 5) * 8;
      bf16x8 af[NA][TM];
#pragma unroll
      for (int p = 0; p < NA; ++p)
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[p][i] = *reinterpret_cast<const bf16x8*>(
              As + ((buf * NA + p) * BM + wm * WM + i * 32 + (lane & 31)) * LDK + kof);
#pragma unroll
      for (int q = 0; q < NB; ++q) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          // Transposing read: within each 16-lane group, lane i receives
          // element i%4 of the 4 values lane 4j + i/4 points at, for j =
          // 0..3. Lane s points at row k0 + s/4, columns nb + 4*(s%4), so
          // lane i gets k rows k0..k0+3 of column nb + i; a second read
          // 4 rows down gives k0+4..k0+7 (the MFMA's 8 k values).
          const int g4 = lane >> 4, s16 = lane & 15;
          const int nb = wn * WN + j * 32 + 16 * (g4 & 1);
          const int kr0 = kk * 16 + 8 * (g4 >> 1) + (s16 >> 2);
          const bf16* bp = Bs + ((buf * NB + q) * BK + kr0) * PB + nb + 4 * (s16 & 3);
          const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(bp));
          const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(bp + 4 * PB));
          const bf16x8 bfr = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int p = 0; p < NA; ++p)
              acc[q][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[p][i], bfr, acc[q][i][j], 0, 0, 0);
          }
        }
      }
    }
  };

  // compute() cut into slices for the rolling refill: MFMA unit u covers
  // (kk = u / TN, B column tile u % TN); the A fragments of a kk are read at
  // its first unit and kept until its last.
  bf16x8 af_s[NA][TM];
  auto compute_units = [&](int buf, int u0, int u1) {
#pragma unroll
    for (int u = u0; u < u1; ++u) {
      const int kk = u / TN, jn = u % TN;
      const int kof = kk * 16 + (lane >> 5) * 8;
      if (jn == 0) {
#pragma unroll
        for (int p = 0; p < NA; ++p)
#pragma unroll
          for (int i = 0; i < TM; ++i)
            af_s[p][i] = *reinterpret_cast<const bf16x8*>(
                As + ((buf * NA + p) * BM + wm * WM + i * 32 + (lane & 31)) * LDK + kof);
      }
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        const int g4 = lane >> 4, s16 = lane & 15;
        const int nb = wn * WN + jn * 32 + 16 * (g4 & 1);
        const int kr0 = kk * 16 + 8 * (g4 >> 1) + (s16 >> 2);
        const bf16* bp = Bs + ((buf * NB + q) * BK + kr0) * PB + nb + 4 * (s16 & 3);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(bp));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(bp + 4 * PB));
        const bf16x8 bfr = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int p = 0; p < NA; ++p)
            acc[q][i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af_s[p][i], bfr, acc[q][i][jn], 0, 0, 0);
      }
    }
  };

  // Pipeline: K steps 0..PD-1 are loaded up front; after step s is computed
  // from LDS buffer s&1, step s+1 moves from its register set into the other
  // buffer and that set is refilled with step s+1+PD. Full groups of PD steps
  // run branch-free; the remaining steps run in a short tail.
  static_assert(PD >= 1 && PD <= 4, "prefetch depth");
  if (nsteps > 0) {
    load_global(kbeg, ic<0>{});
    if constexpr (PD > 1) load_global(kbeg + BK, ic<1>{});
    if constexpr (PD > 2) load_global(kbeg + 2 * BK, ic<2>{});
    if constexpr (PD > 3) load_global(kbeg + 3 * BK, ic<3>{});
    if constexpr (ROLL) {
      // Same store/refill order as the loop body, so the loads in flight at
      // the loop entry are those the loop's waits are counted against.
#pragma unroll
      for (int j = 0; j < AV; ++j) {
        store_a(0, ic<0>{}, j);
        __builtin_amdgcn_sched_barrier(0);
        load_a(kbeg + PD * BK, ic<0>{}, j);
        __builtin_amdgcn_sched_barrier(0);
      }
      store_b(0, ic<0>{});
      __builtin_amdgcn_sched_barrier(0);
      load_b(kbeg + PD * BK, ic<0>{});
      __builtin_amdgcn_sched_barrier(0);
    } else {
      store_lds(0, ic<0>{});
      load_global(kbeg + PD * BK, ic<0>{});
    }
  }
  __syncthreads();
  // Global loads and MFMAs per K step (for the load/MFMA interleave).
  constexpr int NLOADS = AV * AW + KR * NB;
  constexpr int NMFMA = (BK / 16 / KW) * NB * TM * TN * NA;
  constexpr int MPL = NMFMA / NLOADS > 0 ? NMFMA / NLOADS : 1;
  // One K step: step s+1 goes from its register set into the buffer computed
  // on two steps ago (every wave finished reading it before the last
  // barrier), the set is refilled, and step s is computed while the LDS
  // absorbs the stores.
  auto step = [&](int s0, auto j_tag) {
    constexpr int J = decltype(j_tag)::value;
    constexpr int NX = (J + 1) % PD;  // register set of step s + 1
    const int s = s0 + J;
    if constexpr (ROLL) {
      // Each vector's refill is issued as soon as its store has read the
      // registers, so the next step's loads start during this store phase
      // instead of after it.
      // Slice j of this step's MFMAs goes with the store and refill of A
      // vector j: the MFMAs run while the conversion VALU work and the load
      // waits of the slice are issued (the two touch different LDS buffers).
      constexpr int U = (BK / 16) * TN;
#pragma unroll
      for (int j = 0; j < AV; ++j) {
        compute_units(s & 1, j * U / AV, (j + 1) * U / AV);
        store_a((s + 1) & 1, ic<NX>{}, j);
        __builtin_amdgcn_sched_barrier(0);
        load_a(kbeg + (s + 1 + PD) * BK, ic<NX>{}, j);
        __builtin_amdgcn_sched_barrier(0);
      }
      store_b((s + 1) & 1, ic<NX>{});
      __builtin_amdgcn_sched_barrier(0);
      load_b(kbeg + (s + 1 + PD) * BK, ic<NX>{});
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      return;
    }
    store_lds((s + 1) & 1, ic<NX>{});
    // The refill reuses the registers the stores just read: issued earlier,
    // it would need other registers and copies that wait for loads in flight.
    __builtin_amdgcn_sched_barrier(0);
    load_global(kbeg + (s + 1 + PD) * BK, ic<NX>{});
    compute(s & 1);
    // Spread the refill's global loads over the step's MFMAs (one load per
    // two MFMAs) instead of issuing them as one burst the address unit
    // cannot take in: a wave stalled at a load issues no MFMA either.
#pragma unroll
    for (int i = 0; i < NLOADS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one VMEM read
      __builtin_amdgcn_sched_group_barrier(0x008, MPL, 0);  // MPL MFMAs
    }
    __syncthreads();
  };
  int s0 = 0;
  for (; s0 + PD <= nsteps; s0 += PD) {
    step(s0, ic<0>{});
    if constexpr (PD > 1) step(s0, ic<1>{});
    if constexpr (PD > 2) step(s0, ic<2>{});
    if constexpr (PD > 3) step(s0, ic<3>{});
  }
  auto tail = [&](auto j_tag) {
    constexpr int J = decltype(j_tag)::value;
    constexpr int NX = (J + 1) % PD;
    const int s = s0 + J;
    if (s >= nsteps) return;
    if (s + 1 < nsteps) store_lds((s + 1) & 1, ic<NX>{});
    compute(s & 1);
    __syncthreads();
  };
  if constexpr (PD > 1) tail(ic<0>{});
  if constexpr (PD > 2) tail(ic<1>{});
  if constexpr (PD > 3) tail(ic<2>{});

  // ---- 8 waves: group 1's accumulators into group 0's, through LDS --------
  // (the staging buffers are free: every wave passed the last step's
  // barrier). Layout [wave of group][q][i][j][e / 4][lane] of 16-byte
  // quads: consecutive lanes write and read consecutive quads.
  if constexpr (KW == 2) {
    float4* red = reinterpret_cast<float4*>(smem);
    auto slot = [&](int q, int i, int j, int e4) {
      return ((((wave & 3) * NB + q) * TM + i) * TN + j) * 4 * 64 + e4 * 64 + lane;
    };
    if (wk == 1) {
#pragma unroll
      for (int q = 0; q < NB; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4)
              red[slot(q, i, j, e4)] = make_float4(acc[q][i][j][4 * e4], acc[q][i][j][4 * e4 + 1],
                                                   acc[q][i][j][4 * e4 + 2], acc[q][i][j][4 * e4 + 3]);
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int q = 0; q < NB; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
              const float4 o = red[slot(q, i, j, e4)];
              acc[q][i][j][4 * e4] += o.x;
              acc[q][i][j][4 * e4 + 1] += o.y;
              acc[q][i][j][4 * e4 + 2] += o.z;
              acc[q][i][j][4 * e4 + 3] += o.w;
            }
    }
    __syncthreads();  // the row sums below reuse the same LDS
  }

  // ---- row sums of squares (RMSNorm epilogues) ---------------------------
  float* rs_lds = reinterpret_cast<float*>(smem);  // [BM], reuses the A buffers
  if constexpr (is_rms<EPI>()) {
#pragma unroll
    for (int j = 0; j < AV; ++j) {
      float v = sq[j];
      v += __shfl_xor(v, 1, kWave);
      v += __shfl_xor(v, 2, kWave);
      v += __shfl_xor(v, 4, kWave);
      sq[j] = v;  // row (tid + j*NTH)/8, identical across its 8 threads
    }
    if (g.S == 1) {
#pragma unroll
      for (int j = 0; j < AV; ++j)
        if ((tid & 7) == 0) rs_lds[(tid + j * NTH) >> 3] = sq[j];
      __syncthreads();
    } else {
#pragma unroll
      for (int j = 0; j < AV; ++j) {
        const int r = (tid + j * NTH) >> 3;
        // Every N tile computes the same row sums; the first one publishes.
        if ((tid & 7) == 0 && m0 + r < g.M && nt == 0)
          g.rowsq[(static_cast<int64_t>(z) * g.NT + nt) * g.M + m0 + r] = sq[j];
      }
    }
  }

  // Output coordinates of accumulator element e of MFMA tile (i, j):
  // row = 8*(e/4) + 4*(lane/32) + e%4, column = lane%32.
  auto row_of = [&](int i, int e) { return wm * WM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); };
  auto col_of = [&](int j) { return wn * WN + j * 32 + (lane & 31); };

  // An empty contraction (K == 0) leaves zero accumulators and an empty
  // normalised row, whose product is 0: scale 0 rather than 1/0 or 0/0.
  auto scale_of = [&](float sumsq) -> float {
    if (g.K == 0) return 0.f;
    if constexpr (EPI == kRmsSum) return 1.f / sqrtf(sumsq);
    else if constexpr (EPI == kSoftmax) return 1.f / sumsq;
    else if constexpr (EPI == kRmsEps || EPI == kQkv) return 1.f / sqrtf(sumsq / static_cast<float>(g.K) + g.eps);
    else return 1.f;
  };

  auto write_out = [&](int gm, int gn, float v0, float v1) {
    const int64_t o = static_cast<int64_t>(gm) * ldbc + (gn - ncol0);
    if constexpr (EPI == kSiluMul) {
      static_cast<float*>(Cw)[o] = silu(v0) * v1;
    } else {
      (void)v1;
      if (EPI == kPlain && g.c_f32) static_cast<float*>(Cw)[o] = v0;
      else static_cast<bf16*>(Cw)[o] = static_cast<bf16>(v0);
    }
  };

  // With 8 waves group 0 holds the sums and writes the outputs.
  if (KW == 2 && wk != 0) return;

  if (g.S == 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = row_of(i, e);
        const int gm = m0 + r;
        if (gm >= g.M) continue;
        float sc = 1.f;
        if constexpr (is_rms<EPI>()) sc = scale_of(rs_lds[r]);
        if constexpr (EPI == kPlain) {
          if (g.rscale != nullptr) sc = g.rscale[gm];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int gn = n0 + col_of(j);
          if (gn >= g.N) continue;
          write_out(gm, gn, acc[0][i][j][e] * sc, acc[NB - 1][i][j][e]);
        }
      }
    return;
  }

  // ---- split K: publish the partial; splitk_reduce_kernel finishes -------
  const int64_t MN = static_cast<int64_t>(g.M) * g.N;
  if (m0 + BM <= g.M && n0 + BN <= g.N) {
    // Whole tile in range: no per-element guards.
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      float* dst = g.partial + (static_cast<int64_t>(q) * g.S + z) * MN + static_cast<int64_t>(m0) * g.N + n0;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            dst[static_cast<int64_t>(row_of(i, e)) * g.N + col_of(j)] = acc[q][i][j][e];
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < NB; ++q)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int gm = m0 + row_of(i, e);
        if (gm >= g.M) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int gn = n0 + col_of(j);
          if (gn < g.N) g.partial[(static_cast<int64_t>(q) * g.S + z) * MN + static_cast<int64_t>(gm) * g.N + gn] = acc[q][i][j][e];
        }
      }
}

// Split-K fixup: every thread owns 4 consecutive outputs (16-byte loads;
// N % 8 == 0 keeps a quad inside one row), sums the S fp32 partials in split
// order with four splits in flight, applies the epilogue and writes C. The
// whole grid takes part, so the partials (mostly still in the Infinity
// Cache) stream at full rate.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs g, int BN) {
  constexpr int NB = EPI == kSiluMul ? 2 : 1;
  constexpr bool RMS = is_rms<EPI>();
  const int64_t MN = static_cast<int64_t>(g.M) * g.N;
  const int64_t idx = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const int gm = static_cast<int>(min(idx, MN - 1) / g.N), gn = static_cast<int>(idx - static_cast<int64_t>(gm) * g.N);
  // RMSNorm epilogues: the row scales of this block's rows (the block's
  // 1024 outputs span at most 1024 / N + 1 rows, N >= 8) are summed over
  // the splits once, by one thread per row, instead of by every thread.
  // Their loads and the partial loads below are all issued before the first
  // wait, so the two reads overlap; threads past the output load a clamped
  // quad (MN % 8 == 0) and return after the barrier.
  __shared__ float row_scale[129];
  float ss = 0.f;
  bool own_row = false;
  if constexpr (RMS) {
    const int64_t first = static_cast<int64_t>(blockIdx.x) * blockDim.x * 4;
    const int r0 = static_cast<int>(first / g.N);
    const int r1 = static_cast<int>(min(first + static_cast<int64_t>(blockDim.x) * 4, MN) - 1) / g.N;
    const int r = r0 + static_cast<int>(threadIdx.x);
    if (r <= r1) {
      own_row = true;
      // Every N tile holds the same row sums; read tile 0's, in split order.
      const float* rq = g.rowsq + r;
      const int64_t zs = static_cast<int64_t>(g.NT) * g.M;
      int zz = 0;
      for (; zz + 4 <= g.S; zz += 4) {
        const float a0 = rq[(zz + 0) * zs], a1 = rq[(zz + 1) * zs], a2 = rq[(zz + 2) * zs], a3 = rq[(zz + 3) * zs];
        ss = (((ss + a0) + a1) + a2) + a3;
      }
      for (; zz < g.S; ++zz) ss += rq[zz * zs];
    }
  }
  const int64_t lidx = min(idx, MN - 4);
  float v[NB][4];
#pragma unroll
  for (int q = 0; q < NB; ++q) {
    const float* base = g.partial + static_cast<int64_t>(q) * g.S * MN + lidx;
    float t[4] = {0.f, 0.f, 0.f, 0.f};
    int zz = 0;
    for (; zz + 4 <= g.S; zz += 4) {
      const Vec<float> p0 = load_vec(base + (zz + 0) * MN);
      const Vec<float> p1 = load_vec(base + (zz + 1) * MN);
      const Vec<float> p2 = load_vec(base + (zz + 2) * MN);
      const Vec<float> p3 = load_vec(base + (zz + 3) * MN);
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = (((t[e] + p0.v[e]) + p1.v[e]) + p2.v[e]) + p3.v[e];
    }
    for (; zz < g.S; ++zz) {
      const Vec<float> p0 = load_vec(base + zz * MN);
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] += p0.v[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[q][e] = t[e];
  }
  if constexpr (RMS) {
    if (own_row)
      row_scale[threadIdx.x] = EPI == kRmsSum    ? 1.f / sqrtf(ss)
                               : EPI == kSoftmax ? 1.f / ss
                                                 : 1.f / sqrtf(ss / static_cast<float>(g.K) + g.eps);
    __syncthreads();
  }
  if (idx >= MN) return;
  float sc = 1.f;
  (void)BN;
  // Output block of a column-split C (a quad never straddles: ncol % 8 == 0).
  constexpr bool CS = EPI == kColSplit;
  const int csel = CS ? gn / g.ncol : 0;
  void* Cw = CS && csel > 0 ? g.Ccol[csel - 1] : g.C;
  const int64_t oidx = CS ? static_cast<int64_t>(gm) * g.ncol + (gn - csel * g.ncol) : idx;
  if constexpr (RMS) sc = row_scale[gm - static_cast<int>(static_cast<int64_t>(blockIdx.x) * blockDim.x * 4 / g.N)];
  if constexpr (EPI == kPlain) {
    if (g.rscale != nullptr) sc = g.rscale[gm];
  }
  if constexpr (EPI == kSiluMul) {
    Vec<float> o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.v[e] = silu(v[0][e]) * v[1][e];
    store_vec(static_cast<float*>(Cw) + oidx, o);
  } else if (EPI == kPlain && g.c_f32) {
    Vec<float> o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.v[e] = v[0][e] * sc;
    store_vec(static_cast<float*>(Cw) + oidx, o);
  } else {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(v[0][e] * sc);
    *reinterpret_cast<bf16x4*>(static_cast<bf16*>(Cw) + oidx) = o;
  }
}

// ---------------------------------------------------------------------------
// hw variant 2 of the plain GEMM: direct-to-LDS loads (global_load_lds_dwordx4:
// lane i's 16 bytes land at the wave's LDS base + 16 i), so tiles go from
// memory to LDS without passing through registers, and NS LDS stages ring
// with NS - 1 K steps of loads in flight. A wave's wait for its own loads
// (vmcnt) plus the workgroup barrier make a stage visible to every wave; the
// barrier also retires the reads of the stage the next loads overwrite.
// Stage layout (16-byte chunks swizzled so fragment reads spread over banks):
//   A: BM rows x 128 B; chunk kc of row r at slot kc ^ (r & 7);
//   B: 64 k rows x BN columns as loaded; chunk c of row k at slot c ^ bg(k)
//      with bg(k) = 2 ((k & 3) | ((k & 8) >> 1)) (2 (k & 3) for BN = 64), so
//      the 8 rows one transposing read touches use distinct chunk slots.
// Every K step is whole (k % 64 == 0). Rows of A past M and columns of B
// past N are clamped reads that only feed discarded outputs. Steps past the
// workgroup's K range reload its last step into the free stage (never read),
// so the wait count is the same constant every step.
// ---------------------------------------------------------------------------
template <int BN>
__device__ __forceinline__ int dma_bg(int k) {
  if constexpr (BN >= 128) return 2 * ((k & 3) | ((k & 8) >> 1));
  else return 2 * (k & 3);
}

__device__ __forceinline__ void dma16(const void* gptr, void* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(gptr),
                                   (__attribute__((address_space(3))) void*)(lds), 16, 0, 0);
}

// LDS fragment reads of hw variant 2, as inline assembly: the compiler
// treats its own LDS reads after a global_load_lds as possibly aliasing the
// loads in flight and waits for all of them (vmcnt(0)), which would drain
// the stage ring every step. These reads are ordered by the explicit
// vmcnt wait + barrier instead, and their results by lds_wait<N>().
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)(p)));
}

__device__ __forceinline__ bf16x8 lds_read_b128(const void* p) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ i16x4 lds_read_tr(const void* p) {
  i16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}

// Waits until at most N LDS operations are outstanding.
template <int N>
__device__ __forceinline__ void lds_wait() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] and
// [15:14], expcnt[6:4] = 7, lgkmcnt[11:8] = 15).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BM, int BN, int NS>
constexpr size_t dma_lds_bytes() { return static_cast<size_t>(NS) * 128 * (BM + BN); }

template <int BM, int BN, int EPI, int NS>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(GemmArgs g) {
  static_assert(EPI == kPlain, "hw variant 2 serves the plain epilogue");
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int SA = BM * 128, STAGE = (BM + BN) * 128;  // bytes
  constexpr int LA = BM / 32, LB = BN / 32;  // DMA instructions per thread per K step
  constexpr int CPR = BN / 8;                // 16-byte chunks per B row
  constexpr int RPI = 64 / CPR;              // B rows per 1 KiB wave instruction
  static_assert(NS >= 2 && TM >= 1 && TN >= 1, "tile shape");
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int G = g.S * g.MT * g.NT;
  int unit = blockIdx.x;
  if (G % kXcds == 0) unit = (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds;
  const int z = unit / (g.MT * g.NT);
  const int tile = unit - z * g.MT * g.NT;
  const int mt = tile / g.NT, nt = tile - mt * g.NT;
  const int m0 = mt * BM, n0 = nt * BN;
  const int kbeg = z * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const int nsteps = (kend - kbeg) / BK;
  const int klast = kbeg + max(nsteps - 1, 0) * BK;

  const bf16* A = static_cast<const bf16*>(g.A);
  // Per-lane source offsets (elements, without the step's k0).
  int64_t a_off[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int r = (i * 4 + wave) * 8 + (lane >> 3);
    const int kc = (lane & 7) ^ (r & 7);
    a_off[i] = static_cast<int64_t>(min(m0 + r, g.M - 1)) * g.K + kc * 8;
  }
  int b_row[LB], b_col[LB];
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int k = (i * 4 + wave) * RPI + lane / CPR;
    const int c = (lane % CPR) ^ dma_bg<BN>(k);
    b_row[i] = k;
    b_col[i] = min(n0 + c * 8, g.N - 8);
  }

  auto issue = [&](int step, int stage) {
    const int k0 = min(kbeg + step * BK, klast);
    unsigned char* st = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < LA; ++i) dma16(A + a_off[i] + k0, st + (i * 4 + wave) * 1024);
#pragma unroll
    for (int i = 0; i < LB; ++i)
      dma16(g.B + static_cast<int64_t>(k0 + b_row[i]) * g.N + b_col[i], st + SA + (i * 4 + wave) * 1024);
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment reads of one 16-deep slice kk of a stage into register set buf.
  const int g4 = lane >> 4, s16 = lane & 15;
  bf16x8 af[2][TM];
  i16x4 bl[2][TN], bh[2][TN];
  auto read = [&](int stage, int kk, int buf) {
    const unsigned char* sa = smem + stage * STAGE;
    const unsigned char* sb = sa + SA;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm * WM + i * 32 + (lane & 31);
      const int kc = 2 * kk + (lane >> 5);
      af[buf][i] = lds_read_b128(sa + r * 128 + ((kc ^ (r & 7)) << 4));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = wn * WN + j * 32 + 16 * (g4 & 1) + 4 * (s16 & 3);
      const int c = n >> 3, half = (n >> 2) & 1;
      const int k_lo = kk * 16 + 8 * (g4 >> 1) + (s16 >> 2), k_hi = k_lo + 4;
      bl[buf][j] = lds_read_tr(sb + k_lo * (BN * 2) + ((c ^ dma_bg<BN>(k_lo)) << 4) + half * 8);
      bh[buf][j] = lds_read_tr(sb + k_hi * (BN * 2) + ((c ^ dma_bg<BN>(k_hi)) << 4) + half * 8);
    }
  };
  auto mfma = [&](int buf) {
    // The fragments are opaque until here, so no MFMA moves above the wait.
#pragma unroll
    for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[buf][i]));
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      asm volatile("" : "+v"(bl[buf][j]), "+v"(bh[buf][j]));
      const bf16x8 bfr = __builtin_bit_cast(bf16x8, __builtin_shufflevector(bl[buf][j], bh[buf][j], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int i = 0; i < TM; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[buf][i], bfr, acc[i][j], 0, 0, 0);
    }
  };
  constexpr int NR = TM + 2 * TN;  // LDS reads per slice
  static_assert(NR < 16, "reads per slice");

  // Pipeline: step s lives in stage s % NS. Slice kk + 1 is read while slice
  // kk's MFMAs wait only for their own reads; at the last slice of a step the
  // wave finishes its reads of the stage, waits for its loads of the next
  // step, meets the other waves at the barrier, refills the finished stage
  // with step s + NS and reads the next step's first slice, all before the
  // last slice's MFMAs, so no LDS latency is exposed at the step boundary.
  constexpr int L = LA + LB;
  if (nsteps > 0) {
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s, s);
    wait_vmcnt<(NS - 2) * L>();
    __builtin_amdgcn_s_barrier();
    issue(NS - 1, NS - 1);
    read(0, 0, 0);
    int stage = 0;
    for (int t = 0; t < nsteps; ++t) {
      const int next = stage == NS - 1 ? 0 : stage + 1;
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int cur = kk & 1;
        if (kk + 1 < BK / 16) {
          read(stage, kk + 1, cur ^ 1);
          lds_wait<NR>();
        } else if (t + 1 < nsteps) {
          lds_wait<0>();
          wait_vmcnt<(NS - 2) * L>();
          __builtin_amdgcn_s_barrier();
          issue(t + NS, stage);
          read(next, 0, cur ^ 1);
        } else {
          lds_wait<0>();
        }
        mfma(cur);
      }
      stage = next;
    }
    // Drain the loads past the K range before the workgroup's LDS goes away.
    wait_vmcnt<0>();
  }

  auto row_of = [&](int i, int e) { return wm * WM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); };
  auto col_of = [&](int j) { return wn * WN + j * 32 + (lane & 31); };
  if (g.S == 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int gm = m0 + row_of(i, e);
        if (gm >= g.M) continue;
        const float sc = g.rscale != nullptr ? g.rscale[gm] : 1.f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int gn = n0 + col_of(j);
          if (gn >= g.N) continue;
          const int64_t o = static_cast<int64_t>(gm) * g.N + gn;
          if (g.c_f32) static_cast<float*>(g.C)[o] = acc[i][j][e] * sc;
          else static_cast<bf16*>(g.C)[o] = static_cast<bf16>(acc[i][j][e] * sc);
        }
      }
    return;
  }
  const int64_t MN = static_cast<int64_t>(g.M) * g.N;
  float* dst = g.partial + static_cast<int64_t>(z) * MN;
  const bool whole = m0 + BM <= g.M && n0 + BN <= g.N;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int gm = m0 + row_of(i, e);
      if (!whole && gm >= g.M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int gn = n0 + col_of(j);
        if (!whole && gn >= g.N) continue;
        dst[static_cast<int64_t>(gm) * g.N + gn] = acc[i][j][e];
      }
    }
}

// ---------------------------------------------------------------------------
// qkv_cte operand preparation (kernels/qkv_cte/kernel.py:22-27): one
// workgroup per row streams the three residual inputs once, forms
// h = (x + mlp_prev) + attention_prev in fp32 (the reference's order),
// accumulates sum h^2 and writes the GEMM's bf16 A operand:
//   bf16 inputs: A[row] = bf16(h)                          (K' = k)
//   fp32 inputs: A[row] = [hi(h) | lo(h) | hi(h)]           (K' = 3k)
// with hi = bf16(h), lo = bf16(h - hi). Paired with B = [hi(w); hi(w); lo(w)]
// the bf16 GEMM over K' sums hi*hi + lo*hi + hi*lo, leaving only the lo*lo
// term (about 2^-16 relative) out, so fp32 cases keep fp32-level accuracy.
// The row scale rsqrt(sum h^2 / k + eps) goes to `rscale`, applied by the
// GEMM's epilogue; A itself does not depend on it, so no second pass.
// k % 8 == 0 keeps every 8-element group inside one row and 16-byte aligned.
// ---------------------------------------------------------------------------
constexpr int kPrepThreads = 256;

template <typename T>
__global__ __launch_bounds__(kPrepThreads) void qkv_prep_kernel(const T* __restrict__ x,
                                                                const T* __restrict__ mp,
                                                                const T* __restrict__ ap,
                                                                bf16* __restrict__ a,
                                                                float* __restrict__ rscale, int k,
                                                                float eps) {
  constexpr bool F32 = std::is_same<T, float>::value;
  const int row = blockIdx.x;
  const int64_t in_off = static_cast<int64_t>(row) * k;
  bf16* arow = a + static_cast<int64_t>(row) * (F32 ? 3 * k : k);
  float ss = 0.f;
  for (int c = threadIdx.x * 8; c < k; c += kPrepThreads * 8) {
    float h[8];
    if constexpr (F32) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const Vec<float> vx = load_vec_nt(x + in_off + c + 4 * half);
        const Vec<float> vm = load_vec_nt(mp + in_off + c + 4 * half);
        const Vec<float> va = load_vec_nt(ap + in_off + c + 4 * half);
#pragma unroll
        for (int e = 0; e < 4; ++e) h[4 * half + e] = (vx.v[e] + vm.v[e]) + va.v[e];
      }
    } else {
      const Vec<T> vx = load_vec_nt(x + in_off + c);
      const Vec<T> vm = load_vec_nt(mp + in_off + c);
      const Vec<T> va = load_vec_nt(ap + in_off + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = (to_f32(vx.v[e]) + to_f32(vm.v[e])) + to_f32(va.v[e]);
    }
    Vec<bf16> hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ss += h[e] * h[e];
      hi.v[e] = static_cast<bf16>(h[e]);
    }
    store_vec(arow + c, hi);
    if constexpr (F32) {
      Vec<bf16> lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) lo.v[e] = static_cast<bf16>(h[e] - static_cast<float>(hi.v[e]));
      store_vec(arow + k + c, lo);
      store_vec(arow + 2 * k + c, hi);
    }
  }
  __shared__ float part[kPrepThreads / kWave];
  ss = wave_sum(ss);
  if (lane_id() == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kPrepThreads / kWave; ++i) t += part[i];
    rscale[row] = k == 0 ? 0.f : 1.f / sqrtf(t * (1.f / static_cast<float>(k)) + eps);
  }
}

// B operand of the fp32 qkv_cte GEMM: w [k, n] fp32 -> [hi(w); hi(w); lo(w)],
// each plane [k, n] bf16. Every thread converts 8 consecutive elements.
__global__ __launch_bounds__(256) void qkv_split_w_kernel(const float* __restrict__ w,
                                                         bf16* __restrict__ b, int64_t kn) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i >= kn) return;
  const Vec<float> v0 = load_vec_nt(w + i), v1 = load_vec_nt(w + i + 4);
  Vec<bf16> hi, lo;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = e < 4 ? v0.v[e] : v1.v[e - 4];
    hi.v[e] = static_cast<bf16>(f);
    lo.v[e] = static_cast<bf16>(f - static_cast<float>(hi.v[e]));
  }
  store_vec(b + i, hi);
  store_vec(b + kn + i, hi);
  store_vec(b + 2 * kn + i, lo);
}

// A operand of the fp32 matmul: x [m, k] fp32 -> [m, 3k] bf16 rows
// [hi(x) | lo(x) | hi(x)] (paired with w as [hi; hi; lo], as in qkv_cte).
// Every thread converts 8 consecutive elements of one row (k % 8 == 0).
__global__ __launch_bounds__(256) void split_rows_hilo_kernel(const float* __restrict__ x,
                                                             bf16* __restrict__ a, int64_t mk, int k) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i >= mk) return;
  const int64_t row = i / k, col = i - row * k;
  const Vec<float> v0 = load_vec_nt(x + i), v1 = load_vec_nt(x + i + 4);
  Vec<bf16> hi, lo;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = e < 4 ? v0.v[e] : v1.v[e - 4];
    hi.v[e] = static_cast<bf16>(f);
    lo.v[e] = static_cast<bf16>(f - static_cast<float>(hi.v[e]));
  }
  bf16* arow = a + row * 3 * k;
  store_vec(arow + col, hi);
  store_vec(arow + k + col, lo);
  store_vec(arow + 2 * k + col, hi);
}

// ---------------------------------------------------------------------------
// hw variant 3 of qkv_cte (bf16): full-width N tiles with the B operand
// loaded straight into registers.
//
// One workgroup per BM x BN output tile and K range, BN = 64 x waves, so at
// n = 512 one N tile covers every column and each residual row leaves memory
// once per K range. hw variant 2's 256 x 256 tiles read every A row twice,
// once per N tile. Replayed as loads only (A rows plus the B block, 8 waves,
// plain loads), the two patterns take 173 and 161 us at 16384 x 512 x 8192,
// and 154 us for the full-width one with non-temporal A loads, which the
// 256-column pattern cannot use (its second N tile then misses L2: 228 us).
// Wave w owns the output columns 64 w .. 64 w + 63 of the tile and all BM
// rows:
//   * A, h = (x + mlp_prev) + attention_prev (summed in fp32, squares summed
//     for the row scale, rounded to bf16), is staged once per K step in LDS
//     and read by every wave;
//   * B goes from memory straight into the MFMA operand registers. A pre-pass
//     (qkv_pack_w_kernel) lays w out so that each 16-deep slice of a
//     32-column tile is one contiguous KiB holding the 64 lanes' operands in
//     lane order: every B load instruction of a wave reads one whole KiB, and
//     no B byte passes through LDS.
// k order inside a 64-deep step: slice kk of lane half h (lane / 32) holds
// k = 32 h + 8 kk + (0..7). A is read from LDS at that offset and B is packed
// the same way, so each MFMA slice sums over a fixed k set and the four
// slices together cover the step's 64 k values once.
// ---------------------------------------------------------------------------
constexpr int kPackCols = 256;              // columns of w per pre-pass workgroup
constexpr int kPackPitch = kPackCols + 8;   // LDS row pitch (elements), 16-byte aligned rows

// w [K, N] bf16 -> fragments: fragment ((s * nct + ct) * 4 + kk) * 64 + l
// (16 bytes) holds w[k][n] for n = 32 ct + l % 32 and
// k = 64 s + 32 (l / 32) + 8 kk + (0..7); k >= K or n >= N read as 0.
// Grid (Kp / 64, Np / 256): workgroup (s, cg) reads the 64 x 256 block with
// 16-byte row loads into LDS, then writes its 2048 fragments (one
// contiguous 32 KiB run) with each thread gathering 8 rows of one column.
__global__ __launch_bounds__(256) void qkv_pack_w_kernel(const bf16* __restrict__ w, u32x4* __restrict__ out,
                                                         int K, int N, int nct) {
  __shared__ __align__(16) bf16 tile[64 * kPackPitch];
  const int s = blockIdx.x, cg = blockIdx.y;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int v = tid + i * 256;  // 64 rows x 32 vectors of 8 columns
    const int r = v >> 5, c8 = v & 31;
    const int k = s * 64 + r, n = cg * kPackCols + c8 * 8;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (k < K && n < N) val = *reinterpret_cast<const u32x4*>(w + static_cast<int64_t>(k) * N + n);  // N % 8 == 0
    *reinterpret_cast<u32x4*>(tile + r * kPackPitch + c8 * 8) = val;
  }
  __syncthreads();
  u32x4* dst = out + (static_cast<int64_t>(s) * nct + cg * (kPackCols / 32)) * 256;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int f = tid + i * 256;  // (column tile, slice, lane) = (f / 256, f / 64 % 4, f % 64)
    const int l = f & 63, kk = (f >> 6) & 3;
    const int col = (f >> 8) * 32 + (l & 31);
    const int k0 = 32 * (l >> 5) + 8 * kk;
    bf16x8 frag;
#pragma unroll
    for (int e = 0; e < 8; ++e) frag[e] = tile[(k0 + e) * kPackPitch + col];
    dst[f] = __builtin_bit_cast(u32x4, frag);
  }
}

template <int BM, int NW>
__global__ __launch_bounds__(64 * NW) void qkv_wide_kernel(GemmArgs g, const u32x4* __restrict__ wp, int nct) {
  constexpr int NTH = 64 * NW, BN = 64 * NW;
  constexpr int TM = BM / 32;        // 32-row MFMA tiles of a wave
  constexpr int AV = BM * 8 / NTH;   // A vectors (8 k values of one row) per thread per step
  static_assert(AV >= 1 && (BM * 8) % NTH == 0, "tile shape");
  __shared__ __align__(16) bf16 As[2 * BM * LDK];
  __shared__ float rs[BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int G = g.S * g.MT * g.NT;
  int unit = blockIdx.x;
  if (G % kXcds == 0) unit = (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds;
  const int z = unit / (g.MT * g.NT);
  const int tile = unit - z * g.MT * g.NT;
  const int mt = tile / g.NT, nt = tile - mt * g.NT;
  const int m0 = mt * BM, n0 = nt * BN;
  const int kbeg = z * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const int nsteps = max(0, (kend - kbeg + BK - 1) / BK);
  // Loads past the K range re-read its last step (never used): branch-free.
  const int klast = kbeg + max(nsteps - 1, 0) * BK;

  const bf16* X = static_cast<const bf16*>(g.A);
  // A: vector v = tid + j * NTH -> row v / 8, k chunk v % 8 (8 lanes read one
  // row's 128 bytes of a step).
  Vec<bf16> araw[AV][3];
  bool aok[AV];
  float sq[AV];
#pragma unroll
  for (int j = 0; j < AV; ++j) sq[j] = 0.f;
  auto load_a = [&](int k0) __attribute__((always_inline)) {
    const int kl = min(k0, klast);
#pragma unroll
    for (int j = 0; j < AV; ++j) {
      const int v = tid + j * NTH;
      const int r = v >> 3, kc = (v & 7) * 8;
      const int gm = m0 + r;
      aok[j] = gm < g.M && k0 + kc < kend;
      const int64_t off = static_cast<int64_t>(min(gm, g.M - 1)) * g.K + min(kl + kc, g.K - 8);
      araw[j][0] = load_vec_nt(X + off);
      araw[j][1] = load_vec_nt(g.A2 + off);
      araw[j][2] = load_vec_nt(g.A3 + off);
    }
  };
  auto store_a = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < AV; ++j) {
      const int v = tid + j * NTH;
      const int r = v >> 3, kc = (v & 7) * 8;
      Vec<bf16> t;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float h = (to_f32(araw[j][0].v[e]) + to_f32(araw[j][1].v[e])) + to_f32(araw[j][2].v[e]);
        const float x = aok[j] ? h : 0.f;
        sq[j] += x * x;
        t.v[e] = static_cast<bf16>(x);
      }
      store_vec(As + (buf * BM + r) * LDK + kc, t);
    }
  };

  // B fragments of this wave's two 32-column tiles, one per 16-deep slice.
  u32x4 bfr[2][4];
  const u32x4* wcol = wp + static_cast<int64_t>(n0 / 32 + 2 * wave) * 256 + lane;
  auto load_b = [&](int s, int j, int kk) __attribute__((always_inline)) {
    const int sg = min(kbeg + s * BK, klast) / BK;
    bfr[j][kk] = wcol[(static_cast<int64_t>(sg) * nct + j) * 256 + kk * 64];
  };

  floatx16 acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  bf16x8 af[2][TM];
  auto read_a = [&](int buf, int kk, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      af[slot][i] = *reinterpret_cast<const bf16x8*>(As + (buf * BM + 32 * i + (lane & 31)) * LDK + 32 * (lane >> 5) +
                                                     8 * kk);
  };

  // Step s: its A tile in LDS buffer s % 2 and its B fragments in bfr. Each
  // slice's MFMAs are followed by the reload of that slice's B fragments for
  // step s + 1; after slice 1 the next step's A vectors (loaded one step
  // earlier) are summed into the other buffer and step s + 2's are loaded.
  // One barrier per step: it publishes the A tile of step s + 1 and retires
  // every read of the buffer the following step overwrites.
  if (nsteps > 0) {
    load_a(kbeg);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int j = 0; j < 2; ++j) load_b(0, j, kk);
    store_a(0);
    load_a(kbeg + BK);
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
      const int buf = s & 1;
      read_a(buf, 0, 0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk + 1 < 4) read_a(buf, kk + 1, (kk + 1) & 1);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int i = 0; i < TM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk & 1][i], __builtin_bit_cast(bf16x8, bfr[j][kk]),
                                                                acc[i][j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 2; ++j) load_b(s + 1, j, kk);
        if (kk == 1) {
          store_a(buf ^ 1);
          load_a(kbeg + (s + 2) * BK);
        }
      }
      __syncthreads();
    }
  }

  // Row sums of squares: row (tid + j * NTH) / 8 is spread over 8 lanes.
#pragma unroll
  for (int j = 0; j < AV; ++j) {
    float v = sq[j];
    v += __shfl_xor(v, 1, kWave);
    v += __shfl_xor(v, 2, kWave);
    v += __shfl_xor(v, 4, kWave);
    sq[j] = v;
  }
  // Accumulator element e of MFMA tile (i, j): row 32 i + 8 (e / 4) +
  // 4 (lane / 32) + e % 4, column 64 wave + 32 j + lane % 32.
  auto row_of = [&](int i, int e) { return i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); };
  auto col_of = [&](int j) { return wave * 64 + j * 32 + (lane & 31); };

  if (g.S == 1) {
#pragma unroll
    for (int j = 0; j < AV; ++j)
      if ((tid & 7) == 0) rs[(tid + j * NTH) >> 3] = sq[j];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = row_of(i, e);
        const int gm = m0 + r;
        if (gm >= g.M) continue;
        // An empty contraction has zero accumulators and an empty row: 0.
        const float sc = g.K == 0 ? 0.f : 1.f / sqrtf(rs[r] / static_cast<float>(g.K) + g.eps);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int gn = n0 + col_of(j);
          if (gn < g.N) static_cast<bf16*>(g.C)[static_cast<int64_t>(gm) * g.N + gn] = static_cast<bf16>(acc[i][j][e] * sc);
        }
      }
    return;
  }
  // Split K: the partial tile and (first N tile only) the row sums; the
  // splitk_reduce_kernel<kQkv> fixup sums both over the splits.
#pragma unroll
  for (int j = 0; j < AV; ++j) {
    const int r = (tid + j * NTH) >> 3;
    if ((tid & 7) == 0 && m0 + r < g.M && nt == 0) g.rowsq[(static_cast<int64_t>(z) * g.NT + nt) * g.M + m0 + r] = sq[j];
  }
  const int64_t MN = static_cast<int64_t>(g.M) * g.N;
  float* dst = g.partial + static_cast<int64_t>(z) * MN;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int gm = m0 + row_of(i, e);
      if (gm >= g.M) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int gn = n0 + col_of(j);
        if (gn < g.N) dst[static_cast<int64_t>(gm) * g.N + gn] = acc[i][j][e];
      }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
const char* const kTileArgs3[] = {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"};
const char* const kTileArgs4[] = {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K",
                                  "TILES_IN_BLOCK_P"};

struct Plan {
  int BM, BN, kchunk, S, MT, NT;
};

Plan plan_of(int M, int N, int K, int tm, int tn, int tk) {
  Plan p;
  p.BM = 64 * tm;
  p.BN = 64 * tn;
  p.kchunk = kKUnit * tk;
  if (p.kchunk > K) p.kchunk = ((K + BK - 1) / BK) * BK;
  p.S = K > 0 ? (K + p.kchunk - 1) / p.kchunk : 1;
  p.MT = (M + p.BM - 1) / p.BM;
  p.NT = (N + p.BN - 1) / p.BN;
  return p;
}

bool tile_ok(int tm, int tn) {
  // (BM, BN) instantiations: BM in {64, 128, 256}, BN in {64, 128, 256}.
  return (tm == 1 || tm == 2 || tm == 4) && (tn == 1 || tn == 2 || tn == 4);
}

size_t lds_bytes(int BM, int BN, int na, int nb) {
  const size_t b = static_cast<size_t>(BK) * bpitch(BN);
  return static_cast<size_t>(2) * (na * BM * LDK + nb * b) * sizeof(bf16);
}

// Dynamic LDS available to one workgroup (160 KiB on gfx950, less the small
// static allocation of the kernel).
constexpr size_t kMaxLds = 160 * 1024 - 256;

// gemm_kernel's dynamic LDS: the staging buffers, and with 8 waves at least
// the fp32 accumulators of 4 waves (the k-slice groups' sum).
size_t gemm_lds_bytes(int BM, int BN, int na, int nb, int threads) {
  const size_t stage = lds_bytes(BM, BN, na, nb);
  const size_t red = threads > kThreads ? static_cast<size_t>(nb) * BM * BN * sizeof(float) : 0;
  return stage > red ? stage : red;
}

// qkv_cte hw variant 3 counts its tiles differently: TILES_IN_BLOCK_M = BM / 64
// (1 or 2) and TILES_IN_BLOCK_N = BN / 256 (1 or 2: 256 or 512 columns, one
// wave per 64), so its manifest box is exactly its legal set.
bool qkv_wide_tile_ok(int tm, int tn) { return (tm == 1 || tm == 2) && (tn == 1 || tn == 2); }
constexpr int kQkvWideCols = 256;  // columns per TILES_IN_BLOCK_N of hw variant 3

int check_gemm_shape(int64_t M, int64_t N, int64_t K, int tm, int tn, int tk, std::string* why,
                     int threads = kThreads, bool qkv_wide = false) {
  if (M < 0 || N < 0 || K < 0 || M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) {
    *why = "dimension out of range";
    return AXON_EINVAL;
  }
  if (N % 8 != 0 || K % 8 != 0) {
    *why = "n and k must be multiples of 8 (16-byte rows)";
    return AXON_EINVAL;
  }
  if (qkv_wide && !qkv_wide_tile_ok(tm, tn)) {
    *why = "hw variant 3 tiles: TILES_IN_BLOCK_M 1 or 2 (64 or 128 rows), TILES_IN_BLOCK_N 1 or 2 "
           "(256 or 512 columns, one wave per 64)";
    return AXON_EINVAL;
  }
  if (qkv_wide) tn *= kQkvWideCols / 64;  // in 64-column units from here on
  if (!qkv_wide && !tile_ok(tm, tn)) {
    *why = "TILES_IN_BLOCK_M/N must each be 1, 2 or 4 (tiles of 64, 128 or 256)";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(tk, 1, 1 << 20)) {
    *why = "TILES_IN_BLOCK_K must be a positive power of two";
    return AXON_EINVAL;
  }
  // A K range of at least twice k schedules exactly like the next smaller
  // power of two: refused, so each legal tuple is a distinct schedule.
  if (tk > 1 && static_cast<int64_t>(kKUnit / 2) * tk >= K) {
    *why = "TILES_IN_BLOCK_K covers k twice over; a smaller value gives the same schedule";
    return AXON_EINVAL;
  }
  const Plan p = plan_of(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), tm, tn, tk);
  if (!grid_fits(static_cast<int64_t>(p.S) * p.MT * p.NT, 1, threads) ||
      (p.S > 1 && !grid_fits((M * N / 4 + 255) / 256, 1, 256)) ||
      (qkv_wide && !grid_fits((K + 63) / 64, static_cast<int64_t>(p.NT) * p.BN / kPackCols, 256))) {
    *why = "grid too large for one dispatch (fewer than 2^32 work-items)";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Split-K workspace layout: [partials][row sums of squares]; no initial
// content is required (every element read is written first by the same
// launch).
size_t data_bytes(const Plan& p, int M, int N, int nb) {
  if (p.S <= 1) return 0;
  return static_cast<size_t>(nb) * p.S * M * N * sizeof(float) +  // partials
         static_cast<size_t>(p.S) * p.NT * M * sizeof(float);     // row sums of squares
}

size_t gemm_workspace(int M, int N, int K, int tm, int tn, int tk, int nb) {
  const Plan p = plan_of(M, N, K, tm, tn, tk);
  return data_bytes(p, M, N, nb);
}

template <int BM, int BN, int EPI, bool AF, int PD, int NTH = kThreads>
void launch_tile(const GemmArgs& g, hipStream_t st) {
  constexpr int na = AF ? 2 : 1, nb = EPI == kSiluMul ? 2 : 1;
  const size_t lds = gemm_lds_bytes(BM, BN, na, nb, NTH);
  auto fn = gemm_kernel<BM, BN, EPI, AF, PD, NTH>;
  // Raising the dynamic LDS limit is idempotent, so a race between threads
  // doing it for the first time is harmless.
  static std::atomic<bool> configured{false};
  if (!configured.load(std::memory_order_acquire)) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                        static_cast<int>(lds));
    configured.store(true, std::memory_order_release);
  }
  const unsigned blocks = static_cast<unsigned>(g.S * g.MT * g.NT);
  if (blocks == 0) return;  // an empty output (m or n is 0 inside a composite)
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(NTH), lds, st, g);
  if (g.S > 1) {
    const int64_t quads = static_cast<int64_t>(g.M) * g.N / 4;
    hipLaunchKernelGGL(splitk_reduce_kernel<EPI>, dim3(static_cast<unsigned>((quads + 255) / 256)),
                       dim3(256), 0, st, g, BN);
  }
}

// hw variant 2 (direct-to-LDS loads): as many LDS stages as fit, at most 4.
constexpr int dma_ns(int BM, int BN) {
  return static_cast<int>(kMaxLds / (128 * static_cast<size_t>(BM + BN))) < 4
             ? static_cast<int>(kMaxLds / (128 * static_cast<size_t>(BM + BN)))
             : 4;
}

template <int BM, int BN, int EPI>
void launch_dma_tile(const GemmArgs& g, hipStream_t st) {
  constexpr int NS = dma_ns(BM, BN);
  constexpr size_t lds = dma_lds_bytes<BM, BN, NS>();
  static_assert(lds <= kMaxLds, "LDS budget");
  auto fn = gemm_dma_kernel<BM, BN, EPI, NS>;
  static std::atomic<bool> configured{false};
  if (!configured.load(std::memory_order_acquire)) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
    configured.store(true, std::memory_order_release);
  }
  const unsigned blocks = static_cast<unsigned>(g.S * g.MT * g.NT);
  if (blocks == 0) return;  // an empty output (m or n is 0 inside a composite)
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(kThreads), lds, st, g);
  if (g.S > 1) {
    const int64_t quads = static_cast<int64_t>(g.M) * g.N / 4;
    hipLaunchKernelGGL(splitk_reduce_kernel<EPI>, dim3(static_cast<unsigned>((quads + 255) / 256)),
                       dim3(256), 0, st, g, BN);
  }
}

// One GEMM launch's grids (the main kernel and, with split K, the fixup) fit
// one dispatch each.
int gemm_grid_check(const GemmArgs& g, int threads = kThreads) {
  int rc = grid_check("gemm_kernel", static_cast<int64_t>(g.S) * g.MT * g.NT, 1, threads);
  if (rc == AXON_OK && g.S > 1)
    rc = grid_check("splitk_reduce_kernel", (static_cast<int64_t>(g.M) * g.N / 4 + 255) / 256, 1, 256);
  return rc;
}

template <int EPI>
int dispatch_dma(int BM, int BN, const GemmArgs& g, hipStream_t st) {
  if (const int rc = gemm_grid_check(g); rc != AXON_OK) return rc;
#define AXON_GEMM_CASE(bm, bn) \
  if (BM == bm && BN == bn) { launch_dma_tile<bm, bn, EPI>(g, st); return launch_status("gemm_dma_kernel"); }
  AXON_GEMM_CASE(64, 64)
  AXON_GEMM_CASE(64, 128)
  AXON_GEMM_CASE(64, 256)
  AXON_GEMM_CASE(128, 64)
  AXON_GEMM_CASE(128, 128)
  AXON_GEMM_CASE(128, 256)
  AXON_GEMM_CASE(256, 64)
  AXON_GEMM_CASE(256, 128)
  AXON_GEMM_CASE(256, 256)
#undef AXON_GEMM_CASE
  set_error("no GEMM instantiation for this tile");
  return AXON_EINVAL;
}

// Prefetch depth of hw variant 1 (register sets of loads in flight).
constexpr int deep_pd(int BM, int BN) { return BM * BN <= 128 * 128 ? 3 : 2; }

// 8-wave workgroups (hw variant 3 of the plain GEMMs, 2 of the RMSNorm
// GEMMs): the schedule of hw variant 1 with a second group of 4 waves on the
// other half of every K step's k-slices, each thread loading half as much
// per K step, and 4 (up to 128 x 128) or 2 K steps of loads in flight. A CU
// takes in its L2 lines faster with 8 waves issuing loads than with 4 (the
// skinny GEMM's load stream alone: 23.9 us with 4 waves, 18.6 us with 8 at
// 4 steps in flight), and each SIMD has a second wave to issue while the
// other waits for its fragments. 256 x 256 tiles are left out: two waves of
// 128 accumulator registers each per SIMD leave too few for the staging.
constexpr int kWideThreads = 512;
constexpr int wide_pd(int BM, int BN) { return BM * BN <= 128 * 128 ? 4 : 2; }

bool wide_tile_ok(int tm, int tn) { return tile_ok(tm, tn) && tm * tn < 16; }

template <int EPI>
int dispatch_wide(int BM, int BN, const GemmArgs& g, hipStream_t st) {
  if (const int rc = gemm_grid_check(g, kWideThreads); rc != AXON_OK) return rc;
#define AXON_GEMM_CASE(bm, bn)                                                       \
  if (BM == bm && BN == bn) {                                                        \
    launch_tile<bm, bn, EPI, false, wide_pd(bm, bn), kWideThreads>(g, st);           \
    return launch_status("gemm_kernel");                                             \
  }
  AXON_GEMM_CASE(64, 64)
  AXON_GEMM_CASE(64, 128)
  AXON_GEMM_CASE(64, 256)
  AXON_GEMM_CASE(128, 64)
  AXON_GEMM_CASE(128, 128)
  AXON_GEMM_CASE(128, 256)
  AXON_GEMM_CASE(256, 64)
  AXON_GEMM_CASE(256, 128)
#undef AXON_GEMM_CASE
  set_error("no 8-wave GEMM instantiation for this tile");
  return AXON_EINVAL;
}

template <int EPI, bool AF>
int dispatch(int BM, int BN, const GemmArgs& g, hipStream_t st, int variant = 0) {
  if (const int rc = gemm_grid_check(g); rc != AXON_OK) return rc;
#define AXON_GEMM_CASE(bm, bn)                                           \
  if (BM == bm && BN == bn) {                                            \
    if (variant == 1) launch_tile<bm, bn, EPI, AF, deep_pd(bm, bn)>(g, st); \
    else launch_tile<bm, bn, EPI, AF, 1>(g, st);                         \
    return launch_status("gemm_kernel");                                 \
  }
  AXON_GEMM_CASE(64, 64)
  AXON_GEMM_CASE(64, 128)
  AXON_GEMM_CASE(64, 256)
  AXON_GEMM_CASE(128, 64)
  AXON_GEMM_CASE(128, 128)
  AXON_GEMM_CASE(128, 256)
  AXON_GEMM_CASE(256, 64)
  AXON_GEMM_CASE(256, 128)
  AXON_GEMM_CASE(256, 256)
#undef AXON_GEMM_CASE
  set_error("no GEMM instantiation for this tile");
  return AXON_EINVAL;
}

// silu_mlp keeps one register set (its dual-B stage already holds two); its
// stage tiles are narrowed to BM x BN <= 128 x 128 (and BM <= 128 in stage
// 2), so only those shapes are instantiated.
template <int EPI, bool AF>
int dispatch_mlp(int BM, int BN, const GemmArgs& g, hipStream_t st) {
  if (const int rc = gemm_grid_check(g); rc != AXON_OK) return rc;
#define AXON_GEMM_CASE(bm, bn) \
  if (BM == bm && BN == bn) { launch_tile<bm, bn, EPI, AF, 1>(g, st); return launch_status("gemm_kernel"); }
  AXON_GEMM_CASE(64, 64)
  AXON_GEMM_CASE(64, 128)
  AXON_GEMM_CASE(64, 256)
  AXON_GEMM_CASE(128, 64)
  AXON_GEMM_CASE(128, 128)
  if constexpr (!AF) AXON_GEMM_CASE(256, 64)
#undef AXON_GEMM_CASE
  set_error("no GEMM instantiation for this tile");
  return AXON_EINVAL;
}

// Fused qkv_cte GEMM (kQkv): three A loads per 8 values, so the prefetch
// depth is 2 up to 128 x 128 tiles and 1 above (register budget).
constexpr int qkv_pd(int BM, int BN) { return BM * BN <= 128 * 128 ? 2 : 1; }

int dispatch_qkv(int BM, int BN, const GemmArgs& g, hipStream_t st) {
  if (const int rc = gemm_grid_check(g); rc != AXON_OK) return rc;
#define AXON_GEMM_CASE(bm, bn)                                   \
  if (BM == bm && BN == bn) {                                    \
    launch_tile<bm, bn, kQkv, false, qkv_pd(bm, bn)>(g, st);     \
    return launch_status("gemm_kernel");                         \
  }
  AXON_GEMM_CASE(64, 64)
  AXON_GEMM_CASE(64, 128)
  AXON_GEMM_CASE(64, 256)
  AXON_GEMM_CASE(128, 64)
  AXON_GEMM_CASE(128, 128)
  AXON_GEMM_CASE(128, 256)
  AXON_GEMM_CASE(256, 64)
  AXON_GEMM_CASE(256, 128)
  AXON_GEMM_CASE(256, 256)
#undef AXON_GEMM_CASE
  set_error("no GEMM instantiation for this tile");
  return AXON_EINVAL;
}

// qkv_cte hw variant 3: pack w, then the full-width GEMM, then (split K) the
// fixup. Every grid is checked before the first launch.
template <int BM, int NW>
void launch_qkv_wide(const GemmArgs& g, const u32x4* wp, int nct, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>(g.S * g.MT * g.NT);
  hipLaunchKernelGGL((qkv_wide_kernel<BM, NW>), dim3(blocks), dim3(64 * NW), 0, st, g, wp, nct);
  if (g.S > 1) {
    const int64_t quads = static_cast<int64_t>(g.M) * g.N / 4;
    hipLaunchKernelGGL(splitk_reduce_kernel<kQkv>, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                       st, g, 64 * NW);
  }
}

int dispatch_qkv_wide(int BM, int BN, const GemmArgs& g, const bf16* w, u32x4* wp, int kp64, int np, int nct,
                      hipStream_t st) {
  if (const int rc = gemm_grid_check(g, BN); rc != AXON_OK) return rc;
  if (const int rc = grid_check("qkv_pack_w_kernel", kp64 / 64, np / kPackCols, 256); rc != AXON_OK) return rc;
  if (kp64 > 0) {
    hipLaunchKernelGGL(qkv_pack_w_kernel, dim3(static_cast<unsigned>(kp64 / 64), static_cast<unsigned>(np / kPackCols)),
                       dim3(256), 0, st, w, wp, g.K, g.N, nct);
    if (const int rc = launch_status("qkv_pack_w_kernel"); rc != AXON_OK) return rc;
  }
#define AXON_QKV_WIDE_CASE(bm, bn)                                          \
  if (BM == bm && BN == bn) {                                               \
    launch_qkv_wide<bm, bn / 64>(g, wp, nct, st);                           \
    return launch_status("qkv_wide_kernel");                                \
  }
  AXON_QKV_WIDE_CASE(64, 256)
  AXON_QKV_WIDE_CASE(64, 512)
  AXON_QKV_WIDE_CASE(128, 256)
  AXON_QKV_WIDE_CASE(128, 512)
#undef AXON_QKV_WIDE_CASE
  set_error("no qkv_cte hw variant 3 instantiation for this tile");
  return AXON_EINVAL;
}

// Fills a GemmArgs for C = A @ B (+ epilogue); `data` is the partial/row-sum
// region (unused when the plan has S == 1).
GemmArgs make_args(const void* A, const bf16* B, const bf16* B2, void* C, int M, int N, int K,
                   const Plan& p, void* data, int nb, float eps) {
  GemmArgs g{};
  g.A = A;
  g.B = B;
  g.B2 = B2;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.kchunk = p.kchunk;
  g.S = p.S;
  g.MT = p.MT;
  g.NT = p.NT;
  g.eps = eps;
  if (p.S > 1) {
    char* w = static_cast<char*>(data);
    g.partial = reinterpret_cast<float*>(w);
    g.rowsq = reinterpret_cast<float*>(w + static_cast<size_t>(nb) * p.S * M * N * sizeof(float));
  }
  return g;
}

// ---- matmul-like families (dims m, n, k; inputs x[m,k], w[k,n]) ----------
template <int EPI>
int check_mm(const Call& c, std::string* why) {
  if (c.n_tiles != 3 || c.n_dims != 3 || c.n_dtypes != 2) {
    *why = "expected 3 tiles, 3 dims (m, n, k) and 2 dtypes";
    return AXON_EARG;
  }
  if (c.dtype(0) != AXON_BF16 || c.dtype(1) != AXON_BF16) {
    *why = "bf16 inputs only";
    return AXON_EDTYPE;
  }
  // softmax_mm (two hw variants) has no 8-wave schedule.
  const bool wide = EPI != kSoftmax && c.variant == 2;
  if (wide && !wide_tile_ok(c.tile(0), c.tile(1))) {
    *why = "8-wave tiles go up to 256 x 128: TILES_IN_BLOCK_M/N each 1, 2 or 4 with a "
           "product below 16";
    return AXON_EINVAL;
  }
  return check_gemm_shape(c.dim(0), c.dim(1), c.dim(2), c.tile(0), c.tile(1), c.tile(2), why,
                          wide ? kWideThreads : kThreads);
}

// Manifest extent of TILES_IN_BLOCK_K for a contraction of length K: the
// smallest power-of-two multiple of 256 that covers K. A K range need not
// divide K (the last one may be ragged), and check_gemm_shape admits exactly
// the power-of-two ranges up to this extent.
int64_t k_extent(int64_t K) {
  int64_t units = (K + kKUnit - 1) / kKUnit, p = 1;
  while (p < units) p <<= 1;
  return kKUnit * p;
}

int manifest_mm(int, const int64_t* dims, int, Constraint* out, int cap) {
  if (cap < 3) return 0;
  const int64_t m = dims[0] > 0 ? dims[0] : 1, n = dims[1] > 0 ? dims[1] : 1;
  // Tiles of 64..256 that fit the extent (a 64-wide tile is always allowed).
  out[0] = {"TILES_IN_BLOCK_M", m < 256 ? (m < 64 ? 64 : m) : 256, 64, false};
  out[1] = {"TILES_IN_BLOCK_N", n < 256 ? (n < 64 ? 64 : n) : 256, 64, false};
  out[2] = {"TILES_IN_BLOCK_K", k_extent(dims[2]), kKUnit, false};
  return 3;
}

// Occupancy box of a split-K GEMM (C[m, n] over K). The budgeted selection
// (src/axon/candidate_filter.py:106-173 of the reference) seeds the corners of
// the admitted box first, so with three tile arguments and the default budget
// of 8 it benches only corners: over the full 64..256 x 64..256 x 256..K box
// those are the 64 x 64 tiles with one K range (too little work per
// workgroup) and the 256 x 256 tiles over all of K (a handful of workgroups on
// 256 CUs). The box is therefore capped where a workgroup grid stops filling
// the chip: BM x BN is the largest output tile (squarest on ties) that still
// leaves kMinOutputTiles tiles, and the K range the deepest power-of-two
// multiple of 256 that still gives those tiles kMinGroups workgroups. A
// shape too small for either keeps the 64-wide tile and one K unit. Tuples
// outside the box stay legal (check_gemm_shape accepts them) and reachable
// with the candidate filter off.
constexpr int64_t kMinOutputTiles = 32;
constexpr int64_t kMinGroups = 256;

int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

void cap_for_occupancy(int64_t m, int64_t n, int64_t K, Constraint* out) {
  m = std::max<int64_t>(m, 1);
  n = std::max<int64_t>(n, 1);
  int64_t bm = 64, bn = 64, tiles = cdiv64(m, 64) * cdiv64(n, 64);
  for (const int64_t a : {64, 128, 256})
    for (const int64_t b : {64, 128, 256}) {
      const int64_t t = cdiv64(m, a) * cdiv64(n, b);
      const bool larger = a * b > bm * bn || (a * b == bm * bn && std::llabs(a - b) < std::llabs(bm - bn));
      if (t >= kMinOutputTiles && larger) {
        bm = a;
        bn = b;
        tiles = t;
      }
    }
  const int64_t kext = k_extent(K);
  int64_t range = kKUnit;
  while (range * 2 <= kext && tiles * cdiv64(std::max<int64_t>(K, 1), range * 2) >= kMinGroups) range *= 2;
  out[0].extent = std::min(out[0].extent, bm);
  out[1].extent = std::min(out[1].extent, bn);
  out[2].extent = std::min(out[2].extent, range);
}

// Manifest of the plain split-K GEMMs (matmul, rmsnorm_matmul, qkv_cte):
// every legal tuple inside the occupancy box.
int manifest_splitk(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  const int n = manifest_mm(v, dims, dt, out, cap);
  if (n == 3) cap_for_occupancy(dims[0], dims[1], dims[2], out);
  return n;
}

// The plain matmul families have a third hw variant (direct-to-LDS loads)
// that needs whole 64-deep K steps, and a fourth with 8-wave workgroups;
// the RMSNorm GEMMs have the 8-wave schedule as their third.
constexpr int kDmaVariant = 2;
template <int EPI>
constexpr int wide_variant() { return EPI == kPlain ? 3 : 2; }

int check_wide_tile(const Call& c, std::string* why) {
  if (!wide_tile_ok(c.tile(0), c.tile(1))) {
    *why = "8-wave tiles go up to 256 x 128: TILES_IN_BLOCK_M/N each 1, 2 or 4 with a "
           "product below 16";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

// fp32 inputs (hw variants 0 and 1): a prep pass splits x into bf16 rows
// [hi | lo | hi] and w into planes [hi; hi; lo], and the bf16 GEMM over
// K' = 3k sums hi*hi + lo*hi + hi*lo with an fp32 output, leaving out only
// the lo*lo term (about 2^-16 relative).
int plain_kp(int64_t k, int dtype) { return static_cast<int>(dtype == AXON_F32 ? 3 * k : k); }

int check_plain(const Call& c, std::string* why) {
  if (c.n_tiles != 3 || c.n_dims != 3 || c.n_dtypes != 2) {
    *why = "expected 3 tiles, 3 dims (m, n, k) and 2 dtypes";
    return AXON_EARG;
  }
  const int dt = c.dtype(0);
  if ((dt != AXON_BF16 && dt != AXON_F32) || c.dtype(1) != dt) {
    *why = "x and w must both be bf16 or both fp32";
    return AXON_EDTYPE;
  }
  if (dt == AXON_F32) {
    if (c.variant == kDmaVariant || c.variant == wide_variant<kPlain>()) {
      *why = "hw variants 2 and 3 have no fp32 instantiation; fp32 inputs use hw variants 0 and 1";
      return AXON_EDTYPE;
    }
    if (c.dim(2) % 8 != 0 || c.dim(2) > (1 << 28)) {
      *why = "fp32 inputs need k % 8 == 0 (16-byte groups of one row) and k < 2^28";
      return AXON_EINVAL;
    }
  }
  const bool wide = c.variant == wide_variant<kPlain>();
  if (wide) {
    const int rc = check_wide_tile(c, why);
    if (rc != AXON_OK) return rc;
  }
  const int rc = check_gemm_shape(c.dim(0), c.dim(1), plain_kp(c.dim(2), dt), c.tile(0), c.tile(1),
                                  c.tile(2), why, wide ? kWideThreads : kThreads);
  if (rc != AXON_OK) return rc;
  if (c.variant == kDmaVariant && c.dim(2) % BK != 0) {
    *why = "hw variant 2 loads whole 64-deep K steps: k must be a multiple of 64";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

// The 8-wave schedule stops at 256 x 128 tiles: its manifest caps BN at 128
// so the box never admits 256 x 256 (128 x 256 and 64 x 256 stay legal,
// reachable with the candidate filter off).
void cap_wide(Constraint* out, int n) {
  if (n >= 2) out[1].extent = std::min<int64_t>(out[1].extent, 128);
}

int manifest_rms(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  const int n = manifest_splitk(v, dims, dt, out, cap);
  if (v == wide_variant<kRmsEps>()) cap_wide(out, n);
  return n;
}

int manifest_plain(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  const int64_t mnk[3] = {dims[0], dims[1], dt == AXON_F32 ? 3 * dims[2] : dims[2]};
  const int n = manifest_splitk(v, mnk, dt, out, cap);
  if (v == wide_variant<kPlain>()) cap_wide(out, n);
  if ((v == kDmaVariant && (dims[2] % BK != 0 || dt == AXON_F32)) || (v == wide_variant<kPlain>() && dt == AXON_F32))
    for (int i = 0; i < n; ++i) out[i].extent = 0;  // admits no tile
  return n;
}

struct PlainLayout {
  Plan p;
  int kp;
  size_t a, b, data, total;  // byte offsets: A' [m][K'], B' [K'][n] (fp32 only), split-K data
};

PlainLayout plain_layout(const Call& c) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1));
  PlainLayout L;
  L.kp = plain_kp(c.dim(2), c.dtype(0));
  L.p = plan_of(m, n, L.kp, c.tile(0), c.tile(1), c.tile(2));
  L.a = L.b = L.data = 0;
  if (c.dtype(0) == AXON_F32) {
    L.b = align256(static_cast<size_t>(m) * L.kp * sizeof(bf16));
    L.data = L.b + align256(static_cast<size_t>(L.kp) * n * sizeof(bf16));
  }
  L.total = L.data + data_bytes(L.p, m, n, 1);
  return L;
}

size_t workspace_plain(const Call& c) { return plain_layout(c).total; }

template <int EPI>
int launch_mm(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st);

int launch_plain(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  if (c.dtype(0) != AXON_F32) return launch_mm<kPlain>(c, in, out, ws, st);
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1)), k = static_cast<int>(c.dim(2));
  if (m == 0 || n == 0) return AXON_OK;
  if (!aligned16(in[0]) || !aligned16(in[1]) || !aligned16(out[0])) {
    set_error("GEMM buffers must be 16-byte aligned");
    return AXON_EARG;
  }
  const PlainLayout L = plain_layout(c);
  char* base = static_cast<char*>(ws);
  bf16* a = reinterpret_cast<bf16*>(base + L.a);
  bf16* b = reinterpret_cast<bf16*>(base + L.b);
  const int64_t mk = static_cast<int64_t>(m) * k, kn = static_cast<int64_t>(k) * n;
  if (mk > 0) {
    int rc = grid_check("split_rows_hilo_kernel", (mk / 8 + 255) / 256, 1, 256);
    if (rc == AXON_OK) rc = grid_check("qkv_split_w_kernel", (kn / 8 + 255) / 256, 1, 256);
    if (rc != AXON_OK) return rc;
    hipLaunchKernelGGL(split_rows_hilo_kernel, dim3(static_cast<unsigned>((mk / 8 + 255) / 256)), dim3(256), 0,
                       st, static_cast<const float*>(in[0]), a, mk, k);
    rc = launch_status("split_rows_hilo_kernel");
    if (rc != AXON_OK) return rc;
    hipLaunchKernelGGL(qkv_split_w_kernel, dim3(static_cast<unsigned>((kn / 8 + 255) / 256)), dim3(256), 0, st,
                       static_cast<const float*>(in[1]), b, kn);
    rc = launch_status("qkv_split_w_kernel");
    if (rc != AXON_OK) return rc;
  }
  GemmArgs g = make_args(a, b, nullptr, out[0], m, n, L.kp, L.p, base + L.data, 1, 1e-6f);
  g.c_f32 = 1;
  return dispatch<kPlain, false>(L.p.BM, L.p.BN, g, st, c.variant);
}

template <int EPI>
size_t workspace_mm(const Call& c) {
  return gemm_workspace(static_cast<int>(c.dim(0)), static_cast<int>(c.dim(1)),
                        static_cast<int>(c.dim(2)), c.tile(0), c.tile(1), c.tile(2), 1);
}

// fp32 output for fp32 inputs (only the plain matmul families accept them).
void outputs_mm(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, dtypes[0] == AXON_F32 ? AXON_F32 : AXON_BF16};
}

template <int EPI>
int launch_mm(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  const int M = static_cast<int>(c.dim(0)), N = static_cast<int>(c.dim(1)), K = static_cast<int>(c.dim(2));
  if (M == 0 || N == 0) return AXON_OK;
  if (!aligned16(in[0]) || !aligned16(in[1]) || !aligned16(out[0])) {
    set_error("GEMM buffers must be 16-byte aligned");
    return AXON_EARG;
  }
  const Plan p = plan_of(M, N, K, c.tile(0), c.tile(1), c.tile(2));
  const GemmArgs g = make_args(in[0], static_cast<const bf16*>(in[1]), nullptr, out[0], M, N, K, p, ws,
                               1, 1e-6f);
  if constexpr (EPI == kPlain) {
    if (c.variant == kDmaVariant) return dispatch_dma<kPlain>(p.BM, p.BN, g, st);
  }
  if constexpr (EPI == kPlain || EPI == kRmsSum || EPI == kRmsEps) {
    if (c.variant == wide_variant<EPI>()) return dispatch_wide<EPI>(p.BM, p.BN, g, st);
  }
  return dispatch<EPI, false>(p.BM, p.BN, g, st, c.variant);
}

const char* summary_wide() {
  return "bf16 MFMA 32x32x16, 8 waves per BMxBN tile (two groups of 2x2 waves on the two halves of "
         "every K step's k-slices, summed through LDS at the end), 4 K steps (2 above 128x128 tiles) "
         "of global loads in flight in rotating register sets, LDS double "
         "buffer with B staged as loaded and read by the transposing LDS read, split-K with a parallel "
         "fixup kernel, XCD-grouped K ranges, fused row-scale epilogue";
}

// RMSNorm GEMMs: hw variants 0 and 1 as the plain GEMM's, 2 = 8-wave.
const char* summary_mm(int variant);
const char* summary_rms(int variant) { return variant == 2 ? summary_wide() : summary_mm(variant); }

const char* summary_mm(int variant) {
  if (variant == 3) return summary_wide();
  if (variant == kDmaVariant)
    return "bf16 MFMA 32x32x16, 4 waves per BMxBN tile, A and B tiles loaded straight into LDS "
           "(global_load_lds_dwordx4, chunk-swizzled stages, up to 4 stages = 3 K steps in flight), "
           "B fragments by the transposing LDS read, split-K with a parallel fixup kernel, XCD-grouped "
           "K ranges; needs k % 64 == 0";
  return variant == 1
             ? "bf16 MFMA 32x32x16, 4 waves per BMxBN tile, 2-3 K steps of global loads in flight in "
               "rotating register sets, LDS double buffer with B staged as loaded and read by the "
               "transposing LDS read, split-K with a parallel fixup kernel, XCD-grouped K ranges, fused "
               "row-scale epilogue"
             : "bf16 MFMA 32x32x16, 4 waves per BMxBN tile, one K step of loads in flight refilled "
               "vector by vector with the MFMAs sliced between the A stores, LDS double buffer with B "
               "staged as loaded, split-K with a parallel fixup kernel, XCD-grouped K ranges, fused "
               "row-scale epilogue";
}

// ---- silu_mlp (dims m, n, k, p; x[m,k], w1[k,n], w2[k,n], w3[n,p]) --------
int check_mlp(const Call& c, std::string* why) {
  if (c.n_tiles != 4 || c.n_dims != 4 || c.n_dtypes != 4) {
    *why = "expected 4 tiles, 4 dims (m, n, k, p) and 4 dtypes";
    return AXON_EARG;
  }
  for (int i = 0; i < 4; ++i)
    if (c.dtype(i) != AXON_BF16) {
      *why = "bf16 inputs only";
      return AXON_EDTYPE;
    }
  const int64_t m = c.dim(0), n = c.dim(1), k = c.dim(2), p = c.dim(3);
  // Stage 1 (k-contraction) uses M/N/K tiles; stage 2 (n-contraction) uses
  // M/P tiles with the same K range (both narrowed by mlp_tiles).
  int rc = check_gemm_shape(m, n, k, c.tile(0), c.tile(1), c.tile(2), why);
  if (rc != AXON_OK) return rc;
  return check_gemm_shape(m, p, n, c.tile(0), c.tile(3), c.tile(2), why);
}

// Tiles (64-units) the two silu_mlp stages run with: stage 1 holds two
// accumulator sets and two B planes, so BN <= 128 and BM x BN <= 128 x 128;
// stage 2 holds two A planes (fp32 H as bf16 hi + lo), so BM <= 128 and
// BM x BP <= 128 x 128. Larger requested tiles are narrowed to these.
struct MlpTiles {
  int tm1, tn1, tm2, tp2;
};

MlpTiles mlp_tiles(const Call& c) {
  MlpTiles t;
  t.tm1 = c.tile(0);
  t.tn1 = std::max(1, std::min({c.tile(1), 2, 4 / t.tm1}));
  t.tm2 = std::min(c.tile(0), 2);
  t.tp2 = std::max(1, std::min(c.tile(3), 4 / t.tm2));
  return t;
}

int manifest_mlp(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  if (cap < 4) return 0;
  // The K range serves both contractions (over k, then over n).
  const int64_t mnk[3] = {dims[0], dims[1], std::min(dims[1], dims[2])};
  manifest_mm(v, mnk, dt, out, cap);
  const int64_t p = dims[3] > 0 ? dims[3] : 1;
  out[3] = {"TILES_IN_BLOCK_P", p < 256 ? (p < 64 ? 64 : p) : 256, 64, false};
  return 4;
}

struct MlpLayout {
  Plan p1, p2;
  size_t h, data;
};

// silu_mlp workspace: [H fp32 m x n][split-K data of whichever stage needs more].
MlpLayout mlp_layout(const Call& c) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1));
  const int k = static_cast<int>(c.dim(2)), p = static_cast<int>(c.dim(3));
  const MlpTiles t = mlp_tiles(c);
  MlpLayout L;
  L.p1 = plan_of(m, n, k, t.tm1, t.tn1, c.tile(2));
  L.p2 = plan_of(m, p, n, t.tm2, t.tp2, c.tile(2));
  L.h = align256(static_cast<size_t>(m) * n * sizeof(float));
  const size_t d1 = data_bytes(L.p1, m, n, 2), d2 = data_bytes(L.p2, m, p, 1);
  L.data = d1 > d2 ? d1 : d2;
  return L;
}

size_t workspace_mlp(const Call& c) {
  const MlpLayout L = mlp_layout(c);
  return L.h + L.data;
}

void outputs_mlp(const int64_t* dims, const int32_t*, OutDesc* out) {
  out[0] = {2, {dims[0], dims[3]}, AXON_BF16};
}

int launch_mlp(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1));
  const int k = static_cast<int>(c.dim(2)), p = static_cast<int>(c.dim(3));
  if (m == 0 || p == 0) return AXON_OK;
  for (int i = 0; i < 4; ++i)
    if (!aligned16(in[i])) {
      set_error("GEMM buffers must be 16-byte aligned");
      return AXON_EARG;
    }
  const MlpLayout L = mlp_layout(c);
  if (!aligned16(out[0]) || (ws == nullptr && L.h + L.data > 0)) {
    set_error("silu_mlp needs an aligned output and its workspace");
    return AXON_EARG;
  }
  char* base = static_cast<char*>(ws);
  float* H = reinterpret_cast<float*>(base);
  void* data = base + L.h;
  // n == 0: H is empty and the second product (over n) is all zeros.
  if (n > 0) {
    const GemmArgs g1 = make_args(in[0], static_cast<const bf16*>(in[1]), static_cast<const bf16*>(in[2]),
                                  H, m, n, k, L.p1, data, 2, 0.f);
    const int rc = dispatch_mlp<kSiluMul, false>(L.p1.BM, L.p1.BN, g1, st);
    if (rc != AXON_OK) return rc;
  }
  const GemmArgs g2 = make_args(H, static_cast<const bf16*>(in[3]), nullptr, out[0], m, p, n, L.p2,
                                data, 1, 0.f);
  return dispatch_mlp<kPlain, true>(L.p2.BM, L.p2.BN, g2, st);
}

const char* summary_mlp(int) {
  return "stage 1: one MFMA pass over x with both w1 and w2 tiles, H = silu(x w1) * (x w2) kept in "
         "fp32; stage 2: H split into bf16 hi + lo planes (two MFMAs per step) times w3";
}

// ---- qkv_cte (dims m, n, k; x, mlp_prev, attention_prev [m,k], w [k,n]) --
// hw variants 0 and 1: a prep pass writes the GEMM operand, then the GEMM of
// that hw variant runs over K' = k (bf16) or 3k (fp32 hi|lo|hi planes).
// hw variant 2 (bf16 only): no prep pass; the GEMM's A loads read the three
// residual inputs and sum them (kQkv), K' = k.
// hw variant 3 (bf16 only): as 2, over full-width N tiles with w packed into
// MFMA operand order by a pre-pass (qkv_wide_kernel).
constexpr int kQkvFused = 2;
constexpr int kQkvWide = 3;

int qkv_kp(int64_t k, int dtype) { return static_cast<int>(dtype == AXON_F32 ? 3 * k : k); }

int check_qkv(const Call& c, std::string* why) {
  if (c.n_tiles != 3 || c.n_dims != 3 || c.n_dtypes != 4) {
    *why = "expected 3 tiles, 3 dims (m, n, k) and 4 dtypes";
    return AXON_EARG;
  }
  const int dt = c.dtype(0);
  if (dt != AXON_BF16 && dt != AXON_F32) {
    *why = "bf16 or fp32 inputs only";
    return AXON_EDTYPE;
  }
  for (int i = 1; i < 4; ++i)
    if (c.dtype(i) != dt) {
      *why = "all four inputs must share one dtype";
      return AXON_EDTYPE;
    }
  if ((c.variant == kQkvFused || c.variant == kQkvWide) && dt != AXON_BF16) {
    *why = "hw variants 2 and 3 sum bf16 residual inputs inside the GEMM; fp32 inputs use hw variants 0 and 1";
    return AXON_EDTYPE;
  }
  if (c.dim(2) > (1 << 28)) {
    *why = "k out of range";
    return AXON_EINVAL;
  }
  if (c.variant == kQkvWide)
    return check_gemm_shape(c.dim(0), c.dim(1), c.dim(2), c.tile(0), c.tile(1), c.tile(2), why,
                            kQkvWideCols * c.tile(1), true);
  return check_gemm_shape(c.dim(0), c.dim(1), qkv_kp(c.dim(2), dt), c.tile(0), c.tile(1), c.tile(2), why);
}

int manifest_qkv(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  const int64_t mnk[3] = {dims[0], dims[1], dt == AXON_F32 ? 3 * dims[2] : dims[2]};
  int n = 0;
  if (v == kQkvWide) {
    if (cap < 3) return 0;
    // Tiles of 64 or 128 rows and 256 or 512 columns (N counted in units of
    // 256); K range capped where the grid of the largest tile stops reaching
    // kMinGroups workgroups.
    const int64_t m = std::max<int64_t>(dims[0], 1), nn = std::max<int64_t>(dims[1], 1);
    const int64_t bm = m >= 128 ? 128 : 64, bn = nn > 256 ? 512 : 256;
    const int64_t tiles = cdiv64(m, bm) * cdiv64(nn, bn), K = std::max<int64_t>(dims[2], 1);
    const int64_t kext = k_extent(dims[2]);
    int64_t range = kKUnit;
    while (range * 2 <= kext && tiles * cdiv64(K, range * 2) >= kMinGroups) range *= 2;
    out[0] = {"TILES_IN_BLOCK_M", bm, 64, false};
    out[1] = {"TILES_IN_BLOCK_N", bn, kQkvWideCols, false};
    out[2] = {"TILES_IN_BLOCK_K", range, kKUnit, false};
    n = 3;
  } else {
    n = manifest_splitk(v, mnk, dt, out, cap);
  }
  // The fused variants have no fp32 instantiation: an extent of 0 admits no tile.
  if ((v == kQkvFused || v == kQkvWide) && dt != AXON_BF16)
    for (int i = 0; i < n; ++i) out[i].extent = 0;
  return n;
}

struct QkvLayout {
  Plan p;
  int kp;
  size_t scale, a, b, data;  // byte offsets of each region
  size_t total;
};

// qkv_cte workspace: [row scales fp32 m][A' bf16 m x K'][B' bf16 K' x n
// (fp32 inputs only)][split-K data of the GEMM over K']. hw variant 2: the
// split-K data only; hw variant 3: [packed w, Kp x Np bf16 (Kp = k rounded up
// to 64, Np = N tiles x BN)][split-K data].
QkvLayout qkv_layout(const Call& c) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1));
  QkvLayout L;
  L.kp = qkv_kp(c.dim(2), c.dtype(0));
  L.p = plan_of(m, n, L.kp, c.tile(0), c.variant == kQkvWide ? c.tile(1) * (kQkvWideCols / 64) : c.tile(1),
                c.tile(2));
  L.scale = 0;
  if (c.variant == kQkvFused) {  // split-K data only
    L.a = L.b = L.data = 0;
    L.total = data_bytes(L.p, m, n, 1);
    return L;
  }
  if (c.variant == kQkvWide) {
    L.a = L.b = 0;
    const size_t kp64 = (static_cast<size_t>(c.dim(2)) + 63) / 64 * 64;
    L.data = align256(kp64 * static_cast<size_t>(L.p.NT) * L.p.BN * sizeof(bf16));
    L.total = L.data + data_bytes(L.p, m, n, 1);
    return L;
  }
  L.a = align256(static_cast<size_t>(m) * sizeof(float));
  L.b = L.a + align256(static_cast<size_t>(m) * L.kp * sizeof(bf16));
  const size_t bbytes = c.dtype(0) == AXON_F32 ? align256(static_cast<size_t>(L.kp) * n * sizeof(bf16)) : 0;
  L.data = L.b + bbytes;
  L.total = L.data + data_bytes(L.p, m, n, 1);
  return L;
}

size_t workspace_qkv(const Call& c) { return qkv_layout(c).total; }

void outputs_qkv(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, dtypes[0]};
}

int launch_qkv(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1)), k = static_cast<int>(c.dim(2));
  if (m == 0 || n == 0) return AXON_OK;
  for (int i = 0; i < 4; ++i)
    if (!aligned16(in[i])) {
      set_error("qkv_cte buffers must be 16-byte aligned");
      return AXON_EARG;
    }
  const QkvLayout L = qkv_layout(c);
  if (!aligned16(out[0]) || (ws == nullptr && L.total > 0)) {
    set_error("qkv_cte needs an aligned output and its workspace");
    return AXON_EARG;
  }
  const float eps = 1e-6f;
  if (c.variant == kQkvWide) {
    const int kp64 = (k + 63) / 64 * 64, np = L.p.NT * L.p.BN, nct = np / 32;
    u32x4* wp = static_cast<u32x4*>(ws);
    char* base = static_cast<char*>(ws);
    GemmArgs g = make_args(in[0], nullptr, nullptr, out[0], m, n, k, L.p, base + L.data, 1, eps);
    g.A2 = static_cast<const bf16*>(in[1]);
    g.A3 = static_cast<const bf16*>(in[2]);
    return dispatch_qkv_wide(L.p.BM, L.p.BN, g, static_cast<const bf16*>(in[3]), wp, kp64, np, nct, st);
  }
  if (c.variant == kQkvFused) {
    GemmArgs g = make_args(in[0], static_cast<const bf16*>(in[3]), nullptr, out[0], m, n, k, L.p, ws, 1, eps);
    g.A2 = static_cast<const bf16*>(in[1]);
    g.A3 = static_cast<const bf16*>(in[2]);
    return dispatch_qkv(L.p.BM, L.p.BN, g, st);
  }
  const bool f32 = c.dtype(0) == AXON_F32;
  {
    int rc = grid_check("qkv_prep_kernel", m, 1, kPrepThreads);
    if (rc == AXON_OK && f32) rc = grid_check("qkv_split_w_kernel", (static_cast<int64_t>(k) * n / 8 + 255) / 256, 1, 256);
    if (rc != AXON_OK) return rc;
  }
  char* base = static_cast<char*>(ws);
  float* scale = reinterpret_cast<float*>(base + L.scale);
  bf16* a = reinterpret_cast<bf16*>(base + L.a);
  const bf16* b = static_cast<const bf16*>(in[3]);
  if (f32) {
    hipLaunchKernelGGL(qkv_prep_kernel<float>, dim3(m), dim3(kPrepThreads), 0, st,
                       static_cast<const float*>(in[0]), static_cast<const float*>(in[1]),
                       static_cast<const float*>(in[2]), a, scale, k, eps);
    const int64_t kn = static_cast<int64_t>(k) * n;
    bf16* bs = reinterpret_cast<bf16*>(base + L.b);
    if (kn > 0)
      hipLaunchKernelGGL(qkv_split_w_kernel, dim3(static_cast<unsigned>((kn / 8 + 255) / 256)), dim3(256), 0, st,
                         static_cast<const float*>(in[3]), bs, kn);
    b = bs;
  } else {
    hipLaunchKernelGGL(qkv_prep_kernel<bf16>, dim3(m), dim3(kPrepThreads), 0, st,
                       static_cast<const bf16*>(in[0]), static_cast<const bf16*>(in[1]),
                       static_cast<const bf16*>(in[2]), a, scale, k, eps);
  }
  int rc = launch_status("qkv_prep_kernel");
  if (rc != AXON_OK) return rc;
  GemmArgs g = make_args(a, b, nullptr, out[0], m, n, L.kp, L.p, base + L.data, 1, eps);
  g.rscale = scale;
  g.c_f32 = f32 ? 1 : 0;
  return dispatch<kPlain, false>(L.p.BM, L.p.BN, g, st, c.variant);
}

const char* summary_qkv(int variant) {
  if (variant == kQkvWide)
    return "bf16 only: the fused residual sum of hw variant 2 over full-width N tiles (TILES_IN_BLOCK_M "
           "x 64 rows by TILES_IN_BLOCK_N x 256 columns, one wave per 64 columns), so each residual row is "
           "read once per K range; "
           "A staged in LDS, w packed by a pre-pass into MFMA operand order and loaded straight into "
           "registers (one contiguous KiB per wave load), split-K fixup applies the row scale";
  if (variant == kQkvFused)
    return "bf16 only: one GEMM whose A loads read x, mlp_prev and attention_prev and add them in "
           "fp32 (sum of squares taken on the fly, as rmsnorm_matmul_eps), so the residual sum never "
           "touches HBM; 1-2 K steps of loads in flight, split-K fixup applies the row scale";
  return variant == 1
             ? "prep: one pass over the three residual inputs writes the bf16 GEMM operand (fp32: "
               "hi|lo|hi planes, w as hi;hi;lo) and the row scale; GEMM as matmul hw variant 1 with "
               "the row scale applied in the epilogue"
             : "prep: one pass over the three residual inputs writes the bf16 GEMM operand (fp32: "
               "hi|lo|hi planes, w as hi;hi;lo) and the row scale; GEMM as matmul hw variant 0 with "
               "the row scale applied in the epilogue";
}

// ---- transposes between GEMM stages ---------------------------------------
// out[c][r] = in[r][c] for a [R, C] bf16 matrix, through a 64 x 64 LDS tile
// (row pitch 66 elements: the column reads of one wave touch distinct banks).
constexpr int kTp = 64;

// Grid: x over row tiles (the long side here: sequence positions), y over
// column tiles.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const bf16* __restrict__ in,
                                                            bf16* __restrict__ out, int R, int C) {
  __shared__ bf16 tile[kTp][kTp + 2];
  const int r0 = blockIdx.x * kTp, c0 = blockIdx.y * kTp;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < kTp; i += 4) {
    const int r = r0 + ty + i, c = c0 + tx;
    tile[ty + i][tx] = (r < R && c < C) ? in[static_cast<int64_t>(r) * C + c] : static_cast<bf16>(0.f);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTp; i += 4) {
    const int c = c0 + ty + i, r = r0 + tx;
    if (c < C && r < R) out[static_cast<int64_t>(c) * R + r] = tile[tx][ty + i];
  }
}

// The same 64 x 64 tiles moved as 16-byte vectors when R and C are
// multiples of 8 (every vector then lies wholly inside or outside the
// matrix): two vector loads and two vector stores per thread instead of
// sixteen 2-byte ones each. The LDS row pitch of 66 elements (33 words)
// spreads the eight rows a column read gathers over distinct banks.
__global__ __launch_bounds__(256) void transpose_bf16_vec_kernel(const bf16* __restrict__ in,
                                                                bf16* __restrict__ out, int R, int C) {
  constexpr int P = kTp + 2;
  __shared__ __align__(16) bf16 tile[kTp * P];
  const int r0 = blockIdx.x * kTp, c0 = blockIdx.y * kTp;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int v = threadIdx.x + k * 256;
    const int row = v >> 3, ch = v & 7;
    const int r = r0 + row, c = c0 + ch * 8;
    Vec<bf16> x;
    if (r < R && c < C) {
      x = load_vec(in + static_cast<int64_t>(r) * C + c);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x.v[e] = static_cast<bf16>(0.f);
    }
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&x);
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<uint32_t*>(&tile[row * P + ch * 8 + 2 * q]) = w[q];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int v = threadIdx.x + k * 256;
    const int orow = v >> 3, ch = v & 7;  // output row = input column c0 + orow
    const int c = c0 + orow, r = r0 + ch * 8;
    if (c >= C || r >= R) continue;
    Vec<bf16> y;
#pragma unroll
    for (int e = 0; e < 8; ++e) y.v[e] = tile[(ch * 8 + e) * P + orow];
    store_vec(out + static_cast<int64_t>(c) * R + r, y);
  }
}

int launch_transpose(const bf16* in, bf16* out, int R, int C, hipStream_t st) {
  if (R == 0 || C == 0) return AXON_OK;
  if (const int rc = grid_check("transpose_bf16_kernel", (R + kTp - 1) / kTp, (C + kTp - 1) / kTp, 256);
      rc != AXON_OK)
    return rc;
  const dim3 grid((R + kTp - 1) / kTp, (C + kTp - 1) / kTp);
  const bool vec = R % 8 == 0 && C % 8 == 0 && aligned16(in) && aligned16(out);
  if (vec) hipLaunchKernelGGL(transpose_bf16_vec_kernel, grid, dim3(256), 0, st, in, out, R, C);
  else hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, st, in, out, R, C);
  return launch_status("transpose_bf16_kernel");
}

int check_all_bf16(const Call& c, int n, std::string* why) {
  for (int i = 0; i < n; ++i)
    if (c.dtype(i) != AXON_BF16) {
      *why = "bf16 inputs only";
      return AXON_EDTYPE;
    }
  return AXON_OK;
}

// ---- softmax_mm (dims m, n, k; x [m,k], w [k,n]) ---------------------------
// One GEMM (kSoftmax): exp(x) formed as the A tiles are staged, the row sums
// of exp(x) taken on the fly, the output row scaled by 1 / sum in the
// epilogue (or in the split-K fixup). kernels/softmax_mm/kernel.py:7-11.
const char* summary_softmax_mm(int variant) {
  return variant == 1
             ? "one bf16 MFMA GEMM (hw variant 1 schedule) with exp applied to A as it is staged, "
               "row sums of exp taken on the fly and 1/sum applied in the epilogue"
             : "one bf16 MFMA GEMM (hw variant 0 schedule) with exp applied to A as it is staged, "
               "row sums of exp taken on the fly and 1/sum applied in the epilogue";
}

// ---- linear_attention (dims sq, sk, dk, dv; q [sq,dk], key [sk,dk], v [sk,dv])
// out = q (keyᵀ v) (kernels/linear_attention/kernel.py:14-20): key is
// transposed into the workspace, state = keyᵀ v is a split-K GEMM over sk
// (bf16 state, fp32 accumulation), then out = q state over dk.
// Tiles: TILES_IN_BLOCK_P = state rows per tile / 64 (over dk),
// TILES_IN_BLOCK_N = columns per tile / 64 (over dv, both GEMMs),
// TILES_IN_BLOCK_K = state K range / 256 (over sk),
// TILES_IN_BLOCK_M = output rows per tile / 64 (over sq); the output GEMM
// contracts the whole dk in one K range.
int la_tk2(int64_t dk) { return static_cast<int>(k_extent(dk) / kKUnit); }

int check_la(const Call& c, std::string* why) {
  if (c.n_tiles != 4 || c.n_dims != 4 || c.n_dtypes != 3) {
    *why = "expected 4 tiles, 4 dims (sq, sk, dk, dv) and 3 dtypes";
    return AXON_EARG;
  }
  int rc = check_all_bf16(c, 3, why);
  if (rc != AXON_OK) return rc;
  const int64_t sq = c.dim(0), sk = c.dim(1), dk = c.dim(2), dv = c.dim(3);
  if (dk > 65535LL * kTp) {
    *why = "dk out of range";
    return AXON_EINVAL;
  }
  rc = check_gemm_shape(dk, dv, sk, c.tile(3), c.tile(1), c.tile(2), why);
  if (rc != AXON_OK) return rc;
  return check_gemm_shape(sq, dv, dk, c.tile(0), c.tile(1), la_tk2(dk), why);
}

int manifest_la(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  if (cap < 4) return 0;
  const int64_t state[3] = {dims[2], dims[3], dims[1]};  // dk x dv over sk
  manifest_mm(v, state, dt, out, cap);
  const int64_t sq = dims[0] > 0 ? dims[0] : 1;
  out[3] = {"TILES_IN_BLOCK_P", out[0].extent, 64, false};
  out[0] = {"TILES_IN_BLOCK_M", sq < 256 ? (sq < 64 ? 64 : sq) : 256, 64, false};
  return 4;
}

struct LaLayout {
  Plan p1, p2;
  size_t kt, state, data, total;
};

// linear_attention workspace: [keyᵀ bf16 dk x sk][state bf16 dk x dv][split-K
// data of whichever GEMM needs more].
LaLayout la_layout(const Call& c) {
  const int sq = static_cast<int>(c.dim(0)), sk = static_cast<int>(c.dim(1));
  const int dk = static_cast<int>(c.dim(2)), dv = static_cast<int>(c.dim(3));
  LaLayout L;
  L.p1 = plan_of(dk, dv, sk, c.tile(3), c.tile(1), c.tile(2));
  L.p2 = plan_of(sq, dv, dk, c.tile(0), c.tile(1), la_tk2(dk));
  L.kt = 0;
  L.state = align256(static_cast<size_t>(dk) * sk * sizeof(bf16));
  L.data = L.state + align256(static_cast<size_t>(dk) * dv * sizeof(bf16));
  const size_t d1 = data_bytes(L.p1, dk, dv, 1), d2 = data_bytes(L.p2, sq, dv, 1);
  L.total = L.data + (d1 > d2 ? d1 : d2);
  return L;
}

size_t workspace_la(const Call& c) { return la_layout(c).total; }

void outputs_la(const int64_t* dims, const int32_t*, OutDesc* out) {
  out[0] = {2, {dims[0], dims[3]}, AXON_BF16};
}

int launch_la(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  const int sq = static_cast<int>(c.dim(0)), sk = static_cast<int>(c.dim(1));
  const int dk = static_cast<int>(c.dim(2)), dv = static_cast<int>(c.dim(3));
  if (sq == 0 || dv == 0) return AXON_OK;
  for (int i = 0; i < 3; ++i)
    if (!aligned16(in[i])) {
      set_error("linear_attention buffers must be 16-byte aligned");
      return AXON_EARG;
    }
  const LaLayout L = la_layout(c);
  if (!aligned16(out[0]) || ws == nullptr) {
    set_error("linear_attention needs an aligned output and its workspace");
    return AXON_EARG;
  }
  char* base = static_cast<char*>(ws);
  bf16* kt = reinterpret_cast<bf16*>(base + L.kt);
  bf16* state = reinterpret_cast<bf16*>(base + L.state);
  int rc = launch_transpose(static_cast<const bf16*>(in[1]), kt, sk, dk, st);
  if (rc != AXON_OK) return rc;
  const GemmArgs g1 = make_args(kt, static_cast<const bf16*>(in[2]), nullptr, state, dk, dv, sk, L.p1,
                                base + L.data, 1, 0.f);
  rc = dispatch<kPlain, false>(L.p1.BM, L.p1.BN, g1, st, c.variant);
  if (rc != AXON_OK) return rc;
  const GemmArgs g2 = make_args(in[0], state, nullptr, out[0], sq, dv, dk, L.p2, base + L.data, 1, 0.f);
  return dispatch<kPlain, false>(L.p2.BM, L.p2.BN, g2, st, c.variant);
}

const char* summary_la(int variant) {
  return variant == 1
             ? "keyᵀ into the workspace (LDS-tiled transpose), state = keyᵀ v as a split-K bf16 MFMA "
               "GEMM (bf16 state), out = q state; both GEMMs on the hw variant 1 schedule"
             : "keyᵀ into the workspace (LDS-tiled transpose), state = keyᵀ v as a split-K bf16 MFMA "
               "GEMM (bf16 state), out = q state; both GEMMs on the hw variant 0 schedule";
}

// ---- attention (dims m, n, k; x [m,k], w_q, w_k, w_v [k,n]) ----------------
// kernels/attention/kernel.py:7-18: q, k, v = x w_q, x w_k, x w_v (bf16 out,
// fp32 accumulation); kᵀ into the workspace; S = q kᵀ in fp32 (m x m); out =
// softmax(S) v with a bare exp/sum softmax: the kSoftmax GEMM on the fp32 S
// (exp taken in fp32 as S is staged, split into bf16 hi + lo planes so the
// probabilities keep fp32 accuracy), rows scaled by 1 / sum exp.
// Tiles: TILES_IN_BLOCK_M = rows per tile / 64 (all stages),
// TILES_IN_BLOCK_N = columns / 64 of the projections and of the output,
// TILES_IN_BLOCK_P = columns / 64 of S, TILES_IN_BLOCK_K = K range / 256 of
// the S stage (and of the projections when they run as three GEMMs; the
// merged projection and the output stage pick their own, below). The output
// stage holds two A planes, so its tile is narrowed to BM <= 128 and
// BM x BN <= 128 x 128.
// The three projections run as one GEMM over the column-split operand
// [w_q | w_k | w_v] (x read once, one launch, one split-K fixup) whenever
// the projection tile width divides n; otherwise as three GEMMs. The merged
// GEMM takes the fewest K splits (powers of two) that give it at least 128
// workgroups, whatever TILES_IN_BLOCK_K says: its partials are three times
// those of one projection, and at 4096 x 1536 x 4096 two splits (192
// workgroups) run in 76 us where four take 97.
struct AttnPlan {
  Plan proj, proj3, s, pv;
  bool merged;
};

AttnPlan attn_plan(const Call& c) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1)), k = static_cast<int>(c.dim(2));
  const int tm = c.tile(0), tn = c.tile(1), tk = c.tile(2), tp = c.tile(3);
  const int tm2 = std::min(tm, 2), tn2 = std::max(1, std::min(tn, 4 / tm2));
  AttnPlan P;
  P.proj = plan_of(m, n, k, tm, tn, tk);
  {
    int tk_full = 1;  // K range covering all of k, in units of kKUnit
    while (static_cast<int64_t>(kKUnit) * tk_full < k) tk_full *= 2;
    int tk3 = tk_full;
    const Plan whole = plan_of(m, 3 * n, k, tm, tn, tk_full);
    for (int splits = 1; tk3 > 1 && static_cast<int64_t>(whole.MT) * whole.NT * splits < 128; splits *= 2) tk3 /= 2;
    P.proj3 = plan_of(m, 3 * n, k, tm, tn, tk3);
  }
  std::string why;
  P.merged = n > 0 && n % P.proj3.BN == 0 &&
             check_gemm_shape(m, 3 * static_cast<int64_t>(n), k, tm, tn, tk, &why) == AXON_OK;
  P.s = plan_of(m, m, n, tm, tp, tk);
  // The softmax GEMM likewise takes the fewest K splits that give it at
  // least 256 workgroups (4096 x 512 x 4096 on 128 x 128 tiles: two splits,
  // 16 MB of partials, where TILES_IN_BLOCK_K = 2 would make eight and 64 MB;
  // s4k_d512 230 -> 206 us; a 128-workgroup floor is slower here).
  {
    int tk_full = 1;
    while (static_cast<int64_t>(kKUnit) * tk_full < m) tk_full *= 2;
    int tkp = tk_full;
    const Plan whole = plan_of(m, n, m, tm2, tn2, tk_full);
    for (int splits = 1; tkp > 1 && static_cast<int64_t>(whole.MT) * whole.NT * splits < 256; splits *= 2) tkp /= 2;
    P.pv = plan_of(m, n, m, tm2, tn2, tkp);
  }
  return P;
}

int check_attn_qkv(const Call& c, std::string* why) {
  if (c.n_tiles != 4 || c.n_dims != 3 || c.n_dtypes != 4) {
    *why = "expected 4 tiles, 3 dims (m, n, k) and 4 dtypes";
    return AXON_EARG;
  }
  int rc = check_all_bf16(c, 4, why);
  if (rc != AXON_OK) return rc;
  const int64_t m = c.dim(0), n = c.dim(1), k = c.dim(2);
  if (m % 8 != 0) {
    *why = "m must be a multiple of 8 (it is the column count of S)";
    return AXON_EINVAL;
  }
  if (n > 65535LL * kTp) {
    *why = "n out of range";
    return AXON_EINVAL;
  }
  const int tm = c.tile(0), tn = c.tile(1), tk = c.tile(2), tp = c.tile(3);
  rc = check_gemm_shape(m, n, k, tm, tn, tk, why);
  if (rc == AXON_OK) rc = check_gemm_shape(m, m, n, tm, tp, tk, why);
  if (rc == AXON_OK) rc = check_gemm_shape(m, n, m, tm, tn, tk, why);
  return rc;
}

int manifest_attn_qkv(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  if (cap < 4) return 0;
  const int64_t m = dims[0] > 0 ? dims[0] : 1;
  // One K range serves all three contractions (over k, n and m).
  const int64_t mnk[3] = {dims[0], dims[1], std::min({dims[0], dims[1], dims[2]})};
  manifest_mm(v, mnk, dt, out, cap);
  out[3] = {"TILES_IN_BLOCK_P", m < 256 ? (m < 64 ? 64 : m) : 256, 64, false};
  return 4;
}

struct AttnLayout {
  AttnPlan P;
  size_t q, k, v, kt, s, data, total;
};

// attention workspace: [q][k][v] bf16 m x n each, [kᵀ] bf16 n x m, [S] fp32
// m x m, [split-K data of the stage that needs most] (stages run in order
// and share it).
AttnLayout attn_layout(const Call& c) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1));
  AttnLayout L;
  L.P = attn_plan(c);
  const size_t mn = align256(static_cast<size_t>(m) * n * sizeof(bf16));
  L.q = 0;
  L.k = mn;
  L.v = 2 * mn;
  L.kt = 3 * mn;
  L.s = 4 * mn;
  L.data = L.s + align256(static_cast<size_t>(m) * m * sizeof(float));
  const size_t dproj = L.P.merged ? data_bytes(L.P.proj3, m, 3 * n, 1) : data_bytes(L.P.proj, m, n, 1);
  const size_t d = std::max({dproj, data_bytes(L.P.s, m, m, 1), data_bytes(L.P.pv, m, n, 1)});
  L.total = L.data + d;
  return L;
}

size_t workspace_attn_qkv(const Call& c) { return attn_layout(c).total; }

void outputs_attn_qkv(const int64_t* dims, const int32_t*, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, AXON_BF16};
}

int launch_attn_qkv(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  const int m = static_cast<int>(c.dim(0)), n = static_cast<int>(c.dim(1)), k = static_cast<int>(c.dim(2));
  if (m == 0 || n == 0) return AXON_OK;
  for (int i = 0; i < 4; ++i)
    if (!aligned16(in[i])) {
      set_error("attention buffers must be 16-byte aligned");
      return AXON_EARG;
    }
  if (!aligned16(out[0]) || ws == nullptr) {
    set_error("attention needs an aligned output and its workspace");
    return AXON_EARG;
  }
  const AttnLayout L = attn_layout(c);
  char* base = static_cast<char*>(ws);
  bf16* q = reinterpret_cast<bf16*>(base + L.q);
  bf16* kk = reinterpret_cast<bf16*>(base + L.k);
  bf16* v = reinterpret_cast<bf16*>(base + L.v);
  bf16* kt = reinterpret_cast<bf16*>(base + L.kt);
  float* S = reinterpret_cast<float*>(base + L.s);
  void* data = base + L.data;
  bf16* proj_out[3] = {q, kk, v};
  int rc = AXON_OK;
  if (L.P.merged) {
    GemmArgs g = make_args(in[0], static_cast<const bf16*>(in[1]), nullptr, q, m, 3 * n, k, L.P.proj3, data, 1, 0.f);
    g.Bcol[0] = static_cast<const bf16*>(in[2]);
    g.Bcol[1] = static_cast<const bf16*>(in[3]);
    g.Ccol[0] = kk;
    g.Ccol[1] = v;
    g.ncol = n;
    rc = dispatch<kColSplit, false>(L.P.proj3.BM, L.P.proj3.BN, g, st, c.variant);
  } else {
    for (int i = 0; i < 3 && rc == AXON_OK; ++i) {
      const GemmArgs g = make_args(in[0], static_cast<const bf16*>(in[1 + i]), nullptr, proj_out[i], m, n, k,
                                   L.P.proj, data, 1, 0.f);
      rc = dispatch<kPlain, false>(L.P.proj.BM, L.P.proj.BN, g, st, c.variant);
    }
  }
  if (rc == AXON_OK) rc = launch_transpose(kk, kt, m, n, st);
  if (rc != AXON_OK) return rc;
  GemmArgs gs = make_args(q, kt, nullptr, S, m, m, n, L.P.s, data, 1, 0.f);
  gs.c_f32 = 1;
  rc = dispatch<kPlain, false>(L.P.s.BM, L.P.s.BN, gs, st, c.variant);
  if (rc != AXON_OK) return rc;
  const GemmArgs gp = make_args(S, v, nullptr, out[0], m, n, m, L.P.pv, data, 1, 0.f);
  return dispatch_mlp<kSoftmax, true>(L.P.pv.BM, L.P.pv.BN, gp, st);
}

const char* summary_attn_qkv(int variant) {
  return variant == 1
             ? "q, k, v projections and S = q kᵀ (fp32) as bf16 MFMA GEMMs on the hw variant 1 schedule, "
               "kᵀ by an LDS-tiled transpose, then one GEMM over fp32 S with exp on staging (hi + lo "
               "bf16 planes), row sums on the fly and 1/sum in the epilogue"
             : "q, k, v projections and S = q kᵀ (fp32) as bf16 MFMA GEMMs on the hw variant 0 schedule, "
               "kᵀ by an LDS-tiled transpose, then one GEMM over fp32 S with exp on staging (hi + lo "
               "bf16 planes), row sums on the fly and 1/sum in the epilogue";
}

}  // namespace

#define AXON_MM_FAMILY(fn_name, spec_name, EPI)                                                \
  const Family* fn_name() {                                                                  \
    static const Family f = {spec_name,     3,           2,         1,           3,          \
                             kTileArgs3,    3,           summary_rms, manifest_rms, check_mm<EPI>,    \
                             workspace_mm<EPI>, outputs_mm, launch_mm<EPI>};                  \
    return &f;                                                                               \
  }

#define AXON_PLAIN_FAMILY(fn_name, spec_name)                                                    \
  const Family* fn_name() {                                                                    \
    static const Family f = {spec_name,     4,          2,              1,           3,        \
                             kTileArgs3,    3,          summary_mm,     manifest_plain, check_plain, \
                             workspace_plain, outputs_mm, launch_plain};                         \
    return &f;                                                                                 \
  }

AXON_PLAIN_FAMILY(family_matmul, "matmul")
AXON_PLAIN_FAMILY(family_matmul_std002, "matmul_std002")
#undef AXON_PLAIN_FAMILY
AXON_MM_FAMILY(family_rmsnorm_matmul, "rmsnorm_matmul", kRmsSum)
AXON_MM_FAMILY(family_rmsnorm_matmul_eps, "rmsnorm_matmul_eps", kRmsEps)
#undef AXON_MM_FAMILY

const Family* family_silu_mlp() {
  static const Family f = {"silu_mlp", 1, 4, 1, 4, kTileArgs4, 4, summary_mlp, manifest_mlp,
                           check_mlp, workspace_mlp, outputs_mlp, launch_mlp};
  return &f;
}

const Family* family_qkv_cte() {
  static const Family f = {"qkv_cte", 4, 4, 1, 3, kTileArgs3, 3, summary_qkv, manifest_qkv,
                           check_qkv, workspace_qkv, outputs_qkv, launch_qkv};
  return &f;
}

const Family* family_softmax_mm() {
  static const Family f = {"softmax_mm", 2, 2, 1, 3, kTileArgs3, 3, summary_softmax_mm, manifest_mm,
                           check_mm<kSoftmax>, workspace_mm<kSoftmax>, outputs_mm, launch_mm<kSoftmax>};
  return &f;
}

const Family* family_linear_attention() {
  static const Family f = {"linear_attention", 2, 3, 1, 4, kTileArgs4, 4, summary_la, manifest_la,
                           check_la, workspace_la, outputs_la, launch_la};
  return &f;
}

const Family* family_attention_qkv() {
  static const Family f = {"attention", 2, 4, 1, 3, kTileArgs4, 4, summary_attn_qkv, manifest_attn_qkv,
                           check_attn_qkv, workspace_attn_qkv, outputs_attn_qkv, launch_attn_qkv};
  return &f;
}

}  // namespace axon
