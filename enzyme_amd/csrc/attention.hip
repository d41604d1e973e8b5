// Flash attention with bf16 MFMA and an online fp32 softmax.
//
//   attention_causal  O = softmax(Q K^T / sqrt(d) + causal mask) V over
//                     [b, h, s, d] tensors (Q, K, V, O all [b, h, s, d] bf16)
//   attention_nkilib  O = softmax(q @ k_t) V, single head: q [s, d],
//                     k_t [d, s] (K given transposed), v [s, d], no scale,
//                     no mask (kernels/attention_nkilib/kernel.py:14-21; the
//                     reference's bare exp/sum equals the max-shifted softmax
//                     used here)
//
// Schedule (hw variant 0): a workgroup of W waves owns 32*W query rows of one
// (batch, head); each wave owns 32 of them and walks the key/value sequence
// in blocks of BKV keys staged through double-buffered LDS.
// Per block a wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (Q^T
// held in registers for the whole walk), so each lane holds the scores of
// ONE query (lane % 32) for 16 keys per 32-key tile: the row max and row
// sum are in-lane reductions plus one exchange with lane ^ 32. The
// probabilities P^T = exp2(S^T * scale*log2e - m) are converted to bf16 in
// place and are directly the B operand of O^T = V^T P^T: the MFMA's k index
// is mapped to keys {0-3, 8-11 | 4-7, 12-15} (+16) to match the accumulator
// layout. V^T lives in LDS as [d][key] with bits 2 and 3 of the key index
// swapped inside each 16-key group, so the 8 keys a lane needs for one MFMA
// are one contiguous 16-byte read; it is written there as packed key pairs
// (one 32-bit store per d, consecutive lanes on consecutive words, no bank
// conflicts). K lives in LDS as [key][d] (16-byte stores and reads).
// O^T keeps one query per lane too, so the online-softmax rescale is a
// per-lane multiply; it is done only when some lane's running max grows by
// more than 2^8 (a stale max leaves every probability <= 2^8, exact in the
// fp32 sums and in bf16), which after the first block is almost never.
// Causal: key blocks past a wave's last query are skipped, only blocks that
// cross the diagonal (or the end of the sequence) are masked, and the
// heaviest query blocks are scheduled first; the heads are dealt to the 8
// XCDs so each XCD's L2 serves the K/V of h/8 heads only.
// hw variant 1 gives each wave two 32-query tiles: every K and V^T fragment
// read from LDS feeds two MFMAs, halving LDS reads per FLOP, at one wave per
// SIMD (the second tile's accumulators fill the AGPRs).
// hw variant 3 runs hw variant 2's schedule over split key ranges: the
// grid adds a key-range index, each workgroup writes its range's
// unnormalised O^T columns, running max and row sum to the workspace, and a
// second kernel merges the ranges of each query row. It fills the GPU when
// batch * heads * s is small (one head of 1024 queries is 8 workgroups of
// 128 queries otherwise).
// Tile arguments: TILES_IN_BLOCK_M = W / 4 (variant 0: 4 or 8 waves; variant
//                 1: 4 waves; variant 3: W / 2, 2, 4 or 8 waves),
//                 TILES_IN_BLOCK_N = BKV / 32 (variants 1-3: at most 2);
//                 TILES_IN_BLOCK_K = key-range splits (variant 3, 1 to 16;
//                 otherwise pinned to 1); TILES_IN_BLOCK_P is pinned to 1.
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "registry.hpp"

namespace axon {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int D = 128;
constexpr int KP = D + 8;  // Ks row pitch (elements): 16-byte reads of 8 rows hit 32 banks
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.f;  // log2 of the largest un-rescaled probability
constexpr int kXcds = 8;
constexpr int kMaxSplits = 16;  // key ranges of hw variant 3

template <int N>
using ic = std::integral_constant<int, N>;

struct AttnArgs {
  const bf16* q;   // [BH][s][D]
  const bf16* k;   // [BH][s][D], or k_t [D][s] when KT
  const bf16* v;   // [BH][s][D]
  bf16* o;         // [BH][s][D]
  int s;
  int bh;
  int qblocks;
  int xcd_heads;     // heads per XCD when the XCD mapping applies, else 0
  float scale_log2;  // softmax scale * log2(e)
  // Split key ranges (hw variant 3): nsplit ranges of kv_split keys each;
  // partial results go to o_part [nsplit][bh][s][D] (unnormalised fp32) and
  // ml_part [nsplit][bh][s][2] (running max in the exp2 domain, row sum).
  int nsplit;
  int kv_split;
  float* o_part;
  float* ml_part;
};

// Position of key k (0..15 inside its 16-key group) in a V^T row: bits 2 and
// 3 swapped, so keys {0-3, 8-11} and {4-7, 12-15} are contiguous.
__device__ __forceinline__ int vt_pos(int k) {
  return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

__device__ __forceinline__ uint32_t pack2(bf16 lo, bf16 hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
}

template <int W, int TN, int QT, bool CAUSAL, bool KT>
__global__ __launch_bounds__(W * 64) void attn_kernel(AttnArgs a) {
  constexpr int QW = 32 * QT;  // queries per wave
  constexpr int BQ = QW * W;
  constexpr int BKV = 32 * TN;
  constexpr int VP = BKV + 8;  // Vt row pitch (elements)
  constexpr int NT = W * 64;
  // K staging (row layout): BKV*D/8 16-byte vectors.
  constexpr int KITEMS = KT ? (D / 2) * (BKV / 8) : BKV * D / 8;
  constexpr int KI = (KITEMS + NT - 1) / NT;
  // V staging: (BKV/2 key pairs) x (D/8 chunks), two 16-byte loads each.
  constexpr int VITEMS = (BKV / 2) * (D / 8);
  constexpr int VI = (VITEMS + NT - 1) / NT;
  constexpr int KL = KT ? 2 : 1;  // 16-byte loads per K item

  extern __shared__ __align__(16) unsigned char smem[];
  bf16* Ks = reinterpret_cast<bf16*>(smem);  // [2][BKV][KP]
  bf16* Vt = Ks + 2 * BKV * KP;              // [2][D][VP]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;  // half of the wave

  // Block -> (head, query block): heaviest (latest) query blocks first under
  // causal masking; with the XCD mapping, block b runs on XCD b % 8 and that
  // XCD only ever sees heads x, x+8, x+16, ...
  int rank, bh;
  const int bid = static_cast<int>(blockIdx.x);
  if (a.xcd_heads > 0) {
    const int x = bid % kXcds, j = bid / kXcds;
    rank = j / a.xcd_heads;
    bh = x + kXcds * (j % a.xcd_heads);
  } else {
    rank = bid % a.qblocks;
    bh = bid / a.qblocks;
  }
  const int qb = CAUSAL ? a.qblocks - 1 - rank : rank;
  const int64_t base = static_cast<int64_t>(bh) * a.s * D;
  const bf16* Q = a.q + base;
  const bf16* K = a.k + base;
  const bf16* V = a.v + base;
  bf16* O = a.o + base;

  const int q0 = qb * BQ;
  const int qw = q0 + wave * QW;  // this wave's first query
  const int kv_end = CAUSAL ? min(a.s, q0 + BQ) : a.s;
  const int nblocks = (kv_end + BKV - 1) / BKV;
  // Query of this lane in query tile u: qw + 32u + lane % 32.
  auto my_q = [&](int u) { return qw + 32 * u + (lane & 31); };

  // Q^T fragments (B operand): lane holds Q[my_q(u)][step*16 + h*8 .. +8].
  bf16x8 qf[QT][D / 16];
#pragma unroll
  for (int u = 0; u < QT; ++u)
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
      if (my_q(u) < a.s)
        qf[u][st] = *reinterpret_cast<const bf16x8*>(Q + static_cast<int64_t>(my_q(u)) * D + st * 16 + h * 8);
      else
        for (int i = 0; i < 8; ++i) qf[u][st][i] = static_cast<bf16>(0.f);
    }

  // Global -> register staging of one K/V block. Rows past the sequence are
  // read from the last row instead (branch-free loads keep the prefetch in
  // flight across the block's compute): their scores are masked to -inf and
  // their probabilities are 0, so the duplicated rows contribute nothing.
  Vec<bf16> kreg[KI][KL], vreg[VI][2];
  auto load_block = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = min(tid + i * NT, KITEMS - 1);
      if constexpr (!KT) {
        // item -> key item/16, d chunk (item%16)*8
        const int key = min(kv0 + (item >> 4), a.s - 1), dc = (item & 15) * 8;
        kreg[i][0] = load_vec(K + static_cast<int64_t>(key) * D + dc);
      } else {
        // item -> d pair dp = item % 64, key chunk kc = item / 64 (s % 8 == 0)
        const int dp = item % (D / 2), key = min(kv0 + (item / (D / 2)) * 8, a.s - 8);
#pragma unroll
        for (int r = 0; r < 2; ++r)
          kreg[i][r] = load_vec(K + static_cast<int64_t>(2 * dp + r) * a.s + key);
      }
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = min(tid + i * NT, VITEMS - 1);
      // item -> key pair p = item % (BKV/2), d chunk c = item / (BKV/2)
      const int p = item % (BKV / 2), c = item / (BKV / 2);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int key = min(kv0 + 2 * p + r, a.s - 1);
        vreg[i][r] = load_vec(V + static_cast<int64_t>(key) * D + c * 8);
      }
    }
  };

  // Makes a staged vector opaque until its store: otherwise the packing
  // below is placed right after the load and waits for it a block early.
  auto opaque = [](Vec<bf16>& r) {
    u32x4 u = *reinterpret_cast<const u32x4*>(&r);
    asm volatile("" : "+v"(u));
    *reinterpret_cast<u32x4*>(&r) = u;
  };
  auto store_block = [&](int buf) {
    bf16* ks = Ks + buf * BKV * KP;
    bf16* vt = Vt + buf * D * VP;
#pragma unroll
    for (int i = 0; i < KI; ++i)
#pragma unroll
      for (int r = 0; r < KL; ++r) opaque(kreg[i][r]);
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      opaque(vreg[i][0]);
      opaque(vreg[i][1]);
    }
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = tid + i * NT;
      if (KITEMS % NT != 0 && item >= KITEMS) continue;
      if constexpr (!KT) {
        store_vec(ks + (item >> 4) * KP + (item & 15) * 8, kreg[i][0]);
      } else {
        const int dp = item % (D / 2), kc = (item / (D / 2)) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<uint32_t*>(ks + (kc + e) * KP + 2 * dp) = pack2(kreg[i][0].v[e], kreg[i][1].v[e]);
      }
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = tid + i * NT;
      if (VITEMS % NT != 0 && item >= VITEMS) continue;
      const int p = item % (BKV / 2), c = item / (BKV / 2);
      const int k0 = 2 * p;
      const int pos = (k0 & ~15) | vt_pos(k0 & 15);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *reinterpret_cast<uint32_t*>(vt + (c * 8 + e) * VP + pos) = pack2(vreg[i][0].v[e], vreg[i][1].v[e]);
    }
  };

  floatx16 acc_o[QT][D / 32];
#pragma unroll
  for (int u = 0; u < QT; ++u)
#pragma unroll
    for (int t = 0; t < D / 32; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_o[u][t][e] = 0.f;
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    m_run[u] = -INFINITY;
    l_run[u] = 0.f;
  }

  // One key block for this wave; MASK applies the causal / sequence-end mask.
  // Every K and V^T fragment read from LDS feeds the QT query tiles.
  auto process = [&](auto mask_tag, const bf16* ks, const bf16* vt, int kv0) {
    constexpr bool MASK = decltype(mask_tag)::value;
    // S^T = K Q^T: acc_s[u][t] rows = keys t*32.., columns = query tile u.
    floatx16 acc_s[QT][TN];
#pragma unroll
    for (int u = 0; u < QT; ++u)
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_s[u][t][e] = 0.f;
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(ks + (t * 32 + (lane & 31)) * KP + st * 16 + h * 8);
#pragma unroll
        for (int u = 0; u < QT; ++u)
          acc_s[u][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[u][st], acc_s[u][t], 0, 0, 0);
      }
    // P^T in bf16, grouped by MFMA k-step: pf[u][t][ks] holds keys
    // t*32 + ks*16 + {0-3, 8-11} (h = 0) or {4-7, 12-15} (h = 1).
    bf16x8 pf[QT][TN][2];
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if constexpr (MASK) {
            const int key = kv0 + t * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
            if ((CAUSAL && key > my_q(u)) || key >= a.s) acc_s[u][t][e] = -INFINITY;
          }
          mx = fmaxf(mx, acc_s[u][t][e]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mxs = mx * a.scale_log2;
      if (__any(mxs > m_run[u] + kRescaleSlack)) {
        const float m_new = fmaxf(m_run[u], mxs);
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run[u] - m_new);
        l_run[u] *= alpha;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc_o[u][dt][e] *= alpha;
        m_run[u] = m_new;
      }
      const float m_use = m_run[u] == -INFINITY ? 0.f : m_run[u];
      float lblk = 0.f;
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(acc_s[u][t][e], a.scale_log2, -m_use));
          lblk += pv;
          pf[u][t][e >> 3][e & 7] = static_cast<bf16>(pv);
        }
      l_run[u] += lblk + __shfl_xor(lblk, 32, 64);
    }
    // O^T += V^T P^T; the V^T fragment is one 16-byte read (permuted keys).
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vt + (dt * 32 + (lane & 31)) * VP + t * 32 + ks2 * 16 + 8 * h);
#pragma unroll
          for (int u = 0; u < QT; ++u)
            acc_o[u][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[u][t][ks2], acc_o[u][dt], 0, 0, 0);
        }
  };

  if (nblocks > 0) {
    load_block(0);
    store_block(0);
  }
  __syncthreads();

  for (int blk = 0; blk < nblocks; ++blk) {
    const int buf = blk & 1;
    const int kv0 = blk * BKV;
    if (blk + 1 < nblocks) load_block(kv0 + BKV);

    if ((!CAUSAL || kv0 <= qw + QW - 1) && qw < a.s) {
      const bf16* ks = Ks + buf * BKV * KP;
      const bf16* vt = Vt + buf * D * VP;
      const bool mask = (CAUSAL && kv0 + BKV - 1 > qw) || kv0 + BKV > a.s;
      if (mask) process(std::true_type{}, ks, vt, kv0);
      else process(std::false_type{}, ks, vt, kv0);
    }
    // The other buffer was last read before the previous barrier.
    if (blk + 1 < nblocks) store_block(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int u = 0; u < QT; ++u) {
    if (my_q(u) >= a.s) continue;
    const float inv = l_run[u] > 0.f ? 1.f / l_run[u] : 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16x4 out;
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = static_cast<bf16>(acc_o[u][dt][g4 * 4 + i] * inv);
        const int d = dt * 32 + 8 * g4 + 4 * h;
        *reinterpret_cast<bf16x4*>(O + static_cast<int64_t>(my_q(u)) * D + d) = out;
      }
  }
}

// hw variant 2, software-pipelined: K is staged one block ahead of V, so a
// wave computes S(j+1) = K(j+1) Q^T on the matrix cores while it runs the
// softmax of block j on the VALU (the two are independent, and an MFMA keeps
// running while the same wave issues other instructions), then O += V(j)^T
// P(j). At the end of iteration j the block's loads land: K(j+2) into the
// buffer K(j) left (last read in iteration j-1) and V(j+1) into the buffer
// V(j-1) left; one barrier per block. 4 or 8 waves of 32 queries. Causal:
// a wave skips the compute of blocks past its last query (it still stages
// K and V and meets the barrier with the others).
template <int W, int TN, bool CAUSAL, bool KT, bool SPLIT>
__global__ __launch_bounds__(W * 64, W == 4 ? 2 : 1) void attn_sp_kernel(AttnArgs a) {
  constexpr int NT = W * 64;
  constexpr int BQ = 32 * W;
  constexpr int BKV = 32 * TN;
  constexpr int VP = BKV + 8;
  constexpr int KITEMS = KT ? (D / 2) * (BKV / 8) : BKV * D / 8;
  constexpr int KI = (KITEMS + NT - 1) / NT;
  constexpr int VITEMS = (BKV / 2) * (D / 8);
  constexpr int VI = (VITEMS + NT - 1) / NT;
  constexpr int KL = KT ? 2 : 1;

  extern __shared__ __align__(16) unsigned char smem[];
  bf16* Ks = reinterpret_cast<bf16*>(smem);  // [2][BKV][KP]
  bf16* Vt = Ks + 2 * BKV * KP;              // [2][D][VP]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;

  int rank, bh, sp = 0;
  int bid = static_cast<int>(blockIdx.x);
  if constexpr (SPLIT) {
    sp = bid % a.nsplit;
    bid /= a.nsplit;
  }
  if (!SPLIT && a.xcd_heads > 0) {
    const int x = bid % kXcds, j = bid / kXcds;
    rank = j / a.xcd_heads;
    bh = x + kXcds * (j % a.xcd_heads);
  } else {
    rank = bid % a.qblocks;
    bh = bid / a.qblocks;
  }
  const int qb = CAUSAL ? a.qblocks - 1 - rank : rank;
  const int64_t base = static_cast<int64_t>(bh) * a.s * D;
  const bf16* Q = a.q + base;
  const bf16* K = a.k + base;
  const bf16* V = a.v + base;
  bf16* O = a.o + base;

  const int q0 = qb * BQ;
  // Waves w and w + W/2 share a SIMD: pairing an early query tile with a
  // late one gives every SIMD the same number of skipped (fully masked)
  // blocks at the diagonal.
  const int wq = wave < W / 2 ? wave : 3 * W / 2 - 1 - wave;
  const int qw = q0 + wq * 32;
  const int my_q = qw + (lane & 31);
  // Key range [kv_lo, kv_end) of this workgroup (the whole sequence unless
  // the key range is split).
  const int kv_lo = SPLIT ? sp * a.kv_split : 0;
  int kv_end = CAUSAL ? min(a.s, q0 + BQ) : a.s;
  if constexpr (SPLIT) kv_end = min(kv_end, kv_lo + a.kv_split);
  const int nblocks = kv_end > kv_lo ? (kv_end - kv_lo + BKV - 1) / BKV : 0;
  const int klast = kv_lo + max(nblocks - 1, 0) * BKV;

  bf16x8 qf[D / 16];
#pragma unroll
  for (int st = 0; st < D / 16; ++st) {
    if (my_q < a.s)
      qf[st] = *reinterpret_cast<const bf16x8*>(Q + static_cast<int64_t>(my_q) * D + st * 16 + h * 8);
    else
      for (int i = 0; i < 8; ++i) qf[st][i] = static_cast<bf16>(0.f);
  }

  Vec<bf16> kreg[KI][KL], vreg[VI][2];
  auto opaque = [](Vec<bf16>& r) {
    u32x4 u = *reinterpret_cast<const u32x4*>(&r);
    asm volatile("" : "+v"(u));
    *reinterpret_cast<u32x4*>(&r) = u;
  };
  auto load_k = [&](int kv0) {
    kv0 = min(kv0, klast);
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = min(tid + i * NT, KITEMS - 1);
      if constexpr (!KT) {
        const int key = min(kv0 + (item >> 4), a.s - 1), dc = (item & 15) * 8;
        kreg[i][0] = load_vec(K + static_cast<int64_t>(key) * D + dc);
      } else {
        const int dp = item % (D / 2), key = min(kv0 + (item / (D / 2)) * 8, a.s - 8);
#pragma unroll
        for (int r = 0; r < 2; ++r)
          kreg[i][r] = load_vec(K + static_cast<int64_t>(2 * dp + r) * a.s + key);
      }
    }
  };
  auto load_v = [&](int kv0) {
    kv0 = min(kv0, klast);
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = min(tid + i * NT, VITEMS - 1);
      const int p = item % (BKV / 2), c = item / (BKV / 2);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int key = min(kv0 + 2 * p + r, a.s - 1);
        vreg[i][r] = load_vec(V + static_cast<int64_t>(key) * D + c * 8);
      }
    }
  };
  auto store_k = [&](int buf) {
    bf16* ks = Ks + buf * BKV * KP;
#pragma unroll
    for (int i = 0; i < KI; ++i) {
#pragma unroll
      for (int r = 0; r < KL; ++r) opaque(kreg[i][r]);
      const int item = tid + i * NT;
      if (KITEMS % NT != 0 && item >= KITEMS) continue;
      if constexpr (!KT) {
        store_vec(ks + (item >> 4) * KP + (item & 15) * 8, kreg[i][0]);
      } else {
        const int dp = item % (D / 2), kc = (item / (D / 2)) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<uint32_t*>(ks + (kc + e) * KP + 2 * dp) = pack2(kreg[i][0].v[e], kreg[i][1].v[e]);
      }
    }
  };
  auto store_v = [&](int buf) {
    bf16* vt = Vt + buf * D * VP;
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      opaque(vreg[i][0]);
      opaque(vreg[i][1]);
      const int item = tid + i * NT;
      if (VITEMS % NT != 0 && item >= VITEMS) continue;
      const int p = item % (BKV / 2), c = item / (BKV / 2);
      const int k0 = 2 * p;
      const int pos = (k0 & ~15) | vt_pos(k0 & 15);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *reinterpret_cast<uint32_t*>(vt + (c * 8 + e) * VP + pos) = pack2(vreg[i][0].v[e], vreg[i][1].v[e]);
    }
  };

  floatx16 acc_o[D / 32];
#pragma unroll
  for (int t = 0; t < D / 32; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[t][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  floatx16 acc_s[2][TN];  // scores of blocks j (cur) and j+1 (next), by parity
  bf16x8 pf[TN][2];

  auto m1 = [&](floatx16 (&sacc)[TN], int j) {
    const bf16* ks = Ks + (j & 1) * BKV * KP;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[t][e] = 0.f;
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(ks + (t * 32 + (lane & 31)) * KP + st * 16 + h * 8);
        sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], sacc[t], 0, 0, 0);
      }
    }
  };
  auto m2 = [&](int j) {
    const bf16* vt = Vt + (j & 1) * D * VP;
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vt + (dt * 32 + (lane & 31)) * VP + t * 32 + ks2 * 16 + 8 * h);
          acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[t][ks2], acc_o[dt], 0, 0, 0);
        }
  };
  // Iteration j (parity P = j & 1): S(j) is in acc_s[P]. The row max and the
  // (rare) rescale come first; then one branch-free stretch holds the QK^T
  // MFMAs of block j+1 (into acc_s[P ^ 1]), the exponentials of block j and
  // its PV MFMAs, so the scheduler can interleave matrix and vector work.
  // Blocks past a wave's diagonal (or the last block) go through the masked
  // path and contribute probability 0; S of a block past the end is computed
  // from a clamped duplicate and never used.
  auto body = [&](auto mask_tag, auto par_tag, int j) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr int P = decltype(par_tag)::value;
    floatx16 (&sacc)[TN] = acc_s[P];
    const int kv0 = kv_lo + j * BKV;
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        if constexpr (MASK) {
          const int key = kv0 + t * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
          if ((CAUSAL && key > my_q) || key >= a.s) sacc[t][e] = -INFINITY;
        }
        mx = fmaxf(mx, sacc[t][e]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mxs = mx * a.scale_log2;
    if (__any(mxs > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mxs);
      const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[dt][e] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    // A masked block is the wave's last one (its diagonal, or the end of the
    // sequence): no later block needs S(j+1).
    if constexpr (!MASK) m1(acc_s[P ^ 1], j + 1);
    float lblk = 0.f;
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[t][e], a.scale_log2, -m_use));
        lblk += pv;
        pf[t][e >> 3][e & 7] = static_cast<bf16>(pv);
      }
    l_run += lblk + __shfl_xor(lblk, 32, 64);
    m2(j);
  };

  if (nblocks > 0) {
    load_k(kv_lo);
    store_k(0);
    load_k(kv_lo + BKV);
    load_v(kv_lo);
    store_k(1);
    store_v(0);
  }
  __syncthreads();
  if (nblocks > 0) m1(acc_s[0], 0);

  auto iter = [&](int j, auto par_tag) {
    load_k(kv_lo + (j + 2) * BKV);
    load_v(kv_lo + (j + 1) * BKV);
    const int kv0 = kv_lo + j * BKV;
    // A block past the wave's last query contributes nothing, and neither
    // does any later one, whose scores S(j+1) the skipped body would compute.
    if (qw < a.s && !(CAUSAL && kv0 > qw + 31)) {
      if ((CAUSAL && kv0 + BKV - 1 > qw) || kv0 + BKV > a.s) body(std::true_type{}, par_tag, j);
      else body(std::false_type{}, par_tag, j);
    }
    store_k(j & 1);        // K(j+2) into the buffer K(j) left
    store_v((j + 1) & 1);  // V(j+1) into the buffer V(j-1) left
    __syncthreads();
  };
  for (int j = 0; j < nblocks; j += 2) {
    iter(j, ic<0>{});
    if (j + 1 < nblocks) iter(j + 1, ic<1>{});
  }

  if constexpr (SPLIT) {
    // This key range's unnormalised output, running max and row sum (an
    // empty range leaves 0, -inf, 0); the combine kernel merges the ranges.
    if (my_q < a.s) {
      const int64_t row = (static_cast<int64_t>(sp) * a.bh + bh) * a.s + my_q;
      float* op = a.o_part + row * D;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d = dt * 32 + 8 * g4 + 4 * h;
          float4 v;
          v.x = acc_o[dt][g4 * 4 + 0];
          v.y = acc_o[dt][g4 * 4 + 1];
          v.z = acc_o[dt][g4 * 4 + 2];
          v.w = acc_o[dt][g4 * 4 + 3];
          *reinterpret_cast<float4*>(op + d) = v;
        }
      if (h == 0) *reinterpret_cast<float2*>(a.ml_part + row * 2) = make_float2(m_run, l_run);
    }
  } else if (my_q < a.s) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16x4 out;
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = static_cast<bf16>(acc_o[dt][g4 * 4 + i] * inv);
        const int d = dt * 32 + 8 * g4 + 4 * h;
        *reinterpret_cast<bf16x4*>(O + static_cast<int64_t>(my_q) * D + d) = out;
      }
  }
}

// Merges the key ranges of hw variant 3, one wave per query row (two of
// the 128 output columns per lane): with M the largest running max,
// O = sum_r 2^(m_r - M) O_r / sum_r 2^(m_r - M) l_r. Lane r < nsplit loads
// range r's (max, sum) pair, and every range's two output columns are
// loaded in the same round, before the weights are formed, so a row costs
// one memory round trip; the weights then take two wave reductions.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ o_part,
                                                           const float* __restrict__ ml_part,
                                                           bf16* __restrict__ o, int nsplit,
                                                           int64_t rows) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  float2 ml = make_float2(-INFINITY, 0.f);
  if (lane < nsplit) ml = *reinterpret_cast<const float2*>(ml_part + (lane * rows + row) * 2);
  float2 v[kMaxSplits];
#pragma unroll
  for (int r = 0; r < kMaxSplits; ++r)
    if (r < nsplit) v[r] = *reinterpret_cast<const float2*>(o_part + (r * rows + row) * D + 2 * lane);
  const float mx = wave_max(ml.x);
  const float w = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
  const float l = wave_sum(w * ml.y);
  float o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int r = 0; r < kMaxSplits; ++r)
    if (r < nsplit) {
      const float wr = __shfl(w, r, 64);
      o0 += wr * v[r].x;
      o1 += wr * v[r].y;
    }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  bf16 out[2] = {static_cast<bf16>(o0 * inv), static_cast<bf16>(o1 * inv)};
  *reinterpret_cast<uint32_t*>(o + row * D + 2 * lane) = pack2(out[0], out[1]);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
const char* const kTileArgs[] = {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K",
                                 "TILES_IN_BLOCK_P"};

size_t attn_lds(int TN) {
  const int BKV = 32 * TN;
  return static_cast<size_t>(2) * (BKV * KP + D * (BKV + 8)) * sizeof(bf16);
}

// Waves, key-block tiles and query tiles per wave of one tile tuple: hw
// variant 0 runs W = 4 * TILES_IN_BLOCK_M waves (4 or 8) of one 32-query
// tile; hw variant 1 runs 4 waves of two 32-query tiles each.
struct AttnTiles {
  int W, TN, QT;
};

AttnTiles attn_tiles(const Call& c) {
  if (c.variant == 3) return {2 * c.tile(0), c.tile(1), 1};
  return {4 * c.tile(0), c.tile(1), c.variant == 1 ? 2 : 1};
}

// hw variant 3 splits the key range over workgroups and merges the partial
// softmax states in a second kernel; it is offered for up to this many query
// rows (batch * heads * s), where the other variants cannot fill the GPU and
// its workspace (nsplit * rows * 520 bytes) stays below 136 MB.
constexpr int64_t kSplitMaxRows = 16384;

int check_split_tiles(const Call& c, int64_t rows, std::string* why) {
  const int tm = c.tile(0), TN = c.tile(1), ns = c.tile(2);
  if (!(tm == 1 || tm == 2 || tm == 4)) {
    *why = "TILES_IN_BLOCK_M (pairs of waves) must be 1, 2 or 4";
    return AXON_EINVAL;
  }
  if (!(TN == 1 || TN == 2)) {
    *why = "TILES_IN_BLOCK_N (key block / 32) must be 1 or 2";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(ns, 1, kMaxSplits)) {
    *why = "TILES_IN_BLOCK_K (key-range splits) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  if (c.tile(3) != 1) {
    *why = "TILES_IN_BLOCK_P is unused and must be 1";
    return AXON_EINVAL;
  }
  if (rows > kSplitMaxRows) {
    *why = "split key ranges serve at most 16384 query rows (batch * heads * s)";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

int check_tiles(const Call& c, std::string* why) {
  const int tm = c.tile(0), TN = c.tile(1);
  if (c.variant != 1 ? !(tm == 1 || tm == 2) : tm != 1) {
    *why = c.variant != 1 ? "TILES_IN_BLOCK_M (groups of 4 waves) must be 1 or 2"
                          : "TILES_IN_BLOCK_M must be 1 (4 waves of two query tiles)";
    return AXON_EINVAL;
  }
  if (c.variant == 0 ? !(TN == 1 || TN == 2 || TN == 4) : !(TN == 1 || TN == 2)) {
    *why = c.variant == 0 ? "TILES_IN_BLOCK_N (key block / 32) must be 1, 2 or 4"
                          : "TILES_IN_BLOCK_N (key block / 32) must be 1 or 2 with two query tiles per wave";
    return AXON_EINVAL;
  }
  if (c.tile(2) != 1 || c.tile(3) != 1) {
    *why = "TILES_IN_BLOCK_K and TILES_IN_BLOCK_P are unused and must be 1";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

// attention_causal: dims b, h, s, d
int check_causal(const Call& c, std::string* why) {
  if (c.n_tiles != 4 || c.n_dims != 4 || c.n_dtypes != 3) {
    *why = "expected 4 tiles, 4 dims (b, h, s, d) and 3 dtypes";
    return AXON_EARG;
  }
  for (int i = 0; i < 3; ++i)
    if (c.dtype(i) != AXON_BF16) {
      *why = "bf16 inputs only";
      return AXON_EDTYPE;
    }
  if (c.dim(3) != D) {
    *why = "head dim must be 128";
    return AXON_EINVAL;
  }
  if (c.dim(0) < 0 || c.dim(1) < 0 || c.dim(2) < 0 || c.dim(0) * c.dim(1) > (1 << 20) ||
      c.dim(2) > (1 << 24)) {
    *why = "dimension out of range";
    return AXON_EINVAL;
  }
  if (c.variant == 3) return check_split_tiles(c, c.dim(0) * c.dim(1) * c.dim(2), why);
  return check_tiles(c, why);
}

// attention_nkilib: dims s, d
int check_nki(const Call& c, std::string* why) {
  if (c.n_tiles != 4 || c.n_dims != 2 || c.n_dtypes != 3) {
    *why = "expected 4 tiles, 2 dims (s, d) and 3 dtypes";
    return AXON_EARG;
  }
  for (int i = 0; i < 3; ++i)
    if (c.dtype(i) != AXON_BF16) {
      *why = "bf16 inputs only";
      return AXON_EDTYPE;
    }
  if (c.dim(1) != D) {
    *why = "head dim must be 128";
    return AXON_EINVAL;
  }
  if (c.dim(0) < 0 || c.dim(0) > (1 << 24)) {
    *why = "dimension out of range";
    return AXON_EINVAL;
  }
  if (c.dim(0) % 8 != 0) {
    *why = "s must be a multiple of 8 (16-byte rows of k_t)";
    return AXON_EINVAL;
  }
  if (c.variant == 3) return check_split_tiles(c, c.dim(0), why);
  return check_tiles(c, why);
}

int manifest_attn(int variant, Constraint* out, int cap, int64_t s, int64_t rows) {
  if (cap < 4) return 0;
  const int64_t sq = s > 0 ? s : 1;
  const int64_t kmax = variant == 0 ? 128 : 64;  // key block (variants 1-3: at most 64)
  out[0] = {"TILES_IN_BLOCK_M", variant == 1 ? 1 : (variant == 3 ? 4 : 2), 1, false};
  out[1] = {"TILES_IN_BLOCK_N", sq < kmax ? (sq < 32 ? 32 : sq) : kmax, 32, false};
  out[2] = {"TILES_IN_BLOCK_K", variant == 3 ? (rows <= kSplitMaxRows ? kMaxSplits : 0) : 1, 1, false};
  out[3] = {"TILES_IN_BLOCK_P", 1, 1, false};
  return 4;
}

int manifest_causal(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  (void)dt;
  return manifest_attn(v, out, cap, dims[2], dims[0] * dims[1] * dims[2]);
}

int manifest_nki(int v, const int64_t* dims, int dt, Constraint* out, int cap) {
  (void)dt;
  return manifest_attn(v, out, cap, dims[0], dims[0]);
}

// Split key ranges: keys per range (a multiple of the key block) and the
// number of non-empty ranges.
struct SplitPlan {
  int kv_split, nsplit;
};

SplitPlan split_plan(int64_t s, int TN, int ns) {
  const int64_t bkv = 32 * TN;
  const int64_t per = ((s + ns - 1) / ns + bkv - 1) / bkv * bkv;
  const int64_t used = per > 0 ? (s + per - 1) / per : 0;
  return {static_cast<int>(per > 0 ? per : bkv), static_cast<int>(used)};
}

// Workspace of hw variant 3: [nsplit][rows][D] fp32 outputs, then
// [nsplit][rows][2] fp32 (max, sum), at a 256-byte boundary.
size_t split_ws_bytes(int64_t rows, int nsplit, size_t* ml_off) {
  const size_t o = static_cast<size_t>(nsplit) * rows * D * sizeof(float);
  *ml_off = (o + 255) / 256 * 256;
  return *ml_off + static_cast<size_t>(nsplit) * rows * 2 * sizeof(float);
}

size_t workspace_attn(const Call& c, int64_t rows, int64_t s) {
  if (c.variant != 3) return 0;
  const SplitPlan p = split_plan(s, c.tile(1), c.tile(2));
  size_t ml_off;
  return split_ws_bytes(rows, p.nsplit, &ml_off);
}

size_t workspace_causal(const Call& c) {
  return workspace_attn(c, c.dim(0) * c.dim(1) * c.dim(2), c.dim(2));
}

size_t workspace_nki(const Call& c) { return workspace_attn(c, c.dim(0), c.dim(0)); }

void outputs_causal(const int64_t* dims, const int32_t*, OutDesc* out) {
  out[0] = {4, {dims[0], dims[1], dims[2], dims[3]}, AXON_BF16};
}

void outputs_nki(const int64_t* dims, const int32_t*, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, AXON_BF16};
}

template <int W, int TN, int QT, bool CAUSAL, bool KT>
int launch_t(const AttnArgs& a, hipStream_t st) {
  const size_t lds = attn_lds(TN);
  auto fn = attn_kernel<W, TN, QT, CAUSAL, KT>;
  static std::atomic<bool> configured{false};
  if (!configured.load(std::memory_order_acquire)) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                        static_cast<int>(lds));
    configured.store(true, std::memory_order_release);
  }
  const unsigned blocks = static_cast<unsigned>(a.qblocks) * static_cast<unsigned>(a.bh);
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(W * 64), lds, st, a);
  return launch_status("attn_kernel");
}

template <int W, int TN, bool CAUSAL, bool KT, bool SPLIT = false>
int launch_sp(const AttnArgs& a, hipStream_t st) {
  const size_t lds = attn_lds(TN);
  auto fn = attn_sp_kernel<W, TN, CAUSAL, KT, SPLIT>;
  static std::atomic<bool> configured{false};
  if (!configured.load(std::memory_order_acquire)) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
    configured.store(true, std::memory_order_release);
  }
  const unsigned blocks = static_cast<unsigned>(a.qblocks) * static_cast<unsigned>(a.bh) *
                         static_cast<unsigned>(SPLIT ? a.nsplit : 1);
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(W * 64), lds, st, a);
  int rc = launch_status("attn_sp_kernel");
  if (!SPLIT || rc != AXON_OK) return rc;
  const int64_t rows = static_cast<int64_t>(a.bh) * a.s;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, st,
                     a.o_part, a.ml_part, a.o, a.nsplit, rows);
  return launch_status("attn_combine_kernel");
}

template <bool CAUSAL, bool KT>
int dispatch(int W, int TN, int QT, const AttnArgs& a, hipStream_t st, int variant) {
  if (variant == 3) {
    if (W == 2 && TN == 1) return launch_sp<2, 1, CAUSAL, KT, true>(a, st);
    if (W == 2 && TN == 2) return launch_sp<2, 2, CAUSAL, KT, true>(a, st);
    if (W == 4 && TN == 1) return launch_sp<4, 1, CAUSAL, KT, true>(a, st);
    if (W == 4 && TN == 2) return launch_sp<4, 2, CAUSAL, KT, true>(a, st);
    if (W == 8 && TN == 1) return launch_sp<8, 1, CAUSAL, KT, true>(a, st);
    if (W == 8 && TN == 2) return launch_sp<8, 2, CAUSAL, KT, true>(a, st);
    set_error("no split-range attention instantiation for this tile");
    return AXON_EINVAL;
  }
  if (variant == 2) {
    if (W == 4 && TN == 1) return launch_sp<4, 1, CAUSAL, KT>(a, st);
    if (W == 4 && TN == 2) return launch_sp<4, 2, CAUSAL, KT>(a, st);
    if (W == 8 && TN == 1) return launch_sp<8, 1, CAUSAL, KT>(a, st);
    if (W == 8 && TN == 2) return launch_sp<8, 2, CAUSAL, KT>(a, st);
    set_error("no software-pipelined attention instantiation for this tile");
    return AXON_EINVAL;
  }
#define AXON_ATTN_CASE(w, tn, qt) \
  if (W == w && TN == tn && QT == qt) return launch_t<w, tn, qt, CAUSAL, KT>(a, st);
  AXON_ATTN_CASE(4, 1, 1) AXON_ATTN_CASE(4, 2, 1) AXON_ATTN_CASE(4, 4, 1)
  AXON_ATTN_CASE(8, 1, 1) AXON_ATTN_CASE(8, 2, 1) AXON_ATTN_CASE(8, 4, 1)
  AXON_ATTN_CASE(4, 1, 2) AXON_ATTN_CASE(4, 2, 2)
#undef AXON_ATTN_CASE
  set_error("no attention instantiation for this tile");
  return AXON_EINVAL;
}

int launch_common(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st,
                  int64_t bh, int64_t s, bool causal) {
  if (bh == 0 || s == 0) return AXON_OK;
  for (int i = 0; i < 3; ++i)
    if (!aligned16(in[i])) {
      set_error("attention inputs must be 16-byte aligned");
      return AXON_EARG;
    }
  if (!aligned16(out[0])) {
    set_error("attention output must be 16-byte aligned");
    return AXON_EARG;
  }
  const AttnTiles t = attn_tiles(c);
  const int W = t.W, TN = t.TN, QT = t.QT;
  AttnArgs a;
  a.q = static_cast<const bf16*>(in[0]);
  a.k = static_cast<const bf16*>(in[1]);
  a.v = static_cast<const bf16*>(in[2]);
  a.o = static_cast<bf16*>(out[0]);
  a.s = static_cast<int>(s);
  a.bh = static_cast<int>(bh);
  a.qblocks = static_cast<int>((s + 32 * W * QT - 1) / (32 * W * QT));
  {
    const int rc = grid_check("attn_kernel", static_cast<int64_t>(a.qblocks) * a.bh, 1, W * 64);
    if (rc != AXON_OK) return rc;
  }
  // Deal heads to XCDs (workgroup b runs on XCD b % 8) when they split evenly.
  a.xcd_heads = a.bh % kXcds == 0 ? a.bh / kXcds : 0;
  a.nsplit = 1;
  a.kv_split = a.s;
  a.o_part = a.ml_part = nullptr;
  if (c.variant == 3) {
    const SplitPlan p = split_plan(s, TN, c.tile(2));
    size_t ml_off;
    split_ws_bytes(bh * s, p.nsplit, &ml_off);
    a.nsplit = p.nsplit;
    a.kv_split = p.kv_split;
    a.o_part = static_cast<float*>(ws);
    a.ml_part = reinterpret_cast<float*>(static_cast<char*>(ws) + ml_off);
    int rc = grid_check("attn_sp_kernel", static_cast<int64_t>(a.qblocks) * a.bh * a.nsplit, 1, W * 64);
    if (rc == AXON_OK) rc = grid_check("attn_combine_kernel", (bh * s + 3) / 4, 1, 256);
    if (rc != AXON_OK) return rc;
  }
  if (causal) {
    a.scale_log2 = kLog2e / sqrtf(static_cast<float>(D));
    return dispatch<true, false>(W, TN, QT, a, st, c.variant);
  }
  a.scale_log2 = kLog2e;
  return dispatch<false, true>(W, TN, QT, a, st, c.variant);
}

int launch_causal(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  return launch_common(c, in, out, ws, st, c.dim(0) * c.dim(1), c.dim(2), true);
}

int launch_nki(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  return launch_common(c, in, out, ws, st, 1, c.dim(0), false);
}

const char* summary_attn(int variant) {
  return variant == 0
             ? "flash attention: S^T = K Q^T on 32x32x16 bf16 MFMA with Q^T in registers, one query "
               "per lane for an in-lane online softmax (exp2, fp32), P^T kept in registers as the B "
               "operand of O^T = V^T P^T, K and V^T double-buffered in LDS, causal block skipping; "
               "4 or 8 waves of 32 queries"
             : variant == 1
                   ? "flash attention as hw variant 0 with two 32-query tiles per wave (4 waves, one "
                     "per SIMD): every K and V^T fragment read from LDS feeds two MFMAs"
                   : variant == 2
                         ? "flash attention as hw variant 0, software-pipelined: K staged a block ahead "
                           "of V so each wave runs the next block's QK MFMAs under its softmax of this "
                           "block"
                         : "flash attention as hw variant 2 over split key ranges (2, 4 or 8 waves of "
                           "32 queries per workgroup): each range writes its unnormalised output, "
                           "running max and row sum, and a second kernel merges the ranges; fills the "
                           "GPU when batch * heads * s is small";
}

}  // namespace

const Family* family_attention_causal() {
  static const Family f = {"attention_causal", 4, 3, 1, 4, kTileArgs, 4, summary_attn,
                           manifest_causal, check_causal, workspace_causal, outputs_causal, launch_causal};
  return &f;
}

const Family* family_attention_nkilib() {
  static const Family f = {"attention_nkilib", 4, 3, 1, 2, kTileArgs, 4, summary_attn, manifest_nki,
                           check_nki, workspace_nki, outputs_nki, launch_nki};
  return &f;
}

}  // namespace axon
