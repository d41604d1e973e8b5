// Token-major rotate-half RoPE (family "rope_llama3"): q[b, s, hq, d] and
// k[b, s, hkv, d] rotated in one launch with fp32 cos/sin[s, d].
//
// For each head row x and i < d/2 (the rotation of kernels/rope/kernel.py:33-36
// with x_even = x[:d/2], x_odd = x[d/2:]):
//   out[i]       = x[i]       * cos[p, i]       - x[i + d/2] * sin[p, i]
//   out[i + d/2] = x[i + d/2] * cos[p, i + d/2] + x[i]       * sin[p, i + d/2]
// with p = token position (token index mod s).
//
// Schedule (hw variant 0): a thread owns one (token, head group, j) slot,
// j selecting E consecutive rotation pairs (two 16-byte vectors of x, one in
// each half). It loads its cos/sin slices once and reuses them for the H
// heads of its group; heads are interleaved across groups (head = g + i*HG)
// so lanes of one wave touch consecutive head rows. q and k heads form one
// index space (q first), so one launch covers both tensors; x is read once
// and written once.
// Tile arguments: TILES_IN_BLOCK_M = W (waves per workgroup),
//                 TILES_IN_BLOCK_N = H (head rows per thread; hw variant 1:
//                 tokens per workgroup).
#include "common.hpp"
#include "registry.hpp"

namespace axon {
namespace {

template <typename T, int H>
__global__ __launch_bounds__(1024) void rope_tok_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const float* __restrict__ cs,
    const float* __restrict__ sn, T* __restrict__ qo, T* __restrict__ ko, int64_t tokens,
    int64_t s, int hq, int hkv, int d, int HG) {
  constexpr int E = EPV<T>::value;
  const int half = d >> 1;
  const int J = half / E;
  const int64_t slot = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_token = static_cast<int64_t>(HG) * J;
  const int64_t t = slot / per_token;
  if (t >= tokens) return;
  const int rem = static_cast<int>(slot - t * per_token);
  const int g = rem / J;
  const int j = rem - g * J;
  const int64_t pos = t % s;
  const int nh = hq + hkv;

  // cos/sin for the two halves of this thread's E pairs (fp32, 16-byte loads).
  float clo[E], chi[E], slo[E], shi[E];
  const float* crow = cs + pos * d;
  const float* srow = sn + pos * d;
#pragma unroll
  for (int e = 0; e < E; e += 4) {
    const Vec<float> a = load_vec(crow + j * E + e);
    const Vec<float> b = load_vec(crow + half + j * E + e);
    const Vec<float> c = load_vec(srow + j * E + e);
    const Vec<float> dd = load_vec(srow + half + j * E + e);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      clo[e + u] = a.v[u];
      chi[e + u] = b.v[u];
      slo[e + u] = c.v[u];
      shi[e + u] = dd.v[u];
    }
  }

  // All H heads' loads are issued before any arithmetic (heads past the last
  // one re-read the last head and are not stored): with no branch between
  // them the 2H loads are in flight together.
  Vec<T> lo[H], hi[H];
  T* dst[H];
  bool live[H];
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const int h0 = g + i * HG;
    live[i] = h0 < nh;
    const int h = min(h0, nh - 1);
    const T* src = h < hq ? q + (t * hq + h) * d : k + (t * hkv + (h - hq)) * d;
    dst[i] = h < hq ? qo + (t * hq + h) * d : ko + (t * hkv + (h - hq)) * d;
    // q/k are touched exactly once: non-temporal loads and stores stream
    // past the caches (cos/sin above stay cached for the other heads).
    lo[i] = load_vec_nt(src + j * E);
    hi[i] = load_vec_nt(src + half + j * E);
  }
#pragma unroll
  for (int i = 0; i < H; ++i) {
    Vec<T> olo, ohi;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float a = to_f32(lo[i].v[e]);
      const float b = to_f32(hi[i].v[e]);
      olo.v[e] = from_f32<T>(a * clo[e] - b * slo[e]);
      ohi.v[e] = from_f32<T>(b * chi[e] + a * shi[e]);
    }
    if (live[i]) {
      store_vec_nt(dst[i] + j * E, olo);
      store_vec_nt(dst[i] + half + j * E, ohi);
    }
  }
}

// hw variant 1 (token-aligned workgroups): workgroup b owns tokens
// [b * TPB, (b + 1) * TPB) whole. It stages their cos/sin rows in LDS with one
// 16-byte load per vector, so each row leaves HBM once and is read by one
// XCD only (hw variant 0's workgroups straddle tokens, and a token's rows are
// fetched again by the neighbouring workgroup on another XCD: 52.9 MB read
// against 46.1 MB at the Llama-3-8B shape). Slot i of the workgroup is (token
// i / (nh * J), head, pair slice j), j fastest, as in variant 0 with H = 1; a
// thread walks its slots in chunks of U (1-4, the fewest that cover its
// slots in one chunk when they fit) whose x loads are all issued before any
// arithmetic. The first chunk's loads are issued before the LDS barrier.
template <typename T, int kRopeU>
__global__ __launch_bounds__(1024) void rope_tokgroup_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const float* __restrict__ cs,
    const float* __restrict__ sn, T* __restrict__ qo, T* __restrict__ ko, int64_t tokens,
    int64_t s, int hq, int hkv, int d, int TPB) {
  constexpr int E = EPV<T>::value;
  extern __shared__ __align__(16) float rows[];  // [TPB][2][d]: cos row, sin row
  const int half = d >> 1;
  const int J = half / E;
  const int nh = hq + hkv;
  const int per_token = nh * J;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TPB;
  const int ntok = static_cast<int>(min<int64_t>(TPB, tokens - t0));
  const int total = ntok * per_token;
  const int nt = blockDim.x;

  Vec<T> lo[kRopeU], hi[kRopeU];
  int tt[kRopeU], jj[kRopeU];
  T* dst[kRopeU];
  bool live[kRopeU];
  // Issue the x loads of the chunk starting at slot `base` (slots past the
  // end re-read the workgroup's first slot and are not stored).
  auto load_chunk = [&](int base) {
#pragma unroll
    for (int u = 0; u < kRopeU; ++u) {
      const int slot0 = base + u * nt;
      live[u] = slot0 < total;
      const int slot = live[u] ? slot0 : 0;
      tt[u] = slot / per_token;
      const int rem = slot - tt[u] * per_token;
      const int h = rem / J;
      jj[u] = rem - h * J;
      const int64_t t = t0 + tt[u];
      const T* src = h < hq ? q + (t * hq + h) * d : k + (t * hkv + (h - hq)) * d;
      dst[u] = h < hq ? qo + (t * hq + h) * d : ko + (t * hkv + (h - hq)) * d;
      lo[u] = load_vec_nt(src + jj[u] * E);
      hi[u] = load_vec_nt(src + half + jj[u] * E);
    }
  };

  // cos/sin rows of this workgroup's tokens: 2 * d / 4 vectors per token.
  const int vrow = d / 4;
  const int nvec = ntok * 2 * vrow;
  // Branch-free: a vector index past the end re-copies vector 0 (the same
  // value thread 0 writes there), so the loads stay ahead of the x loads and
  // in flight together.
  const int p0 = static_cast<int>(t0 % s);  // position of the workgroup's first token
  const int si = static_cast<int>(s);
  auto row_vec = [&](int i) -> const float4* {
    const int tok = i / (2 * vrow), rem = i - tok * 2 * vrow;
    const int which = rem / vrow, c = rem - which * vrow;
    int pos = p0 + tok;
    while (pos >= si) pos -= si;
    return reinterpret_cast<const float4*>((which ? sn : cs) + static_cast<int64_t>(pos) * d + c * 4);
  };
  const int i0 = threadIdx.x, i1 = threadIdx.x + nt;
  const int c0 = i0 < nvec ? i0 : 0, c1 = i1 < nvec ? i1 : 0;
  const float4 cv0 = *row_vec(c0), cv1 = *row_vec(c1);
  load_chunk(threadIdx.x);
  __builtin_amdgcn_sched_barrier(0);
  reinterpret_cast<float4*>(rows)[c0] = cv0;
  reinterpret_cast<float4*>(rows)[c1] = cv1;
  constexpr int kR = 2;
  for (int i = threadIdx.x + kR * nt; i < nvec; i += nt)  // more than kR vectors per thread
    reinterpret_cast<float4*>(rows)[i] = *row_vec(i);
  __syncthreads();

  for (int base = threadIdx.x;;) {
#pragma unroll
    for (int u = 0; u < kRopeU; ++u) {
      const float* crow = rows + tt[u] * 2 * d;
      const float* srow = crow + d;
      Vec<T> olo, ohi;
#pragma unroll
      for (int e0 = 0; e0 < E; e0 += 4) {
        const float4 c_lo = *reinterpret_cast<const float4*>(crow + jj[u] * E + e0);
        const float4 c_hi = *reinterpret_cast<const float4*>(crow + half + jj[u] * E + e0);
        const float4 s_lo = *reinterpret_cast<const float4*>(srow + jj[u] * E + e0);
        const float4 s_hi = *reinterpret_cast<const float4*>(srow + half + jj[u] * E + e0);
        const float cl[4] = {c_lo.x, c_lo.y, c_lo.z, c_lo.w}, ch[4] = {c_hi.x, c_hi.y, c_hi.z, c_hi.w};
        const float sl[4] = {s_lo.x, s_lo.y, s_lo.z, s_lo.w}, sh[4] = {s_hi.x, s_hi.y, s_hi.z, s_hi.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = to_f32(lo[u].v[e0 + e]);
          const float b = to_f32(hi[u].v[e0 + e]);
          olo.v[e0 + e] = from_f32<T>(a * cl[e] - b * sl[e]);
          ohi.v[e0 + e] = from_f32<T>(b * ch[e] + a * sh[e]);
        }
      }
      if (live[u]) {
        store_vec_nt(dst[u] + jj[u] * E, olo);
        store_vec_nt(dst[u] + half + jj[u] * E, ohi);
      }
    }
    base += kRopeU * nt;
    if (base >= total) break;
    load_chunk(base);
  }
}

// Element-at-a-time fallback for head dims or pointers the vector path
// cannot take: one thread per (token, head, pair).
template <typename T>
__global__ __launch_bounds__(256) void rope_tok_scalar_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const float* __restrict__ cs,
    const float* __restrict__ sn, T* __restrict__ qo, T* __restrict__ ko, int64_t tokens,
    int64_t s, int hq, int hkv, int d) {
  const int half = d >> 1;
  const int nh = hq + hkv;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = tokens * nh * half;
  if (idx >= total) return;
  const int i = static_cast<int>(idx % half);
  const int64_t th = idx / half;
  const int h = static_cast<int>(th % nh);
  const int64_t t = th / nh;
  const int64_t pos = t % s;
  const T* src = h < hq ? q + (t * hq + h) * d : k + (t * hkv + (h - hq)) * d;
  T* dst = h < hq ? qo + (t * hq + h) * d : ko + (t * hkv + (h - hq)) * d;
  const float a = to_f32(src[i]);
  const float b = to_f32(src[i + half]);
  dst[i] = from_f32<T>(a * cs[pos * d + i] - b * sn[pos * d + i]);
  dst[i + half] = from_f32<T>(b * cs[pos * d + i + half] + a * sn[pos * d + i + half]);
}

const char* const kTileArgs[] = {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"};

// dims: b, s, hq, hkv, d
int check_tok(const Call& c, std::string* why) {
  if (c.n_tiles != 2 || c.n_dims != 5 || c.n_dtypes != 4) {
    *why = "expected 2 tiles, 5 dims (b, s, hq, hkv, d) and 4 dtypes";
    return AXON_EARG;
  }
  const int dt = c.dtype(0);
  if ((dt != AXON_BF16 && dt != AXON_F32) || c.dtype(1) != dt) {
    *why = "q and k must share a bf16 or fp32 dtype";
    return AXON_EDTYPE;
  }
  if (c.dtype(2) != AXON_F32 || c.dtype(3) != AXON_F32) {
    *why = "cos/sin must be fp32";
    return AXON_EDTYPE;
  }
  for (int i = 0; i < 5; ++i)
    if (c.dim(i) < 0) {
      *why = "negative dimension";
      return AXON_EINVAL;
    }
  if (c.dim(4) % 2 != 0) {
    *why = "head dim must be even";
    return AXON_EINVAL;
  }
  if (c.dim(2) + c.dim(3) > (1 << 20) || c.dim(4) > (1 << 16)) {
    *why = "head count or head dim out of range";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(c.tile(0), 1, 16)) {
    *why = "TILES_IN_BLOCK_M (waves per workgroup) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(c.tile(1), 1, 16)) {
    *why = c.variant == 1 ? "TILES_IN_BLOCK_N (tokens per workgroup) must be a power of two in [1, 16]"
                          : "TILES_IN_BLOCK_N (heads per thread) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  if (c.variant == 1 && static_cast<int64_t>(c.tile(1)) * 2 * c.dim(4) * 4 > 64 * 1024) {
    *why = "TILES_IN_BLOCK_N: the tokens' cos/sin rows exceed 64 KiB of LDS";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

int manifest_tok(int variant, const int64_t* dims, int, Constraint* out, int cap) {
  if (cap < 2) return 0;
  const int64_t nh = dims[2] + dims[3];
  out[0] = {"TILES_IN_BLOCK_M", 16, 1, false};
  if (variant == 1) {
    // Tokens per workgroup: at most 16, and their cos/sin rows within 64 KiB.
    int64_t t = 16;
    while (t > 1 && t * 2 * dims[4] * 4 > 64 * 1024) t >>= 1;
    out[1] = {"TILES_IN_BLOCK_N", t, 1, false};
  } else {
    out[1] = {"TILES_IN_BLOCK_N", nh < 16 ? (nh > 0 ? nh : 1) : 16, 1, false};
  }
  return 2;
}

size_t no_workspace(const Call&) { return 0; }

void outputs_tok(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  out[0] = {4, {dims[0], dims[1], dims[2], dims[4]}, dtypes[0]};
  out[1] = {4, {dims[0], dims[1], dims[3], dims[4]}, dtypes[0]};
}

template <typename T>
using TokFn = void (*)(const T*, const T*, const float*, const float*, T*, T*, int64_t, int64_t,
                       int, int, int, int);

template <typename T>
TokFn<T> tok_fn(int H) {
  switch (H) {
    case 1: return rope_tok_kernel<T, 1>;
    case 2: return rope_tok_kernel<T, 2>;
    case 4: return rope_tok_kernel<T, 4>;
    case 8: return rope_tok_kernel<T, 8>;
    default: return rope_tok_kernel<T, 16>;
  }
}

template <typename T>
int launch_tok_t(const Call& c, const void* const* in, void* const* out, hipStream_t st) {
  constexpr int E = EPV<T>::value;
  const int64_t b = c.dim(0), s = c.dim(1);
  const int hq = static_cast<int>(c.dim(2)), hkv = static_cast<int>(c.dim(3));
  const int d = static_cast<int>(c.dim(4));
  const int64_t tokens = b * s;
  const int nh = hq + hkv;
  if (tokens == 0 || nh == 0 || d == 0) return AXON_OK;
  const T* q = static_cast<const T*>(in[0]);
  const T* k = static_cast<const T*>(in[1]);
  const float* cs = static_cast<const float*>(in[2]);
  const float* sn = static_cast<const float*>(in[3]);
  T* qo = static_cast<T*>(out[0]);
  T* ko = static_cast<T*>(out[1]);
  bool vec = (d / 2) % E == 0 && (d / 2) % 4 == 0;
  for (const void* p : {in[0], in[1], in[2], in[3], static_cast<const void*>(out[0]),
                        static_cast<const void*>(out[1])})
    vec = vec && aligned16(p);
  if (vec && c.variant == 1) {
    const int W = c.tile(0), TPB = c.tile(1);
    const int bd = W * kWave;
    const size_t lds = static_cast<size_t>(TPB) * 2 * d * sizeof(float);
    if (lds > 64 * 1024) {
      set_error("rope_llama3 v1: TILES_IN_BLOCK_N tokens of cos/sin rows exceed 64 KiB of LDS");
      return AXON_EINVAL;
    }
    const int64_t blocks = (tokens + TPB - 1) / TPB;
    const int rc = grid_check("rope_tokgroup_kernel", blocks, 1, bd);
    if (rc != AXON_OK) return rc;
    // Slots per chunk: enough to cover a workgroup's slots in one chunk when
    // they fit in 4 (fewer idle slots than a fixed 4), else chunks of 4.
    const int64_t per_thread = (static_cast<int64_t>(TPB) * (hq + hkv) * ((d / 2) / E) + bd - 1) / bd;
    auto fn = per_thread <= 1 ? rope_tokgroup_kernel<T, 1>
              : per_thread == 2 ? rope_tokgroup_kernel<T, 2>
              : per_thread == 3 ? rope_tokgroup_kernel<T, 3>
                                : rope_tokgroup_kernel<T, 4>;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(bd), lds, st, q, k, cs, sn, qo, ko, tokens,
                       s, hq, hkv, d, TPB);
    return launch_status("rope_tokgroup_kernel");
  }
  if (vec) {
    const int W = c.tile(0), H = c.tile(1);
    const int HG = (nh + H - 1) / H;
    const int J = (d / 2) / E;
    const int64_t slots = tokens * HG * J;
    const int bd = W * kWave;
    const int rc = grid_check("rope_tok_kernel", (slots + bd - 1) / bd, 1, bd);
    if (rc != AXON_OK) return rc;
    const dim3 grid(static_cast<unsigned>((slots + bd - 1) / bd));
    hipLaunchKernelGGL((tok_fn<T>(H)), grid, dim3(bd), 0, st, q, k, cs, sn, qo, ko, tokens, s, hq,
                       hkv, d, HG);
  } else {
    const int64_t total = tokens * nh * (d / 2);
    const int rc = grid_check("rope_tok_scalar_kernel", (total + 255) / 256, 1, 256);
    if (rc != AXON_OK) return rc;
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    hipLaunchKernelGGL(rope_tok_scalar_kernel<T>, grid, dim3(256), 0, st, q, k, cs, sn, qo, ko,
                       tokens, s, hq, hkv, d);
  }
  return launch_status("rope_tok_kernel");
}

int launch_tok(const Call& c, const void* const* in, void* const* out, void*, hipStream_t st) {
  return c.dtype(0) == AXON_BF16 ? launch_tok_t<bf16>(c, in, out, st)
                                 : launch_tok_t<float>(c, in, out, st);
}

const char* summary_tok(int variant) {
  return variant == 1
             ? "token-major rotate-half, token-aligned workgroups of TILES_IN_BLOCK_N tokens: their "
               "cos/sin rows staged once in LDS (each row read from HBM by one XCD), slots walked in "
               "chunks of 4 with the x loads in flight together; q and k in one launch"
             : "token-major rotate-half: one thread per (token, head group, pair slice), cos/sin "
               "slices loaded once and reused for H interleaved heads; q and k in one launch";
}

}  // namespace

const Family* family_rope_llama3() {
  static const Family f = {"rope_llama3", 2, 4, 2, 5, kTileArgs, 2, summary_tok, manifest_tok,
                           check_tok, no_workspace, outputs_tok, launch_tok};
  return &f;
}

}  // namespace axon
