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
//                 TILES_IN_BLOCK_N = H (head rows per thread).
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
    *why = "TILES_IN_BLOCK_N (heads per thread) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

int manifest_tok(int, const int64_t* dims, int, Constraint* out, int cap) {
  if (cap < 2) return 0;
  const int64_t nh = dims[2] + dims[3];
  out[0] = {"TILES_IN_BLOCK_M", 16, 1, false};
  out[1] = {"TILES_IN_BLOCK_N", nh < 16 ? (nh > 0 ? nh : 1) : 16, 1, false};
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
  if (vec) {
    const int W = c.tile(0), H = c.tile(1);
    const int HG = (nh + H - 1) / H;
    const int J = (d / 2) / E;
    const int64_t slots = tokens * HG * J;
    const int bd = W * kWave;
    const dim3 grid(static_cast<unsigned>((slots + bd - 1) / bd));
    hipLaunchKernelGGL((tok_fn<T>(H)), grid, dim3(bd), 0, st, q, k, cs, sn, qo, ko, tokens, s, hq,
                       hkv, d, HG);
  } else {
    const int64_t total = tokens * nh * (d / 2);
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

const char* summary_tok(int) {
  return "token-major rotate-half: one thread per (token, head group, pair slice), cos/sin "
         "slices loaded once and reused for H interleaved heads; q and k in one launch";
}

}  // namespace

const Family* family_rope_llama3() {
  static const Family f = {"rope_llama3", 1, 4, 2, 5, kTileArgs, 2, summary_tok, manifest_tok,
                           check_tok, no_workspace, outputs_tok, launch_tok};
  return &f;
}

}  // namespace axon
