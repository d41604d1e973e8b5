// Elementwise families: RoPE on the split layout and fused Adam.
//
//   rope        out_even = xe*cos - xo*sin, out_odd = xo*cos + xe*sin
//               over four (half_d, free) tensors      kernels/rope/kernel.py:27-36
//   fused_adam  g = grad + wd*p; m' = b1*m + (1-b1)*g; v' = b2*v + (1-b2)*g^2;
//               p' = p - m' / (sqrt(v')*ibc + eps) * step, with (p, 1) per-row
//               scalars                                 kernels/fused_adam/kernel.py:20-45
//
// Schedule (hw variant 0): the tensors are walked as flat arrays of 16-byte
// vectors; a workgroup of W waves covers V*W*64 consecutive vectors, lane-
// contiguous at each of its V steps, so every access is a full 16-byte
// coalesced load or store and each byte moves exactly once.
// Tile arguments: TILES_IN_BLOCK_M = W (waves per workgroup),
//                 TILES_IN_BLOCK_N = V (16-byte vectors per lane).
//
// This unit is compiled with -ffp-contract=off: Adam's products and sums
// round one at a time, in the order the fp32 CPU reference evaluates them.
#include "common.hpp"
#include "registry.hpp"

namespace axon {
namespace {

constexpr double kBeta1 = 0.9;
constexpr double kBeta2 = 0.999;
// The constants the fp32 reference sees: each double literal rounded to fp32.
constexpr float kB1 = static_cast<float>(kBeta1);
constexpr float kOneMinusB1 = static_cast<float>(1.0 - kBeta1);
constexpr float kB2 = static_cast<float>(kBeta2);
constexpr float kOneMinusB2 = static_cast<float>(1.0 - kBeta2);
constexpr float kAdamEps = static_cast<float>(1e-8);

// ---------------------------------------------------------------------------
// per-element math
// ---------------------------------------------------------------------------
struct RopeMath {
  __device__ static void apply(float xe, float xo, float c, float s, float* oe, float* oo) {
    const float a = xe * c;
    const float b = xo * s;
    const float d = xo * c;
    const float e = xe * s;
    *oe = a - b;
    *oo = d + e;
  }
};

struct AdamMath {
  __device__ static void apply(float p, float g, float m, float v, float step, float ibc, float wd,
                               float* po, float* mo, float* vo) {
    const float wp = wd * p;
    const float gp = g + wp;
    const float m1 = kB1 * m;
    const float m2 = kOneMinusB1 * gp;
    const float mn = m1 + m2;
    const float v1 = kB2 * v;
    const float g2 = gp * gp;
    const float v2 = kOneMinusB2 * g2;
    const float vn = v1 + v2;
    const float sq = sqrtf(vn);
    const float den0 = sq * ibc;
    const float den = den0 + kAdamEps;
    const float q = mn / den;
    const float upd = q * step;
    *po = p - upd;
    *mo = mn;
    *vo = vn;
  }
};

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------
template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void rope_split_kernel(const T* __restrict__ xe,
                                                          const T* __restrict__ xo,
                                                          const T* __restrict__ cs,
                                                          const T* __restrict__ sn,
                                                          T* __restrict__ oe, T* __restrict__ oo,
                                                          int64_t len) {
  constexpr int E = EPV<T>::value;
  const int64_t bd = blockDim.x;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * V * bd + threadIdx.x;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t vi = base + v * bd;
    if constexpr (ALIGNED) {
      const int64_t off = vi * E;
      if (off >= len) continue;
      const Vec<T> a = load_vec_nt(xe + off), b = load_vec_nt(xo + off),
                   c = load_vec_nt(cs + off), s = load_vec_nt(sn + off);
      Vec<T> ra, rb;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float fa, fb;
        RopeMath::apply(to_f32(a.v[e]), to_f32(b.v[e]), to_f32(c.v[e]), to_f32(s.v[e]), &fa, &fb);
        ra.v[e] = from_f32<T>(fa);
        rb.v[e] = from_f32<T>(fb);
      }
      store_vec_nt(oe + off, ra);
      store_vec_nt(oo + off, rb);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int64_t i = vi * E + e;
        if (i >= len) break;
        float fa, fb;
        RopeMath::apply(to_f32(xe[i]), to_f32(xo[i]), to_f32(cs[i]), to_f32(sn[i]), &fa, &fb);
        oe[i] = from_f32<T>(fa);
        oo[i] = from_f32<T>(fb);
      }
    }
  }
}

template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void adam_kernel(
    const T* __restrict__ p, const T* __restrict__ g, const T* __restrict__ m,
    const T* __restrict__ v, const T* __restrict__ step, const T* __restrict__ ibc,
    const T* __restrict__ wd, T* __restrict__ po, T* __restrict__ mo, T* __restrict__ vo,
    int64_t len, int64_t f) {
  constexpr int E = EPV<T>::value;
  const int64_t bd = blockDim.x;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * V * bd + threadIdx.x;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int64_t vi = base + k * bd;
    if constexpr (ALIGNED) {
      const int64_t off = vi * E;
      if (off >= len) continue;
      const int64_t row = off / f;  // f % E == 0: one row per vector
      const float st = to_f32(step[row]), ib = to_f32(ibc[row]), w = to_f32(wd[row]);
      const Vec<T> pv = load_vec_nt(p + off), gv = load_vec_nt(g + off),
                   mv = load_vec_nt(m + off), vv = load_vec_nt(v + off);
      Vec<T> rp, rm, rv;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float a, b, c;
        AdamMath::apply(to_f32(pv.v[e]), to_f32(gv.v[e]), to_f32(mv.v[e]), to_f32(vv.v[e]), st,
                        ib, w, &a, &b, &c);
        rp.v[e] = from_f32<T>(a);
        rm.v[e] = from_f32<T>(b);
        rv.v[e] = from_f32<T>(c);
      }
      store_vec_nt(po + off, rp);
      store_vec_nt(mo + off, rm);
      store_vec_nt(vo + off, rv);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int64_t i = vi * E + e;
        if (i >= len) break;
        const int64_t row = i / f;
        float a, b, c;
        AdamMath::apply(to_f32(p[i]), to_f32(g[i]), to_f32(m[i]), to_f32(v[i]), to_f32(step[row]),
                        to_f32(ibc[row]), to_f32(wd[row]), &a, &b, &c);
        po[i] = from_f32<T>(a);
        mo[i] = from_f32<T>(b);
        vo[i] = from_f32<T>(c);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
const char* const kTileArgs[] = {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"};

int check_ew(const Call& c, int n_in, std::string* why) {
  if (c.n_tiles != 2 || c.n_dims != 2 || c.n_dtypes != n_in) {
    *why = "expected 2 tiles, 2 dims and one dtype per input";
    return AXON_EARG;
  }
  const int dt = c.dtype(0);
  if (dt != AXON_BF16 && dt != AXON_F32) {
    *why = std::string("unsupported dtype ") + dtype_str(dt);
    return AXON_EDTYPE;
  }
  for (int i = 1; i < n_in; ++i)
    if (c.dtype(i) != dt) {
      *why = "all inputs must share one dtype";
      return AXON_EDTYPE;
    }
  if (c.dim(0) < 0 || c.dim(1) < 0) {
    *why = "negative dimension";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(c.tile(0), 1, 16)) {
    *why = "TILES_IN_BLOCK_M (waves per workgroup) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(c.tile(1), 1, 8)) {
    *why = "TILES_IN_BLOCK_N (16-byte vectors per lane) must be a power of two in [1, 8]";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

int manifest_ew(int, const int64_t* dims, int dtype, Constraint* out, int cap) {
  if (cap < 2) return 0;
  const int64_t E = 16 / elem_bytes(dtype);
  const int64_t vecs = (dims[0] * dims[1] + E - 1) / E;
  const int64_t waves = (vecs + kWave - 1) / kWave;
  out[0] = {"TILES_IN_BLOCK_M", waves < 16 ? (waves > 0 ? waves : 1) : 16, 1, false};
  out[1] = {"TILES_IN_BLOCK_N", 8, 1, false};
  return 2;
}

size_t no_workspace(const Call&) { return 0; }

const char* summary_ew(int) {
  return "flat 16-byte-vector stream: W waves per workgroup, V lane-contiguous vectors per lane; "
         "every input byte read once, every output byte written once";
}

// rope ----------------------------------------------------------------------
int check_rope(const Call& c, std::string* why) { return check_ew(c, 4, why); }

void outputs_rope(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, dtypes[0]};
  out[1] = {2, {dims[0], dims[1]}, dtypes[0]};
}

template <typename T, bool A>
void (*rope_fn(int V))(const T*, const T*, const T*, const T*, T*, T*, int64_t) {
  switch (V) {
    case 1: return rope_split_kernel<T, 1, A>;
    case 2: return rope_split_kernel<T, 2, A>;
    case 4: return rope_split_kernel<T, 4, A>;
    default: return rope_split_kernel<T, 8, A>;
  }
}

template <typename T>
int launch_rope_t(const Call& c, const void* const* in, void* const* out, hipStream_t st) {
  const int64_t len = c.dim(0) * c.dim(1);
  if (len == 0) return AXON_OK;
  constexpr int E = EPV<T>::value;
  const int W = c.tile(0), V = c.tile(1);
  const T* a = static_cast<const T*>(in[0]);
  const T* b = static_cast<const T*>(in[1]);
  const T* cs = static_cast<const T*>(in[2]);
  const T* sn = static_cast<const T*>(in[3]);
  T* oe = static_cast<T*>(out[0]);
  T* oo = static_cast<T*>(out[1]);
  bool aligned = len % E == 0;
  for (const void* ptr : {in[0], in[1], in[2], in[3], static_cast<const void*>(out[0]),
                          static_cast<const void*>(out[1])})
    aligned = aligned && aligned16(ptr);
  const int64_t vecs = (len + E - 1) / E;
  const int64_t per_block = static_cast<int64_t>(V) * W * kWave;
  const int rc = grid_check("rope_split_kernel", (vecs + per_block - 1) / per_block, 1, W * kWave);
  if (rc != AXON_OK) return rc;
  const dim3 grid(static_cast<unsigned>((vecs + per_block - 1) / per_block)), block(W * kWave);
  if (aligned)
    hipLaunchKernelGGL((rope_fn<T, true>(V)), grid, block, 0, st, a, b, cs, sn, oe, oo, len);
  else
    hipLaunchKernelGGL((rope_fn<T, false>(V)), grid, block, 0, st, a, b, cs, sn, oe, oo, len);
  return launch_status("rope_split_kernel");
}

int launch_rope(const Call& c, const void* const* in, void* const* out, void*, hipStream_t st) {
  return c.dtype(0) == AXON_BF16 ? launch_rope_t<bf16>(c, in, out, st)
                                 : launch_rope_t<float>(c, in, out, st);
}

// adam ----------------------------------------------------------------------
int check_adam(const Call& c, std::string* why) { return check_ew(c, 7, why); }

void outputs_adam(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  for (int i = 0; i < 3; ++i) out[i] = {2, {dims[0], dims[1]}, dtypes[0]};
}

template <typename T, bool A>
void (*adam_fn(int V))(const T*, const T*, const T*, const T*, const T*, const T*, const T*, T*,
                       T*, T*, int64_t, int64_t) {
  switch (V) {
    case 1: return adam_kernel<T, 1, A>;
    case 2: return adam_kernel<T, 2, A>;
    case 4: return adam_kernel<T, 4, A>;
    default: return adam_kernel<T, 8, A>;
  }
}

template <typename T>
int launch_adam_t(const Call& c, const void* const* in, void* const* out, hipStream_t st) {
  const int64_t f = c.dim(1);
  const int64_t len = c.dim(0) * f;
  if (len == 0) return AXON_OK;
  constexpr int E = EPV<T>::value;
  const int W = c.tile(0), V = c.tile(1);
  const T* x[7];
  for (int i = 0; i < 7; ++i) x[i] = static_cast<const T*>(in[i]);
  T* o[3];
  for (int i = 0; i < 3; ++i) o[i] = static_cast<T*>(out[i]);
  bool aligned = f % E == 0;
  for (int i = 0; i < 4; ++i) aligned = aligned && aligned16(x[i]);
  for (int i = 0; i < 3; ++i) aligned = aligned && aligned16(o[i]);
  const int64_t vecs = (len + E - 1) / E;
  const int64_t per_block = static_cast<int64_t>(V) * W * kWave;
  const int rc = grid_check("adam_kernel", (vecs + per_block - 1) / per_block, 1, W * kWave);
  if (rc != AXON_OK) return rc;
  const dim3 grid(static_cast<unsigned>((vecs + per_block - 1) / per_block)), block(W * kWave);
  if (aligned)
    hipLaunchKernelGGL((adam_fn<T, true>(V)), grid, block, 0, st, x[0], x[1], x[2], x[3], x[4],
                       x[5], x[6], o[0], o[1], o[2], len, f);
  else
    hipLaunchKernelGGL((adam_fn<T, false>(V)), grid, block, 0, st, x[0], x[1], x[2], x[3], x[4],
                       x[5], x[6], o[0], o[1], o[2], len, f);
  return launch_status("adam_kernel");
}

int launch_adam(const Call& c, const void* const* in, void* const* out, void*, hipStream_t st) {
  return c.dtype(0) == AXON_BF16 ? launch_adam_t<bf16>(c, in, out, st)
                                 : launch_adam_t<float>(c, in, out, st);
}

}  // namespace

const Family* family_rope() {
  static const Family f = {"rope", 1, 4, 2, 2, kTileArgs, 2, summary_ew, manifest_ew, check_rope,
                           no_workspace, outputs_rope, launch_rope};
  return &f;
}

const Family* family_fused_adam() {
  static const Family f = {"fused_adam", 1, 7, 3, 2, kTileArgs, 2, summary_ew, manifest_ew,
                           check_adam, no_workspace, outputs_adam, launch_adam};
  return &f;
}

}  // namespace axon
