// Row-wise reductions with the row held in registers: RMSNorm (sum form and
// mean+eps+weight form), LayerNorm and softmax.
//
// Math, per row of x[m, n] with an fp32 accumulator:
//   rmsnorm           y = x / sqrt(sum x^2)                 kernels/rmsnorm/kernel.py:13-20
//   rmsnorm_weighted  y = x * rsqrt(mean x^2 + 1e-6) * w     (RMSNorm with weight and eps)
//   layernorm         y = (x - mu) / sqrt(mean (x - mu)^2 + 1e-6)  kernels/layernorm/kernel.py:17-25
//   softmax           y = exp(x) / sum exp(x), no max shift  kernels/softmax/kernel.py:13-16
//
// Schedule (hw variant 0, "row-resident"): a row is split across Wr waves.
// Each lane owns V 16-byte vectors of it; at vector step v the row's waves
// cover one contiguous 64*E*Wr-element stretch, so every load instruction is
// fully coalesced. The row is read from HBM exactly once and written once:
// the statistics are reduced with a wave64 butterfly and, when Wr > 1,
// across waves through LDS, then the output is formed from the registers.
// R rows share one workgroup (R * Wr waves, at most 16: a larger requested R
// is narrowed to 16 / Wr, so every tuple the manifest admits runs).
//
// Tile arguments: TILES_IN_BLOCK_M = R (rows per workgroup),
//                 TILES_IN_BLOCK_N = V (16-byte vectors per lane per row).
#include "common.hpp"
#include "registry.hpp"

namespace axon {
namespace {

enum RowMode { kRmsSum = 0, kRmsWeighted = 1, kLayerNorm = 2, kSoftmax = 3 };

constexpr float kNormEps = 1e-6f;
constexpr int kMaxWaves = 16;

template <typename T, int V, int MODE, bool ALIGNED>
__global__ __launch_bounds__(1024) void rowwise_kernel(const T* __restrict__ x,
                                                       const T* __restrict__ w,
                                                       T* __restrict__ y, int64_t m,
                                                       int64_t n, int R, int Wr) {
  constexpr int E = EPV<T>::value;
  __shared__ float red[2][kMaxWaves];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = wave / Wr;
  const int wr = wave - r * Wr;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * R + r;
  const bool live = row < m;
  const T* xr = x + (live ? row : 0) * n;
  T* yr = y + (live ? row : 0) * n;
  auto offset = [&](int v) -> int64_t {
    return (static_cast<int64_t>(v * Wr + wr) * kWave + lane) * E;
  };

  // The row stays in registers as loaded (16-byte vectors; elements are
  // widened to fp32 where they are used). Aligned rows (n % E == 0) load
  // branch-free: a vector past the row re-reads the row's first one and is
  // masked, so the V loads, and the weight's, are all in flight together.
  Vec<T> xraw[V];
  bool vin[V];
  Vec<T> wraw[MODE == kRmsWeighted ? V : 1];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t off = offset(v);
    if constexpr (ALIGNED) {
      vin[v] = live && off < n;
      if constexpr (MODE == kRmsWeighted) wraw[v] = load_vec(w + (off < n ? off : 0));
      xraw[v] = load_vec_nt(xr + (vin[v] ? off : 0));  // streamed once
    } else {
      vin[v] = live;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const bool in = live && off + e < n;
        xraw[v].v[e] = in ? xr[off + e] : from_f32<T>(0.f);
        if constexpr (MODE == kRmsWeighted) wraw[v].v[e] = w[off + e < n ? off + e : 0];
      }
    }
  }
  // Keep the scheduler from sinking the weight loads past the reduction.
  __builtin_amdgcn_sched_barrier(0);
  // Element (v, e) as fp32, 0 outside the row.
  auto xat = [&](int v, int e) -> float {
    if constexpr (ALIGNED) return vin[v] ? to_f32(xraw[v].v[e]) : 0.f;
    return to_f32(xraw[v].v[e]);  // out-of-row elements were loaded as 0
  };
  auto in_row = [&](int v, int e) -> bool {
    if constexpr (ALIGNED) return vin[v];
    return vin[v] && offset(v) + e < n;
  };

  // Row total of one per-lane partial: wave butterfly, then LDS across waves.
  auto row_total = [&](float part, int slot) -> float {
    float t = wave_sum(part);
    if (Wr > 1) {
      if (lane == 0) red[slot][wave] = t;
      __syncthreads();
      t = 0.f;
      for (int i = 0; i < Wr; ++i) t += red[slot][r * Wr + i];
    }
    return t;
  };

  float scale = 1.f, shift = 0.f;
  if constexpr (MODE == kRmsSum || MODE == kRmsWeighted) {
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int e = 0; e < E; ++e) s += xat(v, e) * xat(v, e);
    const float tot = row_total(s, 0);
    if constexpr (MODE == kRmsSum) {
      scale = 1.f / sqrtf(tot);
    } else {
      scale = 1.f / sqrtf(tot / static_cast<float>(n) + kNormEps);
    }
  } else if constexpr (MODE == kLayerNorm) {
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int e = 0; e < E; ++e) s += xat(v, e);
    const float mean = row_total(s, 0) / static_cast<float>(n);
    float q = 0.f;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float d = in_row(v, e) ? xat(v, e) - mean : 0.f;
        q += d * d;
      }
    const float var = row_total(q, 1) / static_cast<float>(n);
    scale = 1.f / sqrtf(var + kNormEps);
    shift = mean;
  } else {  // softmax: exp is recomputed for the output (cheaper than holding it)
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int e = 0; e < E; ++e) s += in_row(v, e) ? __expf(xat(v, e)) : 0.f;
    scale = 1.f / row_total(s, 0);
  }

#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t off = offset(v);
    Vec<T> o;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float t;
      if constexpr (MODE == kSoftmax) {
        t = __expf(xat(v, e)) * scale;
      } else {
        t = (xat(v, e) - shift) * scale;
        if constexpr (MODE == kRmsWeighted) t *= to_f32(wraw[v].v[e]);
      }
      o.v[e] = from_f32<T>(t);
    }
    if constexpr (ALIGNED) {
      if (vin[v]) store_vec_nt(yr + off, o);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (in_row(v, e)) yr[off + e] = o.v[e];
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
const char* const kTileArgs[] = {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"};

struct Shape {
  int R, V, Wr, E;
};

Shape shape_of(const Call& c) {
  Shape s;
  s.R = c.tile(0);
  s.V = c.tile(1);
  s.E = 16 / elem_bytes(c.dtype(0));
  if (s.V <= 0) {
    s.Wr = kMaxWaves + 1;
    return s;
  }
  const int64_t per_wave = static_cast<int64_t>(kWave) * s.E * s.V;
  const int64_t waves = (c.dim(1) + per_wave - 1) / per_wave;
  s.Wr = waves < 1 ? 1 : (waves > kMaxWaves ? kMaxWaves + 1 : static_cast<int>(waves));
  // Rows per workgroup, narrowed so R * Wr stays within 16 waves.
  if (s.Wr <= kMaxWaves && s.R * s.Wr > kMaxWaves) s.R = kMaxWaves / s.Wr;
  return s;
}

template <int MODE>
int check_rows(const Call& c, std::string* why) {
  const int n_in = MODE == kRmsWeighted ? 2 : 1;
  if (c.n_tiles != 2 || c.n_dims != 2 || c.n_dtypes != n_in) {
    *why = "expected 2 tile values, 2 dims and one dtype per input";
    return AXON_EARG;
  }
  const int dt = c.dtype(0);
  if (dt != AXON_BF16 && dt != AXON_F32) {
    *why = std::string("unsupported dtype ") + dtype_str(dt);
    return AXON_EDTYPE;
  }
  for (int i = 1; i < n_in; ++i)
    if (c.dtype(i) != dt) {
      *why = "weight dtype must match x";
      return AXON_EDTYPE;
    }
  if (c.dim(0) < 0 || c.dim(1) < 0) {
    *why = "negative dimension";
    return AXON_EINVAL;
  }
  const Shape s = shape_of(c);
  if (!is_pow2_in(c.tile(0), 1, kMaxWaves)) {
    *why = "TILES_IN_BLOCK_M (rows per workgroup) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(s.V, 1, 16)) {
    *why = "TILES_IN_BLOCK_N (16-byte vectors per lane) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  const int64_t span = static_cast<int64_t>(kWave) * s.E;
  if (span * s.V > (c.dim(1) > span ? c.dim(1) : span)) {
    *why = "TILES_IN_BLOCK_N: one wave's vector tile is longer than the row";
    return AXON_EINVAL;
  }
  if (s.Wr > kMaxWaves) {
    *why = "TILES_IN_BLOCK_N: a row needs more than 16 waves at this vector count";
    return AXON_EINVAL;
  }
  if (!grid_fits((c.dim(0) + s.R - 1) / s.R, 1, static_cast<int64_t>(s.R) * s.Wr * kWave)) {
    *why = "too many rows for one dispatch at these tiles (fewer than 2^32 work-items)";
    return AXON_EINVAL;
  }
  return AXON_OK;
}

template <int MODE>
int manifest_rows(int variant, const int64_t* dims, int dtype, Constraint* out, int cap) {
  (void)variant;
  if (cap < 2) return 0;
  const int64_t E = 16 / elem_bytes(dtype);
  const int64_t m = dims[0], n = dims[1];
  const int64_t lane_span = kWave * E;
  out[0] = {"TILES_IN_BLOCK_M", m < kMaxWaves ? (m > 0 ? m : 1) : kMaxWaves, 1, false};
  const int64_t n_ext = n > lane_span ? n : lane_span;
  out[1] = {"TILES_IN_BLOCK_N", n_ext < 16 * lane_span ? n_ext : 16 * lane_span, lane_span, false};
  return 2;
}

template <typename T, int MODE, bool ALIGNED>
using RowFn = void (*)(const T*, const T*, T*, int64_t, int64_t, int, int);

template <typename T, int MODE, bool ALIGNED>
RowFn<T, MODE, ALIGNED> pick(int V) {
  switch (V) {
    case 1: return rowwise_kernel<T, 1, MODE, ALIGNED>;
    case 2: return rowwise_kernel<T, 2, MODE, ALIGNED>;
    case 4: return rowwise_kernel<T, 4, MODE, ALIGNED>;
    case 8: return rowwise_kernel<T, 8, MODE, ALIGNED>;
    default: return rowwise_kernel<T, 16, MODE, ALIGNED>;
  }
}

template <typename T, int MODE>
int launch_typed(const Call& c, const void* const* in, void* const* out, hipStream_t st) {
  const Shape s = shape_of(c);
  const int64_t m = c.dim(0), n = c.dim(1);
  if (m == 0 || n == 0) return AXON_OK;
  const T* x = static_cast<const T*>(in[0]);
  const T* w = MODE == kRmsWeighted ? static_cast<const T*>(in[1]) : nullptr;
  T* y = static_cast<T*>(out[0]);
  const bool aligned = (n % s.E) == 0 && aligned16(x) && aligned16(y) &&
                       (MODE != kRmsWeighted || aligned16(w));
  const int rc = grid_check("rowwise_kernel", (m + s.R - 1) / s.R, 1, static_cast<int64_t>(s.R) * s.Wr * kWave);
  if (rc != AXON_OK) return rc;
  const dim3 grid(static_cast<unsigned>((m + s.R - 1) / s.R));
  const dim3 block(static_cast<unsigned>(s.R * s.Wr * kWave));
  if (aligned) {
    hipLaunchKernelGGL((pick<T, MODE, true>(s.V)), grid, block, 0, st, x, w, y, m, n, s.R, s.Wr);
  } else {
    hipLaunchKernelGGL((pick<T, MODE, false>(s.V)), grid, block, 0, st, x, w, y, m, n, s.R, s.Wr);
  }
  return launch_status("rowwise_kernel");
}

template <int MODE>
int launch_rows(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  (void)ws;
  if (c.dtype(0) == AXON_BF16) return launch_typed<bf16, MODE>(c, in, out, st);
  return launch_typed<float, MODE>(c, in, out, st);
}

size_t no_workspace(const Call&) { return 0; }

void outputs_rows(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, dtypes[0]};
}

const char* summary_rows(int) {
  return "row-resident one-pass: R rows per workgroup, each row split over Wr waves holding V "
         "16-byte vectors per lane; wave64 butterfly + LDS reduction; 1 HBM read + 1 write";
}

}  // namespace

const Family* family_rmsnorm() {
  static const Family f = {"rmsnorm", 1, 1, 1, 2, kTileArgs, 2, summary_rows,
                           manifest_rows<kRmsSum>, check_rows<kRmsSum>, no_workspace, outputs_rows,
                           launch_rows<kRmsSum>};
  return &f;
}

const Family* family_rmsnorm_weighted() {
  static const Family f = {"rmsnorm_weighted", 1, 2, 1, 2, kTileArgs, 2, summary_rows,
                           manifest_rows<kRmsWeighted>, check_rows<kRmsWeighted>, no_workspace, outputs_rows,
                           launch_rows<kRmsWeighted>};
  return &f;
}

const Family* family_layernorm() {
  static const Family f = {"layernorm", 1, 1, 1, 2, kTileArgs, 2, summary_rows,
                           manifest_rows<kLayerNorm>, check_rows<kLayerNorm>, no_workspace, outputs_rows,
                           launch_rows<kLayerNorm>};
  return &f;
}

const Family* family_softmax() {
  static const Family f = {"softmax", 1, 1, 1, 2, kTileArgs, 2, summary_rows,
                           manifest_rows<kSoftmax>, check_rows<kSoftmax>, no_workspace, outputs_rows,
                           launch_rows<kSoftmax>};
  return &f;
}

}  // namespace axon
