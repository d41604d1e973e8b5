// Inclusive prefix sum along the last axis (families "cumsum" and
// "cumsum_probs"; kernels/cumsum/kernel.py:12-13).
//
// Accuracy: the fp32 reference (torch.cumsum on the CPU) accumulates in
// double and rounds each prefix once. Here every chunk is scanned in fp32
// (a thread's serial run, a wave64 shuffle scan, a scan of wave totals in
// LDS: at most ~V*E + 6 + 4 additions deep), and the running offset of all
// earlier chunks is carried in double, so each output is
// round_fp32(double offset + fp32 local prefix). That keeps the relative
// error of every prefix within a few fp32 ulps on positive data instead of
// growing with the row length as a sequential fp32 carry does.
//
// hw variant 0 (row-resident stream): one workgroup per row walks it chunk by
//   chunk, carrying the double offset in registers. 1 read + 1 write.
// hw variant 1 (split rows): rows are cut into chunks handled by separate
//   workgroups. A first kernel writes each chunk's double total to the
//   workspace; the second kernel adds the totals of the earlier chunks of its
//   row and scans its own chunk. Reads the input twice (the second read
//   mostly from the Infinity Cache), writes once; fills the GPU when there
//   are few long rows (64 x 128256).
// Tile arguments: TILES_IN_BLOCK_M = W (waves per workgroup),
//                 TILES_IN_BLOCK_N = V (16-byte vectors per thread per chunk).
#include "common.hpp"
#include "registry.hpp"

namespace axon {
namespace {

constexpr int kMaxW = 16;

// Loads thread `tid`'s V*E consecutive elements of chunk `c0` (blocked
// layout), zero beyond n.
template <typename T, int V, bool ALIGNED>
__device__ __forceinline__ void load_run(const T* __restrict__ row, int64_t c0, int tid,
                                         int64_t n, float (&x)[V * EPV<T>::value]) {
  constexpr int E = EPV<T>::value;
  const int64_t base = c0 + static_cast<int64_t>(tid) * V * E;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t off = base + v * E;
    if constexpr (ALIGNED) {
      if (off < n) {
        const Vec<T> t = load_vec(row + off);
#pragma unroll
        for (int e = 0; e < E; ++e) x[v * E + e] = to_f32(t.v[e]);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) x[v * E + e] = 0.f;
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) x[v * E + e] = off + e < n ? to_f32(row[off + e]) : 0.f;
    }
  }
}

// Inclusive wave64 scan (Hillis-Steele over shuffles).
__device__ __forceinline__ float wave_incl_scan(float v, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float o = __shfl_up(v, off, kWave);
    if (lane >= off) v += o;
  }
  return v;
}

// Scans the chunk held in x (in place, fp32 local inclusive prefixes), adds
// the double `carry`, stores, and returns the chunk total in double (same on
// every thread). Contains __syncthreads: every thread of the block calls it.
template <typename T, int V, bool ALIGNED>
__device__ __forceinline__ double scan_store_chunk(float (&x)[V * EPV<T>::value], T* __restrict__ orow,
                                                   int64_t c0, int64_t n, double carry,
                                                   float* wave_tot) {
  constexpr int E = EPV<T>::value;
  constexpr int R = V * E;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int nw = blockDim.x >> 6;
#pragma unroll
  for (int i = 1; i < R; ++i) x[i] += x[i - 1];
  const float incl = wave_incl_scan(x[R - 1], lane);
  const float excl_lane = incl - x[R - 1];
  if (lane == kWave - 1) wave_tot[wave] = incl;
  __syncthreads();
  float excl_wave = 0.f;
  double total = 0.0;
  for (int w = 0; w < nw; ++w) {
    const float t = wave_tot[w];
    if (w < wave) excl_wave += t;
    total += static_cast<double>(t);
  }
  __syncthreads();  // wave_tot is rewritten by the next chunk
  const float off_f = excl_wave + excl_lane;
  const int64_t base = c0 + static_cast<int64_t>(tid) * R;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t off = base + v * E;
    Vec<T> o;
#pragma unroll
    for (int e = 0; e < E; ++e)
      o.v[e] = from_f32<T>(static_cast<float>(carry + static_cast<double>(x[v * E + e] + off_f)));
    if constexpr (ALIGNED) {
      if (off < n) store_vec(orow + off, o);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (off + e < n) orow[off + e] = o.v[e];
    }
  }
  return total;
}

template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void scan_rows_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                         int64_t n) {
  constexpr int R = V * EPV<T>::value;
  __shared__ float wave_tot[kMaxW];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * n;
  T* yr = y + row * n;
  const int64_t chunk = static_cast<int64_t>(blockDim.x) * R;
  double carry = 0.0;
  for (int64_t c0 = 0; c0 < n; c0 += chunk) {
    float v[R];
    load_run<T, V, ALIGNED>(xr, c0, threadIdx.x, n, v);
    carry += scan_store_chunk<T, V, ALIGNED>(v, yr, c0, n, carry, wave_tot);
  }
}

template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void chunk_total_kernel(const T* __restrict__ x,
                                                           double* __restrict__ totals, int64_t n,
                                                           int nchunks) {
  constexpr int R = V * EPV<T>::value;
  __shared__ double wave_sum_lds[kMaxW];
  const int64_t row = blockIdx.y;
  const int c = blockIdx.x;
  const int64_t chunk = static_cast<int64_t>(blockDim.x) * R;
  float v[R];
  load_run<T, V, ALIGNED>(x + row * n, c * chunk, threadIdx.x, n, v);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i) s += v[i];
  double d = wave_sum(static_cast<double>(s));
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  if (lane == 0) wave_sum_lds[wave] = d;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) t += wave_sum_lds[w];
    totals[row * nchunks + c] = t;
  }
}

template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void chunk_scan_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                          const double* __restrict__ totals,
                                                          int64_t n, int nchunks) {
  constexpr int R = V * EPV<T>::value;
  __shared__ float wave_tot[kMaxW];
  __shared__ double carry_lds;
  const int64_t row = blockIdx.y;
  const int c = blockIdx.x;
  const int64_t chunk = static_cast<int64_t>(blockDim.x) * R;
  float v[R];
  load_run<T, V, ALIGNED>(x + row * n, c * chunk, threadIdx.x, n, v);
  if (threadIdx.x < kWave) {
    // Sum of the earlier chunk totals of this row, in double.
    double s = 0.0;
    for (int i = threadIdx.x; i < c; i += kWave) s += totals[row * nchunks + i];
    s = wave_sum(s);
    if (threadIdx.x == 0) carry_lds = s;
  }
  __syncthreads();
  const double carry = carry_lds;
  scan_store_chunk<T, V, ALIGNED>(v, y + row * n, c * chunk, n, carry, wave_tot);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
const char* const kTileArgs[] = {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"};

int64_t chunk_elems(const Call& c) {
  return static_cast<int64_t>(c.tile(0)) * kWave * c.tile(1) * (16 / elem_bytes(c.dtype(0)));
}

int check_scan(const Call& c, std::string* why) {
  if (c.n_tiles != 2 || c.n_dims != 2 || c.n_dtypes != 1) {
    *why = "expected 2 tiles, 2 dims and 1 dtype";
    return AXON_EARG;
  }
  const int dt = c.dtype(0);
  if (dt != AXON_BF16 && dt != AXON_F32) {
    *why = std::string("unsupported dtype ") + dtype_str(dt);
    return AXON_EDTYPE;
  }
  if (c.dim(0) < 0 || c.dim(1) < 0 || c.dim(0) > 65535 * 1024LL) {
    *why = "dimension out of range";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(c.tile(0), 1, kMaxW)) {
    *why = "TILES_IN_BLOCK_M (waves per workgroup) must be a power of two in [1, 16]";
    return AXON_EINVAL;
  }
  if (!is_pow2_in(c.tile(1), 1, 8)) {
    *why = "TILES_IN_BLOCK_N (vectors per thread) must be a power of two in [1, 8]";
    return AXON_EINVAL;
  }
  if (c.variant == 1) {
    const int64_t nchunks = (c.dim(1) + chunk_elems(c) - 1) / chunk_elems(c);
    if (nchunks > 65535 || c.dim(0) > 65535) {
      *why = "split-row scan needs at most 65535 chunks per row and 65535 rows";
      return AXON_EINVAL;
    }
  }
  return AXON_OK;
}

int manifest_scan(int variant, const int64_t* dims, int dtype, Constraint* out, int cap) {
  if (cap < 2) return 0;
  const int64_t E = 16 / elem_bytes(dtype);
  const int64_t n = dims[1] > 0 ? dims[1] : 1;
  // Waves per workgroup: a workgroup never spans more lanes than the row has
  // vectors (variant 0), or more than a quarter of them (variant 1, so each
  // row splits into at least a few chunks).
  int64_t lanes = (n + E - 1) / E;
  if (variant == 1) lanes = lanes / 4 > 0 ? lanes / 4 : 1;
  const int64_t w = (lanes + kWave - 1) / kWave;
  out[0] = {"TILES_IN_BLOCK_M", w < kMaxW ? w : kMaxW, 1, false};
  out[1] = {"TILES_IN_BLOCK_N", 8, 1, false};
  return 2;
}

size_t workspace_scan(const Call& c) {
  if (c.variant != 1) return 0;
  const int64_t nchunks = (c.dim(1) + chunk_elems(c) - 1) / chunk_elems(c);
  return static_cast<size_t>(c.dim(0) * nchunks) * sizeof(double);
}

void outputs_scan(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, dtypes[0]};
}

#define AXON_SCAN_PICK(KERNEL, T, A, V)      \
  switch (V) {                               \
    case 1: return KERNEL<T, 1, A>;          \
    case 2: return KERNEL<T, 2, A>;          \
    case 4: return KERNEL<T, 4, A>;          \
    default: return KERNEL<T, 8, A>;         \
  }

template <typename T, bool A>
void (*rows_fn(int V))(const T*, T*, int64_t) { AXON_SCAN_PICK(scan_rows_kernel, T, A, V) }
template <typename T, bool A>
void (*tot_fn(int V))(const T*, double*, int64_t, int) { AXON_SCAN_PICK(chunk_total_kernel, T, A, V) }
template <typename T, bool A>
void (*cscan_fn(int V))(const T*, T*, const double*, int64_t, int) {
  AXON_SCAN_PICK(chunk_scan_kernel, T, A, V)
}

template <typename T, bool A>
int launch_scan_ta(const Call& c, const T* x, T* y, void* ws, hipStream_t st) {
  const int64_t m = c.dim(0), n = c.dim(1);
  const int W = c.tile(0), V = c.tile(1);
  const dim3 block(W * kWave);
  if (c.variant == 0) {
    hipLaunchKernelGGL((rows_fn<T, A>(V)), dim3(static_cast<unsigned>(m)), block, 0, st, x, y, n);
    return launch_status("scan_rows_kernel");
  }
  const int64_t ce = chunk_elems(c);
  const int nchunks = static_cast<int>((n + ce - 1) / ce);
  double* totals = static_cast<double*>(ws);
  const dim3 grid(nchunks, static_cast<unsigned>(m));
  hipLaunchKernelGGL((tot_fn<T, A>(V)), grid, block, 0, st, x, totals, n, nchunks);
  int rc = launch_status("chunk_total_kernel");
  if (rc != AXON_OK) return rc;
  hipLaunchKernelGGL((cscan_fn<T, A>(V)), grid, block, 0, st, x, y, totals, n, nchunks);
  return launch_status("chunk_scan_kernel");
}

template <typename T>
int launch_scan_t(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  const int64_t m = c.dim(0), n = c.dim(1);
  if (m == 0 || n == 0) return AXON_OK;
  const T* x = static_cast<const T*>(in[0]);
  T* y = static_cast<T*>(out[0]);
  const bool aligned = n % EPV<T>::value == 0 && aligned16(x) && aligned16(y);
  return aligned ? launch_scan_ta<T, true>(c, x, y, ws, st) : launch_scan_ta<T, false>(c, x, y, ws, st);
}

int launch_scan(const Call& c, const void* const* in, void* const* out, void* ws, hipStream_t st) {
  return c.dtype(0) == AXON_BF16 ? launch_scan_t<bf16>(c, in, out, ws, st)
                                 : launch_scan_t<float>(c, in, out, ws, st);
}

const char* summary_scan(int variant) {
  return variant == 0
             ? "row-resident stream: one workgroup per row, fp32 chunk scans (thread run, wave64 "
               "shuffle scan, LDS wave totals) with a double carry; 1 read + 1 write"
             : "split rows: chunk totals (double) to workspace, then each chunk adds its row's "
               "earlier totals and scans; fills the GPU for few long rows";
}

}  // namespace

const Family* family_cumsum() {
  static const Family f = {"cumsum", 2, 1, 1, 2, kTileArgs, 2, summary_scan, manifest_scan,
                           check_scan, workspace_scan, outputs_scan, launch_scan};
  return &f;
}

const Family* family_cumsum_probs() {
  static const Family f = {"cumsum_probs", 2, 1, 1, 2, kTileArgs, 2, summary_scan, manifest_scan,
                           check_scan, workspace_scan, outputs_scan, launch_scan};
  return &f;
}

}  // namespace axon
