// Inclusive prefix sum along the last axis (families "cumsum" and
// "cumsum_probs"; kernels/cumsum/kernel.py:12-13).
//
// Accuracy: the fp32 reference (torch.cumsum on the CPU) accumulates in
// double and rounds each prefix once. Here a chunk is scanned in fp32 (each
// lane's E elements serially, a wave64 shuffle scan per step, a running wave
// offset across the V steps), while the offsets of earlier waves and chunks
// are carried in double, so each output is round_fp32(double offset + fp32
// chunk-local prefix). The fp32 part is at most E + 6 + V additions deep, so
// the relative error of a prefix of positive terms stays within a few ulps
// however long the row is.
//
// Layout (both variants): a workgroup's chunk is W waves x 64 lanes x V
// steps x E elements. Each wave owns a contiguous run of 64*V*E elements and
// at step v its lanes read one lane-contiguous stretch of 64 16-byte
// vectors, so every load and store instruction is fully coalesced.
//
// hw variant 0 (row-resident stream): one workgroup per row walks it chunk by
//   chunk, carrying the double offset. 1 read + 1 write.
// hw variant 1 (split rows): rows are cut into chunks handled by separate
//   workgroups. A first kernel writes each chunk's double total to the
//   workspace; the second adds the totals of the earlier chunks of its row and
//   scans its own chunk. The input is read twice (the second read mostly from
//   the Infinity Cache), written once; this fills the GPU when there are few
//   long rows (64 x 128256).
// hw variant 2 (single pass, published chunk totals): one launch, 1 read +
//   1 write. Workgroup b owns chunk b (row-major), loads it, publishes its
//   chunk total as one 64-bit word {launch tag, fp32 total} and sums the
//   totals of the earlier chunks of its row as they appear (one poll round
//   per lane in the common case). The tag is unique per launch (a counter in
//   the library), so words left by earlier launches never match and the
//   workspace needs no reset. Correctness never depends on the order in
//   which workgroups are dispatched: a lane polls an earlier chunk's word at
//   most `max_polls` times, and a total that has not appeared by then is
//   recomputed by the waiting wave from the input itself, in the publisher's
//   own summation order, so it equals the published value bit for bit. The
//   wait is then bounded by max_polls sleeps plus one chunk read per missing
//   total, and every workgroup finishes. The workspace header's word 0
//   counts the totals recomputed since the workspace was zeroed (a
//   diagnostic; nothing reads it to decide a result).
// Tile arguments: TILES_IN_BLOCK_M = W (waves per workgroup),
//                 TILES_IN_BLOCK_N = V (16-byte vectors per lane per chunk).
#include <atomic>

#include "common.hpp"
#include "registry.hpp"

namespace axon {
namespace {

constexpr int kMaxW = 16;

// x[v][e] <- element (wbase + (v*64 + lane)*E + e) of `row`, zero past n.
template <typename T, int V, bool ALIGNED, bool NT>
__device__ __forceinline__ void load_striped(const T* __restrict__ row, int64_t wbase, int lane,
                                             int64_t n, float (&x)[V][EPV<T>::value]) {
  constexpr int E = EPV<T>::value;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t off = wbase + static_cast<int64_t>(v * kWave + lane) * E;
    if constexpr (ALIGNED) {
      // n % E == 0: a vector is all in or all out. Branch-free (a vector past
      // n re-reads the row's first one and is zeroed), so the V loads are in
      // flight together.
      const bool in = off < n;
      const int64_t at = in ? off : 0;
      const Vec<T> t = NT ? load_vec_nt(row + at) : load_vec(row + at);
#pragma unroll
      for (int e = 0; e < E; ++e) x[v][e] = in ? to_f32(t.v[e]) : 0.f;
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) x[v][e] = off + e < n ? to_f32(row[off + e]) : 0.f;
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

// Turns x into wave-local inclusive prefixes (fp32) and returns the wave's
// total (same on every lane).
template <int V, int E>
__device__ __forceinline__ float wave_scan_run(float (&x)[V][E], int lane) {
  float run = 0.f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
#pragma unroll
    for (int e = 1; e < E; ++e) x[v][e] += x[v][e - 1];
    const float t = x[v][E - 1];
    const float incl = wave_incl_scan(t, lane);
    const float base = run + (incl - t);
#pragma unroll
    for (int e = 0; e < E; ++e) x[v][e] += base;
    run += __shfl(incl, kWave - 1, kWave);
  }
  return run;
}

// Scans the chunk held in x (striped), adds `carry`, stores, and returns the
// chunk total in double (same on every thread). Contains __syncthreads:
// every thread of the block calls it.
template <typename T, int V, bool ALIGNED>
__device__ __forceinline__ double scan_store_chunk(float (&x)[V][EPV<T>::value], T* __restrict__ orow,
                                                   int64_t c0, int64_t n, double carry,
                                                   float* wave_tot) {
  constexpr int E = EPV<T>::value;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const float wt = wave_scan_run<V, E>(x, lane);
  if (lane == 0) wave_tot[wave] = wt;
  __syncthreads();
  double before = 0.0, total = 0.0;
  for (int w = 0; w < nw; ++w) {
    const double t = static_cast<double>(wave_tot[w]);
    if (w < wave) before += t;
    total += t;
  }
  __syncthreads();  // wave_tot is rewritten by the next chunk
  const double off = carry + before;
  const int64_t wbase = c0 + static_cast<int64_t>(wave) * kWave * V * E;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t o0 = wbase + static_cast<int64_t>(v * kWave + lane) * E;
    Vec<T> o;
#pragma unroll
    for (int e = 0; e < E; ++e) o.v[e] = from_f32<T>(static_cast<float>(off + static_cast<double>(x[v][e])));
    if constexpr (ALIGNED) {
      if (o0 < n) store_vec_nt(orow + o0, o);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (o0 + e < n) orow[o0 + e] = o.v[e];
    }
  }
  return total;
}

template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void scan_rows_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                         int64_t n) {
  constexpr int E = EPV<T>::value;
  __shared__ float wave_tot[kMaxW];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * n;
  T* yr = y + row * n;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t per_wave = static_cast<int64_t>(kWave) * V * E;
  const int64_t chunk = static_cast<int64_t>(blockDim.x >> 6) * per_wave;
  double carry = 0.0;
  for (int64_t c0 = 0; c0 < n; c0 += chunk) {
    float v[V][E];
    load_striped<T, V, ALIGNED, true>(xr, c0 + (threadIdx.x >> 6) * per_wave, lane, n, v);
    carry += scan_store_chunk<T, V, ALIGNED>(v, yr, c0, n, carry, wave_tot);
  }
}

template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void chunk_total_kernel(const T* __restrict__ x,
                                                           double* __restrict__ totals, int64_t n,
                                                           int nchunks) {
  constexpr int E = EPV<T>::value;
  __shared__ double wave_sum_lds[kMaxW];
  const int64_t row = blockIdx.y;
  const int c = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int64_t per_wave = static_cast<int64_t>(kWave) * V * E;
  const int64_t c0 = static_cast<int64_t>(c) * (blockDim.x >> 6) * per_wave;
  float v[V][E];
  // Regular (cached) loads: the scan pass re-reads this chunk right after.
  load_striped<T, V, ALIGNED, false>(x + row * n, c0 + wave * per_wave, lane, n, v);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) s += v[i][e];
  const double d = wave_sum(static_cast<double>(s));
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
  constexpr int E = EPV<T>::value;
  __shared__ float wave_tot[kMaxW];
  __shared__ double carry_lds;
  const int64_t row = blockIdx.y;
  const int c = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int64_t per_wave = static_cast<int64_t>(kWave) * V * E;
  const int64_t c0 = static_cast<int64_t>(c) * (blockDim.x >> 6) * per_wave;
  float v[V][E];
  load_striped<T, V, ALIGNED, true>(x + row * n, c0 + wave * per_wave, lane, n, v);
  if (threadIdx.x < kWave) {
    // Sum of the earlier chunk totals of this row, in double.
    double s = 0.0;
    for (int i = threadIdx.x; i < c; i += kWave) s += totals[row * nchunks + i];
    s = wave_sum(s);
    if (threadIdx.x == 0) carry_lds = s;
  }
  __syncthreads();
  const double carry = carry_lds;
  scan_store_chunk<T, V, ALIGNED>(v, y + row * n, c0, n, carry, wave_tot);
}

// Single-pass workspace: a header (word 0: count of recomputed chunk totals)
// padded to 256 bytes, then one 64-bit slot per chunk (row-major).
constexpr size_t kOnepassHeader = 256;

// fp32 sum of one thread's V x E elements, in the order every total of the
// single-pass variant uses (v outer, e inner).
template <int V, int E>
__device__ __forceinline__ float thread_total(const float (&x)[V][E]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) s += x[i][e];
  return s;
}

// The total of the chunk starting at c0, computed by one wave exactly as the
// chunk's own workgroup computes it before publishing: per wave w of that
// workgroup, the double wave64 sum of its threads' fp32 totals, added in w
// order in double. Same value on every lane.
template <typename T, int V, bool ALIGNED>
__device__ double recompute_chunk_total(const T* __restrict__ xr, int64_t c0, int64_t n, int nw,
                                        int lane) {
  constexpr int E = EPV<T>::value;
  const int64_t per_wave = static_cast<int64_t>(kWave) * V * E;
  double t = 0.0;
  for (int w = 0; w < nw; ++w) {
    float v[V][E];
    load_striped<T, V, ALIGNED, false>(xr, c0 + w * per_wave, lane, n, v);
    t += wave_sum(static_cast<double>(thread_total<V, E>(v)));
  }
  return t;
}

template <typename T, int V, bool ALIGNED>
__global__ __launch_bounds__(1024) void scan_onepass_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                            unsigned* hdr, unsigned long long* slots,
                                                            int64_t n, int nchunks, unsigned tag,
                                                            unsigned max_polls) {
  constexpr int E = EPV<T>::value;
  __shared__ float wave_tot[kMaxW];
  __shared__ double part[kMaxW];
  __shared__ double s_carry;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const unsigned b = blockIdx.x;
  const int64_t row = b / static_cast<unsigned>(nchunks);
  const int c = static_cast<int>(b - row * nchunks);
  const int64_t per_wave = static_cast<int64_t>(kWave) * V * E;
  const int64_t chunk = static_cast<int64_t>(nw) * per_wave;
  const int64_t c0 = static_cast<int64_t>(c) * chunk;
  const T* xr = x + row * n;
  float v[V][E];
  load_striped<T, V, ALIGNED, true>(xr, c0 + wave * per_wave, lane, n, v);

  // Publish this chunk's total (not needed by the last chunk of a row).
  const double d = wave_sum(static_cast<double>(thread_total<V, E>(v)));
  if (lane == 0) part[wave] = d;
  __syncthreads();
  if (threadIdx.x == 0 && c + 1 < nchunks) {
    double t = 0.0;
    for (int w = 0; w < nw; ++w) t += part[w];
    const unsigned long long word =
        (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(static_cast<float>(t));
    __hip_atomic_store(&slots[b], word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Carry: the totals of chunks 0..c-1 of this row (wave 0, one chunk per
  // lane per round of 64).
  if (wave == 0) {
    double acc = 0.0;
    const int64_t rowbase = row * nchunks;
    for (int base = 0; base < c; base += kWave) {
      const int i = base + lane;
      bool have = false;
      float t = 0.f;
      if (i < c) {
        for (unsigned polls = 0; polls < max_polls; ++polls) {
          const unsigned long long w =
              __hip_atomic_load(&slots[rowbase + i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (static_cast<unsigned>(w >> 32) == tag) {
            t = __uint_as_float(static_cast<unsigned>(w));
            have = true;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
        }
      }
      // Totals that did not appear within the bound: the wave sums each of
      // those chunks from x (bounded work, same value as the publisher's).
      unsigned long long missing = __ballot(i < c && !have);
      if (missing != 0ull && lane == 0)
        __hip_atomic_fetch_add(&hdr[0], static_cast<unsigned>(__popcll(missing)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      while (missing != 0ull) {
        const int f = __builtin_ctzll(missing);
        missing &= missing - 1ull;
        const double tot = recompute_chunk_total<T, V, ALIGNED>(xr, (base + f) * chunk, n, nw, lane);
        if (lane == f) t = static_cast<float>(tot);
      }
      if (i < c) acc += static_cast<double>(t);
    }
    acc = wave_sum(acc);
    if (lane == 0) s_carry = acc;
  }
  __syncthreads();
  scan_store_chunk<T, V, ALIGNED>(v, y + row * n, c0, n, s_carry, wave_tot);
}

// Launch tags of the single-pass variant: unique per launch in this process
// (0 is never used, so a zero-filled workspace matches nothing).
std::atomic<unsigned> g_scan_tag{0};

unsigned next_scan_tag() {
  unsigned t = g_scan_tag.fetch_add(1, std::memory_order_relaxed) + 1;
  if (t == 0) t = g_scan_tag.fetch_add(1, std::memory_order_relaxed) + 1;
  return t;
}

// How many times a single-pass lane polls for an earlier chunk's total before
// recomputing it (each poll is one L2 load and a short sleep; a total
// normally appears within a few polls).
constexpr unsigned kDefaultPolls = 1u << 12;
std::atomic<unsigned> g_scan_polls{kDefaultPolls};

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
  if (c.variant == 2) {
    const int64_t nchunks = (c.dim(1) + chunk_elems(c) - 1) / chunk_elems(c);
    if (c.dim(0) * nchunks > (1LL << 31) - 1) {
      *why = "single-pass scan needs fewer than 2^31 chunks in total";
      return AXON_EINVAL;
    }
  }
  const int64_t nchunks = c.variant == 0 ? 1 : (c.dim(1) + chunk_elems(c) - 1) / chunk_elems(c);
  const bool fits = c.variant == 1 ? grid_fits(nchunks, c.dim(0), c.tile(0) * kWave)
                                   : grid_fits(c.dim(0) * nchunks, 1, c.tile(0) * kWave);
  if (!fits) {
    *why = "too many workgroups for one dispatch at these tiles (fewer than 2^32 work-items)";
    return AXON_EINVAL;
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
  if (variant >= 1) lanes = lanes / 4 > 0 ? lanes / 4 : 1;
  const int64_t w = (lanes + kWave - 1) / kWave;
  out[0] = {"TILES_IN_BLOCK_M", w < kMaxW ? w : kMaxW, 1, false};
  out[1] = {"TILES_IN_BLOCK_N", 8, 1, false};
  return 2;
}

size_t workspace_scan(const Call& c) {
  if (c.variant == 0) return 0;
  const int64_t nchunks = (c.dim(1) + chunk_elems(c) - 1) / chunk_elems(c);
  const size_t slots = static_cast<size_t>(c.dim(0) * nchunks) * 8;  // double / 64-bit word
  return c.variant == 1 ? slots : kOnepassHeader + slots;
}

// The single-pass variant's slots must not hold a word whose tag matches the
// launch: zero the whole workspace when it held anything but this variant's
// own words.
size_t zeroed_scan(const Call& c) { return c.variant == 2 ? workspace_scan(c) : 0; }

void outputs_scan(const int64_t* dims, const int32_t* dtypes, OutDesc* out) {
  out[0] = {2, {dims[0], dims[1]}, dtypes[0]};
}

#define AXON_SCAN_PICK(KERNEL, T, A, V) \
  switch (V) {                          \
    case 1: return KERNEL<T, 1, A>;     \
    case 2: return KERNEL<T, 2, A>;     \
    case 4: return KERNEL<T, 4, A>;     \
    default: return KERNEL<T, 8, A>;    \
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
void (*onepass_fn(int V))(const T*, T*, unsigned*, unsigned long long*, int64_t, int, unsigned,
                          unsigned) {
  AXON_SCAN_PICK(scan_onepass_kernel, T, A, V)
}

template <typename T, bool A>
int launch_scan_ta(const Call& c, const T* x, T* y, void* ws, hipStream_t st) {
  const int64_t m = c.dim(0), n = c.dim(1);
  const int W = c.tile(0), V = c.tile(1);
  const dim3 block(W * kWave);
  if (c.variant == 0) {
    const int rc = grid_check("scan_rows_kernel", m, 1, W * kWave);
    if (rc != AXON_OK) return rc;
    hipLaunchKernelGGL((rows_fn<T, A>(V)), dim3(static_cast<unsigned>(m)), block, 0, st, x, y, n);
    return launch_status("scan_rows_kernel");
  }
  const int64_t ce = chunk_elems(c);
  const int nchunks = static_cast<int>((n + ce - 1) / ce);
  if (c.variant == 2) {
    const int rc = grid_check("scan_onepass_kernel", m * nchunks, 1, W * kWave);
    if (rc != AXON_OK) return rc;
    const unsigned nblocks = static_cast<unsigned>(m * nchunks);
    unsigned* hdr = static_cast<unsigned*>(ws);
    auto* slots = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + kOnepassHeader);
    hipLaunchKernelGGL((onepass_fn<T, A>(V)), dim3(nblocks), block, 0, st, x, y, hdr, slots, n,
                       nchunks, next_scan_tag(), g_scan_polls.load(std::memory_order_relaxed));
    return launch_status("scan_onepass_kernel");
  }
  double* totals = static_cast<double*>(ws);
  int rc = grid_check("chunk_total_kernel", nchunks, m, W * kWave);
  if (rc != AXON_OK) return rc;
  const dim3 grid(nchunks, static_cast<unsigned>(m));
  hipLaunchKernelGGL((tot_fn<T, A>(V)), grid, block, 0, st, x, totals, n, nchunks);
  rc = launch_status("chunk_total_kernel");
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
  if (variant == 2)
    return "single pass: each chunk publishes a {launch tag, fp32 total} word and adds the "
           "published totals of its row's earlier chunks (double carry), recomputing from the "
           "input any total that does not appear within the poll bound; 1 read + 1 write, one "
           "launch";
  return variant == 0
             ? "row-resident stream: one workgroup per row, striped coalesced chunks scanned in "
               "fp32 (lane run, wave64 shuffle scan per step) with double wave/chunk offsets; "
               "1 read + 1 write"
             : "split rows: chunk totals (double) to workspace, then each chunk adds its row's "
               "earlier totals and scans; fills the GPU for few long rows";
}

}  // namespace

unsigned set_scan_poll_bound(unsigned polls) {
  return g_scan_polls.exchange(polls, std::memory_order_relaxed);
}

const Family* family_cumsum() {
  static const Family f = {"cumsum", 3, 1, 1, 2, kTileArgs, 2, summary_scan, manifest_scan,
                           check_scan, workspace_scan, outputs_scan, launch_scan, zeroed_scan};
  return &f;
}

const Family* family_cumsum_probs() {
  static const Family f = {"cumsum_probs", 3, 1, 1, 2, kTileArgs, 2, summary_scan, manifest_scan,
                           check_scan, workspace_scan, outputs_scan, launch_scan, zeroed_scan};
  return &f;
}

}  // namespace axon
