// The C ABI (include/axon_hip.h) over the static family registry.
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "common.hpp"
#include "registry.hpp"

namespace axon {

const Family* family_rmsnorm();
const Family* family_rmsnorm_weighted();
const Family* family_layernorm();
const Family* family_softmax();
const Family* family_rope();
const Family* family_rope_llama3();
const Family* family_fused_adam();
const Family* family_cumsum();
const Family* family_cumsum_probs();
const Family* family_matmul();
const Family* family_matmul_std002();
const Family* family_rmsnorm_matmul();
const Family* family_rmsnorm_matmul_eps();
const Family* family_silu_mlp();
const Family* family_attention_causal();
const Family* family_attention_nkilib();
const Family* family_qkv_cte();
const Family* family_softmax_mm();
const Family* family_linear_attention();
const Family* family_attention_qkv();

namespace {

using FamilyFn = const Family* (*)();
const FamilyFn kFamilyFns[] = {
    family_rmsnorm,        family_rmsnorm_weighted,   family_layernorm,     family_softmax,
    family_rope,           family_rope_llama3,        family_fused_adam,    family_cumsum,
    family_cumsum_probs,   family_matmul,             family_matmul_std002, family_rmsnorm_matmul,
    family_rmsnorm_matmul_eps, family_silu_mlp,  family_attention_causal, family_attention_nkilib,
    family_qkv_cte,        family_softmax_mm,         family_linear_attention, family_attention_qkv,
};
constexpr int kNumFamilies = sizeof(kFamilyFns) / sizeof(kFamilyFns[0]);

const Family* family_at(int i) { return kFamilyFns[i](); }

thread_local std::string g_last_error;

const Family* find(const char* name) {
  if (name == nullptr) return nullptr;
  for (int i = 0; i < kNumFamilies; ++i)
    if (strcmp(family_at(i)->name, name) == 0) return family_at(i);
  return nullptr;
}

int write_text(const std::string& s, char* buf, size_t len) {
  if (buf == nullptr || len < s.size() + 1) {
    set_error("buffer of " + std::to_string(len) + " bytes is too small for " +
              std::to_string(s.size() + 1));
    return AXON_EBUFFER;
  }
  memcpy(buf, s.c_str(), s.size() + 1);
  return AXON_OK;
}

std::string json_str(const char* s) {
  std::string r = "\"";
  for (const char* p = s; *p; ++p) {
    if (*p == '"' || *p == '\\') r += '\\';
    r += *p;
  }
  return r + "\"";
}

// Resolves family + variant and validates the argument counts shared by
// check/workspace/launch.
int resolve(const char* kernel, int variant, const Call& c, const Family** out) {
  const Family* f = find(kernel);
  if (f == nullptr) {
    set_error(std::string("no HIP kernel family for spec '") + (kernel ? kernel : "(null)") + "'");
    return AXON_ENOKERNEL;
  }
  if (variant < 0 || variant >= f->n_variants) {
    set_error(std::string(f->name) + ": hw_variant " + std::to_string(variant) +
              " out of range [0, " + std::to_string(f->n_variants) + ")");
    return AXON_ENOKERNEL;
  }
  if (c.n_tiles != f->n_tiles || c.n_dims != f->n_dims || c.n_dtypes != f->n_inputs ||
      (c.n_tiles > 0 && c.tiles == nullptr) || (c.n_dims > 0 && c.dims == nullptr) ||
      (c.n_dtypes > 0 && c.dtypes == nullptr)) {
    set_error(std::string(f->name) + ": expected " + std::to_string(f->n_tiles) + " tiles, " +
              std::to_string(f->n_dims) + " dims, " + std::to_string(f->n_inputs) +
              " dtypes; got " + std::to_string(c.n_tiles) + ", " + std::to_string(c.n_dims) +
              ", " + std::to_string(c.n_dtypes));
    return AXON_EARG;
  }
  *out = f;
  return AXON_OK;
}

int checked(const char* kernel, const Call& c, const Family** f) {
  int rc = resolve(kernel, c.variant, c, f);
  if (rc != AXON_OK) return rc;
  std::string why;
  rc = (*f)->check(c, &why);
  if (rc != AXON_OK) set_error(std::string((*f)->name) + " v" + std::to_string(c.variant) + ": " + why);
  return rc;
}

}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }

int grid_check(const char* what, int64_t gx, int64_t gy, int64_t threads) {
  if (grid_fits(gx, gy, threads)) return AXON_OK;
  set_error(std::string(what) + ": " + std::to_string(gx) + " x " + std::to_string(gy) + " workgroups of " +
            std::to_string(threads) +
            " threads exceed one dispatch (at most 2^31 - 1 x 65535 workgroups, fewer than 2^32 work-items)");
  return AXON_EINVAL;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return AXON_EHIP;
  }
  return AXON_OK;
}

// Plain 16-byte vector copy, grid-stride, for traffic-counter calibration.
__global__ __launch_bounds__(256) void copy_kernel(const uint4* __restrict__ src,
                                                   uint4* __restrict__ dst, size_t n16) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    __builtin_nontemporal_store(
        __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + i),
        reinterpret_cast<u32x4*>(dst) + i);
}

// One-shot copy: every thread moves V vectors (its loads all in flight
// before its stores), one block per 256 * V vectors.
template <int V>
__global__ __launch_bounds__(256) void copy_oneshot_kernel(const uint4* __restrict__ src,
                                                          uint4* __restrict__ dst, size_t n16) {
  const size_t base = static_cast<size_t>(blockIdx.x) * blockDim.x * V + threadIdx.x;
  u32x4 r[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const size_t i = base + static_cast<size_t>(v) * blockDim.x;
    r[v] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + (i < n16 ? i : 0));
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const size_t i = base + static_cast<size_t>(v) * blockDim.x;
    if (i < n16) __builtin_nontemporal_store(r[v], reinterpret_cast<u32x4*>(dst) + i);
  }
}

// Workspace of axon_variant_launch_noalloc: one array per GPU, held for the
// life of the process. Calls on one GPU share it (and race when they
// overlap); it keeps the last call's contents, so the part a kernel needs at
// zero is cleared before each launch.
constexpr size_t kScratchBytes = size_t{32} << 20;
static_assert(kScratchBytes % 16 == 0, "the zero fill writes whole 16-byte vectors");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current GPU's `scratch`, looked up once per device
// (the array's name in host code is not a device address).
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
    return AXON_EHIP;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("device index " + std::to_string(dev) + " beyond the scratch table");
    return AXON_EHIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      return AXON_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return AXON_OK;
}

__global__ __launch_bounds__(256) void zero_kernel(uint4* __restrict__ p, size_t n16) {
  const uint4 z = {0u, 0u, 0u, 0u};
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = z;
}

}  // namespace axon

using namespace axon;

extern "C" {

int axon_abi_version(void) { return AXON_ABI_VERSION; }

const char* axon_last_error(void) { return g_last_error.c_str(); }

int axon_kernel_count(void) { return kNumFamilies; }

const char* axon_kernel_name(int index) {
  if (index < 0 || index >= kNumFamilies) return nullptr;
  return family_at(index)->name;
}

int axon_kernel_variants(const char* kernel) {
  const Family* f = find(kernel);
  return f ? f->n_variants : 0;
}

int axon_variant_describe(const char* kernel, int hw_variant, char* buf, size_t buf_len) {
  const Family* f = find(kernel);
  if (f == nullptr || hw_variant < 0 || hw_variant >= f->n_variants) {
    set_error(std::string("unknown kernel/variant ") + (kernel ? kernel : "(null)") + " v" +
              std::to_string(hw_variant));
    return AXON_ENOKERNEL;
  }
  std::string s = "{\"kernel\": " + json_str(f->name) +
                  ", \"hw_variant\": " + std::to_string(hw_variant) + ", \"tile_args\": [";
  for (int i = 0; i < f->n_tiles; ++i) s += (i ? ", " : "") + json_str(f->tile_args[i]);
  s += "], \"n_inputs\": " + std::to_string(f->n_inputs) +
       ", \"n_outputs\": " + std::to_string(f->n_outputs) +
       ", \"n_dims\": " + std::to_string(f->n_dims) +
       ", \"summary\": " + json_str(f->summary(hw_variant)) + "}";
  return write_text(s, buf, buf_len);
}

int axon_variant_manifest(const char* kernel, int hw_variant, const int64_t* dims, int n_dims,
                          int dtype, char* buf, size_t buf_len) {
  const Family* f = find(kernel);
  if (f == nullptr || hw_variant < 0 || hw_variant >= f->n_variants) {
    set_error(std::string("unknown kernel/variant ") + (kernel ? kernel : "(null)") + " v" +
              std::to_string(hw_variant));
    return AXON_ENOKERNEL;
  }
  if (n_dims != f->n_dims || dims == nullptr) {
    set_error(std::string(f->name) + ": expected " + std::to_string(f->n_dims) + " dims");
    return AXON_EARG;
  }
  if (dtype != AXON_BF16 && dtype != AXON_F16 && dtype != AXON_F32) {
    set_error("unknown dtype code " + std::to_string(dtype));
    return AXON_EDTYPE;
  }
  Constraint recs[8];
  const int k = f->manifest(hw_variant, dims, dtype, recs, 8);
  std::string s = "{\"version\": 1, \"constraints\": [";
  for (int i = 0; i < k; ++i) {
    s += (i ? ", " : "");
    s += "{\"tile_arg\": " + json_str(recs[i].tile_arg) +
         ", \"extent\": " + std::to_string(recs[i].extent) +
         ", \"tile_size\": " + std::to_string(recs[i].tile_size) +
         ", \"require_divisible\": " + (recs[i].require_divisible ? "true" : "false") + "}";
  }
  s += "]}";
  return write_text(s, buf, buf_len);
}

int axon_variant_outputs(const char* kernel, const int64_t* dims, int n_dims,
                         const int32_t* dtypes, int n_dtypes, int max_rank, int64_t* shapes,
                         int32_t* ranks, int32_t* out_dtypes, int cap) {
  const Family* f = find(kernel);
  if (f == nullptr) {
    set_error(std::string("no HIP kernel family for spec '") + (kernel ? kernel : "(null)") + "'");
    return -AXON_ENOKERNEL;
  }
  if (n_dims != f->n_dims || n_dtypes != f->n_inputs || dims == nullptr || dtypes == nullptr ||
      shapes == nullptr || ranks == nullptr || out_dtypes == nullptr) {
    set_error(std::string(f->name) + ": bad arguments to axon_variant_outputs");
    return -AXON_EARG;
  }
  if (cap < f->n_outputs) {
    set_error(std::string(f->name) + ": room for " + std::to_string(f->n_outputs) + " outputs needed");
    return -AXON_EBUFFER;
  }
  OutDesc d[8];
  f->outputs(dims, dtypes, d);
  for (int i = 0; i < f->n_outputs; ++i) {
    if (d[i].rank > max_rank) {
      set_error(std::string(f->name) + ": output rank exceeds max_rank");
      return -AXON_EBUFFER;
    }
    ranks[i] = d[i].rank;
    out_dtypes[i] = d[i].dtype;
    for (int k = 0; k < d[i].rank; ++k) shapes[i * max_rank + k] = d[i].shape[k];
  }
  return f->n_outputs;
}

int axon_variant_check(const char* kernel, int hw_variant, const int32_t* tiles, int n_tiles,
                       const int64_t* dims, int n_dims, const int32_t* dtypes, int n_dtypes) {
  const Call c{hw_variant, tiles, n_tiles, dims, n_dims, dtypes, n_dtypes};
  const Family* f = nullptr;
  return checked(kernel, c, &f);
}

size_t axon_variant_workspace(const char* kernel, int hw_variant, const int32_t* tiles,
                              int n_tiles, const int64_t* dims, int n_dims,
                              const int32_t* dtypes, int n_dtypes) {
  const Call c{hw_variant, tiles, n_tiles, dims, n_dims, dtypes, n_dtypes};
  const Family* f = nullptr;
  if (checked(kernel, c, &f) != AXON_OK) return 0;
  return f->workspace(c);
}

}  // extern "C"

namespace {

// Argument checks shared by both launch entry points. Sets *empty when every
// output has zero elements (the launch is then a no-op: empty tensors may
// carry null data pointers).
int check_launch_args(const Family* f, const Call& c, const void* const* inputs, int n_in,
                      void* const* outputs, int n_out, bool* empty) {
  if (n_in != f->n_inputs || n_out != f->n_outputs || inputs == nullptr || outputs == nullptr) {
    set_error(std::string(f->name) + ": expected " + std::to_string(f->n_inputs) + " inputs and " +
              std::to_string(f->n_outputs) + " outputs");
    return AXON_EARG;
  }
  *empty = false;
  OutDesc d[8];
  if (f->n_outputs <= 8) {
    f->outputs(c.dims, c.dtypes, d);
    bool all_empty = true;
    for (int i = 0; i < f->n_outputs; ++i) {
      int64_t e = 1;
      for (int r = 0; r < d[i].rank; ++r) e *= d[i].shape[r];
      all_empty = all_empty && e == 0;
    }
    if (all_empty) {
      *empty = true;
      return AXON_OK;
    }
  }
  for (int i = 0; i < n_in; ++i)
    if (inputs[i] == nullptr) {
      set_error(std::string(f->name) + ": input " + std::to_string(i) + " is null");
      return AXON_EARG;
    }
  for (int i = 0; i < n_out; ++i)
    if (outputs[i] == nullptr) {
      set_error(std::string(f->name) + ": output " + std::to_string(i) + " is null");
      return AXON_EARG;
    }
  return AXON_OK;
}

}  // namespace

extern "C" {

int axon_variant_launch(const char* kernel, int hw_variant, const int32_t* tiles, int n_tiles,
                        const int64_t* dims, int n_dims, const int32_t* dtypes, int n_dtypes,
                        const void* const* inputs, int n_in, void* const* outputs, int n_out,
                        void* workspace, size_t workspace_bytes, axon_stream_t stream) {
  const Call c{hw_variant, tiles, n_tiles, dims, n_dims, dtypes, n_dtypes};
  const Family* f = nullptr;
  int rc = checked(kernel, c, &f);
  if (rc != AXON_OK) return rc;
  bool empty = false;
  rc = check_launch_args(f, c, inputs, n_in, outputs, n_out, &empty);
  if (rc != AXON_OK || empty) return rc;
  const size_t need = f->workspace(c);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error(std::string(f->name) + ": workspace of " + std::to_string(need) +
              " bytes required, got " + std::to_string(workspace_bytes));
    return AXON_EWORKSPACE;
  }
  return f->launch(c, inputs, outputs, workspace, reinterpret_cast<hipStream_t>(stream));
}

int axon_variant_launch_noalloc(const char* kernel, int hw_variant, const int32_t* tiles,
                                int n_tiles, const int64_t* dims, int n_dims,
                                const int32_t* dtypes, int n_dtypes, const void* const* inputs,
                                int n_in, void* const* outputs, int n_out, axon_stream_t stream) {
  const Call c{hw_variant, tiles, n_tiles, dims, n_dims, dtypes, n_dtypes};
  const Family* f = nullptr;
  int rc = checked(kernel, c, &f);
  if (rc != AXON_OK) return rc;
  bool empty = false;
  rc = check_launch_args(f, c, inputs, n_in, outputs, n_out, &empty);
  if (rc != AXON_OK || empty) return rc;
  const size_t need = f->workspace(c);
  if (need > kScratchBytes) {
    set_error(std::string(f->name) + " v" + std::to_string(hw_variant) + ": needs " +
              std::to_string(need) + " bytes of workspace, above the " +
              std::to_string(kScratchBytes) +
              "-byte static workspace of axon_variant_launch_noalloc; use axon_variant_launch "
              "with a caller workspace");
    return AXON_EWORKSPACE;
  }
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_address(&ws);
    if (rc != AXON_OK) return rc;
    const size_t zero = f->workspace_zeroed != nullptr ? f->workspace_zeroed(c) : 0;
    if (zero > 0) {
      const size_t n16 = (zero + 15) / 16;  // within the array: kScratchBytes % 16 == 0
      size_t blocks = (n16 + 255) / 256;
      if (blocks > 1024) blocks = 1024;
      hipLaunchKernelGGL(zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                         static_cast<uint4*>(ws), n16);
      rc = launch_status("zero_kernel");
      if (rc != AXON_OK) return rc;
    }
  }
  return f->launch(c, inputs, outputs, ws, st);
}

int axon_copy(const void* src, void* dst, size_t bytes, axon_stream_t stream) {
  return axon_copy_shape(src, dst, bytes, 0, stream);
}

int axon_copy_shape(const void* src, void* dst, size_t bytes, int shape, axon_stream_t stream) {
  if (src == nullptr || dst == nullptr || (bytes & 15u) || !aligned16(src) || !aligned16(dst)) {
    set_error("axon_copy: pointers must be 16-byte aligned and bytes a multiple of 16");
    return AXON_EARG;
  }
  if (shape < 0 || shape > 3) {
    set_error("axon_copy_shape: shape must be 0..3");
    return AXON_EARG;
  }
  if (bytes == 0) return AXON_OK;
  const size_t n16 = bytes / 16;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint4* s = static_cast<const uint4*>(src);
  uint4* d = static_cast<uint4*>(dst);
  if (shape == 1 || shape == 2) {
    const int V = shape == 1 ? 8 : 4;
    const size_t blocks = (n16 + 256 * V - 1) / (256 * V);
    if (const int rc = grid_check("axon_copy_shape (one-shot)", static_cast<int64_t>(blocks), 1, 256);
        rc != AXON_OK)
      return rc;
    if (V == 8)
      hipLaunchKernelGGL(copy_oneshot_kernel<8>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                         st, s, d, n16);
    else
      hipLaunchKernelGGL(copy_oneshot_kernel<4>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                         st, s, d, n16);
    return launch_status("copy_oneshot_kernel");
  }
  size_t blocks = (n16 + 255) / 256;
  const size_t cap = shape == 0 ? 256 * 64 : 1024;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, s, d, n16);
  return launch_status("copy_kernel");
}

uint32_t axon_scan_poll_bound(uint32_t polls) { return axon::set_scan_poll_bound(polls); }

}  // extern "C"
