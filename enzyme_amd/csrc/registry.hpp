// Internal registry types shared by the kernel families and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "axon_hip.h"

namespace axon {

// One `__axon_tile_constraints__` record.
struct Constraint {
  const char* tile_arg;
  int64_t extent;
  int64_t tile_size;
  bool require_divisible;
};

// Everything a family needs to judge or run one (variant, tiles, dims) key.
struct Call {
  int variant;
  const int32_t* tiles;
  int n_tiles;
  const int64_t* dims;
  int n_dims;
  const int32_t* dtypes;
  int n_dtypes;

  int64_t dim(int i) const { return dims[i]; }
  int tile(int i) const { return tiles[i]; }
  int dtype(int i) const { return dtypes[i]; }
};

// Shape and element type of one output.
struct OutDesc {
  int rank;
  int64_t shape[6];
  int dtype;
};

struct Family {
  const char* name;  // the spec name this family serves
  int n_variants;
  int n_inputs;
  int n_outputs;
  int n_dims;
  const char* const* tile_args;
  int n_tiles;
  const char* (*summary)(int variant);
  // Fills at most `cap` records; returns how many were written.
  int (*manifest)(int variant, const int64_t* dims, int dtype, Constraint* out, int cap);
  // AXON_OK, or an AXON_E* code with `why` filled in.
  int (*check)(const Call& c, std::string* why);
  size_t (*workspace)(const Call& c);
  // Fills one record per output from the dims and input dtypes.
  void (*outputs)(const int64_t* dims, const int32_t* dtypes, OutDesc* out);
  int (*launch)(const Call& c, const void* const* in, void* const* out, void* ws,
                hipStream_t stream);
  // Bytes at the start of the workspace that must hold zeros when it last
  // served a different kernel (null: none; every byte is written before it
  // is read).
  size_t (*workspace_zeroed)(const Call& c) = nullptr;
};

// Records `msg` as the calling thread's last error.
void set_error(const std::string& msg);

// Returns AXON_OK or AXON_EHIP after the last enqueue.
int launch_status(const char* what);

// A dispatch holds at most 2^31 - 1 workgroups along x, at most 65535 along
// y, and fewer than 2^32 work-items in total.
inline bool grid_fits(int64_t gx, int64_t gy, int64_t threads) {
  return gx >= 0 && gy >= 0 && gx <= (1LL << 31) - 1 && gy <= 65535 && threads > 0 &&
         (gx == 0 || gy == 0 || gx * gy <= 0xFFFFFFFFLL / threads);
}

// AXON_OK when a launch of gx x gy workgroups of `threads` threads fits one
// dispatch; otherwise records why (naming `what`) and returns AXON_EINVAL.
int grid_check(const char* what, int64_t gx, int64_t gy, int64_t threads);

inline bool is_pow2_in(int v, int lo, int hi) {
  return v >= lo && v <= hi && (v & (v - 1)) == 0;
}

inline const char* dtype_str(int d) {
  switch (d) {
    case AXON_BF16: return "bfloat16";
    case AXON_F16: return "float16";
    case AXON_F32: return "float32";
    default: return "unknown";
  }
}

inline int elem_bytes(int d) { return d == AXON_F32 ? 4 : 2; }

// Poll bound of the single-pass cumsum variant (scan.hip); returns the
// previous bound.
unsigned set_scan_poll_bound(unsigned polls);

}  // namespace axon
