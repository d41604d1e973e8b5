// Shared device helpers for the gfx950 kernel set: element types, 16-byte
// vector loads/stores, fp32 conversion and wave64 reductions/scans.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "axon_hip.h"

namespace axon {

using bf16 = __bf16;
using f16 = _Float16;

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Scalar conversions. float -> bf16 lowers to v_cvt_pk_bf16_f32 (round to
// nearest even) on gfx950.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return static_cast<bf16>(v); }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }

// ---------------------------------------------------------------------------
// 16-byte vectors: EPV<T> elements per vector (8 for 16-bit types, 4 for fp32).
// ---------------------------------------------------------------------------
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct EPV {
  static constexpr int value = 16 / sizeof(T);
};

template <typename T>
struct alignas(16) Vec {
  T v[EPV<T>::value];
};

template <typename T>
__device__ __forceinline__ Vec<T> load_vec(const T* p) {
  Vec<T> r;
  *reinterpret_cast<u32x4*>(&r) = *reinterpret_cast<const u32x4*>(p);
  return r;
}

template <typename T>
__device__ __forceinline__ void store_vec(T* p, const Vec<T>& r) {
  *reinterpret_cast<u32x4*>(p) = *reinterpret_cast<const u32x4*>(&r);
}

// Non-temporal variants for streams that are read or written exactly once.
template <typename T>
__device__ __forceinline__ Vec<T> load_vec_nt(const T* p) {
  Vec<T> r;
  const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  *reinterpret_cast<u32x4*>(&r) = u;
  return r;
}

template <typename T>
__device__ __forceinline__ void store_vec_nt(T* p, const Vec<T>& r) {
  __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&r),
                              reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// wave64 reductions (butterfly over all 64 lanes; every lane gets the result)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Launch-shape checks used by every family before any kernel is enqueued.
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace axon
