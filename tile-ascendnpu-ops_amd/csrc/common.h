// Shared device helpers for the gfx950 TileOPs kernels: element types,
// 128-bit vector access, fp32 <-> fp16/bf16 conversion and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tileops_hip.h"

namespace tileops {

typedef _Float16 f16;
typedef __bf16 bf16;

// 128-bit payload used for every coalesced global load/store.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Element traits: how many elements fit in 16 bytes and how to move them
// through fp32.  Conversions to the narrow types round to nearest even
// (v_cvt_f16_f32 / v_cvt_pk_bf16_f32), the same rounding torch applies in
// `.to(dtype)`.
template <typename T> struct Elem;

template <> struct Elem<float> {
  static constexpr int kVec = 4;
  __device__ __forceinline__ static float to_f32(float v) { return v; }
  __device__ __forceinline__ static float from_f32(float v) { return v; }
};

template <> struct Elem<f16> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float to_f32(f16 v) { return (float)v; }
  __device__ __forceinline__ static f16 from_f32(float v) { return (f16)v; }
};

template <> struct Elem<bf16> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float to_f32(bf16 v) { return (float)v; }
  __device__ __forceinline__ static bf16 from_f32(float v) { return (bf16)v; }
};

// A 16-byte bundle of kVec elements of T, loadable with one global_load_dwordx4.
template <typename T> struct alignas(16) Pack {
  T v[Elem<T>::kVec];
};

template <typename T>
__device__ __forceinline__ Pack<T> load_pack(const T* p) {
  return *reinterpret_cast<const Pack<T>*>(p);
}

// Streaming (non-temporal) variants: data touched exactly once should not
// evict reusable lines from L2 / MALL.
template <typename T>
__device__ __forceinline__ Pack<T> load_pack_nt(const T* p) {
  u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return *reinterpret_cast<Pack<T>*>(&r);
}

template <typename T>
__device__ __forceinline__ void store_pack_nt(T* p, const Pack<T>& v) {
  __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&v),
                              reinterpret_cast<u32x4*>(p));
}

__device__ __forceinline__ bool is_aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline bool host_aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Number of workgroups for a grid-stride streaming kernel: enough waves in
// flight to saturate HBM on 256 CUs (8 XCDs x 32 CUs), never more than the
// work needs.
inline int64_t stream_grid(int64_t work_items, int block) {
  int64_t need = (work_items + block - 1) / block;
  const int64_t cap = 256 * 16;  // 16 workgroups of 256 threads per CU
  if (need < 1) need = 1;
  return need < cap ? need : cap;
}

// Compute units of the current device, queried once per device (persistent
// grids size themselves from it).
inline int device_cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// A streamed operand up to this size may still sit in the 256 MB Infinity
// Cache when it is read again soon (a decode loop over a small model, a
// repeated call): kernels read such operands with plain loads and larger
// ones, which cannot stay resident, with non-temporal loads.
constexpr int64_t kCacheFitBytes = int64_t(128) << 20;

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // namespace tileops

namespace tileops {

// Butterfly reductions across the 64 lanes of a wavefront (ds_swizzle /
// ds_bpermute under __shfl_xor); every lane ends with the full result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

}  // namespace tileops
