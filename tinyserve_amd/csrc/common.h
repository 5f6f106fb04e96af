// Device-side building blocks shared by the gfx950 kernels: element types, 16-byte
// vector loads/stores, wave64 cross-lane exchanges and fp32 helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <stdint.h>

#include "../../include/tinyserve_amd.h"

namespace ts {

using f16 = _Float16;
using bf16 = __bf16;

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// 16 bytes moved as one global_load_dwordx4 / global_store_dwordx4.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Pack16 {
  static constexpr int N = 16 / sizeof(T);
  union {
    u32x4 raw;
    T v[16 / sizeof(T)];
  };
};

template <typename T>
__device__ __forceinline__ float to_f32(T x) {
  return static_cast<float>(x);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  return static_cast<T>(x);  // round to nearest even for f16 and bf16
}

template <typename T>
__device__ __forceinline__ Pack16<T> load16(const T* p) {
  Pack16<T> r;
  r.raw = *reinterpret_cast<const u32x4*>(p);
  return r;
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const Pack16<T>& x) {
  *reinterpret_cast<u32x4*>(p) = x.raw;
}

// x from the lane whose id is (this lane's id) XOR OFF. OFF < 32 stays inside a
// 32-lane half and uses ds_swizzle's xor mode (no address computation); OFF == 32
// crosses the halves through ds_bpermute.
template <int OFF>
__device__ __forceinline__ float xor_lane(float x) {
  static_assert(OFF > 0 && OFF <= 32 && (OFF & (OFF - 1)) == 0, "power-of-2 offset");
  if constexpr (OFF == 32) {
    return __shfl_xor(x, 32);
  } else {
    constexpr int pattern = (OFF << 10) | 0x1f;  // and_mask 31, or_mask 0, xor_mask OFF
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), pattern));
  }
}

// Sum / max over groups of N consecutive lanes (N a power of 2 <= 64); every lane of a
// group ends with the group's total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += xor_lane<1>(x);
  if constexpr (N >= 4) x += xor_lane<2>(x);
  if constexpr (N >= 8) x += xor_lane<4>(x);
  if constexpr (N >= 16) x += xor_lane<8>(x);
  if constexpr (N >= 32) x += xor_lane<16>(x);
  if constexpr (N >= 64) x += xor_lane<32>(x);
  return x;
}

// Max / sum of x over lanes l and l ^ 32 (the two 32-lane halves), via gfx950's
// v_permlane32_swap: with both operands x, one result holds x of this lane and the other
// x of the partner lane (in either order per half), so max/sum of the pair is the answer.
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// RMSNorm's output element: y = (T)(x * r) * w, the multiply by w in T's precision (exact
// product, one rounding), as layers.py:14-38 computes it in the model dtype.
template <typename T>
__device__ __forceinline__ T norm_scale(T x, float r, T w) {
  const T xn = from_f32<T>(to_f32(x) * r);
  return from_f32<T>(to_f32(xn) * to_f32(w));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

inline int ilog2(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

inline bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

inline int elem_size(int dtype) { return dtype == TS_F32 ? 4 : 2; }

// Compute units of the current device (cached per device; 256 on MI355X).
inline int compute_units() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int hit = cache[dev].load(std::memory_order_relaxed);
    if (hit > 0) return hit;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

}  // namespace ts
