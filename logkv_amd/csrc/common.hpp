// Shared device helpers for the LogKV HIP kernels (gfx950, wave64).
//
// Float rules used by every kernel:
//  * no fused multiply-add: the library is built with -ffp-contract=off, so
//    each a*b+c is a rounded product followed by a rounded add;
//  * feature-axis sums use `wave_dsum`: lane l accumulates t[l], t[l+64], ...
//    in order, then the 64 partials are folded by an xor butterfly, which
//    leaves in every lane the value of the halving tree p[i] += p[i+32],
//    p[i] += p[i+16], ..., p[i] += p[i+1];
//  * token-axis sums run sequentially in row order;
//  * bf16 stores round to nearest, ties to even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/logkv_hip.h"

namespace logkv {

// Address-space-qualified pointers: loads and stores through them compile to
// global_* / ds_* instructions instead of flat_* ones, which the compiler must
// fence against both memory counters (a generic pointer might be LDS).
#if defined(__HIP_DEVICE_COMPILE__)
#define LOGKV_G __attribute__((address_space(1)))
#define LOGKV_S __attribute__((address_space(3)))
#else
#define LOGKV_G
#define LOGKV_S
#endif

template <typename T>
__device__ __forceinline__ LOGKV_G T* gp(T* p) {
  return (LOGKV_G T*)p;
}
template <typename T>
__device__ __forceinline__ const LOGKV_G T* gp(const T* p) {
  return (const LOGKV_G T*)p;
}

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Butterfly over the 64 lanes of a wave; every lane ends with the canonical sum.
__device__ __forceinline__ float wave_tree(float s) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_xor(s, off, kWave);
  return s;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

__device__ __forceinline__ int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }
__device__ __forceinline__ int64_t imax64(int64_t a, int64_t b) { return a > b ? a : b; }

}  // namespace logkv
