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

#include <mutex>
#include <vector>

#include "../../include/logkv_hip.h"

namespace logkv {

// Why a launch function refused before enqueueing anything (a host-side check
// failed); the C ABI puts it in the text logkv_last_error returns. Defined in
// capi.hip.
extern thread_local const char* g_refusal;
inline int refuse(const char* why) {
  g_refusal = why;
  return LOGKV_ERUNTIME;
}

// Lets kernel `fn` launch with `bytes` of dynamic LDS on the current device.
// Above the 64 KiB default the limit is raised once per (kernel, device) and
// remembered, so steady-state launches make no attribute call.
inline bool allow_dynamic_lds(const void* fn, size_t bytes) {
  if (bytes <= 64 * 1024) return true;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    g_refusal = "no current HIP device";
    return false;
  }
  struct Limit {
    const void* fn;
    int dev;
    size_t bytes;
  };
  static std::mutex mu;
  static std::vector<Limit> limits;
  std::lock_guard<std::mutex> lock(mu);
  Limit* hit = nullptr;
  for (Limit& e : limits)
    if (e.fn == fn && e.dev == dev) hit = &e;
  if (hit && hit->bytes >= bytes) return true;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)) != hipSuccess) {
    g_refusal = "the device refused the kernel's dynamic LDS size";
    return false;
  }
  if (hit) hit->bytes = bytes;
  else limits.push_back(Limit{fn, dev, bytes});
  return true;
}

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

// dst[i] = src[i] for i < n by the threads of a block (thread tid of nthr): each
// thread issues up to kStageLoads loads before its first store, so staging a
// table into LDS waits on one load latency per kStageLoads * nthr elements
// instead of one per nthr (a plain strided loop waits on every load).
constexpr int kStageLoads = 16;
template <typename T, typename Dst, typename Src>
__device__ __forceinline__ void stage_copy(Dst dst, Src src, int n, int tid, int nthr) {
  if (n <= nthr) {   // one element per thread at most
    if (tid < n) dst[tid] = src[tid];
    return;
  }
  for (int i0 = tid; i0 < n; i0 += kStageLoads * nthr) {
    T v[kStageLoads];
#pragma unroll
    for (int q = 0; q < kStageLoads; ++q) {
      const int i = i0 + q * nthr;
      v[q] = i < n ? src[i] : T{};
    }
#pragma unroll
    for (int q = 0; q < kStageLoads; ++q) {
      const int i = i0 + q * nthr;
      if (i < n) dst[i] = v[q];
    }
  }
}

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

// Element d of a row as float, 0 for d >= D (D >= 1). The load is issued
// unconditionally with the index clamped into the row, so it needs no branch
// that would wait on it.
__device__ __forceinline__ float feat_or_zero(const LOGKV_G uint16_t* row, int d, int D) {
  const float x = bf16_to_f32(row[d < D ? d : D - 1]);
  return d < D ? x : 0.f;
}

__device__ __forceinline__ float feat_or_zero(const LOGKV_G float* row, int d, int D) {
  const float x = row[d < D ? d : D - 1];
  return d < D ? x : 0.f;
}

// The same sum as wave_tree (offsets 32, 16, 8, 4, 2, 1; lane l adds lane
// l + offset, which is what lane 0 of the xor butterfly adds), formed toward
// lane 0 with the gfx950 permlane swaps (lanes 0-31 read 32-63, rows 0/2 read
// rows 1/3) and DPP row shifts (lane l reads l + n within its 16-lane row),
// then read from lane 0. Every lane of the wave must be active.
__device__ __forceinline__ float wave_sum0(float s) {
  s = s + __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false)[1]);
  s = s + __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false)[1]);
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x108, 0xf, 0xf, false));  // row_shl:8
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x104, 0xf, 0xf, false));  // row_shl:4
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x102, 0xf, 0xf, false));  // row_shl:2
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x101, 0xf, 0xf, false));  // row_shl:1
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(s)));
}

// Four canonical sums at once, each exactly wave_sum0 of its value: the first
// permlane32 swap pairs a with b (lanes 0-31 fold a, lanes 32-63 fold b) and c
// with d; the permlane16 swap of the two results leaves rows 0..3 folding a, c,
// b, d; the row shifts finish all four. Every lane of the wave must be active.
__device__ __forceinline__ void wave_sum4(float a, float b, float c, float d, float& sa, float& sb, float& sc,
                                          float& sd) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const float ab = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(d), false, false);
  const float cd = __uint_as_float(q[0]) + __uint_as_float(q[1]);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(ab), __float_as_uint(cd), false, false);
  float s = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x108, 0xf, 0xf, false));  // row_shl:8
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x104, 0xf, 0xf, false));  // row_shl:4
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x102, 0xf, 0xf, false));  // row_shl:2
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x101, 0xf, 0xf, false));  // row_shl:1
  sa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
  sc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 16));
  sb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
  sd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 48));
}

__device__ __forceinline__ double readlane_f64(double x, int lane) {
  const long long bits = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(bits), lane);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(bits >> 32), lane);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<uint32_t>(lo));
}

// a / b rounded to float exactly as IEEE float division, from b's double
// reciprocal r = 1 / (double)b: the double product a * r is within 2^-52
// (relative) of a / b, while a quotient of two floats that is not itself a
// float lies at least 2^-50 (relative) from every float rounding boundary,
// normal or subnormal; so rounding the product to float gives the correctly
// rounded quotient (and an exact quotient stays exact). Three instructions
// per quotient once r is known.
__device__ __forceinline__ float div_by_rcp(float a, double r) {
  return static_cast<float>(static_cast<double>(a) * r);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

__device__ __forceinline__ int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }
__device__ __forceinline__ int64_t imax64(int64_t a, int64_t b) { return a > b ? a : b; }

}  // namespace logkv
