// Attach routing on the device: position order, frozen-center decisions, farthest-point seeds.
//
// Follows litgpt/log_kv_route_triton.py:841-917 (fused attach decisions) and
// litgpt/log_kv_cache.py:4597-4680 (position order, seeding planner), redesigned
// for wave64: one wave evaluates one row against every cluster, holding features
// l, l+64, ... of the row in lane l; distances are folded with the canonical
// butterfly (common.hpp), so every lane holds the same decision inputs.
#include "route.hpp"

namespace logkv {

// ---------------------------------------------------------------------------
// Position order per batch row: stable argsort of positions, padding last.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void order_kernel(const int64_t* __restrict__ pos, int64_t pos_sb,
                                                     const int32_t* __restrict__ counts, int32_t tokens,
                                                     int32_t* __restrict__ order, int32_t* __restrict__ clear,
                                                     int n_clear) {
  __shared__ uint64_t keys[kMaxOrderRows];
  const int b = blockIdx.x;
  // Optional status words for the launches that follow, cleared in stream order.
  if (clear && b == 0 && static_cast<int>(threadIdx.x) < n_clear) clear[threadIdx.x] = 0;
  int n = counts ? counts[b] : tokens;
  n = n < 0 ? 0 : (n > tokens ? tokens : n);
  const int64_t* p = pos + b * pos_sb;
  int32_t* out = order + static_cast<int64_t>(b) * tokens;
  // Already non-decreasing (the common case: a contiguous recent window) ->
  // the stable order is the identity.
  int unsorted = 0;
  for (int t = threadIdx.x; t + 1 < n; t += blockDim.x) unsorted |= p[t] > p[t + 1];
  if (!__syncthreads_or(unsorted)) {
    for (int t = threadIdx.x; t < tokens; t += blockDim.x) out[t] = t;
    return;
  }
  int width = 1;
  while (width < tokens) width <<= 1;
  for (int t = threadIdx.x; t < width; t += blockDim.x) {
    uint64_t key;
    if (t < n) key = (static_cast<uint64_t>(p[t]) << kOrderIndexBits) | static_cast<uint64_t>(t);
    else key = (~0ull << kOrderIndexBits) | static_cast<uint64_t>(t < tokens ? t : kOrderIndexMask);
    keys[t] = key;
  }
  __syncthreads();
  for (int size = 2; size <= width; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < width; t += blockDim.x) {
        const int partner = t ^ stride;
        if (partner > t) {
          const bool up = (t & size) == 0;
          const uint64_t a = keys[t], c = keys[partner];
          if ((a > c) == up) {
            keys[t] = c;
            keys[partner] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int t = threadIdx.x; t < tokens; t += blockDim.x) out[t] = static_cast<int32_t>(keys[t] & kOrderIndexMask);
}

// ---------------------------------------------------------------------------
// Frozen-center decisions (litgpt/log_kv_route_triton.py:841-917): one thread
// per (row, cluster) pair over a tile of rows staged in LDS.
//
// Every distance keeps the canonical order of wave_sum0: leaf l (0..63) sums
// features l, l + 64, ... in order; leaves fold as a balanced tree (l with
// l + 32, then + 16, ..., + 1). One thread evaluates the whole tree, leaves
// visited depth-first (bit-reversed leaf order), so no cross-lane reduction
// is needed. Rows and centers are stored leaf-major: leaf l's NJ features
// are adjacent (one LDS read), rows padded by two words against bank
// conflicts between the rows a wave reads together.
// ---------------------------------------------------------------------------
template <int NJ>
__host__ __device__ constexpr int leaf_stride() { return kWave * NJ + 2; }

struct DotEx {
  float dot, ex;
};

template <int NJ, int LEVEL, int L0>
__device__ __forceinline__ DotEx canon_tree(const float* x, const float* m) {
  if constexpr (LEVEL == 0) {
    DotEx r;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float a = x[L0 * NJ + j], b = m[L0 * NJ + j];
      const float diff = a - b;
      r.dot = j == 0 ? a * b : r.dot + a * b;
      r.ex = j == 0 ? diff * diff : r.ex + diff * diff;
    }
    return r;
  } else {
    const DotEx lo = canon_tree<NJ, LEVEL - 1, L0>(x, m);
    // Subtrees of 8 leaves are scheduled one after the other, which bounds
    // the LDS values in flight (and the registers holding them).
    if constexpr (LEVEL == 4) __builtin_amdgcn_sched_barrier(0);
    const DotEx hi = canon_tree<NJ, LEVEL - 1, L0 + (1 << (6 - LEVEL))>(x, m);
    return DotEx{lo.dot + hi.dot, lo.ex + hi.ex};
  }
}

// Canonical sum of squares of one leaf-major row.
template <int NJ, int LEVEL, int L0>
__device__ __forceinline__ float canon_sq(const float* x) {
  if constexpr (LEVEL == 0) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) s = j == 0 ? x[L0 * NJ] * x[L0 * NJ] : s + x[L0 * NJ + j] * x[L0 * NJ + j];
    return s;
  } else {
    const float lo = canon_sq<NJ, LEVEL - 1, L0>(x);
    if constexpr (LEVEL == 4) __builtin_amdgcn_sched_barrier(0);
    return lo + canon_sq<NJ, LEVEL - 1, L0 + (1 << (6 - LEVEL))>(x);
  }
}

template <int NJ>
__host__ __device__ constexpr int attach_tile() { return NJ <= 2 ? 64 : 16; }   // rows per block (32 and 128 measured slower)

template <int NJ>
__host__ __device__ inline size_t attach_shmem(int K) {
  constexpr int R = attach_tile<NJ>();
  return static_cast<size_t>(R + K) * leaf_stride<NJ>() * 4 + static_cast<size_t>(R) * K * 8 +
         static_cast<size_t>(R + K) * 4 + static_cast<size_t>(R) * 12 + 64;
}

constexpr int kAttachMaxThreads = 512;

// Leaves 4 lq .. 4 lq + 3 of a leaf-major row: v[j][e] is feature 4 lq + e + 64 j.
template <int NJ>
__device__ __forceinline__ void stage_leaves(float* row, const float (&v)[NJ][4], int lq) {
  float* p = row + 4 * lq * NJ;
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int j = 0; j < NJ; ++j) p[e * NJ + j] = v[j][e];
}

template <int NJ>
__global__ __launch_bounds__(kAttachMaxThreads) void attach_kernel(LadderArgs c, RowsArgs r, RouteParams prm,
                                                     const int32_t* __restrict__ order,
                                                     int8_t* __restrict__ assign, float* __restrict__ s_win) {
  constexpr int R = attach_tile<NJ>(), LS = leaf_stride<NJ>();
  extern __shared__ __align__(16) float att[];
  const int K = c.k_max, D = c.dk;
  float* x_l = att;                        // [R][LS] rows, leaf-major
  float* mu_l = x_l + R * LS;              // [K][LS] centers, leaf-major
  float* dot_s = mu_l + K * LS;            // [R * K]
  float* ex_s = dot_s + R * K;             // [R * K]
  float* xx_s = ex_s + R * K;              // [R]
  float* mm_s = xx_s + R;                  // [K]
  int32_t* t_s = reinterpret_cast<int32_t*>(mm_s + K);                 // [R] row index in the flush
  int64_t* pos_s = reinterpret_cast<int64_t*>(
      reinterpret_cast<uintptr_t>(t_s + R + 1) & ~uintptr_t(7));       // [R]
  const int lane_ix = blockIdx.y;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  const int n = valid_rows(r, b);
  const int tile0 = blockIdx.x * R;
  const int rows = max(0, min(R, n - tile0));
  const int tid = static_cast<int>(threadIdx.x), nthr = static_cast<int>(blockDim.x);
  // Centers and rows into LDS (features past D are zero).
  const LOGKV_G float* mu = gp(c.centroid) + static_cast<int64_t>(lane_ix) * K * D;
  // Staged four leaves at a time: features 4 lq + e + 64 j (e < 4) of every
  // j are one 16-byte (center, f32) or 8-byte (row, bf16) load each.
  constexpr int LQ = kWave / 4;
  for (int i = tid; i < K * LQ; i += nthr) {
    const int cc = i / LQ, lq = i % LQ;
    float v[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int f = 4 * lq + kWave * j;
      float4 x = {0.f, 0.f, 0.f, 0.f};
      if (f < D) x = *reinterpret_cast<const LOGKV_G float4*>(mu + cc * D + f);
      v[j][0] = x.x;
      v[j][1] = x.y;
      v[j][2] = x.z;
      v[j][3] = x.w;
    }
    stage_leaves<NJ>(mu_l + cc * LS, v, lq);
  }
  for (int i = tid; i < rows; i += nthr) {
    const int t = order[static_cast<int64_t>(b) * r.tokens + tile0 + i];
    t_s[i] = t;
    pos_s[i] = r.pos[b * r.pos_sb + t];
  }
  // The lane's cluster state for the decisions (alive bits, p_hi per cluster).
  __shared__ int64_t phi_s[kMaxClusters];
  __shared__ int32_t ntot_s[kMaxClusters];
  __shared__ uint32_t alive_s;
  if (tid < kWave) {
    const bool live = tid < K && c.alive[lane_ix * K + tid];
    const uint64_t bits = __ballot(live);
    if (tid < K) {
      phi_s[tid] = c.p_hi_c[static_cast<int64_t>(lane_ix) * K + tid];
      ntot_s[tid] = c.n_total[static_cast<int64_t>(lane_ix) * K + tid];
    }
    if (tid == 0) alive_s = static_cast<uint32_t>(bits);
  }
  __syncthreads();
  const LOGKV_G uint16_t* kbase = gp(r.k + b * r.k_sb + g * r.k_sg);
  for (int i = tid; i < rows * LQ; i += nthr) {
    const int rr = i / LQ, lq = i % LQ;
    const LOGKV_G uint16_t* row = kbase + static_cast<int64_t>(t_s[rr]) * r.k_st;
    float v[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int f = 4 * lq + kWave * j;
      uint2 x = {0u, 0u};
      if (f < D) x = *reinterpret_cast<const LOGKV_G uint2*>(row + f);
      v[j][0] = __uint_as_float(x.x << 16);
      v[j][1] = __uint_as_float(x.x & 0xffff0000u);
      v[j][2] = __uint_as_float(x.y << 16);
      v[j][3] = __uint_as_float(x.y & 0xffff0000u);
    }
    stage_leaves<NJ>(x_l + rr * LS, v, lq);
  }
  __syncthreads();
  if (tid < rows) xx_s[tid] = canon_sq<NJ, 6, 0>(x_l + tid * LS);
  else if (tid >= R && tid < R + K) mm_s[tid - R] = canon_sq<NJ, 6, 0>(mu_l + (tid - R) * LS);
  for (int p = tid; p < rows * K; p += nthr) {
    const int rr = p / K, cc = p % K;
    const DotEx de = canon_tree<NJ, 6, 0>(x_l + rr * LS, mu_l + cc * LS);
    dot_s[p] = de.dot;
    ex_s[p] = de.ex;
  }
  __syncthreads();
  if (tid < rows) {
    const uint32_t alive_bits = alive_s;
    const bool any_alive = alive_bits != 0;
    const bool any_free = alive_bits != ((K >= 32) ? 0xffffffffu : ((1u << K) - 1u));
    const float radius = prm.lam * c.s_h[lane_ix];
    const int64_t* phi = phi_s;
    const float xx = xx_s[tid];
    const int64_t pos = pos_s[tid];
    float best = __builtin_inff(), s_winner = 0.f, best_e = __builtin_inff();
    int winner = 0, nearest = 0;
    for (int cc = 0; cc < K; ++cc) {
      const float semantic = fmaxf((xx + mm_s[cc]) - 2.0f * dot_s[tid * K + cc], 0.0f);
      const bool live = (alive_bits >> cc) & 1u;
      if (cc == 0) s_winner = semantic;
      if (live) {
        const int64_t gi = pos - phi[cc];
        const float gap = static_cast<float>(gi > 0 ? gi : 0);
        const float cost = semantic + prm.eta * (gap / (gap + prm.g0));
        if (cost < best) {
          best = cost;
          winner = cc;
          s_winner = semantic;
        }
        const float ex = ex_s[tid * K + cc];
        if (ex < best_e) {
          best_e = ex;
          nearest = cc;
        }
      }
    }
    // With a capacity cap a frozen join also needs room for one more row in
    // the winner (litgpt/log_kv_cache.py:2677-2680); the per-cluster room and
    // the orphans are settled by the capped seed launch.
    const bool capped = prm.hard_cap > 0.f;
    bool direct = any_alive && (s_winner <= radius);
    if (capped) direct = direct && static_cast<float>(ntot_s[winner] + 1) <= prm.hard_cap;
    int out;
    if (!any_free && !capped) out = direct ? winner : nearest;
    else out = direct ? winner : -1;
    const int s = tile0 + tid;
    assign[static_cast<int64_t>(lane_ix) * r.tokens + s] = static_cast<int8_t>(out);
    if (any_free || capped) s_win[static_cast<int64_t>(lane_ix) * r.tokens + s] = s_winner;
  }
  // Padding rows of the lane keep -1.
  for (int s = tile0 + tid; s < tile0 + R && s < r.tokens; s += nthr)
    if (s >= n) assign[static_cast<int64_t>(lane_ix) * r.tokens + s] = -1;
}

// ---------------------------------------------------------------------------
// Frozen-center decisions for 128-feature rows with a matrix-core screen (the
// decisions of attach_kernel, bit for bit).
//
// A wave takes 32 rows at a time. Lane r + 32 h holds features 16 j + 8 h + e
// (j, e < 8) of row r: the A operand of v_mfma_f32_32x32x16_bf16 for k step j,
// and whole leaves of the canonical tree (leaf L's features L and L + 64 sit
// in the same lane; only the fold of leaves L and L + 8 and the last fold of
// the two half sums cross to the partner lane).
//
// Screen: each center is split into two bf16 parts, hi + mid, within 2^-16
// (relative) of the f32 center, so 16 products give every (row, cluster) dot
// product d~ = x.m within about 2^-15 sum|x m| <= 2^-15 sqrt(xx mm) (the
// residual plus the matrix core's accumulation, if it rounds like a chain of
// f32 adds). From d~ and the canonical norms each live cluster gets its cost
// c~ and squared difference v~ = (xx + mm) - 2 d~, with the bounds
// D = 2^-11 (sqrt(xx) sqrt(mm) + |v~| + |t~|) + 2^-80 on |c~ - cost| and
// D' = 2^-11 (xx + mm + |v~|) + 2^-80 on |v~ - canonical squared difference|
// (generous for every rounding on either side, the temporal term t~ taken
// with a hardware reciprocal). A cluster can win only if c~ - D <= min(c~ + D)
// and be the nearest only if v~ - D' <= min(v~ + D'): the canonical trees run
// for those candidates only, the winner's dot always (its semantic distance
// is compared with the radius and stored). The two lanes of a row screen
// alternate clusters and merge their minima and candidate masks. A lane with a
// center whose sum of squares is above 2^60 or not finite, and a row with such
// a sum or a non-finite screened value, evaluate every cluster canonically.
// ---------------------------------------------------------------------------
typedef __bf16 att_bf16x8 __attribute__((ext_vector_type(8)));
typedef float att_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kAttachMfmaWaves = 4;
constexpr int kAttachTilesPerWave = 2;   // 32-row tiles per wave (the block's centers are staged once)
constexpr int kCenterPitchF = 132;   // floats per staged f32 center (16 B of padding)
constexpr int kCenterPitchB = 136;   // bf16 per staged center part (16 B of padding)
constexpr int kCenterParts = 2;      // bf16 parts per center (hi, mid)

__host__ __device__ inline size_t attach_mfma_shmem(int K) {
  return static_cast<size_t>(K) * kCenterPitchF * 4 + static_cast<size_t>(kCenterParts * K) * kCenterPitchB * 2 +
         static_cast<size_t>(kAttachMfmaWaves) * 2 * 32 * (K + 1) * 4;
}

// min / or of a value over the two lanes of a row (lanes r and r + 32).
__device__ __forceinline__ float pair_min(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fminf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ uint32_t pair_or(uint32_t v) {
  const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return p[0] | p[1];
}

__device__ __forceinline__ void unpack_bf16x8(const uint4 q, float (&f)[8]) {
  f[0] = __uint_as_float(q.x << 16);
  f[1] = __uint_as_float(q.x & 0xffff0000u);
  f[2] = __uint_as_float(q.y << 16);
  f[3] = __uint_as_float(q.y & 0xffff0000u);
  f[4] = __uint_as_float(q.z << 16);
  f[5] = __uint_as_float(q.z & 0xffff0000u);
  f[6] = __uint_as_float(q.w << 16);
  f[7] = __uint_as_float(q.w & 0xffff0000u);
}

__device__ __forceinline__ void load_f32x8(const float* p, float (&f)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x;
  f[1] = a.y;
  f[2] = a.z;
  f[3] = a.w;
  f[4] = b.x;
  f[5] = b.y;
  f[6] = b.z;
  f[7] = b.w;
}

// The canonical tree of canon_tree / canon_sq for a row held as above, against
// center m (f32, natural feature order): KIND 0 the row's sum of squares, 1 the
// dot product, 2 the squared difference. Both lanes of the row must be active;
// both return the same value.
template <int KIND>
__device__ __forceinline__ float pair_tree(const uint4 (&xq)[8], const float* m, int h) {
  float p2[8];
#pragma unroll
  for (int jp = 0; jp < 2; ++jp) {
    if (jp == 1) __builtin_amdgcn_sched_barrier(0);   // one half of the center's loads in flight at a time
    float lf[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int j = jp + 2 * q;     // leaves 16 j + 8 h + e: features j and j + 4 of the lane
      float xa[8], xb[8], ma[8], mb[8];
      unpack_bf16x8(xq[j], xa);
      unpack_bf16x8(xq[j + 4], xb);
      if constexpr (KIND != 0) {
        load_f32x8(m + 16 * j + 8 * h, ma);
        load_f32x8(m + 16 * (j + 4) + 8 * h, mb);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (KIND == 0) {
          lf[q][e] = xa[e] * xa[e] + xb[e] * xb[e];
        } else if constexpr (KIND == 1) {
          lf[q][e] = xa[e] * ma[e] + xb[e] * mb[e];
        } else {
          const float da = xa[e] - ma[e], db = xb[e] - mb[e];
          lf[q][e] = da * da + db * db;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p1 = lf[0][e] + lf[1][e];   // leaves L and L + 32
      p2[e] = jp == 0 ? p1 : p2[e] + p1;      // then L and L + 16
    }
  }
  // Leaves L and L + 8 sit in the two lanes of the row: the low lane folds the
  // even e, the high lane the odd e (one permlane32 swap per pair).
  float q4[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(p2[2 * k]), __float_as_uint(p2[2 * k + 1]),
                                                     false, false);
    q4[k] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  const float s = (q4[0] + q4[2]) + (q4[1] + q4[3]);   // + 4, + 2
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);   // + 1
}

// Marks the packed row as rewritten, so the loops over candidate clusters
// unpack it per evaluation instead of hoisting all 64 unpacked features.
__device__ __forceinline__ void keep_packed(uint4 (&xq)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(xq[j].x), "+v"(xq[j].y), "+v"(xq[j].z), "+v"(xq[j].w));
}

// Wave-local LDS exchange point: the wave's earlier LDS writes are seen by its
// later reads from any lane.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(kAttachMfmaWaves* kWave) void attach_mfma_kernel(
    LadderArgs c, RowsArgs r, RouteParams prm, const int32_t* __restrict__ order, int8_t* __restrict__ assign,
    float* __restrict__ s_win, int tiles_per_wave) {
  extern __shared__ __align__(16) float att[];
  const int K = c.k_max, tp = K + 1;
  float* mf = att;                                                              // [K][132] f32 centers
  uint16_t* bs = reinterpret_cast<uint16_t*>(mf + K * kCenterPitchF);          // [2][K][136] bf16 parts
  float* tw = reinterpret_cast<float*>(bs + kCenterParts * K * kCenterPitchB); // [waves][2][32][K + 1]
  __shared__ float mm_s[kMaxClusters], sm_s[kMaxClusters];
  __shared__ int64_t phi_s[kMaxClusters];
  __shared__ int32_t ntot_s[kMaxClusters];
  __shared__ uint32_t alive_s;
  const int lane_ix = blockIdx.y;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  const int n = valid_rows(r, b);
  const int tid = static_cast<int>(threadIdx.x), l = lane_id(), w = wave_id();
  // Centers: f32 copies for the canonical trees and the three bf16 parts.
  const LOGKV_G float* mu = gp(c.centroid) + static_cast<int64_t>(lane_ix) * K * 128;
  for (int i = tid; i < K * 32; i += static_cast<int>(blockDim.x)) {
    const int cc = i >> 5, q = i & 31;
    const float4 v = *reinterpret_cast<const LOGKV_G float4*>(mu + cc * 128 + 4 * q);
    *reinterpret_cast<float4*>(mf + cc * kCenterPitchF + 4 * q) = v;
    const float e[4] = {v.x, v.y, v.z, v.w};
    uint16_t part[kCenterParts][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      part[0][k] = f32_to_bf16(e[k]);
      part[1][k] = f32_to_bf16(e[k] - bf16_to_f32(part[0][k]));
    }
#pragma unroll
    for (int pt = 0; pt < kCenterParts; ++pt)
      *reinterpret_cast<uint2*>(bs + (pt * K + cc) * kCenterPitchB + 4 * q) =
          make_uint2(part[pt][0] | (static_cast<uint32_t>(part[pt][1]) << 16),
                     part[pt][2] | (static_cast<uint32_t>(part[pt][3]) << 16));
  }
  if (tid < kWave) {
    const bool live = tid < K && c.alive[lane_ix * K + tid];
    const uint64_t bits = __ballot(live);
    if (tid < K) {
      phi_s[tid] = c.p_hi_c[static_cast<int64_t>(lane_ix) * K + tid];
      ntot_s[tid] = c.n_total[static_cast<int64_t>(lane_ix) * K + tid];
    }
    if (tid == 0) alive_s = static_cast<uint32_t>(bits);
  }
  __syncthreads();
  // Canonical squared norms of the centers (leaf l: features l and l + 64).
  for (int cc = w; cc < K; cc += kAttachMfmaWaves) {
    const float a = mf[cc * kCenterPitchF + l], a2 = mf[cc * kCenterPitchF + l + 64];
    const float s = wave_tree(a * a + a2 * a2);
    if (l == 0) {
      mm_s[cc] = s;
      sm_s[cc] = __builtin_amdgcn_sqrtf(s);
    }
  }
  __syncthreads();
  bool lane_ok = true;
  for (int cc = 0; cc < K; ++cc) lane_ok = lane_ok && mm_s[cc] <= 0x1p60f;
  const uint32_t alive_bits = alive_s;
  const uint32_t all_bits = K >= 32 ? 0xffffffffu : ((1u << K) - 1u);
  const bool any_alive = alive_bits != 0;
  const bool any_free = alive_bits != all_bits;
  const bool capped = prm.hard_cap > 0.f;
  const float radius = prm.lam * c.s_h[lane_ix];
  const float inf = __builtin_inff();
  float* t0 = tw + w * 2 * 32 * tp;   // d~, then the winner screen's lower bounds
  float* t1 = t0 + 32 * tp;           // the nearest screen's lower bounds
  const int rr = l & 31, h = l >> 5;
  const int colc = rr < K ? rr : K - 1;
  const LOGKV_G uint16_t* kbase = gp(r.k + b * r.k_sb + g * r.k_sg) + 8 * h;
  const int tiles = (r.tokens + 31) / 32;
  for (int it = 0; it < tiles_per_wave; ++it) {
    const int tile = (static_cast<int>(blockIdx.x) * tiles_per_wave + it) * kAttachMfmaWaves + w;
    if (tile >= tiles) break;
    const int s = tile * 32 + rr;
    const bool valid = s < n;
    int64_t pos = 0;
    uint4 xq[8];
    if (valid) {
      const int t = order[static_cast<int64_t>(b) * r.tokens + s];
      pos = r.pos[b * r.pos_sb + t];
      const LOGKV_G uint16_t* row = kbase + static_cast<int64_t>(t) * r.k_st;
#pragma unroll
      for (int j = 0; j < 8; ++j) xq[j] = *reinterpret_cast<const LOGKV_G uint4*>(row + 16 * j);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) xq[j] = make_uint4(0u, 0u, 0u, 0u);
    }
    // Screened dot products (parts accumulated smallest first).
    att_f32x16 acc = {};
#pragma unroll
    for (int pt = kCenterParts - 1; pt >= 0; --pt) {
      const uint16_t* bp = bs + (pt * K + colc) * kCenterPitchB + 8 * h;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        uint4 bq = *reinterpret_cast<const uint4*>(bp + 16 * ks);
        if (rr >= K) bq = make_uint4(0u, 0u, 0u, 0u);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(att_bf16x8, xq[ks]),
                                                      __builtin_bit_cast(att_bf16x8, bq), acc, 0, 0, 0);
      }
    }
    if (rr < K) {
#pragma unroll
      for (int i = 0; i < 16; ++i) t0[(8 * (i >> 2) + 4 * h + (i & 3)) * tp + rr] = acc[i];
    }
    const float xx = pair_tree<0>(xq, nullptr, h);
    wave_lds_sync();
    if (valid) {
      float* d0 = t0 + rr * tp;
      float* d1 = t1 + rr * tp;
      bool ok = lane_ok && xx <= 0x1p60f;
      const float sx = __builtin_amdgcn_sqrtf(xx);
      float U = inf, Un = inf;
      for (int cc = h; cc < K; cc += 2) {
        if (!((alive_bits >> cc) & 1u)) continue;
        const float mmc = mm_s[cc];
        const float v = (xx + mmc) - 2.0f * d0[cc];
        const int64_t gi = pos - phi_s[cc];
        const float gap = static_cast<float>(gi > 0 ? gi : 0);
        const float tq = prm.eta * (gap * __builtin_amdgcn_rcpf(gap + prm.g0));
        const float cost = fmaxf(v, 0.f) + tq;
        const float dw = 0x1p-11f * ((sx * sm_s[cc] + fabsf(v)) + fabsf(tq)) + 0x1p-80f;
        const float dn = 0x1p-11f * ((xx + mmc) + fabsf(v)) + 0x1p-80f;
        ok = ok && fabsf(cost) <= 0x1p100f && dw <= 0x1p100f;
        U = fminf(U, cost + dw);
        Un = fminf(Un, v + dn);
        d0[cc] = cost - dw;
        d1[cc] = v - dn;
      }
      U = pair_min(U);
      Un = pair_min(Un);
      ok = pair_or(ok ? 0u : 1u) == 0u;
      uint32_t sw = all_bits, sn = alive_bits;
      if (ok) {
        sw = 0u;
        sn = 0u;
        for (int cc = h; cc < K; cc += 2) {
          if (!((alive_bits >> cc) & 1u)) continue;
          if (d0[cc] <= U) sw |= 1u << cc;
          if (d1[cc] <= Un) sn |= 1u << cc;
        }
        sw = pair_or(sw);
        sn = pair_or(sn);
        if (sw == 0u) sw = 1u;   // no live cluster: the winner stays cluster 0
      }
      // Canonical costs of the candidates, in cluster order as attach_kernel.
      float best = inf, s_winner = 0.f;
      int winner = 0;
      for (uint32_t m = sw; m; m &= m - 1u) {
        const int cc = __builtin_ctz(m);
        keep_packed(xq);
        const float dot = pair_tree<1>(xq, mf + cc * kCenterPitchF, h);
        const float semantic = fmaxf((xx + mm_s[cc]) - 2.0f * dot, 0.0f);
        if (cc == 0) s_winner = semantic;
        if ((alive_bits >> cc) & 1u) {
          const int64_t gi = pos - phi_s[cc];
          const float gap = static_cast<float>(gi > 0 ? gi : 0);
          const float cost = semantic + prm.eta * (gap / (gap + prm.g0));
          if (cost < best) {
            best = cost;
            winner = cc;
            s_winner = semantic;
          }
        }
      }
      bool direct = any_alive && (s_winner <= radius);
      if (capped) direct = direct && static_cast<float>(ntot_s[winner] + 1) <= prm.hard_cap;
      int out;
      if (!any_free && !capped) {
        out = winner;
        if (!direct) {
          int nearest = 0;
          if (ok && __popc(sn) == 1) {
            nearest = __builtin_ctz(sn);
          } else {
            float best_e = inf;
            for (uint32_t m = sn; m; m &= m - 1u) {
              const int cc = __builtin_ctz(m);
              keep_packed(xq);
              const float ex = pair_tree<2>(xq, mf + cc * kCenterPitchF, h);
              if (ex < best_e) {
                best_e = ex;
                nearest = cc;
              }
            }
          }
          out = nearest;
        }
      } else {
        out = direct ? winner : -1;
      }
      if (h == 0) {
        assign[static_cast<int64_t>(lane_ix) * r.tokens + s] = static_cast<int8_t>(out);
        if (any_free || capped) s_win[static_cast<int64_t>(lane_ix) * r.tokens + s] = s_winner;
      }
    } else if (h == 0 && s < r.tokens) {
      assign[static_cast<int64_t>(lane_ix) * r.tokens + s] = -1;   // padding rows of the lane
    }
    wave_lds_sync();
  }
}

// Canonical squared distance between a row (held in x[]) and another bf16 row.
__device__ __forceinline__ float row_d2_bf16(const float* x, const uint16_t* other, int D, int J) {
  const int l = lane_id();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxDim / kWave; ++j) {
    if (j < J) {
      const int d = l + j * kWave;
      const float diff = d < D ? x[j] - bf16_to_f32(other[d]) : 0.f;
      s = j == 0 ? diff * diff : s + diff * diff;
    }
  }
  return wave_sum0(s);
}

// Block-wide argmax (first index on ties) of (value, index) pairs.
__device__ __forceinline__ void block_argmax(float& v, int& i, float* sv, int* si) {
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, kWave);
    const int oi = __shfl_xor(i, off, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
  const int w = wave_id(), nw = blockDim.x / kWave;
  __syncthreads();
  if (lane_id() == 0) {
    sv[w] = v;
    si[w] = i;
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
  for (int k = 1; k < nw; ++k)
    if (sv[k] > v || (sv[k] == v && si[k] < i)) {
      v = sv[k];
      i = si[k];
    }
  __syncthreads();
}

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off, kWave);
    v = o < v ? o : v;
  }
  return v;
}

// ---------------------------------------------------------------------------
// Seeds for lanes with free cluster slots (one block per lane), then the
// orphans' clusters.
//
// CAPPED (a capacity cap, litgpt/log_kv_cache.py:4497-4516, :4734-4822): the
// lane's decisions are kept in LDS. First every cluster keeps its first
// max(0, cap - n_total) direct rows in offset order and the rest become
// orphans; after the seeds, each remaining orphan in position order takes the
// nearest candidate cluster that still has room (room = cap - n_total - the
// rows it already took: its kept direct rows, or 1 for a seeded slot), or the
// nearest candidate when none has room. The distances go to `cap_dist` in
// orphan order, then one wave walks them in chunks staged through LDS.
// ---------------------------------------------------------------------------
template <bool CAPPED>
__global__ __launch_bounds__(1024) void seed_kernel(LadderArgs c, RowsArgs r, RouteParams prm,
                                                    const int32_t* __restrict__ order, int8_t* __restrict__ assign,
                                                    const float* __restrict__ s_win, float* __restrict__ dist,
                                                    float* __restrict__ cap_dist) {
  __shared__ float cand_s[kMaxClusters * kMaxDim];
  __shared__ float red_v[16];
  __shared__ int red_i[16];
  __shared__ int picks_s[kMaxClusters];
  __shared__ int free_s[kMaxClusters];
  __shared__ int kept_s[kMaxClusters];
  __shared__ int n_orphan_s;
  __shared__ int8_t as_l[CAPPED ? kMaxOrderRows : 1];
  __shared__ int16_t idx_l[CAPPED ? kMaxOrderRows : 1];
  const int lane_ix = blockIdx.x;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  const int K = c.k_max, D = c.dk, J = (D + kWave - 1) / kWave;
  const int n = valid_rows(r, b);
  const int tid = static_cast<int>(threadIdx.x), nthr = static_cast<int>(blockDim.x);
  const int l = lane_id(), w = wave_id(), nw = nthr / kWave;
  int n_free = 0;
  for (int cc = 0; cc < K; ++cc)
    if (!c.alive[lane_ix * K + cc]) {
      if (tid == 0) free_s[n_free] = cc;
      ++n_free;
    }
  if ((!CAPPED && n_free == 0) || n == 0) return;
  int8_t* as_g = assign + static_cast<int64_t>(lane_ix) * r.tokens;
  int8_t* as = CAPPED ? as_l : as_g;
  const float* sw = s_win + static_cast<int64_t>(lane_ix) * r.tokens;
  const int32_t* ord = order + static_cast<int64_t>(b) * r.tokens;
  const uint16_t* kbase = r.k + b * r.k_sb + g * r.k_sg;
  const int32_t* ntot = c.n_total + static_cast<int64_t>(lane_ix) * K;
  if constexpr (CAPPED) {
    // idx_l: position-order index of each offset (the lane's rows 0..n-1 are
    // a permutation of the first n offsets).
    for (int s = tid; s < n; s += nthr) {
      as_l[s] = as_g[s];
      idx_l[s] = -1;
    }
    __syncthreads();
    for (int s = tid; s < n; s += nthr) {
      const int o = ord[s];
      if (o >= 0 && o < n) idx_l[o] = static_cast<int16_t>(s);
    }
    __syncthreads();
    if (w == 0) {
      const int room = l < K ? max(0, prm.hard_cap_rows - ntot[l]) : 0;
      const uint64_t below = (1ull << l) - 1ull;
      int run = 0;   // lane cc: direct rows of cluster cc met so far, in offset order
      for (int t0 = 0; t0 < n; t0 += kWave) {
        const int t = t0 + l;
        const int s = t < n ? idx_l[t] : -1;
        const int a = s >= 0 && s < n ? as_l[s] : -1;
        bool demote = false;
        for (int cc = 0; cc < K; ++cc) {
          const uint64_t m = __ballot(a == cc);
          if (m == 0) continue;
          const int base = __shfl(run, cc, kWave), room_cc = __shfl(room, cc, kWave);
          if (a == cc) demote = base + __popcll(m & below) >= room_cc;
          if (l == cc) run += __popcll(m);
        }
        if (demote) as_l[s] = -1;
      }
      if (l < K) kept_s[l] = min(run, room);
    }
  }
  if (tid == 0) n_orphan_s = 0;
  __syncthreads();
  int mine = 0;
  float v = -__builtin_inff();
  int vi = 0x7fffffff;
  for (int s = tid; s < n; s += nthr) {
    if (as[s] < 0) {
      ++mine;
      const float val = sw[s];
      if (val > v || (val == v && s < vi)) {
        v = val;
        vi = s;
      }
    }
  }
  atomicAdd(&n_orphan_s, mine);
  __syncthreads();
  const int n_orphan = n_orphan_s;
  if (n_orphan == 0) {
    if constexpr (CAPPED)
      for (int s = tid; s < n; s += nthr) as_g[s] = as_l[s];
    return;
  }
  int n_use = n_free < n_orphan ? n_free : n_orphan;
  block_argmax(v, vi, red_v, red_i);
  int pick = vi;
  // Every pick is an unpicked orphan with a finite score while n_use <= orphans;
  // a non-finite score (NaN keys) could leave no valid index: seed fewer then.
  if (n_use > 0 && (pick < 0 || pick >= n)) {
    if constexpr (!CAPPED) return;
    n_use = 0;
  }
  if (n_use > 0 && tid == 0) picks_s[0] = pick;
  // While seeding, the rows' running distances live in LDS (the candidate
  // centers take the space afterwards); a wave takes kSeedRows rows at a time,
  // their loads issued together, and holds the pick row in registers.
  float* ds_l = cand_s;
  constexpr int kSeedRows = 4, JM = kMaxDim / kWave;
  for (int step = 0; step + 1 < n_use; ++step) {
    // dist = min(dist, d2(., pick)), with the pick itself masked; argmax -> next pick.
    const uint16_t* prow = kbase + static_cast<int64_t>(ord[pick]) * r.k_st;
    float xp[JM];
#pragma unroll
    for (int j = 0; j < JM; ++j) xp[j] = feat_or_zero(gp(prow), l + j * kWave, D);
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    for (int s0 = w * kSeedRows; s0 < n; s0 += nw * kSeedRows) {
      float x[kSeedRows][JM];
#pragma unroll
      for (int u = 0; u < kSeedRows; ++u) {
        const uint16_t* row = kbase + static_cast<int64_t>(ord[min(s0 + u, n - 1)]) * r.k_st;
#pragma unroll
        for (int j = 0; j < JM; ++j) x[u][j] = feat_or_zero(gp(row), l + j * kWave, D);
      }
#pragma unroll
      for (int u = 0; u < kSeedRows; ++u) {
        const int s = s0 + u;
        if (s >= n) break;
        float e = 0.f;
#pragma unroll
        for (int j = 0; j < JM; ++j) {
          if (j < J) {
            const float diff = l + j * kWave < D ? x[u][j] - xp[j] : 0.f;
            e = j == 0 ? diff * diff : e + diff * diff;
          }
        }
        const float d2 = wave_sum0(e);
        float val;
        if (step == 0) val = as[s] < 0 ? d2 : -__builtin_inff();
        else val = fminf(ds_l[s], d2);
        if (s == pick) val = -__builtin_inff();
        if (l == 0) ds_l[s] = val;
        if (val > bv || (val == bv && s < bi)) {
          bv = val;
          bi = s;
        }
      }
    }
    block_argmax(bv, bi, red_v, red_i);
    if (bi < 0 || bi >= n) {
      n_use = step + 1;
      break;
    }
    pick = bi;
    if (tid == 0) picks_s[step + 1] = pick;
    __syncthreads();
  }
  __syncthreads();
  // Candidate centers: live centroids, seed rows at the free slots.
  const float* mu = c.centroid + static_cast<int64_t>(lane_ix) * K * D;
  for (int i = tid; i < K * D; i += nthr) cand_s[i] = mu[i];
  __syncthreads();
  for (int i = tid; i < n_use * D; i += nthr) {
    const int k = i / D, d = i % D;
    const uint16_t* row = kbase + static_cast<int64_t>(ord[picks_s[k]]) * r.k_st;
    cand_s[free_s[k] * D + d] = bf16_to_f32(row[d]);
  }
  __syncthreads();
  uint32_t cand_bits = 0;
  for (int cc = 0; cc < K; ++cc) cand_bits |= (c.alive[lane_ix * K + cc] ? 1u : 0u) << cc;
  for (int k = 0; k < n_use; ++k) cand_bits |= 1u << free_s[k];
  if constexpr (!CAPPED) {
    // Every orphan's nearest candidate, kSeedRows rows of a wave at a time.
    for (int s0 = w * kSeedRows; s0 < n; s0 += nw * kSeedRows) {
      float x[kSeedRows][JM];
      bool orphan[kSeedRows];
#pragma unroll
      for (int u = 0; u < kSeedRows; ++u) {
        orphan[u] = s0 + u < n && as[s0 + u] < 0;
        const uint16_t* row = kbase + static_cast<int64_t>(ord[min(s0 + u, n - 1)]) * r.k_st;
#pragma unroll
        for (int j = 0; j < JM; ++j) x[u][j] = orphan[u] ? feat_or_zero(gp(row), l + j * kWave, D) : 0.f;
      }
      float best[kSeedRows];
      int arg[kSeedRows];
#pragma unroll
      for (int u = 0; u < kSeedRows; ++u) {
        best[u] = __builtin_inff();
        arg[u] = 0;
      }
      for (int cc = 0; cc < K; ++cc) {
        float cj[JM];
#pragma unroll
        for (int j = 0; j < JM; ++j) cj[j] = j < J && l + j * kWave < D ? cand_s[cc * D + l + j * kWave] : 0.f;
        const bool cand = (cand_bits >> cc) & 1u;
#pragma unroll
        for (int u = 0; u < kSeedRows; ++u) {
          float e = 0.f;
#pragma unroll
          for (int j = 0; j < JM; ++j) {
            if (j < J) {
              const float diff = l + j * kWave < D ? x[u][j] - cj[j] : 0.f;
              e = j == 0 ? diff * diff : e + diff * diff;
            }
          }
          e = wave_sum0(e);
          if (cand && e < best[u]) {
            best[u] = e;
            arg[u] = cc;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kSeedRows; ++u)
        if (orphan[u] && l == 0) as[s0 + u] = static_cast<int8_t>(arg[u]);
    }
    __syncthreads();
    if (tid < n_use) as[picks_s[tid]] = static_cast<int8_t>(free_s[tid]);
  } else {
    // Seeds open their slots; the remaining orphans in position order -> idx_l.
    if (tid < n_use) as_l[picks_s[tid]] = static_cast<int8_t>(free_s[tid]);
    __syncthreads();
    __shared__ int n_rest_s;
    if (w == 0) {
      int count = 0;
      for (int s0 = 0; s0 < n; s0 += kWave) {
        const bool orphan = s0 + l < n && as_l[s0 + l] < 0;
        const uint64_t m = __ballot(orphan);
        if (orphan) idx_l[count + __popcll(m & ((1ull << l) - 1ull))] = static_cast<int16_t>(s0 + l);
        count += __popcll(m);
      }
      if (l == 0) n_rest_s = count;
    }
    __syncthreads();
    const int n_rest = n_rest_s;
    float* cd = cap_dist + static_cast<int64_t>(lane_ix) * r.tokens * K;
    for (int i = w; i < n_rest; i += nw) {
      const int s = idx_l[i];
      float x[kMaxDim / kWave];
      const uint16_t* row = kbase + static_cast<int64_t>(ord[s]) * r.k_st;
#pragma unroll
      for (int j = 0; j < kMaxDim / kWave; ++j) {
        const int d = l + j * kWave;
        x[j] = feat_or_zero(gp(row), d, D);
      }
      for (int cc = 0; cc < K; ++cc) {
        float e = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxDim / kWave; ++j) {
          if (j < J) {
            const int d = l + j * kWave;
            const float diff = d < D ? x[j] - cand_s[cc * D + d] : 0.f;
            e = j == 0 ? diff * diff : e + diff * diff;
          }
        }
        e = wave_sum0(e);
        if (l == 0) cd[static_cast<int64_t>(i) * K + cc] = ((cand_bits >> cc) & 1u) ? e : __builtin_inff();
      }
    }
    __threadfence();
    __syncthreads();
    // Rooms, in lane cc of the walking wave.
    int room = 0;
    if (l < K && ((cand_bits >> l) & 1u)) {
      bool seeded = false;
      for (int k = 0; k < n_use; ++k) seeded |= free_s[k] == l;
      room = max(0, prm.hard_cap_rows - ntot[l] - (seeded ? 1 : kept_s[l]));
    }
    const int chunk = (kMaxClusters * kMaxDim) / K;
    for (int i0 = 0; i0 < n_rest; i0 += chunk) {
      const int rows = min(chunk, n_rest - i0);
      for (int e = tid; e < rows * K; e += nthr) cand_s[e] = cd[static_cast<int64_t>(i0) * K + e];
      __syncthreads();
      if (w == 0) {
        for (int i = 0; i < rows; ++i) {
          const float e = l < K ? cand_s[i * K + l] : __builtin_inff();
          const uint64_t key = (static_cast<uint64_t>(__float_as_uint(e)) << 32) | static_cast<uint32_t>(l);
          uint64_t best = wave_min_u64(l < K && room > 0 ? key : ~0ull);
          // Every cluster full: the nearest one (litgpt/log_kv_cache.py:4816-4819).
          if (best == ~0ull) best = wave_min_u64(l < K ? key : ~0ull);
          const int chosen = static_cast<int>(best & 0xffffffffu);
          if (l == chosen) --room;
          if (l == 0) as_l[idx_l[i0 + i]] = static_cast<int8_t>(chosen);
        }
      }
      __syncthreads();
    }
    for (int s = tid; s < n; s += nthr) as_g[s] = as_l[s];
  }
}

int launch_order(const RowsArgs& r, int n_batch, int32_t* order, int32_t* clear, hipStream_t stream, int n_clear) {
  hipLaunchKernelGGL(order_kernel, dim3(n_batch), dim3(1024), 0, stream, r.pos, r.pos_sb, r.counts, r.tokens, order,
                     clear, n_clear);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_route(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                 hipStream_t stream) {
  const int lanes = c.n_batch * c.n_groups;
  hipLaunchKernelGGL(order_kernel, dim3(c.n_batch), dim3(1024), 0, stream, r.pos, r.pos_sb, r.counts, r.tokens,
                     ws.order, static_cast<int32_t*>(nullptr), 0);
  if (r.tokens > 0) {
    const int nj = (c.dk + kWave - 1) / kWave;
    auto attach = [&](auto kernel, int tile, size_t shmem) {
      if (!allow_dynamic_lds(reinterpret_cast<const void*>(kernel), shmem)) return false;
      // One thread per (row, cluster) pair of a tile where it fits.
      const int threads = std::min(kAttachMaxThreads, std::max(256, (tile * c.k_max + kWave - 1) / kWave * kWave));
      hipLaunchKernelGGL(kernel, dim3((r.tokens + tile - 1) / tile, lanes), dim3(threads), shmem, stream, c, r, p,
                         ws.order, ws.assign, ws.s_win);
      return true;
    };
    // 128-feature rows that allow 16-byte loads take the matrix-core screen.
    const bool aligned16 = (reinterpret_cast<uintptr_t>(r.k) & 15u) == 0 && r.k_sb % 8 == 0 && r.k_sg % 8 == 0 &&
                           r.k_st % 8 == 0;
    bool ok;
    if (c.dk == 128 && c.k_max >= 1 && aligned16) {
      const size_t shmem = attach_mfma_shmem(c.k_max);
      ok = allow_dynamic_lds(reinterpret_cast<const void*>(attach_mfma_kernel), shmem);
      if (ok) {
        const int tiles = (r.tokens + 31) / 32;
        // Two tiles per wave share a block's staged centers; a small launch takes one, for more blocks.
        const int tpw = static_cast<int64_t>(tiles) * lanes >= 4096 ? kAttachTilesPerWave : 1;
        const int per_block = kAttachMfmaWaves * tpw;
        hipLaunchKernelGGL(attach_mfma_kernel, dim3((tiles + per_block - 1) / per_block, lanes),
                           dim3(kAttachMfmaWaves * kWave), shmem, stream, c, r, p, ws.order, ws.assign, ws.s_win, tpw);
      }
    } else if (nj == 1) ok = attach(attach_kernel<1>, attach_tile<1>(), attach_shmem<1>(c.k_max));
    else if (nj == 2) ok = attach(attach_kernel<2>, attach_tile<2>(), attach_shmem<2>(c.k_max));
    else if (nj == 3) ok = attach(attach_kernel<3>, attach_tile<3>(), attach_shmem<3>(c.k_max));
    else ok = attach(attach_kernel<4>, attach_tile<4>(), attach_shmem<4>(c.k_max));
    if (!ok) return LOGKV_ERUNTIME;
    if (p.hard_cap > 0.f)
      hipLaunchKernelGGL(seed_kernel<true>, dim3(lanes), dim3(1024), 0, stream, c, r, p, ws.order, ws.assign,
                         ws.s_win, ws.dist, ws.cap_dist);
    else
      hipLaunchKernelGGL(seed_kernel<false>, dim3(lanes), dim3(1024), 0, stream, c, r, p, ws.order, ws.assign,
                         ws.s_win, ws.dist, static_cast<float*>(nullptr));
  }
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
