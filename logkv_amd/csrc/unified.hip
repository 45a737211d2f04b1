// Unified (Ward / radius) route on the device.
//
// Follows litgpt/log_kv_cache.py:3589-3688 (the route), :448-637 (the
// incremental mutual-nearest rounds of _UnifiedReduceTorch and the Triton
// UnifiedReduce, litgpt/log_kv_route_triton.py:197-838), :3544-3568 (labels),
// docs/semantic-unified-routing.md:11-96. Per lane (batch row, KV group):
//   1. candidates: the flushed rows start as singletons and merge in mutual-
//      nearest Ward pairs while the radius bound stays under sqrt(lambda s_h);
//   2. budget: old live clusters and candidates merge until at most K remain;
//   3. old-old merges (ladder re-appends, in ladder.hip) and the commit of the
//      rows into their final clusters (the attach commit).
// A round's plan runs on one workgroup per lane with the per-row state (cached
// row minima, masses, radii, flags, pair table) in LDS; its Lance-Williams
// updates and rescans, which read and write the squared distance matrix in
// HBM, run on many workgroups per lane; the state passes between the launches
// through a per-lane global image, and no launch waits on the host. Every element operation keeps
// the reference's float32 order (_unified_pair_cost, _merge); the initial
// squared distances and the radius check's exact distances are canonical
// wave sums of squared differences (common.hpp).
#include <vector>

#include "route.hpp"
#include "unified.hpp"

namespace logkv {

namespace {

constexpr int kReduceThreads = 1024;
constexpr int kReduceWaves = kReduceThreads / kWave;
constexpr uint64_t kInfKey = 0x7F800000ull << 32;
constexpr uint8_t kAlive = 1, kValid = 2, kKeep = 4, kMerged = 8, kRejected = 16, kDirty = 32;
// Frozen-center sweeps: in a pair of the round (or its partner), and the lower row of a sweep's pair.
constexpr uint8_t kMatched = 64, kSweep = 128;

__device__ __forceinline__ uint64_t pack_cost(float cost, int key) {
  const uint32_t bits = cost == 0.f ? 0u : __float_as_uint(cost);
  return (static_cast<uint64_t>(bits) << 32) | static_cast<uint32_t>(key);
}

__device__ __forceinline__ float key_cost(uint64_t k) { return __uint_as_float(static_cast<uint32_t>(k >> 32)); }

// Ward cost of merging rows of masses mi, mj at squared distance d2, +inf when
// not allowed (litgpt/log_kv_cache.py:437-445, same operation order).
template <bool LIMIT>
__device__ __forceinline__ float ward_cost(float d2, float mi, float mj, float ri, float rj, float limit,
                                           bool valid) {
  const float sum = mi + mj;
  const float denom = sum < 1.f ? 1.f : sum;
  valid = valid && mi > 0.f && mj > 0.f;
  if (LIMIT) {
    const float distance = sqrtf(d2);
    const float x = ri + (mj / denom) * distance, y = rj + (mi / denom) * distance;
    valid = valid && (x < y ? y : x) <= limit;
  }
  return valid ? d2 * (mi * mj / denom) : __builtin_inff();
}

// Screening form of ward_cost: the quotients from v_rcp_f32 and the distance
// from v_sqrt_f32 (each within 1 ulp), so a finite result is within 2^-20
// (relative) of ward_cost's, and +inf means the pair is certainly not allowed.
// `border` is set for an allowed-looking pair whose radius test lies within
// 2^-16 of the limit, or whose d2 is below 2^-96 (where v_sqrt_f32 and the
// relative bound do not hold): only ward_cost decides those. A result of 0
// is +0.
template <bool LIMIT>
__device__ __forceinline__ float screen_cost(float d2, float mi, float mj, float ri, float rj, float limit, bool valid,
                                             bool& border) {
  const float sum = mi + mj;
  const float denom = sum < 1.f ? 1.f : sum;
  valid = valid && mi > 0.f && mj > 0.f;
  const float inv = __builtin_amdgcn_rcpf(denom);
  bool near_edge = d2 < 0x1p-96f;
  if (LIMIT) {
    const float distance = __builtin_amdgcn_sqrtf(d2);
    const float x = ri + (mj * inv) * distance, y = rj + (mi * inv) * distance;
    const float mx = x < y ? y : x;
    const bool over = mx > limit * (1.f + 0x1p-16f);
    near_edge = near_edge || mx >= limit * (1.f - 0x1p-16f);
    valid = valid && !over;
  }
  border = valid && near_edge;
  const float c = d2 * ((mi * mj) * inv);
  return valid ? (c > 0.f ? c : 0.f) : __builtin_inff();
}

// Cut-off of the screen: a pair whose screened cost exceeds m (1 + 2^-16),
// where m is the least screened cost of a non-border pair of the same set,
// has an exact cost above that pair's exact cost, so it cannot hold the
// set's minimum key.
__device__ __forceinline__ float screen_cutoff(float m) { return m * (1.f + 0x1p-16f); }

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off, kWave);
    v = o < v ? o : v;
  }
  return v;
}

// Minimum over the 64 lanes, formed toward lane 0 with the permlane swaps and
// DPP row shifts of wave_sum0 and read from lane 0 (uniform result). Every
// lane of the wave must be active.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  auto mn = [](uint32_t x, uint32_t y) { return x < y ? x : y; };
  v = mn(v, __builtin_amdgcn_permlane32_swap(v, v, false, false)[1]);
  v = mn(v, __builtin_amdgcn_permlane16_swap(v, v, false, false)[1]);
  const int i = static_cast<int>(v);
  v = mn(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(i, i, 0x108, 0xf, 0xf, false)));  // row_shl:8
  const int j = static_cast<int>(v);
  v = mn(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(j, j, 0x104, 0xf, 0xf, false)));  // row_shl:4
  const int k = static_cast<int>(v);
  v = mn(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(k, k, 0x102, 0xf, 0xf, false)));  // row_shl:2
  const int m = static_cast<int>(v);
  v = mn(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(m, m, 0x101, 0xf, 0xf, false)));  // row_shl:1
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// Minimum packed key over the 64 lanes (uniform): the least cost bits, then
// the least low word among the lanes that hold them. Every lane must be active.
__device__ __forceinline__ uint64_t wave_min_key(uint64_t k) {
  const uint32_t hi = wave_min_u32(static_cast<uint32_t>(k >> 32));
  const uint32_t lo = wave_min_u32(static_cast<uint32_t>(k >> 32) == hi ? static_cast<uint32_t>(k) : 0xFFFFFFFFu);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

struct ReduceLds {
  uint64_t* packed;   // [M] cached row minimum: cost bits << 32 | (row ^ col)
  uint64_t* keys;     // [P2] proposals sorted by (cost, row)
  float* mass;        // [M]
  float* radius;      // [M]
  float* p_alpha;     // [M/2] per merge of the round
  float* p_beta;
  float* p_shift;
  int16_t* best;      // [M]
  int16_t* pair_of;   // [M] merge index of a kept row
  uint8_t* flags;     // [M]
};

__host__ __device__ inline int half_up(int m) { return (m + 1) / 2; }
__host__ __device__ inline int pow2_at_least(int n) {
  int w = 1;
  while (w < n) w <<= 1;
  return w;
}

__host__ __device__ inline size_t reduce_lds_bytes(int M) {
  const int H = half_up(M), P2 = pow2_at_least(H > 0 ? H : 1);
  return static_cast<size_t>(M) * 8 + static_cast<size_t>(P2) * 8 + static_cast<size_t>(M) * 8 +
         static_cast<size_t>(H) * 12 + static_cast<size_t>(M) * 5 + 64;
}

__device__ inline ReduceLds carve_lds(uint8_t* dyn, int M) {
  const int H = half_up(M), P2 = pow2_at_least(H > 0 ? H : 1);
  ReduceLds s;
  s.packed = reinterpret_cast<uint64_t*>(dyn);
  s.keys = s.packed + M;
  s.mass = reinterpret_cast<float*>(s.keys + P2);
  s.radius = s.mass + M;
  s.p_alpha = s.radius + M;
  s.p_beta = s.p_alpha + H;
  s.p_shift = s.p_beta + H;
  s.best = reinterpret_cast<int16_t*>(s.p_shift + H);
  s.pair_of = s.best + M;
  s.flags = reinterpret_cast<uint8_t*>(s.pair_of + M);
  return s;
}

// Packed minimum of row r over the live columns (litgpt/log_kv_cache.py:
// 473-488); the row's own column contributes (inf, key 0), so a row without a
// finite cost packs to the infinite key (the minimum starts there). With
// `live`, only the listed columns are visited: a dead column has mass 0, so
// its key is (inf, r ^ c) >= the infinite key and never the minimum.
template <bool LIMIT>
__device__ uint64_t scan_row(const ReduceLds& s, const float* dist, int M, int n, int r, float limit,
                             const int16_t* live = nullptr, int n_live = 0) {
  const float mr = s.mass[r], rr = s.radius[r];
  uint64_t best = kInfKey;
  const float* row = dist + static_cast<int64_t>(r) * M;
  const int end = live ? n_live : n;
  for (int idx = lane_id(); idx < end; idx += kWave) {
    const int c = live ? live[idx] : idx;
    const float cost = ward_cost<LIMIT>(row[c], mr, s.mass[c], rr, s.radius[c], limit, c != r);
    const uint64_t k = pack_cost(cost, r ^ c);
    best = k < best ? k : best;
  }
  return wave_min_u64(best);
}

// Packed minimum of row r over the columns not matched this round (a matched
// column takes mass 0, litgpt/log_kv_cache.py:473-488 with `excluded`), for
// the budget stage's frozen-center sweeps (no radius limit).
__device__ uint64_t scan_row_unmatched(const ReduceLds& s, const float* dist, int M, int n, int r) {
  const float mr = s.mass[r];
  uint64_t best = kInfKey;
  const float* row = dist + static_cast<int64_t>(r) * M;
  for (int c = lane_id(); c < n; c += kWave) {
    const float mc = (s.flags[c] & kMatched) ? 0.f : s.mass[c];
    const float cost = ward_cost<false>(row[c], mr, mc, 0.f, 0.f, 0.f, c != r);
    const uint64_t k = pack_cost(cost, r ^ c);
    best = k < best ? k : best;
  }
  return wave_min_u64(best);
}

// Partner named by a packed row minimum (the low word is row ^ col).
__device__ __forceinline__ int key_partner(uint64_t k, int r, int M) {
  const int p = static_cast<int>(static_cast<uint32_t>(k) ^ static_cast<uint32_t>(r));
  return p < 0 ? 0 : (p > M - 1 ? M - 1 : p);
}

}  // namespace

// Rows -> f32 nodes with mass 1 (rows past the lane's count: mass 0), one block per (row tile, lane).
__global__ __launch_bounds__(256) void load_nodes_kernel(RowsArgs r, int n_groups, UnifiedBufs u) {
  const int lane = blockIdx.y, b = lane / n_groups, g = lane % n_groups;
  const int n = valid_rows(r, b), M = u.M, D = u.D;
  const uint16_t* kb = r.k + b * r.k_sb + g * r.k_sg;
  float* mu = u.mu1 + static_cast<int64_t>(lane) * M * D;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < M * D; i += gridDim.x * 256) {
    const int row = i / D, d = i - row * D;
    mu[i] = row < n ? bf16_to_f32(kb[static_cast<int64_t>(row) * r.k_st + d]) : 0.f;
  }
  for (int i = blockIdx.x * 256 + threadIdx.x; i < M; i += gridDim.x * 256)
    u.mass1[static_cast<int64_t>(lane) * M + i] = i < n ? 1.f : 0.f;
  if (blockIdx.x == 0 && threadIdx.x == 0) u.count1[lane] = n;
}

// Squared distances of every pair of a lane's nodes, as the canonical wave sum
// of squared differences of the one-row-per-wave form: leaf l adds the
// squared differences of features l, l + 64, ... in order, and the 64 leaves
// fold as a halving tree (l with l + 32, then + 16, ..., + 1). Here a thread
// evaluates whole pairs: the tree depth first (the left subtree, lower leaf
// indices, before the right), which is the same sum. A block takes a tile of
// kDistRows rows x kDistCols columns (features staged in LDS, feature-major),
// a thread kDistR x kDistC pairs; every pair (i, j) with i < j < n is written
// to both (i, j) and (j, i), the diagonal is zero. Tiles wholly below the
// diagonal or past the node count return at once.
constexpr int kDistRows = 32, kDistCols = 64, kDistR = 2, kDistC = 4;
constexpr int kDistThreads = (kDistRows / kDistR) * (kDistCols / kDistC);
// Feature-major LDS rows padded so a thread's kDistR row values and kDistC
// column values of one feature are each one aligned vector read.
constexpr int kDistRowLd = kDistRows + kDistR, kDistColLd = kDistCols + kDistC;
static_assert((kDistR == 2 || kDistR == 4) && kDistC == 4, "the tile reads are float2 / float4");

template <int J>
struct DistTile {
  const float* xs;   // [64 J][kDistRowLd]
  const float* ys;   // [64 J][kDistColLd]
  int r0, c0;        // the thread's first row / column in the tile
  // Leaf 8 hi + low of every pair of the thread: sum over q < J of (x - y)^2
  // at feature leaf + 64 q, in q order. xb / yb point at feature `low` of the
  // thread's rows / columns, so the reads take compile-time offsets.
  __device__ __forceinline__ void leaf(const float* xb, const float* yb, int hi, float (&out)[kDistR * kDistC]) const {
#pragma unroll
    for (int q = 0; q < J; ++q) {
      float x[kDistR];
      if constexpr (kDistR == 4) {
        const float4 x4 = *reinterpret_cast<const float4*>(xb + (8 * hi + 64 * q) * kDistRowLd);
        x[0] = x4.x, x[1] = x4.y, x[2] = x4.z, x[3] = x4.w;
      } else {
        const float2 x2 = *reinterpret_cast<const float2*>(xb + (8 * hi + 64 * q) * kDistRowLd);
        x[0] = x2.x, x[1] = x2.y;
      }
      const float4 y4 = *reinterpret_cast<const float4*>(yb + (8 * hi + 64 * q) * kDistColLd);
      const float y[kDistC] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
      for (int r = 0; r < kDistR; ++r)
#pragma unroll
        for (int c = 0; c < kDistC; ++c) {
          const float diff = x[r] - y[c];
          out[r * kDistC + c] = q == 0 ? diff * diff : out[r * kDistC + c] + diff * diff;
        }
    }
  }
  // The 64-leaf tree, depth first: position k = 8 kk + j of the depth-first
  // order is leaf 8 bitrev3(j) + bitrev3(kk); positions are combined as a
  // binary counter (a carry folds into the pending left sibling, left + right),
  // levels 0-2 inside a group of eight positions, levels 3-5 across groups.
  __device__ __forceinline__ void tree(float (&root)[kDistR * kDistC]) const {
    constexpr int E = kDistR * kDistC;
    float s3[E], s4[E], s5[E];
    for (int kk = 0; kk < 8; ++kk) {
      const int low = ((kk & 1) << 2) | (kk & 2) | ((kk >> 2) & 1);   // bitrev3(kk)
      const float* xb = xs + low * kDistRowLd + r0;
      const float* yb = ys + low * kDistColLd + c0;
      float s0[E], s1[E], s2[E], c[E];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int hi = ((j & 1) << 2) | (j & 2) | ((j >> 2) & 1);     // bitrev3(j)
        leaf(xb, yb, hi, c);
        if ((j & 1) == 0) {
#pragma unroll
          for (int e = 0; e < E; ++e) s0[e] = c[e];
          continue;
        }
#pragma unroll
        for (int e = 0; e < E; ++e) c[e] = s0[e] + c[e];
        if ((j & 2) == 0) {
#pragma unroll
          for (int e = 0; e < E; ++e) s1[e] = c[e];
          continue;
        }
#pragma unroll
        for (int e = 0; e < E; ++e) c[e] = s1[e] + c[e];
        if ((j & 4) == 0) {
#pragma unroll
          for (int e = 0; e < E; ++e) s2[e] = c[e];
          continue;
        }
#pragma unroll
        for (int e = 0; e < E; ++e) c[e] = s2[e] + c[e];
      }
      // c: the level-3 node of this group of eight.
      if ((kk & 1) == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) s3[e] = c[e];
        continue;
      }
#pragma unroll
      for (int e = 0; e < E; ++e) c[e] = s3[e] + c[e];
      if ((kk & 2) == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) s4[e] = c[e];
        continue;
      }
#pragma unroll
      for (int e = 0; e < E; ++e) c[e] = s4[e] + c[e];
      if ((kk & 4) == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) s5[e] = c[e];
        continue;
      }
#pragma unroll
      for (int e = 0; e < E; ++e) root[e] = s5[e] + c[e];
    }
  }
};

template <int J>
__global__ __launch_bounds__(kDistThreads) void dist_kernel(const float* __restrict__ mu, const int32_t* __restrict__ count,
                                                   float* __restrict__ dist, int M, int D) {
  extern __shared__ __align__(16) float tile_s[];
  const int lane = blockIdx.z, n = count[lane];
  const int i0 = blockIdx.x * kDistRows, j0 = blockIdx.y * kDistCols;
  if (i0 >= n || j0 >= n || j0 + kDistCols - 1 < i0) return;
  const float* base = mu + static_cast<int64_t>(lane) * M * D;
  float* xs = tile_s;
  float* ys = tile_s + 64 * J * kDistRowLd;
  const int t = threadIdx.x;
  for (int e = t; e < kDistRows * 64 * J; e += kDistThreads) {
    const int r = e / (64 * J), d = e - r * (64 * J);
    xs[d * kDistRowLd + r] = i0 + r < n && d < D ? base[static_cast<int64_t>(i0 + r) * D + d] : 0.f;
  }
  for (int e = t; e < kDistCols * 64 * J; e += kDistThreads) {
    const int c = e / (64 * J), d = e - c * (64 * J);
    ys[d * kDistColLd + c] = j0 + c < n && d < D ? base[static_cast<int64_t>(j0 + c) * D + d] : 0.f;
  }
  __syncthreads();
  const int tr = t / (kDistCols / kDistC), tc = t % (kDistCols / kDistC);
  const DistTile<J> tl{xs, ys, kDistR * tr, kDistC * tc};
  float v[kDistR * kDistC];
  tl.tree(v);
  float* dl = dist + static_cast<int64_t>(lane) * M * M;
#pragma unroll
  for (int r = 0; r < kDistR; ++r) {
    const int i = i0 + kDistR * tr + r;
#pragma unroll
    for (int c = 0; c < kDistC; ++c) {
      const int j = j0 + kDistC * tc + c;
      if (i < n && j < n && j > i) {
        dl[static_cast<int64_t>(i) * M + j] = v[r * kDistC + c];
        dl[static_cast<int64_t>(j) * M + i] = v[r * kDistC + c];
      } else if (i < n && j == i) {
        dl[static_cast<int64_t>(i) * M + i] = 0.f;
      }
    }
  }
}

size_t dist_lds_bytes(int D) {
  const int J = (D + 63) / 64;
  return static_cast<size_t>(64) * J * (kDistRowLd + kDistColLd) * 4;
}

int launch_dist(const float* mu, const int32_t* count, float* dist, int M, int D, int lanes, hipStream_t stream) {
  const dim3 grid((M + kDistRows - 1) / kDistRows, (M + kDistCols - 1) / kDistCols, lanes);
  const size_t lds = dist_lds_bytes(D);
  const int J = (D + 63) / 64;
  const void* fn = J == 1 ? reinterpret_cast<const void*>(&dist_kernel<1>)
                 : J == 2 ? reinterpret_cast<const void*>(&dist_kernel<2>)
                 : J == 3 ? reinterpret_cast<const void*>(&dist_kernel<3>)
                          : reinterpret_cast<const void*>(&dist_kernel<4>);
  if (!allow_dynamic_lds(fn, lds)) return LOGKV_ERUNTIME;
  if (J == 1) hipLaunchKernelGGL(dist_kernel<1>, grid, dim3(kDistThreads), lds, stream, mu, count, dist, M, D);
  else if (J == 2) hipLaunchKernelGGL(dist_kernel<2>, grid, dim3(kDistThreads), lds, stream, mu, count, dist, M, D);
  else if (J == 3) hipLaunchKernelGGL(dist_kernel<3>, grid, dim3(kDistThreads), lds, stream, mu, count, dist, M, D);
  else hipLaunchKernelGGL(dist_kernel<4>, grid, dim3(kDistThreads), lds, stream, mu, count, dist, M, D);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

// ---------------------------------------------------------------------------
// One stage's rounds (litgpt/log_kv_cache.py:490-637). A round is three
// phases: the plan (proposals, exact radius check, the stable sort by cost,
// merges of masses, radii and centers), one block per lane with the lane's row
// state in LDS; the Lance-Williams rows of the kept rows with their cost
// pushes, and the rescans of the rows whose partner merged or whose proposal
// was rejected, both spread over many blocks per lane. Between launches the
// row state lives in a per-lane global image with the LDS layout. A fixed
// number of rounds is enqueued (a finished lane's launches return at once);
// the finish kernel runs any rounds left on one block per lane, so nothing
// waits on the host. Every element operation is the one-block reducer's.

constexpr int kPhaseThreads = 256;
constexpr int kPhaseWaves = kPhaseThreads / kWave;
constexpr int kPhaseBlocks = 64;      // blocks per lane of the Lance-Williams / rescan phases
// Rounds enqueued as phase launches before the finish kernel: the radius
// stage of a 4096-row flush of clustered keys ends in about 20 rounds, the
// budget stage in 40 to 50 (an idle round still costs its three launches; a
// tail round on the finish kernel's one block costs about what a pipelined
// round of that size does).
constexpr int kPipelinedRounds[2] = {40, 24};   // [LIMIT]

__device__ inline ReduceLds image_of(const ReduceArgs& a, int lane) {
  return carve_lds(a.image + static_cast<int64_t>(lane) * a.image_stride, a.M);
}

// Proposals .. merges of one round on state `s` (the block's LDS). Returns the
// round's merge count; sh[0] = count, sh[1] = ntrace on entry and exit.
// Frozen-center sweeps of a budget round (litgpt/log_kv_cache.py:561-588),
// after the round's mutual proposals (kValid): the proposals and their
// partners are matched; per pass, the unmatched rows whose restricted partner
// is matched rescan the unmatched columns (restricted minima in
// a.restricted, starting as the cached ones, which stay untouched), then the
// unmatched rows whose restricted minima name each other (finite) pair up:
// the lower row takes kValid | kSweep and its mate in pair_of. Up to
// passes - 1 passes; a pass that adds no pair ends them (a later pass would
// rescan nothing). Every row's mate is left in pair_of (its cached partner
// unless a sweep paired it). Returns the pairs added; *scans gets the rows
// rescanned.
__device__ int frozen_sweeps(const ReduceLds& s, const ReduceArgs& a, int lane, int n, int* scans) {
  __shared__ int s_added, s_scans;
  const int M = a.M, t = threadIdx.x, l = lane_id(), w = wave_id();
  const float* dist = a.dist + static_cast<int64_t>(lane) * M * M;
  uint64_t* restricted = a.restricted + static_cast<int64_t>(lane) * M;
  for (int r = t; r < n; r += kReduceThreads) {
    restricted[r] = s.packed[r];
    s.pair_of[r] = s.best[r];
    if (s.flags[r] & kValid) {
      s.flags[r] |= kMatched;
      s.flags[s.best[r]] |= kMatched;
    }
  }
  if (t == 0) {
    s_added = 0;
    s_scans = 0;
  }
  __syncthreads();
  int total = 0;
  for (int pass = 1; pass < a.passes; ++pass) {
    for (int r = w; r < n; r += kReduceWaves) {
      const uint8_t fl = s.flags[r];
      if (!(fl & kAlive) || (fl & kMatched)) continue;
      if (!(s.flags[key_partner(restricted[r], r, M)] & kMatched)) continue;
      const uint64_t k = scan_row_unmatched(s, dist, M, n, r);
      if (l == 0) {
        restricted[r] = k;
        atomicAdd(&s_scans, 1);
      }
    }
    __syncthreads();
    for (int r = t; r < n; r += kReduceThreads) {
      const uint8_t fl = s.flags[r];
      if (!(fl & kAlive) || (fl & kMatched)) continue;
      const uint64_t k = restricted[r];
      const int p = key_partner(k, r, M);
      if (r < p && key_partner(restricted[p], p, M) == r && key_cost(k) < __builtin_inff() &&
          !(s.flags[p] & kMatched))
        s.flags[r] = fl | kSweep;
    }
    __syncthreads();
    for (int r = t; r < n; r += kReduceThreads) {
      const uint8_t fl = s.flags[r];
      if ((fl & kSweep) && !(fl & kMatched)) {
        const int p = key_partner(restricted[r], r, M);
        s.flags[r] = fl | kMatched | kValid;
        s.flags[p] |= kMatched;
        s.pair_of[r] = static_cast<int16_t>(p);
        atomicAdd(&s_added, 1);
      }
    }
    __syncthreads();
    const int added = s_added - total;
    total = s_added;
    __syncthreads();
    if (added == 0) break;
  }
  *scans = s_scans;
  __syncthreads();
  return total;
}

template <bool LIMIT>
__device__ void plan_phase(const ReduceLds& s, const ReduceArgs& a, int lane, int n, float limit, int* sh,
                           int* s_nprop, int* s_nvalid, int& nprop_out, int& n_ok_out, int& sweep_scans) {
  const int M = a.M, D = a.D, t = threadIdx.x, l = lane_id(), w = wave_id();
  float* dist = a.dist + static_cast<int64_t>(lane) * M * M;
  float* mu = a.mu + static_cast<int64_t>(lane) * M * D;
  int32_t* trace = a.trace + static_cast<int64_t>(lane) * M * 2;
  for (int i = t; i < M; i += kReduceThreads) s.flags[i] &= kAlive;
  // Proposals: every row's cached partner; a pair is proposed by its lower row.
  for (int r = t; r < M; r += kReduceThreads) {
    int bst = static_cast<int>(static_cast<uint32_t>(s.packed[r]) ^ static_cast<uint32_t>(r));
    bst = bst < 0 ? 0 : (bst > M - 1 ? M - 1 : bst);
    s.best[r] = static_cast<int16_t>(bst);
  }
  if (t == 0) {
    *s_nprop = 0;
    *s_nvalid = 0;
  }
  __syncthreads();
  int mine = 0;
  for (int r = t; r < n; r += kReduceThreads) {
    const int bst = s.best[r];
    const bool v = (s.flags[r] & kAlive) && r < bst && s.best[bst] == r && key_cost(s.packed[r]) < __builtin_inff();
    if (v) {
      s.flags[r] |= kValid;
      ++mine;
    }
  }
  if (mine) atomicAdd(s_nprop, mine);
  __syncthreads();
  const int nprop = *s_nprop;
  if (LIMIT) {
    // Exact radius check of every proposal (litgpt/log_kv_cache.py:503-525).
    for (int r = w; r < n; r += kReduceWaves) {
      if (!(s.flags[r] & kValid)) continue;
      const int o = s.best[r];
      const float* xr = mu + static_cast<int64_t>(r) * D;
      const float* xo = mu + static_cast<int64_t>(o) * D;
      float acc = 0.f;
      for (int q = 0; q * kWave < D; ++q) {
        const int d = l + q * kWave;
        const float diff = feat_or_zero(gp(xr), d, D) - feat_or_zero(gp(xo), d, D);
        acc = q == 0 ? diff * diff : acc + diff * diff;
      }
      const float exact2 = wave_sum0(acc);
      if (l == 0) {
        const float exact = sqrtf(exact2);
        const float ma = s.mass[r], mb = s.mass[o];
        const float sum = ma + mb;
        const float denom = sum < 1.f ? 1.f : sum;
        const float x = s.radius[r] + (mb / denom) * exact, y = s.radius[o] + (ma / denom) * exact;
        const float verified = x < y ? y : x;
        a.bound[static_cast<int64_t>(lane) * M + r] = verified;
        if (verified > limit) {
          dist[static_cast<int64_t>(r) * M + o] = exact2;
          dist[static_cast<int64_t>(o) * M + r] = exact2;
          s.flags[r] = static_cast<uint8_t>((s.flags[r] | kRejected) & ~kValid);
          s.flags[o] |= kRejected;
        }
      }
    }
    __syncthreads();
  }
  // Frozen-center sweeps (budget stage, passes > 1): more pairs of the round.
  const bool sweeps = !LIMIT && a.passes > 1;
  int extra = 0;
  sweep_scans = 0;
  if (sweeps) extra = frozen_sweeps(s, a, lane, n, &sweep_scans);
  const uint64_t* restricted = sweeps ? a.restricted + static_cast<int64_t>(lane) * M : nullptr;
  // Surviving proposals sorted by (cost, row) (a stable argsort by cost); a
  // sweep's pair is priced by its restricted minimum.
  for (int r = t; r < n; r += kReduceThreads) {
    const uint8_t fl = s.flags[r];
    if (fl & kValid) {
      const int at = atomicAdd(s_nvalid, 1);
      const uint64_t k = (fl & kSweep) ? restricted[r] : s.packed[r];
      s.keys[at] = (k & 0xFFFFFFFF00000000ull) | static_cast<uint32_t>(r);
    }
  }
  __syncthreads();
  const int nv = *s_nvalid;
  const int width = pow2_at_least(nv > 0 ? nv : 1);
  for (int i = nv + t; i < width; i += kReduceThreads) s.keys[i] = ~0ull;
  __syncthreads();
  for (int size = 2; size <= width; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < width; i += kReduceThreads) {
        const int p = i ^ stride;
        if (p > i) {
          const bool up = (i & size) == 0;
          const uint64_t x = s.keys[i], y = s.keys[p];
          if ((x > y) == up) {
            s.keys[i] = y;
            s.keys[p] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  const int budget = sh[0] - a.target;
  const int n_ok = nv < budget ? nv : (budget > 0 ? budget : 0);
  // Merges: centers (one wave per merge, lanes over the features), then pair
  // scalars, masses and radii (litgpt/log_kv_cache.py:589-606).
  for (int p = w; p < n_ok; p += kReduceWaves) {
    const int ra = static_cast<int>(s.keys[p] & 0xFFFFFFFFu), rb = sweeps ? s.pair_of[ra] : s.best[ra];
    const float ma = s.mass[ra], mb = s.mass[rb];
    const float total = ma + mb;
    const float scale = total < 1.f ? 1.f : total;
    float* ua = mu + static_cast<int64_t>(ra) * D;
    const float* ub = mu + static_cast<int64_t>(rb) * D;
    for (int d = l; d < D; d += kWave) ua[d] = (ma * ua[d] + mb * ub[d]) / scale;
  }
  __syncthreads();
  for (int p = t; p < n_ok; p += kReduceThreads) {
    const int ra = static_cast<int>(s.keys[p] & 0xFFFFFFFFu), rb = sweeps ? s.pair_of[ra] : s.best[ra];
    // A kept row's best names its mate from here on (the Lance-Williams phase
    // reads it); the dirty rule reads the best of rows that are not kept.
    s.best[ra] = static_cast<int16_t>(rb);
    const float ma = s.mass[ra], mb = s.mass[rb];
    const float dab = dist[static_cast<int64_t>(ra) * M + rb];
    const float total = ma + mb;
    const float alpha = ma / total, beta = mb / total;
    s.p_alpha[p] = alpha;
    s.p_beta[p] = beta;
    s.p_shift[p] = alpha * beta * dab;
    s.pair_of[ra] = static_cast<int16_t>(p);
    s.flags[ra] |= kKeep | kMerged;
    s.flags[rb] = static_cast<uint8_t>((s.flags[rb] | kMerged) & ~kAlive);
    s.mass[ra] = total;
    s.mass[rb] = 0.f;
    if (LIMIT) s.radius[ra] = a.bound[static_cast<int64_t>(lane) * M + ra];
    trace[2 * (sh[1] + p)] = ra;
    trace[2 * (sh[1] + p) + 1] = rb;
  }
  __syncthreads();
  nprop_out = nprop + extra;
  n_ok_out = n_ok;
}

// Lance-Williams updates of merge p's kept row over columns [c0, c1) (or live
// columns live[c0 .. c1) when `live` is given; a dead column is never written
// and its key is never a minimum) (one wave, litgpt/log_kv_cache.py:607-626):
// the row and its mirror, each column's cost pushed into the column's cached
// minimum; returns the row's minimum key over those columns.
template <bool LIMIT>
__device__ uint64_t lw_columns(const ReduceLds& s, float* dist, int M, int n, int p, int c0, int c1, float limit,
                               const int16_t* live = nullptr) {
  const int l = lane_id();
  const int ra = static_cast<int>(s.keys[p] & 0xFFFFFFFFu), rb = s.best[ra];
  const float alpha = s.p_alpha[p], beta = s.p_beta[p], shift = s.p_shift[p];
  const float total = s.mass[ra], rad = s.radius[ra];
  float* row_a = dist + static_cast<int64_t>(ra) * M;
  const float* row_b = dist + static_cast<int64_t>(rb) * M;
  uint64_t rmin = kInfKey;
  for (int idx = c0 + l; idx < c1; idx += kWave) {
    const int c = live ? live[idx] : idx;
    const uint8_t fl = s.flags[c];
    const bool alive_c = fl & kAlive, keep_c = fl & kKeep;
    const float x_aa = row_a[c], x_ba = row_b[c];
    float nw = alpha * x_aa + beta * x_ba - shift;
    if (keep_c && c != ra) {
      const int q = s.best[c], pc = s.pair_of[c];
      const float qa = s.p_alpha[pc], qb = s.p_beta[pc], qs = s.p_shift[pc];
      const float x_ab = row_a[q], x_bb = row_b[q];
      const float own = qa * nw + qb * (alpha * x_ab + beta * x_bb - shift) - qs;
      const float other = alpha * (qa * x_aa + qb * x_ab - qs) + beta * (qa * x_ba + qb * x_bb - qs) - shift;
      nw = ra < c ? own : other;
    }
    nw = nw < 0.f ? 0.f : nw;
    if (c == ra) nw = 0.f;
    if (alive_c) {
      row_a[c] = nw;
      if (!keep_c) dist[static_cast<int64_t>(c) * M + ra] = nw;
    }
    const bool valid = alive_c && c != ra;
    const float cost = ward_cost<LIMIT>(nw, total, s.mass[c], rad, s.radius[c], limit, valid);
    const uint64_t k = pack_cost(cost, ra ^ c);
    // Keys only fall during the phase, so a key at or above the one read now
    // cannot be the final minimum: the atomic is issued only when it can lower
    // it, and never for a row the round rescans.
    if (cost < __builtin_inff() && !keep_c && !(fl & kDirty) && k < s.packed[c])
      atomicMin(reinterpret_cast<unsigned long long*>(&s.packed[c]), static_cast<unsigned long long>(k));
    rmin = k < rmin ? k : rmin;
  }
  return wave_min_u64(rmin);
}

// A row rescans when its partner merged or its proposal was rejected.
__device__ __forceinline__ bool is_dirty(const ReduceLds& s, int r) {
  const uint8_t fl = s.flags[r];
  return (fl & kAlive) && !(fl & kKeep) && ((s.flags[s.best[r]] & kMerged) || (fl & kRejected));
}

// Stage setup: every lane's image (masses, zero radii, live flags, infinite
// keys), every row in both lists (the first scan is a rescan of every row
// over every column) and round bookkeeping.
__global__ __launch_bounds__(kPhaseThreads) void reduce_init_kernel(ReduceArgs a) {
  const int lane = blockIdx.y, M = a.M;
  const int n = a.count[lane];
  const ReduceLds s = image_of(a, lane);
  int16_t* lists = a.live + static_cast<int64_t>(lane) * 3 * M;
  for (int i = blockIdx.x * kPhaseThreads + threadIdx.x; i < M; i += gridDim.x * kPhaseThreads) {
    s.mass[i] = i < n ? a.mass[static_cast<int64_t>(lane) * M + i] : 0.f;
    s.radius[i] = 0.f;
    s.flags[i] = i < n ? kAlive : 0;
    s.packed[i] = kInfKey;
    s.best[i] = static_cast<int16_t>(i);
    if (i < n) {
      lists[i] = static_cast<int16_t>(i);
      lists[M + i] = static_cast<int16_t>(i);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    LaneCtl c{};
    c.count = n;
    c.active = n > a.target ? 1 : 0;
    c.work = c.active;
    c.n_live = n;
    c.n_dirty = n;
    c.scan_elems = c.active ? n * n : 0;   // the first scan runs only for an active stage
    a.ctl[lane] = c;
  }
}

// Round phase 1: the plan on one block per lane (image -> LDS -> image). Kept
// rows' keys are reset to +inf for the Lance-Williams phase's minima.
template <bool LIMIT>
__global__ __launch_bounds__(kReduceThreads) void reduce_plan_kernel(ReduceArgs a) {
  extern __shared__ __align__(16) uint8_t dyn[];
  __shared__ int sh[2], s_nprop, s_nvalid;
  const int lane = blockIdx.x, M = a.M, t = threadIdx.x;
  LaneCtl ctl = a.ctl[lane];
  if (!ctl.active) {
    if (t == 0) a.ctl[lane].work = 0;
    return;
  }
  const int n = a.count[lane];
  const size_t bytes = reduce_lds_bytes(M);
  const uint8_t* img = a.image + static_cast<int64_t>(lane) * a.image_stride;
  for (size_t i = t * 16; i + 16 <= bytes; i += kReduceThreads * 16)
    *reinterpret_cast<uint4*>(dyn + i) = *reinterpret_cast<const uint4*>(img + i);
  if (t == 0) {
    sh[0] = ctl.count;
    sh[1] = ctl.ntrace;
  }
  __syncthreads();
  const ReduceLds s = carve_lds(dyn, M);
  int nprop, n_ok, sweep_scans;
  plan_phase<LIMIT>(s, a, lane, n, LIMIT ? a.limit[lane] : 0.f, sh, &s_nprop, &s_nvalid, nprop, n_ok, sweep_scans);
  for (int p = t; p < n_ok; p += kReduceThreads) s.packed[static_cast<int>(s.keys[p] & 0xFFFFFFFFu)] = kInfKey;
  // The live rows after the merges, ascending (the columns the Lance-Williams
  // and rescan phases visit: a dead column's key is never a minimum), the
  // rows to rescan, ascending, their cached minima reset for the rescan's
  // atomic minima, and the kept rows, ascending (the Lance-Williams tiles take
  // neighbouring kept rows, so their mirror writes into a row share lines).
  __shared__ int s_live, s_dirty, s_kept, part_s[3 * kReduceWaves];
  int16_t* live = a.live + static_cast<int64_t>(lane) * 3 * M;
  int16_t* dirty = live + M;
  int16_t* kept = live + 2 * M;
  if (t == 0) {
    s_live = 0;
    s_dirty = 0;
    s_kept = 0;
  }
  __syncthreads();
  for (int c0 = 0; c0 < n; c0 += kReduceThreads) {
    const int c = c0 + t;
    const bool on = c < n && (s.flags[c] & kAlive);
    const bool re = c < n && is_dirty(s, c);
    const bool kp = c < n && (s.flags[c] & kKeep);
    const uint64_t below = (1ull << lane_id()) - 1ull;
    const uint64_t mask = __ballot(on), mask_re = __ballot(re), mask_kp = __ballot(kp);
    if (lane_id() == 0) {
      part_s[wave_id()] = __popcll(mask);
      part_s[kReduceWaves + wave_id()] = __popcll(mask_re);
      part_s[2 * kReduceWaves + wave_id()] = __popcll(mask_kp);
    }
    __syncthreads();
    int base = s_live, base_re = s_dirty, base_kp = s_kept;
    for (int q = 0; q < wave_id(); ++q) {
      base += part_s[q];
      base_re += part_s[kReduceWaves + q];
      base_kp += part_s[2 * kReduceWaves + q];
    }
    if (on) live[base + __popcll(mask & below)] = static_cast<int16_t>(c);
    if (re) {
      dirty[base_re + __popcll(mask_re & below)] = static_cast<int16_t>(c);
      s.packed[c] = kInfKey;
      s.flags[c] |= kDirty;
    }
    if (kp) kept[base_kp + __popcll(mask_kp & below)] = static_cast<int16_t>(c);
    __syncthreads();
    if (t == 0) {
      int total = 0, total_re = 0, total_kp = 0;
      for (int q = 0; q < kReduceWaves; ++q) {
        total += part_s[q];
        total_re += part_s[kReduceWaves + q];
        total_kp += part_s[2 * kReduceWaves + q];
      }
      s_live += total;
      s_dirty += total_re;
      s_kept += total_kp;
    }
    __syncthreads();
  }
  uint8_t* out = a.image + static_cast<int64_t>(lane) * a.image_stride;
  for (size_t i = t * 16; i + 16 <= bytes; i += kReduceThreads * 16)
    *reinterpret_cast<uint4*>(out + i) = *reinterpret_cast<const uint4*>(dyn + i);
  if (t == 0) {
    const int count = ctl.count - n_ok;
    const bool remaining = count > a.target;
    ctl.count = count;
    ctl.ntrace += n_ok;
    ctl.n_ok = n_ok;
    ctl.nprop = nprop;
    ctl.work = nprop > 0 ? 1 : 0;
    ctl.active = remaining && nprop > 0 ? 1 : 0;
    ctl.stuck = remaining && nprop == 0 ? 1 : 0;
    ctl.rounds += 1;
    ctl.n_live = s_live;
    ctl.n_dirty = s_dirty;
    ctl.lw_elems += n_ok * s_live;
    ctl.scan_elems += s_dirty * s_live + sweep_scans * (count + n_ok);   // sweeps scan before the merges
    if (ctl.rounds >= 2 * M + 7) ctl.active = 0;
    a.ctl[lane] = ctl;
  }
}

// Round phase 2: the Lance-Williams rows of the round's kept rows
// (litgpt/log_kv_cache.py:607-626) as wave tiles: up to kLwRows kept rows
// (neighbours in row order) x kLwCols * 64 live columns (kLwCols per lane,
// the columns' state held across the rows). Each element is lw_columns'
// update: the row and, for a column
// that is not kept, its mirror; the screen leaves only the elements that can
// hold the kept row's minimum key (an atomic minimum per tile) or lower a
// column's cached minimum to evaluate ward_cost.
constexpr int kLwCols = 4, kLwRows = 16, kLwTile = kLwCols * kWave;

template <bool LIMIT>
__global__ __launch_bounds__(kPhaseThreads) void reduce_lw_kernel(ReduceArgs a) {
  const int lane = blockIdx.y, M = a.M, l = lane_id();
  const LaneCtl ctl = a.ctl[lane];
  if (!ctl.work) return;
  const ReduceLds s = image_of(a, lane);
  float* dist = a.dist + static_cast<int64_t>(lane) * M * M;
  const float limit = LIMIT ? a.limit[lane] : 0.f;
  const int16_t* live = a.live + static_cast<int64_t>(lane) * 3 * M;
  const int16_t* kept = live + 2 * M;
  const int n_live = ctl.n_live, n_ok = ctl.n_ok;
  const int col_chunks = (n_live + kLwTile - 1) / kLwTile, waves = gridDim.x * kPhaseWaves;
  // Merges per item: up to kLwRows, fewer when that would leave waves idle.
  const int rows = max(1, min(kLwRows, n_ok * col_chunks / waves));
  const int items = col_chunks * ((n_ok + rows - 1) / rows);
  for (int it = blockIdx.x * kPhaseWaves + wave_id(); it < items; it += waves) {
    const int pg = it / col_chunks, cc = it - pg * col_chunks;
    int col[kLwCols];
    uint8_t fl[kLwCols];
    float mc[kLwCols], rc[kLwCols], thr[kLwCols];
#pragma unroll
    for (int e = 0; e < kLwCols; ++e) {
      const int idx = cc * kLwTile + e * kWave + l;
      col[e] = idx < n_live ? live[idx] : -1;
      const int c = col[e] >= 0 ? col[e] : 0;
      fl[e] = col[e] >= 0 ? s.flags[c] : 0;
      mc[e] = s.mass[c];
      rc[e] = s.radius[c];
      // A kept or rescanned column takes no push (-1); keys only fall during
      // the phase, so the cost read now bounds every key that can still lower it.
      thr[e] = col[e] >= 0 && !(fl[e] & (kKeep | kDirty)) ? key_cost(s.packed[c]) : -1.f;
    }
    const int p1 = min(n_ok, (pg + 1) * rows);
    for (int j = pg * rows; j < p1; ++j) {
      const int ra = kept[j], rb = s.best[ra], p = s.pair_of[ra];
      const float alpha = s.p_alpha[p], beta = s.p_beta[p], shift = s.p_shift[p];
      const float total = s.mass[ra], rad = s.radius[ra];
      float* row_a = dist + static_cast<int64_t>(ra) * M;
      const float* row_b = dist + static_cast<int64_t>(rb) * M;
      float x_aa[kLwCols], x_ba[kLwCols], nw[kLwCols], sc[kLwCols];
      bool border[kLwCols];
#pragma unroll
      for (int e = 0; e < kLwCols; ++e) {
        const int c = col[e] >= 0 ? col[e] : ra;
        x_aa[e] = row_a[c];
        x_ba[e] = row_b[c];
      }
      float m = __builtin_inff();
#pragma unroll
      for (int e = 0; e < kLwCols; ++e) {
        const int c = col[e];
        float v = alpha * x_aa[e] + beta * x_ba[e] - shift;
        if (c >= 0 && (fl[e] & kKeep) && c != ra) {
          const int q = s.best[c], pc = s.pair_of[c];
          const float qa = s.p_alpha[pc], qb = s.p_beta[pc], qs = s.p_shift[pc];
          const float x_ab = row_a[q], x_bb = row_b[q];
          const float own = qa * v + qb * (alpha * x_ab + beta * x_bb - shift) - qs;
          const float other = alpha * (qa * x_aa[e] + qb * x_ab - qs) + beta * (qa * x_ba[e] + qb * x_bb - qs) - shift;
          v = ra < c ? own : other;
        }
        v = v < 0.f ? 0.f : v;
        if (c == ra) v = 0.f;
        nw[e] = v;
        if (c >= 0) {
          row_a[c] = v;
          if (!(fl[e] & kKeep)) dist[static_cast<int64_t>(c) * M + ra] = v;
        }
        sc[e] = screen_cost<LIMIT>(v, total, mc[e], rad, rc[e], limit, c >= 0 && c != ra, border[e]);
        if (!border[e]) m = sc[e] < m ? sc[e] : m;
      }
      const float cut = screen_cutoff(__uint_as_float(wave_min_u32(__float_as_uint(m))));
      uint64_t best = kInfKey;
#pragma unroll
      for (int e = 0; e < kLwCols; ++e) {
        const bool open = border[e] || sc[e] < __builtin_inff();
        const bool near_row = open && (border[e] || sc[e] <= cut);
        const bool near_col = open && thr[e] >= 0.f && (border[e] || sc[e] <= screen_cutoff(thr[e]));
        if (near_row || near_col) {
          const float cost = ward_cost<LIMIT>(nw[e], total, mc[e], rad, rc[e], limit, true);
          const uint64_t k = pack_cost(cost, ra ^ col[e]);
          if (near_row) best = k < best ? k : best;
          if (near_col && cost < __builtin_inff() && k < s.packed[col[e]])
            atomicMin(reinterpret_cast<unsigned long long*>(&s.packed[col[e]]), static_cast<unsigned long long>(k));
        }
      }
      best = wave_min_key(best);
      if (l == 0 && best < kInfKey)
        atomicMin(reinterpret_cast<unsigned long long*>(&s.packed[ra]), static_cast<unsigned long long>(best));
    }
  }
}

// Round phase 3 (and the stage's first scan): the cached minimum of every
// listed row over the live columns, as atomic minima of wave tiles. A wave
// takes up to kScanRows listed rows x kScanCols * 64 live columns (kScanCols per
// lane, the columns' masses and radii held across the rows); per row, the
// screen leaves only the lanes whose pairs can hold the tile's minimum key
// to evaluate ward_cost.
constexpr int kScanCols = 8, kScanRows = 16, kScanChunk = kScanCols * kWave;

template <bool LIMIT>
__global__ __launch_bounds__(kPhaseThreads) void reduce_rescan_kernel(ReduceArgs a) {
  const int lane = blockIdx.y, M = a.M, l = lane_id();
  const LaneCtl ctl = a.ctl[lane];
  if (!ctl.work) return;
  const ReduceLds s = image_of(a, lane);
  const float* dist = a.dist + static_cast<int64_t>(lane) * M * M;
  const float limit = LIMIT ? a.limit[lane] : 0.f;
  const int16_t* live = a.live + static_cast<int64_t>(lane) * 3 * M;
  const int16_t* dirty = live + M;
  const int n_live = ctl.n_live, n_dirty = ctl.n_dirty;
  const int col_chunks = (n_live + kScanChunk - 1) / kScanChunk, waves = gridDim.x * kPhaseWaves;
  // Rows per item: up to kScanRows, fewer when that would leave waves idle.
  const int rows = max(1, min(kScanRows, n_dirty * col_chunks / waves));
  const int items = col_chunks * ((n_dirty + rows - 1) / rows);
  for (int it = blockIdx.x * kPhaseWaves + wave_id(); it < items; it += waves) {
    const int rg = it / col_chunks, cc = it - rg * col_chunks;
    int col[kScanCols];
    float mc[kScanCols], rc[kScanCols];
#pragma unroll
    for (int e = 0; e < kScanCols; ++e) {
      const int idx = cc * kScanChunk + e * kWave + l;
      col[e] = idx < n_live ? live[idx] : -1;
      mc[e] = col[e] >= 0 ? s.mass[col[e]] : 0.f;
      rc[e] = col[e] >= 0 ? s.radius[col[e]] : 0.f;
    }
    const int q1 = min(n_dirty, (rg + 1) * rows);
    for (int q = rg * rows; q < q1; ++q) {
      const int r = dirty[q];
      const float mr = s.mass[r], rr = s.radius[r];
      const float* row = dist + static_cast<int64_t>(r) * M;
      float d2[kScanCols], sc[kScanCols];
      bool border[kScanCols];
#pragma unroll
      for (int e = 0; e < kScanCols; ++e) d2[e] = row[col[e] >= 0 ? col[e] : 0];
      float m = __builtin_inff();
#pragma unroll
      for (int e = 0; e < kScanCols; ++e) {
        sc[e] = screen_cost<LIMIT>(d2[e], mr, mc[e], rr, rc[e], limit, col[e] >= 0 && col[e] != r, border[e]);
        if (!border[e]) m = sc[e] < m ? sc[e] : m;
      }
      const float cut = screen_cutoff(__uint_as_float(wave_min_u32(__float_as_uint(m))));
      uint64_t best = kInfKey;
#pragma unroll
      for (int e = 0; e < kScanCols; ++e) {
        if (border[e] || (sc[e] < __builtin_inff() && sc[e] <= cut)) {
          const uint64_t k = pack_cost(ward_cost<LIMIT>(d2[e], mr, mc[e], rr, rc[e], limit, true), r ^ col[e]);
          best = k < best ? k : best;
        }
      }
      best = wave_min_key(best);
      if (l == 0 && best < kInfKey)
        atomicMin(reinterpret_cast<unsigned long long*>(&s.packed[r]), static_cast<unsigned long long>(best));
    }
  }
}

// The stage's end on one block per lane: any rounds left (one block runs
// every phase, the image in LDS), then the survivors, merge count and stuck
// flag.
template <bool LIMIT>
__global__ __launch_bounds__(kReduceThreads) void reduce_finish_kernel(ReduceArgs a) {
  extern __shared__ __align__(16) uint8_t dyn[];
  __shared__ int sh[2], s_nprop, s_nvalid, s_rescans;
  const int lane = blockIdx.x, M = a.M, t = threadIdx.x, l = lane_id(), w = wave_id();
  const int n = a.count[lane];
  LaneCtl ctl = a.ctl[lane];
  const size_t bytes = reduce_lds_bytes(M);
  const uint8_t* img = a.image + static_cast<int64_t>(lane) * a.image_stride;
  for (size_t i = t * 16; i + 16 <= bytes; i += kReduceThreads * 16)
    *reinterpret_cast<uint4*>(dyn + i) = *reinterpret_cast<const uint4*>(img + i);
  if (t == 0) {
    sh[0] = ctl.count;
    sh[1] = ctl.ntrace;
  }
  __syncthreads();
  const ReduceLds s = carve_lds(dyn, M);
  float* dist = a.dist + static_cast<int64_t>(lane) * M * M;
  const float limit = LIMIT ? a.limit[lane] : 0.f;
  while (ctl.active) {
    int nprop, n_ok, sweep_scans;
    plan_phase<LIMIT>(s, a, lane, n, limit, sh, &s_nprop, &s_nvalid, nprop, n_ok, sweep_scans);
    if (t == 0) s_rescans = 0;
    for (int p = w; p < n_ok; p += kReduceWaves) {
      const uint64_t rmin = lw_columns<LIMIT>(s, dist, M, n, p, 0, n, limit);
      if (l == 0) s.packed[static_cast<int>(s.keys[p] & 0xFFFFFFFFu)] = rmin;
    }
    __syncthreads();
    for (int r = w; r < n; r += kReduceWaves) {
      if (!is_dirty(s, r)) continue;
      const uint64_t k = scan_row<LIMIT>(s, dist, M, n, r, limit);
      if (l == 0) {
        s.packed[r] = k;
        atomicAdd(&s_rescans, 1);
      }
    }
    __syncthreads();
    ctl.scan_elems += sweep_scans * ctl.count;
    const int count = ctl.count - n_ok;
    const bool remaining = count > a.target;
    ctl.lw_elems += n_ok * count;
    ctl.scan_elems += s_rescans * count;
    ctl.count = count;
    ctl.ntrace += n_ok;
    ctl.stuck = remaining && nprop == 0 ? 1 : 0;
    ctl.active = remaining && nprop > 0 ? 1 : 0;
    ctl.rounds += 1;
    if (ctl.rounds >= 2 * M + 7) ctl.active = 0;
    if (t == 0) {
      sh[0] = ctl.count;
      sh[1] = ctl.ntrace;
    }
    __syncthreads();
  }
  for (int i = t; i < M; i += kReduceThreads)
    a.alive_out[static_cast<int64_t>(lane) * M + i] = (s.flags[i] & kAlive) ? 1 : 0;
  if (t == 0) {
    a.n_trace[lane] = ctl.ntrace;
    a.stuck[lane] = ctl.stuck;
    if (a.stats) {
      int32_t* st = a.stats + static_cast<int64_t>(lane) * a.stats_stride;
      st[0] = n;
      st[1] = ctl.rounds;
      st[2] = ctl.ntrace;
      st[3] = ctl.lw_elems;
      st[4] = ctl.scan_elems;
      st[5] = ctl.stuck;
    }
  }
}

// One stage: setup, the pipelined rounds, the finish.
template <bool LIMIT>
int launch_reduce(const ReduceArgs& a, int lanes, hipStream_t stream) {
  if (!a.dist || !a.mu || !a.mass || !a.count || !a.image || !a.ctl || !a.live || !a.alive_out || !a.trace ||
      !a.n_trace || !a.stuck || !a.bound || (LIMIT && !a.limit))
    return refuse("unified reducer: a workspace buffer of the stage is NULL");
  if (a.image_stride < static_cast<int64_t>(reduce_lds_bytes(a.M)))
    return refuse("unified reducer: the per-lane state image is smaller than the reducer's LDS layout");
  if (!LIMIT && a.passes > 1 && !a.restricted)
    return refuse("unified reducer: frozen-center sweeps without their restricted-minimum buffer");
  const size_t lds = reduce_lds_bytes(a.M);
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&reduce_plan_kernel<LIMIT>), lds) ||
      !allow_dynamic_lds(reinterpret_cast<const void*>(&reduce_finish_kernel<LIMIT>), lds))
    return LOGKV_ERUNTIME;
  const dim3 phase(kPhaseBlocks, lanes);
  hipLaunchKernelGGL(reduce_init_kernel, dim3(std::max(1, std::min(16, a.M / kPhaseThreads)), lanes),
                     dim3(kPhaseThreads), 0, stream, a);
  hipLaunchKernelGGL(reduce_rescan_kernel<LIMIT>, phase, dim3(kPhaseThreads), 0, stream, a);
  for (int round = 0; round < kPipelinedRounds[LIMIT]; ++round) {
    hipLaunchKernelGGL(reduce_plan_kernel<LIMIT>, dim3(lanes), dim3(kReduceThreads), lds, stream, a);
    hipLaunchKernelGGL(reduce_lw_kernel<LIMIT>, phase, dim3(kPhaseThreads), 0, stream, a);
    hipLaunchKernelGGL(reduce_rescan_kernel<LIMIT>, phase, dim3(kPhaseThreads), 0, stream, a);
  }
  hipLaunchKernelGGL(reduce_finish_kernel<LIMIT>, dim3(lanes), dim3(kReduceThreads), lds, stream, a);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

// ---------------------------------------------------------------------------
// Full-recompute rounds of a capacity-capped unified route
// (litgpt/log_kv_cache.py:3445-3519; pairs :3067-3117 in the unfused form;
// merges _semantic_unified_merge_pack :3134-3156). Each round prices the
// current nodes afresh: their squared distances (dist_kernel, the canonical
// sums), every row's least cost with the radius bound (candidate stage) and
// without pairs whose total mass exceeds the cap, mutual minima with the
// row ^ col tie rule in (cost, row) order; in the budget stage a lane with no
// capped pair takes its uncapped ones. Candidate pairs are re-checked from
// their exact distances. The first count - target pairs merge into their lower
// rows (mass-weighted centers, summed masses, the pair's radius bound) and the
// survivors are compacted in order, so row indices, and with them the ties,
// are those of the compacted nodes. The host polls the lanes between batches of
// rounds (a round with no pair, or at the target, ends a lane).
constexpr int kRoundPoll = 8;   // rounds enqueued between the host's polls

// Cost of a pair of current nodes (round_pairs' order: Ward cost, radius
// bound > limit -> +inf); the capped cost is +inf too when the total mass
// exceeds the cap.
template <bool LIMIT>
__device__ __forceinline__ void round_cost(float d2, float mi, float mj, float ri, float rj, float limit, float cap,
                                           bool valid, float& cost, float& capped) {
  const float total = mi + mj;
  const float denom = total < 1.f ? 1.f : total;
  valid = valid && mi > 0.f && mj > 0.f;
  cost = valid ? d2 * (mi * mj / denom) : __builtin_inff();
  if (LIMIT) {
    const float distance = sqrtf(d2);
    const float x = ri + (mj / denom) * distance, y = rj + (mi / denom) * distance;
    if ((x < y ? y : x) > limit) cost = __builtin_inff();
  }
  capped = total > cap ? __builtin_inff() : cost;
}

__global__ __launch_bounds__(kPhaseThreads) void rounds_init_kernel(RoundArgs a) {
  const int lane = blockIdx.y, M = a.M, D = a.D;
  const int n = a.count[lane];
  for (int i = blockIdx.x * kPhaseThreads + threadIdx.x; i < M; i += gridDim.x * kPhaseThreads) {
    const int64_t at = static_cast<int64_t>(lane) * M + i;
    a.cmass[0][at] = i < n ? a.mass[at] : 0.f;
    a.crad[0][at] = 0.f;
    a.croot[0][at] = i;
    if (i < n)
      for (int d = 0; d < D; ++d) a.cmu[0][at * D + d] = a.mu[at * D + d];
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    a.n_cur[lane] = n;
    a.cbuf[lane] = 0;
    a.dcount[lane] = n > a.target ? n : 0;
    a.n_trace[lane] = 0;
    a.stuck[lane] = 0;
    a.rounds[lane] = 0;
  }
}

// Every current row's least capped and uncapped keys (one wave per row).
template <bool LIMIT>
__global__ __launch_bounds__(kPhaseThreads) void rounds_min_kernel(RoundArgs a, int src) {
  const int lane = blockIdx.y, M = a.M, n = a.dcount[lane];
  if (n == 0) return;
  const float limit = LIMIT ? a.limit[lane] : 0.f;
  const float* mass = a.cmass[src] + static_cast<int64_t>(lane) * M;
  const float* rad = a.crad[src] + static_cast<int64_t>(lane) * M;
  const float* dist = a.dist + static_cast<int64_t>(lane) * M * M;
  for (int r = blockIdx.x * kPhaseWaves + wave_id(); r < n; r += gridDim.x * kPhaseWaves) {
    const float mr = mass[r], rr = rad[r];
    uint64_t kc = kInfKey, ka = kInfKey;
    for (int c = lane_id(); c < n; c += kWave) {
      float cost, capped;
      round_cost<LIMIT>(dist[static_cast<int64_t>(r) * M + c], mr, mass[c], rr, rad[c], limit, a.cap, c != r, cost,
                        capped);
      const uint64_t k1 = pack_cost(capped, r ^ c), k2 = pack_cost(cost, r ^ c);
      kc = k1 < kc ? k1 : kc;
      ka = k2 < ka ? k2 : ka;
    }
    kc = wave_min_u64(kc);
    ka = wave_min_u64(ka);
    if (lane_id() == 0) {
      a.keys[(static_cast<int64_t>(lane) * M + r) * 2] = kc;
      a.keys[(static_cast<int64_t>(lane) * M + r) * 2 + 1] = ka;
    }
  }
}

// One round of a lane on one block: pairs, budget, merges into the other
// buffer set, compaction, trace.
template <bool LIMIT>
__global__ __launch_bounds__(kReduceThreads) void rounds_pair_kernel(RoundArgs a, int src) {
  extern __shared__ __align__(16) uint8_t dyn[];
  __shared__ int s_nprop, s_nkeep, s_n, part_s[kReduceWaves];
  const int lane = blockIdx.x, M = a.M, D = a.D, t = threadIdx.x, l = lane_id(), w = wave_id();
  const int n = a.dcount[lane];
  if (n == 0) return;
  const int dst = src ^ 1;
  const int64_t lm = static_cast<int64_t>(lane) * M;
  const float* mu = a.cmu[src] + lm * D;
  const float* mass = a.cmass[src] + lm;
  const float* rad = a.crad[src] + lm;
  const int32_t* root = a.croot[src] + lm;
  const uint64_t* keys = a.keys + lm * 2;
  // LDS: sort keys [P2], partner [M], new index [M], exact distance of a kept pair [M / 2 + 1].
  const int P2 = pow2_at_least(half_up(M) > 0 ? half_up(M) : 1);
  uint64_t* sk = reinterpret_cast<uint64_t*>(dyn);
  int16_t* partner = reinterpret_cast<int16_t*>(sk + P2);
  int16_t* nidx = partner + M;
  float* pdist = reinterpret_cast<float*>(nidx + M);
  auto key_of = [&](int r, int which) { return keys[2 * r + which]; };
  auto mate = [&](uint64_t k, int r) { return key_partner(k, r, M); };
  // Capped proposals (the lower row of each mutual pair); none: the uncapped ones (budget stage).
  int which = 0;
  for (int pass = 0; pass < 2; ++pass) {
    if (t == 0) s_nprop = 0;
    __syncthreads();
    for (int r = t; r < n; r += kReduceThreads) {
      const uint64_t k = key_of(r, which);
      const int b = mate(k, r);
      if (r < b && mate(key_of(b, which), b) == r && key_cost(k) < __builtin_inff()) {
        const int at = atomicAdd(&s_nprop, 1);
        sk[at] = (k & 0xFFFFFFFF00000000ull) | static_cast<uint32_t>(r);
      }
    }
    __syncthreads();
    if (s_nprop > 0 || !a.strict || which == 1) break;
    which = 1;
  }
  const int nv = s_nprop;
  const int width = pow2_at_least(nv > 0 ? nv : 1);
  for (int i = nv + t; i < width; i += kReduceThreads) sk[i] = ~0ull;
  __syncthreads();
  for (int size = 2; size <= width; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < width; i += kReduceThreads) {
        const int p = i ^ stride;
        if (p > i) {
          const bool up = (i & size) == 0;
          const uint64_t x = sk[i], y = sk[p];
          if ((x > y) == up) {
            sk[i] = y;
            sk[p] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  // Candidate stage: each pair's bound from its exact distance (one wave per pair); a pair that
  // fails is marked (top bit of its key) and skipped in place.
  for (int p = w; LIMIT && p < nv; p += kReduceWaves) {
    const int ra = static_cast<int>(sk[p] & 0xFFFFFFFFu), rb = mate(key_of(ra, which), ra);
    float acc = 0.f;
    for (int q = 0; q * kWave < D; ++q) {
      const int d = l + q * kWave;
      const float diff = (d < D ? mu[static_cast<int64_t>(ra) * D + d] : 0.f) -
                         (d < D ? mu[static_cast<int64_t>(rb) * D + d] : 0.f);
      acc = q == 0 ? diff * diff : acc + diff * diff;
    }
    const float exact = sqrtf(wave_sum0(acc));
    if (l == 0) {
      pdist[p] = exact;
      const float ma = mass[ra], mb = mass[rb];
      const float sum = ma + mb;
      const float den = sum < 1.f ? 1.f : sum;
      const float x = rad[ra] + mb / den * exact, y = rad[rb] + ma / den * exact;
      if ((x < y ? y : x) > a.limit[lane]) sk[p] |= 0x8000000000000000ull;   // rejected
    }
  }
  __syncthreads();
  // Kept pairs in order: the first count - target that passed (a rejected pair keeps its place and
  // takes no budget).
  if (t == 0) {
    const int budget = n - a.target;
    int kept = 0;
    for (int p = 0; p < nv; ++p) {
      const bool ok = !(sk[p] >> 63) && kept < budget;
      if (ok) ++kept;
      else sk[p] |= 0x8000000000000000ull;
    }
    s_nkeep = kept;
  }
  for (int r = t; r < n; r += kReduceThreads) partner[r] = -1;
  __syncthreads();
  const int nk = s_nkeep;
  // Each kept pair marks its rows: the lower row gets the pair's index, the other is retired.
  for (int p = t; p < nv; p += kReduceThreads) {
    if (sk[p] >> 63) continue;
    const int ra = static_cast<int>(sk[p] & 0xFFFFFFFFu), rb = mate(key_of(ra, which), ra);
    partner[ra] = static_cast<int16_t>(p);      // pair index of a kept lower row
    partner[rb] = static_cast<int16_t>(-2);     // retired
  }
  __syncthreads();
  // Trace in kept order (input ids), by one thread (nk is at most n / 2).
  if (t == 0) {
    int32_t* tr = a.trace + lm * 2;
    int at = a.n_trace[lane];
    for (int p = 0; p < nv; ++p) {
      if (sk[p] >> 63) continue;
      const int ra = static_cast<int>(sk[p] & 0xFFFFFFFFu), rb = mate(key_of(ra, which), ra);
      tr[2 * at] = root[ra];
      tr[2 * at + 1] = root[rb];
      ++at;
    }
    a.n_trace[lane] = at;
  }
  // New indices of the survivors (ballot prefix sums, row order).
  if (t == 0) s_n = 0;
  __syncthreads();
  for (int c0 = 0; c0 < n; c0 += kReduceThreads) {
    const int r = c0 + t;
    const bool on = r < n && partner[r] != -2;
    const uint64_t mask = __ballot(on);
    if (l == 0) part_s[w] = __popcll(mask);
    __syncthreads();
    int base = s_n;
    for (int q = 0; q < w; ++q) base += part_s[q];
    if (on) nidx[r] = static_cast<int16_t>(base + __popcll(mask & ((1ull << l) - 1ull)));
    __syncthreads();
    if (t == 0) {
      int total = 0;
      for (int q = 0; q < kReduceWaves; ++q) total += part_s[q];
      s_n += total;
    }
    __syncthreads();
  }
  const int n_new = s_n;
  // Survivors into the other buffer set: a kept lower row merges (one wave per row).
  float* omu = a.cmu[dst] + lm * D;
  for (int r = w; r < n; r += kReduceWaves) {
    const int pr = partner[r];
    if (pr == -2) continue;
    const int i = nidx[r];
    const int64_t o = lm + i;
    if (pr < 0) {
      for (int d = l; d < D; d += kWave) omu[static_cast<int64_t>(i) * D + d] = mu[static_cast<int64_t>(r) * D + d];
      if (l == 0) {
        a.cmass[dst][o] = mass[r];
        a.crad[dst][o] = LIMIT ? rad[r] : 0.f;
        a.croot[dst][o] = root[r];
      }
      continue;
    }
    const int rb = mate(key_of(r, which), r);
    const float ma = mass[r], mb = mass[rb];
    const float comb = ma + mb;
    const float scale = comb < 1.f ? 1.f : comb;
    for (int d = l; d < D; d += kWave)
      omu[static_cast<int64_t>(i) * D + d] =
          (ma * mu[static_cast<int64_t>(r) * D + d] + mb * mu[static_cast<int64_t>(rb) * D + d]) / scale;
    if (l == 0) {
      a.cmass[dst][o] = comb;
      if (LIMIT) {
        const float dd = pdist[pr];
        const float x = rad[r] + mb / scale * dd, y = rad[rb] + ma / scale * dd;
        a.crad[dst][o] = x < y ? y : x;
      } else {
        a.crad[dst][o] = 0.f;
      }
      a.croot[dst][o] = root[r];
    }
  }
  for (int i = n_new + t; i < M; i += kReduceThreads) a.cmass[dst][lm + i] = 0.f;
  if (t == 0) {
    a.n_cur[lane] = n_new;
    a.cbuf[lane] = dst;
    const bool more = nk > 0 && n_new > a.target;
    a.dcount[lane] = more ? n_new : 0;
    a.rounds[lane] += 1;
    if (nk == 0 && a.strict && n > a.target) a.stuck[lane] = 1;
  }
}

// The stage's outputs in the incremental reducer's form: survivors by input
// id, their final centers at their input rows, merge count, stuck flag.
__global__ __launch_bounds__(kPhaseThreads) void rounds_finish_kernel(RoundArgs a) {
  const int lane = blockIdx.x, M = a.M, D = a.D, t = threadIdx.x;
  const int64_t lm = static_cast<int64_t>(lane) * M;
  const int n = a.n_cur[lane];
  const int src = a.cbuf[lane];   // the buffer set of the lane's last round
  for (int i = t; i < M; i += kPhaseThreads) a.alive_out[lm + i] = 0;
  __syncthreads();
  for (int i = t; i < n; i += kPhaseThreads) {
    const int r = a.croot[src][lm + i];
    a.alive_out[lm + r] = 1;
    for (int d = 0; d < D; ++d) a.mu[(lm + r) * D + d] = a.cmu[src][(lm + i) * D + d];
  }
  if (t == 0 && a.stats) {
    int32_t* st = a.stats + lane * static_cast<int64_t>(a.stats_stride);
    st[0] = a.count[lane];
    st[1] = a.rounds[lane];
    st[2] = a.n_trace[lane];
    st[3] = 0;
    st[4] = 0;
    st[5] = a.stuck[lane];
  }
}

size_t rounds_pair_lds(int M) {
  const int P2 = pow2_at_least(half_up(M) > 0 ? half_up(M) : 1);
  return static_cast<size_t>(P2) * 8 + static_cast<size_t>(M) * 4 + static_cast<size_t>(half_up(M) + 1) * 4 + 16;
}

// One stage of full-recompute rounds; the host reads the lanes' round flags
// after every kRoundPoll rounds (the stream is synchronized there).
template <bool LIMIT>
int launch_rounds(const RoundArgs& a, int lanes, hipStream_t stream) {
  if (!a.mu || !a.mass || !a.count || (LIMIT && !a.limit) || !a.n_cur || !a.dcount || !a.cbuf || !a.keys || !a.dist ||
      !a.alive_out || !a.trace || !a.n_trace || !a.stuck || !a.rounds)
    return refuse("unified rounds: a workspace buffer of the stage is NULL");
  for (int s = 0; s < 2; ++s)
    if (!a.cmu[s] || !a.cmass[s] || !a.crad[s] || !a.croot[s])
      return refuse("unified rounds: a node buffer of the stage is NULL");
  const size_t lds = rounds_pair_lds(a.M);
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&rounds_pair_kernel<LIMIT>), lds)) return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(rounds_init_kernel, dim3(std::max(1, std::min(16, a.M / kPhaseThreads)), lanes),
                     dim3(kPhaseThreads), 0, stream, a);
  std::vector<int32_t> host(lanes);
  int src = 0;
  for (int round = 0; round < 2 * a.M + 8; ++round) {
    if (round > 0 && round % kRoundPoll == 0) {
      if (hipMemcpyAsync(host.data(), a.dcount, sizeof(int32_t) * lanes, hipMemcpyDeviceToHost, stream) !=
              hipSuccess ||
          hipStreamSynchronize(stream) != hipSuccess)
        return LOGKV_ERUNTIME;
      bool any = false;
      for (int32_t v : host) any = any || v > 0;
      if (!any) break;
    }
    int rc = launch_dist(a.cmu[src], a.dcount, a.dist, a.M, a.D, lanes, stream);
    if (rc) return rc;
    hipLaunchKernelGGL(rounds_min_kernel<LIMIT>, dim3(kPhaseBlocks, lanes), dim3(kPhaseThreads), 0, stream, a, src);
    hipLaunchKernelGGL(rounds_pair_kernel<LIMIT>, dim3(lanes), dim3(kReduceThreads), lds, stream, a, src);
    src ^= 1;
  }
  hipLaunchKernelGGL(rounds_finish_kernel, dim3(lanes), dim3(kPhaseThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

// Leaf -> compact surviving row (litgpt/log_kv_cache.py:3553-3568): parents
// from the trace, pointer jumping to the roots, roots numbered in order.
__global__ __launch_bounds__(1024) void labels_kernel(const uint8_t* __restrict__ alive, const int32_t* __restrict__ trace,
                                                      const int32_t* __restrict__ n_trace,
                                                      const int32_t* __restrict__ count, int M,
                                                      int32_t* __restrict__ label, int32_t* __restrict__ n_roots) {
  extern __shared__ __align__(16) uint8_t dyn[];
  __shared__ int wave_sum[16];
  int32_t* parent = reinterpret_cast<int32_t*>(dyn);
  int32_t* compact = parent + M;
  const int lane = blockIdx.x, n = count[lane], t = threadIdx.x;
  const uint8_t* al = alive + static_cast<int64_t>(lane) * M;
  const int32_t* tr = trace + static_cast<int64_t>(lane) * M * 2;
  for (int i = t; i < n; i += 1024) parent[i] = i;
  __syncthreads();
  for (int p = t; p < n_trace[lane]; p += 1024) parent[tr[2 * p + 1]] = tr[2 * p];
  __syncthreads();
  for (;;) {
    int changed = 0;
    for (int i = t; i < n; i += 1024) {
      const int up = parent[parent[i]];
      if (up != parent[i]) {
        parent[i] = up;
        changed = 1;
      }
    }
    if (!__syncthreads_or(changed)) break;
  }
  // Ranks of the roots among the survivors, in row order.
  int carry = 0;
  for (int base = 0; base < n; base += 1024) {
    const int i = base + t;
    const int v = i < n && al[i] ? 1 : 0;
    const uint64_t ballot = __ballot(v);
    const int ln = lane_id(), wv = wave_id();
    const int before = __popcll(ballot & ((ln == 0) ? 0ull : (~0ull >> (kWave - ln))));
    if (ln == 0) wave_sum[wv] = __popcll(ballot);
    __syncthreads();
    int off = carry;
    for (int q = 0; q < wv; ++q) off += wave_sum[q];
    if (v) compact[i] = off + before;
    int tot = 0;
    for (int q = 0; q < 16; ++q) tot += wave_sum[q];
    carry += tot;
    __syncthreads();
  }
  for (int i = t; i < n; i += 1024) label[static_cast<int64_t>(lane) * M + i] = compact[parent[i]];
  if (t == 0) n_roots[lane] = carry;
}

// Stage-2 nodes of a lane (litgpt/log_kv_cache.py:3624-3655): old live
// clusters in ascending id (center, mass n_total), then the candidates in
// root order (center, mass = member count).
__global__ __launch_bounds__(256) void stage2_kernel(LadderArgs c, UnifiedBufs u) {
  __shared__ int old_s[kMaxClusters];
  __shared__ int n_old_s;
  extern __shared__ __align__(16) uint8_t dyn[];
  int32_t* members = reinterpret_cast<int32_t*>(dyn);   // [M]
  int32_t* roots = members + u.M;                       // [M]
  const int lane = blockIdx.x, K = c.k_max, M = u.M, D = u.D, t = threadIdx.x;
  const int n1 = u.count1[lane];
  if (n1 == 0) {
    if (t == 0) {
      u.count2[lane] = 0;
      u.n_old[lane] = 0;
    }
    return;
  }
  if (t == 0) {
    int k = 0;
    for (int cc = 0; cc < K; ++cc)
      if (c.alive[static_cast<int64_t>(lane) * K + cc]) {
        old_s[k] = cc;
        u.old_ids[static_cast<int64_t>(lane) * kMaxClusters + k] = cc;
        ++k;
      }
    n_old_s = k;
  }
  const int nr = u.n_roots1[lane];
  for (int i = t; i < nr; i += 256) members[i] = 0;
  __syncthreads();
  const int n_old = n_old_s;
  const uint8_t* al = u.alive1 + static_cast<int64_t>(lane) * M;
  const int32_t* lab = u.label1 + static_cast<int64_t>(lane) * M;
  for (int i = t; i < n1; i += 256) {
    atomicAdd(&members[lab[i]], 1);
    if (al[i]) roots[lab[i]] = i;
  }
  __syncthreads();
  float* mu2 = u.mu2 + static_cast<int64_t>(lane) * M * D;
  const float* mu1 = u.mu1 + static_cast<int64_t>(lane) * M * D;
  float* mass2 = u.mass2 + static_cast<int64_t>(lane) * M;
  const int m2 = n_old + nr;
  for (int i = t; i < m2 * D; i += 256) {
    const int row = i / D, d = i - row * D;
    mu2[i] = row < n_old ? c.centroid[(static_cast<int64_t>(lane) * K + old_s[row]) * c.dk + d]
                         : mu1[static_cast<int64_t>(roots[row - n_old]) * D + d];
  }
  for (int i = t; i < m2; i += 256)
    mass2[i] = i < n_old ? static_cast<float>(c.n_total[static_cast<int64_t>(lane) * K + old_s[i]])
                         : static_cast<float>(members[i - n_old]);
  if (t == 0) {
    u.count2[lane] = m2;
    u.n_old[lane] = n_old;
  }
}

// Final cluster of every row (position order, as the attach decisions) and
// the lane's old-old merges in trace order (litgpt/log_kv_cache.py:3656-3686):
// a root that is an old cluster keeps its id, a new root opens the next free
// id (free after the old-old merges), in root order.
__global__ __launch_bounds__(256) void final_kernel(LadderArgs c, RowsArgs r, UnifiedBufs u, const int32_t* order,
                                                    int8_t* assign) {
  __shared__ int target_s[kMaxClusters];
  __shared__ int n_target_s;
  const int lane = blockIdx.x, K = c.k_max, M = u.M, t = threadIdx.x;
  const int b = lane / c.n_groups;
  const int n1 = u.count1[lane];
  int32_t* jobs = u.jobs + static_cast<int64_t>(lane) * kMaxClusters * 2;
  if (n1 == 0) {
    if (t == 0) u.n_jobs[lane] = 0;
    return;
  }
  const int n_old = u.n_old[lane], m2 = u.count2[lane];
  const int32_t* old = u.old_ids + static_cast<int64_t>(lane) * kMaxClusters;
  if (t == 0) {
    const int32_t* tr = u.trace2 + static_cast<int64_t>(lane) * M * 2;
    uint32_t alive = 0;
    for (int cc = 0; cc < K; ++cc) alive |= (c.alive[static_cast<int64_t>(lane) * K + cc] ? 1u : 0u) << cc;
    int nj = 0;
    for (int p = 0; p < u.n_trace2[lane]; ++p) {
      const int x = tr[2 * p], y = tr[2 * p + 1];
      if (y < n_old) {
        jobs[2 * nj] = old[x];
        jobs[2 * nj + 1] = old[y];
        alive &= ~(1u << old[y]);
        ++nj;
      }
    }
    u.n_jobs[lane] = nj;
    const uint8_t* al = u.alive2 + static_cast<int64_t>(lane) * M;
    int k = 0, next_free = 0;
    for (int i = 0; i < m2 && k < kMaxClusters; ++i) {
      if (!al[i]) continue;
      if (i < n_old) {
        target_s[k] = old[i];
      } else {
        while (next_free < K && ((alive >> next_free) & 1u)) ++next_free;
        target_s[k] = next_free;
        alive |= 1u << next_free;
      }
      ++k;
    }
    n_target_s = k;
  }
  __syncthreads();
  const int n_target = n_target_s;
  const int T = r.tokens;
  const int32_t* ord = order + static_cast<int64_t>(b) * T;
  const int32_t* lab1 = u.label1 + static_cast<int64_t>(lane) * M;
  const int32_t* lab2 = u.label2 + static_cast<int64_t>(lane) * M;
  int8_t* as = assign + static_cast<int64_t>(lane) * T;
  // (A root past the table only arises when the budget stage is stuck, which the host rejects.)
  for (int s = t; s < T; s += 256) {
    const int root = s < n1 ? lab2[n_old + lab1[ord[s]]] : -1;
    as[s] = root >= 0 && root < n_target ? static_cast<int8_t>(target_s[root]) : -1;
  }
}

int launch_unified_plan(const LadderArgs& c, const RowsArgs& r, const UnifiedBufs& u, const Workspace& ws,
                        hipStream_t stream) {
  const int lanes = c.n_batch * c.n_groups, M = u.M, D = u.D;
  int rc = launch_order(r, c.n_batch, ws.order, nullptr, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(load_nodes_kernel, dim3(std::max(1, std::min(64, M * D / 4096)), lanes), dim3(256), 0, stream, r,
                     c.n_groups, u);
  // A capacity cap runs the full-recompute rounds (litgpt/log_kv_cache.py:3283-3288), else the
  // incremental reducer.
  const bool capped = u.cap > 0.f;
  auto rounds_args = [&](float* mu, const float* mass, const int32_t* count, const float* limit, int target,
                         int strict, uint8_t* alive, int32_t* trace, int32_t* n_trace, int32_t* stuck,
                         int32_t* stats) {
    return RoundArgs{mu, mass, count, limit, target, M, D, strict, u.cap,
                     {u.cmu[0], u.cmu[1]}, {u.cmass[0], u.cmass[1]}, {u.crad[0], u.crad[1]},
                     {u.croot[0], u.croot[1]}, u.n_cur, u.cbuf, u.dcount, u.keys, u.dist, alive, trace, n_trace,
                     stuck, u.rounds, stats, 2 * kStatsInts};
  };
  if (capped) {
    if ((rc = launch_rounds<true>(rounds_args(u.mu1, u.mass1, u.count1, u.limit, 1, 0, u.alive1, u.trace1,
                                              u.n_trace1, u.stuck1, u.stats),
                                  lanes, stream)))
      return rc;
  } else {
    if ((rc = launch_dist(u.mu1, u.count1, u.dist, M, D, lanes, stream))) return rc;
    ReduceArgs a1{u.dist, u.mu1, u.mass1, u.count1, u.limit, 1, M, D, u.alive1, u.trace1, u.n_trace1, u.stuck1,
                  u.bound, u.image, u.image_stride, u.ctl, u.live, u.stats, 2 * kStatsInts, 1, nullptr};
    if ((rc = launch_reduce<true>(a1, lanes, stream))) return rc;
  }
  const size_t lab_lds = static_cast<size_t>(M) * 8;
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&labels_kernel), lab_lds)) return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(labels_kernel, dim3(lanes), dim3(1024), lab_lds, stream, u.alive1, u.trace1, u.n_trace1, u.count1,
                     M, u.label1, u.n_roots1);
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&stage2_kernel), lab_lds)) return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(stage2_kernel, dim3(lanes), dim3(256), lab_lds, stream, c, u);
  if (capped) {
    if ((rc = launch_rounds<false>(rounds_args(u.mu2, u.mass2, u.count2, nullptr, c.k_max, 1, u.alive2, u.trace2,
                                               u.n_trace2, u.stuck2, u.stats ? u.stats + kStatsInts : nullptr),
                                   lanes, stream)))
      return rc;
  } else {
    if ((rc = launch_dist(u.mu2, u.count2, u.dist, M, D, lanes, stream))) return rc;
    ReduceArgs a2{u.dist, u.mu2, u.mass2, u.count2, nullptr, c.k_max, M, D, u.alive2, u.trace2, u.n_trace2,
                  u.stuck2, u.bound, u.image, u.image_stride, u.ctl, u.live, u.stats ? u.stats + kStatsInts : nullptr,
                  2 * kStatsInts, u.passes, u.restricted};
    if ((rc = launch_reduce<false>(a2, lanes, stream))) return rc;
  }
  hipLaunchKernelGGL(labels_kernel, dim3(lanes), dim3(1024), lab_lds, stream, u.alive2, u.trace2, u.n_trace2, u.count2,
                     M, u.label2, u.n_roots2);
  hipLaunchKernelGGL(final_kernel, dim3(lanes), dim3(256), 0, stream, c, r, u, ws.order, ws.assign);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

size_t unified_reduce_lds(int M) { return reduce_lds_bytes(M); }

int64_t unified_image_stride(int M) { return (static_cast<int64_t>(reduce_lds_bytes(M)) + 255) / 256 * 256; }

__global__ __launch_bounds__(256) void summary_kernel(const int32_t* __restrict__ n_jobs,
                                                      const int32_t* __restrict__ stuck, int lanes, int tokens,
                                                      int32_t* __restrict__ summary) {
  int most = 0, any = 0;
  for (int i = threadIdx.x; tokens && i < lanes; i += 256) {
    most = max(most, n_jobs[i]);
    any |= stuck[i];
  }
  for (int off = 32; off >= 1; off >>= 1) {
    most = max(most, __shfl_xor(most, off, kWave));
    any |= __shfl_xor(any, off, kWave);
  }
  __shared__ int m_s[4], a_s[4];
  if (lane_id() == 0) {
    m_s[wave_id()] = most;
    a_s[wave_id()] = any;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    summary[0] = max(max(m_s[0], m_s[1]), max(m_s[2], m_s[3]));
    summary[1] = a_s[0] | a_s[1] | a_s[2] | a_s[3];
  }
}

int launch_unified_summary(const LadderArgs& c, const UnifiedBufs& u, int32_t* summary, int tokens,
                           hipStream_t stream) {
  hipLaunchKernelGGL(summary_kernel, dim3(1), dim3(256), 0, stream, u.n_jobs, u.stuck2, c.n_batch * c.n_groups,
                     tokens, summary);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
