// Chunk attention on the matrix cores: many query rows per KV group (a prefill
// or training chunk) over the packed rows [pooled | exact | recent | current].
//
// Same math as the decode kernel (litgpt/log_kv_cache.py:6428-6464, :6751-6758):
// softmax(scale * [q, 1/scale] . [k, bias]) v, the last `causal_tail` rows
// causal against the query rows. Flash attention with gfx950's
// v_mfma_f32_32x32x16_bf16: a block of 8 waves (one per CU, two per SIMD)
// owns 256 query rows of one KV group, a wave 32 of them (one per lane
// column), so each staged K / V tile serves 256 queries. Per 64-row key tile,
// staged in LDS (K row-major, V transposed):
//   S^T = K Q^T   (keys x queries; each lane holds 16 keys of its own query),
//   online softmax per lane (its query's max and sum, the other 16 keys of the
//   32-key block in lane ^ 32),
//   O^T += V^T P^T (dv x queries) with v_mfma_f32_32x32x16_f16: P 2^15 in
//   fp16 (11 significant bits, RNE) against an fp16 copy of V 2^-k made per
//   launch, k chosen per lane so its largest magnitude lands in [2^15, 2^16);
//   the copy is exact when the lane's nonzero magnitudes span at most 29
//   binades (all land in fp16's normal range), and the output is scaled back
//   by 2^(k - 15) after the division by the softmax sum, so any bf16 exponent
//   works. fp16 P rounds P to 2^-11 relative, so an output errs by at most
//   2^-11 of its values' weighted mean magnitude. A lane whose V spans more
//   binades, or holds an infinity, NaN or subnormal, reads its bf16 V rows
//   instead and splits P 2^15 into high and low bf16 parts (two products per
//   step, P kept to about 2^-16).
// Queries live in registers for the whole key range; the K / V tiles are
// double-buffered in LDS with one barrier per tile.
// The P^T operand is the lane's own score registers: MFMA B operand element j
// of a 16-key step s is key 16s + 8(j/4) + 4(lane/32) + j%4, which is exactly
// accumulator element 8(s%2) + j of S^T block s/2, so V^T is read with the same
// key order and no data moves between lanes.
#include <algorithm>
#include <type_traits>

#include "route.hpp"

namespace logkv {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kWavesPerBlock = 8;                 // waves per block, each owning 32 query rows
constexpr int kThreads = 64 * kWavesPerBlock;
constexpr int kQRows = 32 * kWavesPerBlock;       // query rows per block
constexpr int kBlocksPerCu = 8 / kWavesPerBlock;  // resident blocks per CU (two waves per SIMD)
constexpr int kKeys = 64;        // key rows per staged tile
constexpr int kMaxSteps = 9;     // 16-wide steps of the packed width (<= 144)
constexpr int kLdK = 152;        // K tile row stride in LDS (bf16)
constexpr int kLdV = kKeys + 4;  // V^T row stride in LDS (bf16; 34 dwords: 16 rows' 8-byte reads hit distinct banks)
constexpr int kMaxDvBlocks = 4;  // dv <= 128
constexpr int kVSlices = 64;     // row slices of a lane's V in the fp16 copy
// vshift of a lane whose V has no exact fp16 copy (the bf16 path reads its rows).
constexpr int kBf16Lane = 1 << 20;
// P is scaled by 2^kPShift before its fp16 rounding (P <= 1, so P 2^15 < 65504).
constexpr int kPShift = 15;

__device__ __forceinline__ __bf16 to_bf16(float x) { return static_cast<__bf16>(x); }

// max / sum of the values of lanes l and l ^ 32, in every lane: one permlane
// swap leaves {x[l], x[l ^ 32]} in its two results (lower-half lane's value
// first), no LDS round trip.
__device__ __forceinline__ float pair_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The block's logical (query block, split, lane) in a grid of (query blocks,
// splits, lanes). Workgroups go to the 8 XCDs round robin in dispatch order,
// and each XCD has its own L2: dispatched block n takes logical block
// (n % 8) (N / 8) + n / 8 (N blocks, a multiple of 8), so an XCD runs one
// contiguous range of logical blocks - whole lanes when the lane count is a
// multiple of 8 - and a lane's K / V tiles, read by all of its query blocks,
// are fetched into one L2 instead of eight.
struct ChunkBlock {
  int qb, split, lane;
};
__device__ __forceinline__ ChunkBlock chunk_block() {
  const int nx = static_cast<int>(gridDim.x), ny = static_cast<int>(gridDim.y);
  const int n = nx * ny * static_cast<int>(gridDim.z);
  int lin = static_cast<int>(blockIdx.x) + nx * (static_cast<int>(blockIdx.y) + ny * static_cast<int>(blockIdx.z));
  if (n % 8 == 0) lin = (lin % 8) * (n / 8) + lin / 8;
  return ChunkBlock{lin % nx, (lin / nx) % ny, lin / (nx * ny)};
}

}  // namespace

// splits == 1: the block writes the output. splits > 1: block (x, s) covers the
// s-th of `splits` equal parts (whole 64-row tiles) of its queries' key range
// and writes partials [m, l, acc[dv]] per query (m in the base-2 domain).
// NKS 16-wide steps of the packed width and NDV 32-wide blocks of dv at
// compile time (straight-line tile code); columns past the packed width and
// V^T rows past dv are zero, so a kernel with more steps or blocks than the
// shape needs gives the same result.
// BF16V: the body of a lane without an exact fp16 V copy (vshift kBf16Lane).
template <int NKS, int NDV, bool BF16V>
__device__ __forceinline__ void chunk_body(const logkv_attention_args& a, const int32_t* __restrict__ width_ptr,
                                           int splits, float* __restrict__ part, const uint16_t* __restrict__ v16,
                                           int kv, const ChunkBlock blk_id) {
  // Two K / V^T tile buffers: tile i + 1 is written into the other buffer while
  // tile i is read, so one barrier per tile orders both.
  __shared__ __align__(16) uint16_t k_s[2][kKeys * kLdK];
  __shared__ __align__(16) uint16_t vt_s[2][kMaxDvBlocks * 32 * kLdV];
  const int lane_ix = blk_id.lane, split = blk_id.split, G = a.n_groups;
  const int b = lane_ix / G, g = lane_ix % G;
  const int rep = a.n_heads / G, nq = rep * a.tq;
  const int w = wave_id(), l = lane_id(), h = l >> 5, col = l & 31;
  const int dim = a.dim, ndv = a.dv / 32;
  const int qi = blk_id.qb * kQRows + w * 32 + col;
  const bool q_ok = qi < nq;
  const int qc = q_ok ? qi : nq - 1;
  const int head = g * rep + qc / a.tq, t = qc % a.tq;
  const int total = min(*width_ptr + a.tail + (a.alpha_count_dev ? *a.alpha_count_dev : 0), a.cap);
  const int tail0 = total - a.causal_tail;
  // Last key row any query of the block can see.
  const int q_first = blk_id.qb * kQRows, q_last = min(q_first + kQRows, nq) - 1;
  const int t_max = q_first / a.tq == q_last / a.tq ? q_last % a.tq : a.tq - 1;
  const int key_end = a.causal_tail ? min(total, tail0 + t_max + 1) : total;
  // This block's part of the key range, in whole tiles.
  const int tiles = (key_end + kKeys - 1) / kKeys, per = (tiles + splits - 1) / splits;
  const int k_begin = min(split * per, tiles) * kKeys, k_stop = min(min((split + 1) * per, tiles) * kKeys, key_end);

  // The lane's query [q, 1/scale, 0...] as MFMA B fragments (dims 16 ks + 8 h
  // .. + 8), held in registers for the whole key range.
  bf16x8 qf[NKS];
  {
    const LOGKV_G uint16_t* qrow = gp(a.q) + b * a.q_sb + head * a.q_sh + t * a.q_st;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      uint16_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = 16 * ks + 8 * h + j;
        e[j] = d < a.dk ? qrow[d] : (d == a.dk ? f32_to_bf16(a.inv_scale_bf16) : uint16_t(0));
      }
      qf[ks] = __builtin_bit_cast(bf16x8, make_uint4(e[0] | (uint32_t(e[1]) << 16), e[2] | (uint32_t(e[3]) << 16),
                                                     e[4] | (uint32_t(e[5]) << 16), e[6] | (uint32_t(e[7]) << 16)));
    }
  }
  // Columns past the packed width and V^T rows past dv stay zero in every
  // tile of both buffers.
  for (int i = threadIdx.x; i < 2 * kKeys * (kLdK - dim); i += blockDim.x) {
    const int bf = i / (kKeys * (kLdK - dim)), rest = i - bf * kKeys * (kLdK - dim);
    const int r = rest / (kLdK - dim), c = dim + rest % (kLdK - dim);
    k_s[bf][r * kLdK + c] = 0;
  }
  for (int i = threadIdx.x; i < 2 * (32 * NDV - a.dv) * kLdV; i += blockDim.x) {
    const int bf = i / ((32 * NDV - a.dv) * kLdV), rest = i - bf * (32 * NDV - a.dv) * kLdV;
    vt_s[bf][a.dv * kLdV + rest] = 0;
  }
  f32x16 o[NDV];
#pragma unroll
  for (int blk = 0; blk < NDV; ++blk)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[blk][i] = 0.f;
  float m = -__builtin_inff(), lsum = 0.f;   // running maximum of s * scale * log2(e), and the sum
  const LOGKV_G uint16_t* kbase = gp(a.k) + static_cast<int64_t>(lane_ix) * a.cap * dim;
  // The lane's V source: its fp16 copy (V 2^-k), or its bf16 packed rows.
  const LOGKV_G uint16_t* vbase = BF16V ? gp(a.v) + static_cast<int64_t>(lane_ix) * a.cap * dim
                                        : gp(v16) + static_cast<int64_t>(lane_ix) * a.cap * a.dv;
  const int vstride = BF16V ? dim : a.dv;
  const int units = dim / 8;
  const int vunits = a.dv / 8;
  // Each thread's staging tasks are the same in every tile: up to kKTasks
  // 16-byte K units (row, unit) and kVTasks V tasks (key pair, 8-wide dv unit).
  constexpr int kKTasks = (kKeys * kMaxSteps * 2 + kThreads - 1) / kThreads, kVTasks = (kKeys / 2) * 16 / kThreads;
  int k_row[kKTasks], k_goff[kKTasks], k_loff[kKTasks];
#pragma unroll
  for (int q = 0; q < kKTasks; ++q) {
    const int i = threadIdx.x + kThreads * q;
    const bool ok = i < kKeys * units;
    const int r = ok ? i / units : kKeys, u = ok ? i - (i / units) * units : 0;
    k_row[q] = r;
    k_goff[q] = 8 * u;
    k_loff[q] = r * kLdK + 8 * u;
  }
  int v_pair[kVTasks], v_unit[kVTasks];
#pragma unroll
  for (int q = 0; q < kVTasks; ++q) {
    const int i = threadIdx.x + kThreads * q;
    v_pair[q] = i < (kKeys / 2) * vunits ? i % (kKeys / 2) : -1;
    v_unit[q] = i / (kKeys / 2);
  }
  // Registers of the next tile (loaded while the current one is computed).
  uint4 kx[kKTasks], vx[kVTasks][2];
  auto load_tile = [&](int t0) {
    const int rows = min(kKeys, k_stop - t0);
#pragma unroll
    for (int q = 0; q < kKTasks; ++q) {
      const int r = min(k_row[q], rows - 1);
      kx[q] = *(const LOGKV_G uint4*)(kbase + static_cast<int64_t>(t0 + r) * dim + k_goff[q]);
      if (k_row[q] >= rows) kx[q] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < kVTasks; ++q) {
      const int kp = v_pair[q] < 0 ? 0 : v_pair[q];
      const int r0 = min(2 * kp, rows - 1), r1 = min(2 * kp + 1, rows - 1);
      vx[q][0] = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(t0 + r0) * vstride + 8 * v_unit[q]);
      vx[q][1] = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(t0 + r1) * vstride + 8 * v_unit[q]);
      if (2 * kp >= rows) vx[q][0] = make_uint4(0, 0, 0, 0);
      if (2 * kp + 1 >= rows) vx[q][1] = make_uint4(0, 0, 0, 0);
    }
  };
  // K rows row-major; V transposed: each task's two key rows of one 8-wide dv
  // unit become 8 dwords (key pairs). Rows past the end are zeros.
  auto store_tile = [&](int bf) {
#pragma unroll
    for (int q = 0; q < kKTasks; ++q)
      if (k_row[q] < kKeys) *reinterpret_cast<uint4*>(&k_s[bf][k_loff[q]]) = kx[q];
#pragma unroll
    for (int q = 0; q < kVTasks; ++q) {
      if (v_pair[q] < 0) continue;
      const uint32_t a0[4] = {vx[q][0].x, vx[q][0].y, vx[q][0].z, vx[q][0].w};
      const uint32_t a1[4] = {vx[q][1].x, vx[q][1].y, vx[q][1].z, vx[q][1].w};
      const int r0 = 2 * v_pair[q], u = v_unit[q];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = __builtin_amdgcn_perm(a1[j], a0[j], 0x05040100u);   // low halves of rows r0, r0 + 1
        const uint32_t hi = __builtin_amdgcn_perm(a1[j], a0[j], 0x07060302u);   // high halves
        *reinterpret_cast<uint32_t*>(&vt_s[bf][(8 * u + 2 * j) * kLdV + r0]) = lo;
        *reinterpret_cast<uint32_t*>(&vt_s[bf][(8 * u + 2 * j + 1) * kLdV + r0]) = hi;
      }
    }
  };
  const int ntiles = k_begin < k_stop ? (k_stop - k_begin + kKeys - 1) / kKeys : 0;
  if (ntiles > 0) {
    load_tile(k_begin);
    store_tile(0);
    if (ntiles > 1) load_tile(k_begin + kKeys);
  }
  __syncthreads();

  const float c2 = a.scale * 1.44269504088896341f;
  // One key tile; MASKED tiles evaluate the row and causal masks, the others
  // (every row present, none past the causal limit) skip them.
  auto tile = [&](int it, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int t0 = k_begin + it * kKeys, bf = it & 1;
    const int rows = min(kKeys, k_stop - t0);
    const uint16_t* kt = k_s[bf];
    const uint16_t* vt = vt_s[bf];
    // S^T = K Q^T over the packed width, the two 32-key blocks' chains
    // interleaved.
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb][i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(kt + col * kLdK + 16 * ks + 8 * h);
      const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(kt + (32 + col) * kLdK + 16 * ks + 8 * h);
      s[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k0, qf[ks], s[0], 0, 0, 0);
      s[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k1, qf[ks], s[1], 0, 0, 0);
    }
    // Online softmax of this lane's query in the base-2 domain: with c2 = scale
    // * log2(e), p = 2^(s c2 - m) where m is the running maximum of s c2.
    float mx = -__builtin_inff();
    if constexpr (MASKED) {
      // Visible keys of this lane's query: t0 .. t0 + lim - 1 (past the rows,
      // and past tail0 + t under the causal mask, are masked); element i of
      // block kb is key t0 + 32 kb + 8 (i / 4) + 4 h + i % 4.
      const int lim = (a.causal_tail ? min(rows, tail0 + t + 1 - t0) : rows) - 4 * h;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[kb][i] = 32 * kb + 8 * (i / 4) + (i % 4) < lim ? s[kb][i] : -__builtin_inff();
          mx = fmaxf(mx, s[kb][i]);
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    }
    mx = pair_max32(mx);
    const float m_new = fmaxf(m, mx * c2);
    const float mb = m_new == -__builtin_inff() ? 0.f : m_new;
    const float corr = __builtin_amdgcn_exp2f(m - mb);
    // p' = 2^(s c2 - m + 15) = P 2^15; the sum is taken of p' and scaled
    // back by 2^-15 (exact).
    const float arg0 = static_cast<float>(kPShift) - mb;
    float sum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], c2, arg0));
        s[kb][i] = p;
        sum += p;
      }
    }
    sum = pair_sum32(sum) * __builtin_ldexpf(1.f, -kPShift);
    lsum = lsum * corr + sum;
    m = m_new;
    if (__ballot(corr != 1.f)) {
#pragma unroll
      for (int blk = 0; blk < NDV; ++blk)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[blk][i] *= corr;
    }
    // O^T += V^T P^T, four 16-key steps, P rounded to fp16 (bf16 lanes: P as
    // high + low bf16 parts against the bf16 V rows).
    if constexpr (BF16V) {
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p0 = s[st / 2][8 * (st % 2) + 2 * j], p1 = s[st / 2][8 * (st % 2) + 2 * j + 1];
          const uint16_t h0 = f32_to_bf16(p0), h1 = f32_to_bf16(p1);
          const float r0 = p0 - __uint_as_float(static_cast<uint32_t>(h0) << 16);
          const float r1 = p1 - __uint_as_float(static_cast<uint32_t>(h1) << 16);
          hw[j] = h0 | (static_cast<uint32_t>(h1) << 16);
          lw[j] = f32_to_bf16(r0) | (static_cast<uint32_t>(f32_to_bf16(r1)) << 16);
        }
        const bf16x8 ph = __builtin_bit_cast(bf16x8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
        const bf16x8 pl = __builtin_bit_cast(bf16x8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
#pragma unroll
        for (int blk = 0; blk < NDV; ++blk) {
          const uint16_t* vr = vt + (32 * blk + col) * kLdV + 16 * st + 4 * h;
          const uint2 v0 = *reinterpret_cast<const uint2*>(vr);
          const uint2 v1 = *reinterpret_cast<const uint2*>(vr + 8);
          const bf16x8 vb = __builtin_bit_cast(bf16x8, make_uint4(v0.x, v0.y, v1.x, v1.y));
          o[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, ph, o[blk], 0, 0, 0);
          o[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, pl, o[blk], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      f16x2 pw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p0 = s[st / 2][8 * (st % 2) + 2 * j], p1 = s[st / 2][8 * (st % 2) + 2 * j + 1];
        pw[j] = __builtin_convertvector(f32x2{p0, p1}, f16x2);   // RNE
      }
      const f16x8 ph = __builtin_bit_cast(f16x8, make_uint4(__builtin_bit_cast(uint32_t, pw[0]),
                                                            __builtin_bit_cast(uint32_t, pw[1]),
                                                            __builtin_bit_cast(uint32_t, pw[2]),
                                                            __builtin_bit_cast(uint32_t, pw[3])));
      f16x8 vf[NDV];
#pragma unroll
      for (int blk = 0; blk < NDV; ++blk) {
        const uint16_t* vr = vt + (32 * blk + col) * kLdV + 16 * st + 4 * h;
        const uint2 v0 = *reinterpret_cast<const uint2*>(vr);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vr + 8);
        vf[blk] = __builtin_bit_cast(f16x8, make_uint4(v0.x, v0.y, v1.x, v1.y));
      }
#pragma unroll
      for (int blk = 0; blk < NDV; ++blk) o[blk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[blk], ph, o[blk], 0, 0, 0);
    }
    }
    if (it + 1 < ntiles) {
      store_tile(bf ^ 1);
      if (it + 2 < ntiles) load_tile(t0 + 2 * kKeys);
    }
    __syncthreads();
  };
  // Tiles below min(k_stop, tail0) (tail0 only under the causal mask) are full.
  const int full_end = a.causal_tail ? min(k_stop, tail0) : k_stop;
  const int n_full = min(ntiles, full_end > k_begin ? (full_end - k_begin) / kKeys : 0);
  for (int it = 0; it < n_full; ++it) tile(it, std::false_type{});
  for (int it = n_full; it < ntiles; ++it) tile(it, std::true_type{});
  if (!q_ok) return;
  if (splits > 1) {
    float* pp = part + ((static_cast<int64_t>(lane_ix) * splits + split) * nq + qi) * (a.dv + 2);
    if (h == 0) {
      pp[0] = m;
      pp[1] = lsum;
    }
#pragma unroll
    for (int blk = 0; blk < NDV; ++blk) {
      if (blk < ndv) {
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int d = 32 * blk + 8 * i4 + 4 * h;
#pragma unroll
          for (int j = 0; j < 4; ++j) pp[2 + d + j] = o[blk][4 * i4 + j];
        }
      }
    }
    return;
  }
  // o holds 2^(15 - k) sum P V: divided by the sum, then scaled by 2^(k - 15) exactly.
  const int oexp = (BF16V ? 0 : kv) - kPShift;
  LOGKV_G uint16_t* orow = gp(a.out) + b * a.o_sb + head * a.o_sh + t * a.o_st;
#pragma unroll
  for (int blk = 0; blk < NDV; ++blk) {
    if (blk < ndv) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d = 32 * blk + 8 * i4 + 4 * h;
        float y[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = __builtin_ldexpf(o[blk][4 * i4 + j] / lsum, oexp);
        const uint32_t lo = static_cast<uint32_t>(f32_to_bf16(y[0])) | (static_cast<uint32_t>(f32_to_bf16(y[1])) << 16);
        const uint32_t hi = static_cast<uint32_t>(f32_to_bf16(y[2])) | (static_cast<uint32_t>(f32_to_bf16(y[3])) << 16);
        *(LOGKV_G uint2*)(orow + d) = make_uint2(lo, hi);
      }
    }
  }
}

template <int NKS, int NDV>
__global__ __launch_bounds__(kThreads, kBlocksPerCu) void chunk_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr,
                                                       int splits, float* __restrict__ part,
                                                       const uint16_t* __restrict__ v16,
                                                       const int32_t* __restrict__ vshift) {
  const ChunkBlock id = chunk_block();
  const int kv = vshift[id.lane];
  if (kv == kBf16Lane) chunk_body<NKS, NDV, true>(a, width_ptr, splits, part, v16, kv, id);
  else chunk_body<NKS, NDV, false>(a, width_ptr, splits, part, v16, kv, id);
}

// The fp16 copy of the packed V (rows [0, total) of every lane, dv features):
// vmax_kernel takes the largest and the smallest nonzero bf16 magnitude (as
// bits) of each of a lane's kVSlices row slices; vconv_kernel reduces them to
// the lane's shift k = E_max - 15 (E_max the largest value's exponent, so the
// largest scaled magnitude is in [2^15, 2^16) and at most 65280) and writes V
// 2^-k as fp16 by moving the exponent field (exact: bf16 has 8 significant
// bits, fp16 11, and every nonzero value lands in fp16's normal range when
// E_max - E_min <= 29). Other lanes - wider spans, infinities, NaNs, bf16
// subnormals - get vshift = kBf16Lane and no copy.
__device__ __forceinline__ int chunk_rows(const logkv_attention_args& a, const int32_t* width_ptr) {
  return min(*width_ptr + a.tail + (a.alpha_count_dev ? *a.alpha_count_dev : 0), a.cap);
}

__global__ __launch_bounds__(256) void vmax_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr,
                                                   int32_t* __restrict__ vmax) {
  const int slice = blockIdx.x, lane_ix = blockIdx.y;
  const int total = chunk_rows(a, width_ptr);
  const int per = (total + kVSlices - 1) / kVSlices, r0 = slice * per, r1 = min(total, r0 + per);
  const int units = a.dv / 8;
  const LOGKV_G uint16_t* vbase = gp(a.v) + static_cast<int64_t>(lane_ix) * a.cap * a.dim;
  uint32_t mx = 0, mn = 0xffffu;   // largest magnitude, smallest nonzero one (0xffff: none)
  for (int i = threadIdx.x; i < (r1 - r0) * units; i += blockDim.x) {
    const int row = r0 + i / units, u = i % units;
    const uint4 x = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(row) * a.dim + 8 * u);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t m0 = w[j] & 0x7fffu, m1 = (w[j] >> 16) & 0x7fffu;
      mx = max(mx, max(m0, m1));
      mn = min(mn, min(m0 ? m0 : 0xffffu, m1 ? m1 : 0xffffu));
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), off, 64)));
    mn = min(mn, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mn), off, 64)));
  }
  __shared__ uint32_t red[2][4];
  if (lane_id() == 0) {
    red[0][wave_id()] = mx;
    red[1][wave_id()] = mn;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t* out = vmax + 2 * (lane_ix * kVSlices + slice);
    out[0] = static_cast<int32_t>(max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3])));
    out[1] = static_cast<int32_t>(min(min(red[1][0], red[1][1]), min(red[1][2], red[1][3])));
  }
}

__global__ __launch_bounds__(256) void vconv_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr,
                                                    const int32_t* __restrict__ vmax, int32_t* __restrict__ vshift,
                                                    uint16_t* __restrict__ v16) {
  const int slice = blockIdx.x, lane_ix = blockIdx.y;
  __shared__ int shift_s;
  if (threadIdx.x < kWave) {
    const int4 pair = *reinterpret_cast<const int4*>(vmax + 2 * (lane_ix * kVSlices + 2 * threadIdx.x % kVSlices));
    uint32_t mx = static_cast<uint32_t>(max(pair.x, pair.z)), mn = static_cast<uint32_t>(min(pair.y, pair.w));
    for (int off = 32; off >= 1; off >>= 1) {
      mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), off, 64)));
      mn = min(mn, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mn), off, 64)));
    }
    if (threadIdx.x == 0) {
      // Exponent fields (biased by 127): 0 is a subnormal, 255 an infinity or NaN.
      const int emax = static_cast<int>(mx >> 7), emin = static_cast<int>(mn >> 7);
      const bool exact = mx == 0 || (emax < 255 && emin >= 1 && emax - emin <= 29);
      shift_s = exact ? (mx == 0 ? 0 : emax - 127 - 15) : kBf16Lane;
      if (slice == 0) vshift[lane_ix] = shift_s;
    }
  }
  __syncthreads();
  const int k = shift_s;
  if (k == kBf16Lane) return;
  const int total = chunk_rows(a, width_ptr);
  const int per = (total + kVSlices - 1) / kVSlices, r0 = slice * per, r1 = min(total, r0 + per);
  const int units = a.dv / 8;
  const LOGKV_G uint16_t* vbase = gp(a.v) + static_cast<int64_t>(lane_ix) * a.cap * a.dim;
  uint16_t* obase = v16 + static_cast<int64_t>(lane_ix) * a.cap * a.dv;
  // bf16 exponent field e (value 1.m 2^(e - 127)) -> fp16 field e - 127 - k + 15, in [1, 30] here.
  const int ebias = 127 + k - 15;
  auto conv = [&](uint32_t x) -> uint32_t {
    const uint32_t mag = x & 0x7fffu;
    const uint32_t h = mag ? ((static_cast<uint32_t>(static_cast<int>(mag >> 7) - ebias) << 10) | ((mag & 0x7fu) << 3))
                           : 0u;
    return h | ((x >> 15) << 15);
  };
  for (int i = threadIdx.x; i < (r1 - r0) * units; i += blockDim.x) {
    const int row = r0 + i / units, u = i % units;
    const uint4 x = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(row) * a.dim + 8 * u);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = conv(w[j] & 0xffffu) | (conv(w[j] >> 16) << 16);
    *reinterpret_cast<uint4*>(obase + static_cast<int64_t>(row) * a.dv + 8 * u) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Partials of the key-range splits combined in split order: eight queries per
// block, 32 threads per query, four output features per thread (dv <= 128). A
// partial's maximum m is of s * scale * log2(e), so a split's weight is
// 2^(m_split - m).
constexpr int kCombineQueries = 8;
__global__ __launch_bounds__(256) void chunk_combine_kernel(logkv_attention_args a, const float* __restrict__ part,
                                                            int splits, const int32_t* __restrict__ vshift) {
  const int lane_ix = blockIdx.y, G = a.n_groups;
  const int b = lane_ix / G, g = lane_ix % G;
  const int rep = a.n_heads / G, nq = rep * a.tq;
  const int qi = blockIdx.x * kCombineQueries + static_cast<int>(threadIdx.x) / 32;
  const int d = 4 * (static_cast<int>(threadIdx.x) % 32);
  if (qi >= nq || d >= a.dv) return;
  const int stride = a.dv + 2;
  const float* base = part + (static_cast<int64_t>(lane_ix) * splits * nq + qi) * stride;
  const int64_t step = static_cast<int64_t>(nq) * stride;
  float m = -__builtin_inff();
  for (int sp = 0; sp < splits; ++sp) m = fmaxf(m, base[sp * step]);
  float lsum = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < splits; ++sp) {
    const float* pp = base + sp * step;
    if (pp[0] == -__builtin_inff()) continue;
    const float f = __builtin_amdgcn_exp2f(pp[0] - m);   // maxima are in the base-2 domain
    lsum += pp[1] * f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] += pp[2 + d + j] * f;
  }
  const int head = g * rep + qi / a.tq, t = qi % a.tq;
  // Partials hold 2^(15 - k) sum P V (see chunk_kernel's output).
  const int kv = vshift[lane_ix], oexp = (kv == kBf16Lane ? 0 : kv) - kPShift;
  float y[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = __builtin_ldexpf(acc[j] / lsum, oexp);
  LOGKV_G uint16_t* o = gp(a.out) + b * a.o_sb + head * a.o_sh + t * a.o_st + d;
  const uint32_t lo = static_cast<uint32_t>(f32_to_bf16(y[0])) | (static_cast<uint32_t>(f32_to_bf16(y[1])) << 16);
  const uint32_t hi = static_cast<uint32_t>(f32_to_bf16(y[2])) | (static_cast<uint32_t>(f32_to_bf16(y[3])) << 16);
  *reinterpret_cast<LOGKV_G uint2*>(o) = make_uint2(lo, hi);
}

// Key-range splits: enough blocks for one resident round (kBlocksPerCu per
// CU of the 256), at most one split per 1024 rows of the packed capacity.
int chunk_splits(const logkv_attention_args& a) {
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  const int64_t blocks = static_cast<int64_t>((nq + kQRows - 1) / kQRows) * a.n_batch * a.n_groups;
  const int64_t target = 256 * kBlocksPerCu;
  int splits = static_cast<int>((target + blocks - 1) / blocks);
  splits = std::min(splits, std::max(1, a.cap / 1024));
  return std::max(1, std::min(splits, 16));
}

// Workspace: [partials of the key-range splits (splits > 1)] [vmax: lanes x
// kVSlices x 2] [vshift: lanes] [fp16 V: lanes x cap x dv], regions 256-byte
// aligned.
struct ChunkWs {
  float* part;
  int32_t* vmax;
  int32_t* vshift;
  uint16_t* v16;
  int64_t bytes;
};

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

static ChunkWs chunk_ws(const logkv_attention_args& a, void* base) {
  const int splits = chunk_splits(a);
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  const int64_t lanes = static_cast<int64_t>(a.n_batch) * a.n_groups;
  uint8_t* b = static_cast<uint8_t*>(base);
  int64_t off = 0;
  ChunkWs w{};
  w.part = splits > 1 && b ? reinterpret_cast<float*>(b + off) : nullptr;
  if (splits > 1) off += align256(lanes * splits * nq * (a.dv + 2) * 4);
  w.vmax = b ? reinterpret_cast<int32_t*>(b + off) : nullptr;
  off += align256(lanes * kVSlices * 2 * 4);
  w.vshift = b ? reinterpret_cast<int32_t*>(b + off) : nullptr;
  off += align256(lanes * 4);
  w.v16 = b ? reinterpret_cast<uint16_t*>(b + off) : nullptr;
  off += align256(lanes * a.cap * a.dv * 2);
  w.bytes = off;
  return w;
}

int64_t chunk_workspace_floats(const logkv_attention_args& a) { return chunk_ws(a, nullptr).bytes / 4; }

int launch_chunk_attention(const logkv_attention_args& a, const int32_t* width, float* ws, hipStream_t stream) {
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  const int splits = chunk_splits(a);
  const ChunkWs w = chunk_ws(a, ws);
  const dim3 grid((nq + kQRows - 1) / kQRows, splits, a.n_batch * a.n_groups);
  const dim3 vgrid(kVSlices, a.n_batch * a.n_groups);
  hipLaunchKernelGGL(vmax_kernel, vgrid, dim3(256), 0, stream, a, width, w.vmax);
  hipLaunchKernelGGL(vconv_kernel, vgrid, dim3(256), 0, stream, a, width, w.vmax, w.vshift, w.v16);
  // Shapes with at most 5 steps and 2 dv blocks (head dim 64) take the
  // smaller kernel; every other shape runs the full 9 x 4 one on zero padding.
  if (a.dim <= 80 && a.dv <= 64)
    hipLaunchKernelGGL((chunk_kernel<5, 2>), grid, dim3(kThreads), 0, stream, a, width, splits, w.part, w.v16,
                       w.vshift);
  else
    hipLaunchKernelGGL((chunk_kernel<kMaxSteps, kMaxDvBlocks>), grid, dim3(kThreads), 0, stream, a, width, splits,
                       w.part, w.v16, w.vshift);
  if (splits > 1)
    hipLaunchKernelGGL(chunk_combine_kernel, dim3((nq + kCombineQueries - 1) / kCombineQueries, a.n_batch * a.n_groups),
                       dim3(256), 0, stream, a, w.part, splits, w.vshift);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
