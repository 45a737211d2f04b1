// Attention readout: mid-anchor slot plan, packed K/V workspace, decode attention.
//
// Plan (litgpt/log_kv_cache.py:5979-6007): per lane, occupied slots cluster by
// cluster, top level first, slots in order; anchor (2*sum_wp + w) // (2*w) with
// w as an integer >= 1; valid = w > 0. The pooled width is the largest lane
// count; it stays on the device, so readout never waits for the host.
//
// Pack (litgpt/log_kv_pack.py:27-72, litgpt/log_kv_pack_triton.py:12-92): rows
// [pooled | exact pool | recent | current] of width `dim`; pooled and exact keys
// rotated (rotate-half RoPE) at their anchor, the products rounded to bf16
// first when the tables are bf16; column dk holds log(max(w, 1)) for valid
// pooled rows, 0 for valid exact / recent / current rows, -10000 for invalid
// rows, which are zero otherwise.
//
// Decode attention (litgpt/log_kv_cache.py:6428-6464, :6751-6758):
// softmax(scale * [q, 1/scale] . [k, bias]) v over the packed rows, the last
// `causal_tail` rows causal against the queries, query head h reading KV group
// h / (Hq / G). Flash-decoding: row splits per lane, each staging 64-row K and
// V tiles in LDS with an online softmax; a second kernel combines the splits in
// a fixed order.
#include <algorithm>
#include <type_traits>

#include "route.hpp"

namespace logkv {

namespace {

typedef __bf16 rd_bf16x2 __attribute__((ext_vector_type(2)));
constexpr int kPlanThreads = 1024;
constexpr int kTile = 64;          // rows per staged K/V tile
constexpr int kSplitRows = 512;    // rows per attention split (staged decode kernel)
constexpr int kStreamRows = 512;   // most rows per split of the streaming kernel when the grid is not the limit
constexpr int kStreamBlocks = 640;    // streaming blocks per launch at most: 2.5 per CU, so splits are long enough to
                                      // amortize a block's start and end (1280 / 1024 / 512 / 320 measured slower)
constexpr int kMaxQ = 16;          // queries per KV group (heads per group x query rows)
constexpr int kMaxPacked = 264;    // packed row width limit (dk + 1 rounded to 8, dv)
constexpr int kAccPerThread = kMaxQ * kMaxDim / 256;   // outputs per thread of a 256-thread split block

struct PlanCtx {
  const LOGKV_G int16_t* count;    // [lanes, K, L]
  int K, L;
};

// Lane pooled-row prefix over (cluster, level top-down) blocks -> plan table
// [lanes, K*L + 1] (offsets), plus the maximum lane count at table[lanes*(K*L+1)].
// One thread per lane; a lane's counts are loaded kPlanChunk at a time, all
// before the chunk's prefix stores.
constexpr int kPlanChunk = 32;

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(logkv_readout_view c, int32_t* __restrict__ table) {
  __shared__ int wave_max[kPlanThreads / kWave];
  const int lanes = c.n_batch * c.n_groups;
  const int L = c.levels, KL = c.k_max * L;
  int best = 0;
  for (int lane = threadIdx.x; lane < lanes; lane += kPlanThreads) {
    const LOGKV_G int16_t* cnt = gp(c.level_count) + static_cast<int64_t>(lane) * KL;
    LOGKV_G int32_t* row = gp(table) + static_cast<int64_t>(lane) * (KL + 1);
    int acc = 0;
    for (int j0 = 0; j0 < KL; j0 += kPlanChunk) {
      int v[kPlanChunk];
#pragma unroll
      for (int q = 0; q < kPlanChunk; ++q) {
        // Table entry j = cc * L + k is cluster cc's level L - 1 - k (top level first).
        const int j = min(j0 + q, KL - 1), cc = j / L, k = j - cc * L;
        v[q] = cnt[cc * L + (L - 1 - k)];
      }
#pragma unroll
      for (int q = 0; q < kPlanChunk; ++q) {
        if (j0 + q < KL) {
          row[j0 + q] = acc;
          acc += v[q];
        }
      }
    }
    row[KL] = acc;
    best = acc > best ? acc : best;
  }
  for (int off = kWave / 2; off >= 1; off >>= 1) best = max(best, __shfl_xor(best, off, kWave));
  if (lane_id() == 0) wave_max[wave_id()] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    int m = 0;
    for (int i = 0; i < kPlanThreads / kWave; ++i) m = wave_max[i] > m ? wave_max[i] : m;
    table[static_cast<int64_t>(lanes) * (KL + 1)] = m;
  }
}

__device__ __forceinline__ float lo_bf16(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

__device__ __forceinline__ float table_at(const void* t, int64_t i, int bf16) {
  return bf16 ? bf16_to_f32(gp(static_cast<const uint16_t*>(t))[i]) : gp(static_cast<const float*>(t))[i];
}

constexpr int kPackRows = 64;   // packed rows per pack block
constexpr int kPackBatch = 4;   // units per thread whose loads are issued before their arithmetic

// Source of one packed row.
struct PackSrc {
  const LOGKV_G uint16_t* k;
  const LOGKV_G uint16_t* v;
  int64_t pos;
  float bias;     // column dk: log(max(w, 1)) / 0 for valid rows, -10000 for invalid ones
  int flags;      // bit 0 valid, bit 1 rotate, bit 2 row exists in the output
};

__device__ __forceinline__ void store_bf16x4(LOGKV_G uint16_t* dst, const float* o) {
  uint2 packed;
  packed.x = static_cast<uint32_t>(f32_to_bf16(o[0])) | (static_cast<uint32_t>(f32_to_bf16(o[1])) << 16);
  packed.y = static_cast<uint32_t>(f32_to_bf16(o[2])) | (static_cast<uint32_t>(f32_to_bf16(o[3])) << 16);
  *reinterpret_cast<LOGKV_G uint2*>(dst) = packed;
}

// Packed key feature d: rotate-half RoPE at the row's anchor for rotated rows
// (products rounded to bf16 first with bf16 tables), the row's bias at column
// dk, zero past it and for invalid rows.
__device__ __forceinline__ float rope_out(const logkv_readout_view& c, const PackSrc& r, int d, float x, float other,
                                          float cs, float sn, int half, bool valid) {
  float kx = x;
  if ((r.flags & 2) && d < c.rope_n) {
    const float rot = d < half ? -other : other;
    float a = kx * cs, bb = rot * sn;
    if (c.table_bf16) {
      a = round_bf16(a);
      bb = round_bf16(bb);
    }
    kx = round_bf16(a + bb);
  }
  return d < c.dk ? (valid ? kx : 0.f) : (d == c.dk ? r.bias : 0.f);
}

// The K and V units (4 features each) of a tile: kPackBatch (row, unit)
// items per thread with all their loads (row features, rotate-half partners,
// table entries, value features: one vector load each) issued before the
// arithmetic. Needs contiguous tables with 4-aligned position strides and
// rope_n a multiple of 8, so a unit lies wholly on one side of half, of
// rope_n and of dk (dk, dv multiples of 4).
template <bool BF16_TABLE>
__device__ __forceinline__ void pack_units_vec(const logkv_readout_view& c, const logkv_pack_args& p,
                                               const PackSrc* src, int s0, int lane, int units, int half) {
  const int tid = static_cast<int>(threadIdx.x), nthr = static_cast<int>(blockDim.x);
  const int items = kPackRows * units;
  // Row of item i = floor((i + 0.5) / units) in float: the quotient is at
  // least 0.5 / units (>= 1/132) from an integer and the float error is below
  // 64 * 2^-23, so truncation gives the exact row.
  const float inv_units = 1.0f / static_cast<float>(units);
  using TableUnit = typename std::conditional<BF16_TABLE, uint2, float4>::type;
  for (int i0 = tid; i0 < items; i0 += kPackBatch * nthr) {
    uint2 xu[kPackBatch], pu[kPackBatch], vu[kPackBatch];
    TableUnit cu[kPackBatch], su[kPackBatch];
    int rr[kPackBatch], d0s[kPackBatch];
#pragma unroll
    for (int q = 0; q < kPackBatch; ++q) {
      const int i = min(i0 + q * nthr, items - 1);
      rr[q] = static_cast<int>((static_cast<float>(i) + 0.5f) * inv_units);
      d0s[q] = 4 * (i - rr[q] * units);
      const PackSrc& r = src[rr[q]];
      const int d0r = d0s[q];
      const int d0 = d0r < c.dk ? d0r : 0;
      const int pd = d0 < c.rope_n ? (d0 < half ? d0 + half : d0 - half) : d0;
      const int rd = d0 < c.rope_n ? d0 : 0;
      const int64_t pos = r.pos < 0 ? 0 : (r.pos >= c.rope_rows ? c.rope_rows - 1 : r.pos);
      xu[q] = *reinterpret_cast<const LOGKV_G uint2*>(r.k + d0);
      pu[q] = *reinterpret_cast<const LOGKV_G uint2*>(r.k + pd);
      vu[q] = *reinterpret_cast<const LOGKV_G uint2*>(r.v + (d0r < c.dv ? d0r : 0));
      if constexpr (BF16_TABLE) {
        cu[q] = *reinterpret_cast<const LOGKV_G uint2*>(gp(static_cast<const uint16_t*>(c.cos)) + pos * c.cos_s0 + rd);
        su[q] = *reinterpret_cast<const LOGKV_G uint2*>(gp(static_cast<const uint16_t*>(c.sin)) + pos * c.sin_s0 + rd);
      } else {
        cu[q] = *reinterpret_cast<const LOGKV_G float4*>(gp(static_cast<const float*>(c.cos)) + pos * c.cos_s0 + rd);
        su[q] = *reinterpret_cast<const LOGKV_G float4*>(gp(static_cast<const float*>(c.sin)) + pos * c.sin_s0 + rd);
      }
    }
#pragma unroll
    for (int q = 0; q < kPackBatch; ++q) {
      if (i0 + q * nthr >= items) break;
      const PackSrc& r = src[rr[q]];
      if (!(r.flags & 4)) continue;
      const int d0 = d0s[q];
      const bool valid = r.flags & 1;
      // Copied rows keep their bf16 bits; rotated features and the bias are
      // bf16-exact floats (rounded already), whose high halves are the bits.
      uint2 ok = valid ? xu[q] : make_uint2(0u, 0u);
      if (d0 < c.dk) {
        if (valid && (r.flags & 2) && d0 < c.rope_n) {
          // Rotate-half RoPE: x cos + rot sin, rot = -partner below half (products
          // rounded to bf16 first with bf16 tables), rounded to bf16.
          const float sign = d0 < half ? -1.f : 1.f;
          const float x[4] = {lo_bf16(xu[q].x), hi_bf16(xu[q].x), lo_bf16(xu[q].y), hi_bf16(xu[q].y)};
          const float other[4] = {lo_bf16(pu[q].x), hi_bf16(pu[q].x), lo_bf16(pu[q].y), hi_bf16(pu[q].y)};
          float cs[4], sn[4];
          if constexpr (BF16_TABLE) {
            cs[0] = lo_bf16(cu[q].x); cs[1] = hi_bf16(cu[q].x); cs[2] = lo_bf16(cu[q].y); cs[3] = hi_bf16(cu[q].y);
            sn[0] = lo_bf16(su[q].x); sn[1] = hi_bf16(su[q].x); sn[2] = lo_bf16(su[q].y); sn[3] = hi_bf16(su[q].y);
          } else {
            cs[0] = cu[q].x; cs[1] = cu[q].y; cs[2] = cu[q].z; cs[3] = cu[q].w;
            sn[0] = su[q].x; sn[1] = su[q].y; sn[2] = su[q].z; sn[3] = su[q].w;
          }
          uint32_t o[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float a = x[k] * cs[k], bb = (sign * other[k]) * sn[k];
            if constexpr (BF16_TABLE) {
              a = round_bf16(a);
              bb = round_bf16(bb);
            }
            o[k] = f32_to_bf16(a + bb);
          }
          ok = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
        }
      } else {
        // Column dk holds the bias (dk is a multiple of 4: first of its unit).
        ok = make_uint2(d0 == c.dk ? static_cast<uint32_t>(f32_to_bf16(r.bias)) : 0u, 0u);
      }
      const int64_t orow = (static_cast<int64_t>(lane) * p.out_cap + s0 + rr[q]) * p.dim;
      *reinterpret_cast<LOGKV_G uint2*>(gp(p.out_k) + orow + d0) = ok;
      const uint2 ov = valid && d0 < c.dv ? vu[q] : make_uint2(0u, 0u);
      *reinterpret_cast<LOGKV_G uint2*>(gp(p.out_v) + orow + d0) = ov;
    }
  }
}

// Block (tile of kPackRows packed rows, lane). One thread per row resolves its
// source (pooled rows by binary search over the lane's plan row, held in LDS);
// then one thread per (row, 4-feature unit) writes the K and V units, every
// load of a unit issued before its arithmetic.
__global__ __launch_bounds__(256) void pack_kernel(logkv_readout_view c, logkv_pack_args p,
                                                   const int32_t* __restrict__ table) {
  __shared__ int32_t prow[kMaxClusters * kMaxLevels + 1];
  __shared__ PackSrc src[kPackRows];
  const int lanes = c.n_batch * c.n_groups;
  const int lane = blockIdx.y;
  const int b = lane / c.n_groups, g = lane % c.n_groups;
  const int KL = c.k_max * c.levels;
  const int tid = static_cast<int>(threadIdx.x);
  const int width = table[static_cast<int64_t>(lanes) * (KL + 1)];
  const int alpha_count = c.alpha_count_dev ? *c.alpha_count_dev : c.alpha_count;
  const int tail_rows = alpha_count + c.recent_count + p.cur_len;
  const int first = p.skip_pooled ? width + alpha_count + p.recent_start : 0;   // packed index of item 0
  const int items = p.skip_pooled ? tail_rows - alpha_count - p.recent_start : width + tail_rows;
  const int i0 = blockIdx.x * kPackRows;
  if (i0 >= items) return;
  const LOGKV_G int32_t* row_tab = gp(table) + static_cast<int64_t>(lane) * (KL + 1);
  for (int i = tid; i <= KL; i += blockDim.x) prow[i] = row_tab[i];
  __syncthreads();
  const int dk = c.dk, dv = c.dv;
  if (tid < kPackRows) {
    const int s = first + i0 + tid;
    PackSrc r{gp(c.level_k), gp(c.level_v), 0, -10000.0f, 0};
    if (i0 + tid < items && s < p.out_cap) {
      r.flags = 4;
      if (s < width) {
        if (s < prow[KL]) {
          int lo = 0;   // largest block whose prefix is <= s (empty blocks share their successor's prefix)
          for (int len = KL; len > 1;) {
            const int half = len >> 1;
            lo = prow[lo + half] <= s ? lo + half : lo;
            len -= half;
          }
          const int cc = lo / c.levels, e = c.levels - 1 - lo % c.levels;
          const int64_t phys = ((static_cast<int64_t>(lane) * c.k_max + cc) * c.levels + e) * c.slots + (s - prow[lo]);
          const float w = gp(c.level_w)[phys];
          if (w > 0.f) {
            const int64_t wi = static_cast<int64_t>(w) > 1 ? static_cast<int64_t>(w) : 1;
            const int64_t swp = gp(c.level_sum_wp)[phys];
            const int64_t num = 2 * swp + wi, den = 2 * wi;
            r.pos = num >= 0 ? num / den : -((-num + den - 1) / den);
            r.k = gp(c.level_k) + phys * dk;
            r.v = gp(c.level_v) + phys * dv;
            r.bias = round_bf16(logf(w > 1.f ? w : 1.f));
            r.flags |= 3;
          }
        }
      } else if (s < width + alpha_count) {
        const int i = s - width;
        if (gp(c.alpha_valid)[static_cast<int64_t>(b) * c.alpha_cap + i] != 0) {
          r.pos = gp(c.alpha_pos)[static_cast<int64_t>(b) * c.alpha_cap + i];
          r.k = gp(c.alpha_k) + (static_cast<int64_t>(lane) * c.alpha_cap + i) * dk;
          r.v = gp(c.alpha_v) + (static_cast<int64_t>(lane) * c.alpha_cap + i) * dv;
          r.bias = 0.f;
          r.flags |= 3;
        }
      } else if (s < width + alpha_count + c.recent_count) {
        const int i = s - width - alpha_count;
        r.k = gp(c.recent_k) + (static_cast<int64_t>(lane) * c.recent_cap + i) * dk;
        r.v = gp(c.recent_v) + (static_cast<int64_t>(lane) * c.recent_cap + i) * dv;
        r.bias = 0.f;
        r.flags |= 1;
      } else {
        const int i = s - width - alpha_count - c.recent_count;
        r.k = gp(p.cur_k) + b * p.ck_sb + g * p.ck_sg + static_cast<int64_t>(i) * p.ck_st;
        r.v = gp(p.cur_v) + b * p.cv_sb + g * p.cv_sg + static_cast<int64_t>(i) * p.cv_st;
        r.bias = 0.f;
        r.flags |= 1;
      }
    }
    src[tid] = r;
    if (p.out_w && (r.flags & 4)) {
      // Per-row mass and validity of the packed rows (an attention state's slot_w /
      // slot_valid): a pooled slot's stored mass (0 for padding), 1 or 0 for an
      // exact row by its flag, 1 for recent and current rows.
      float w_out = 1.f;
      if (s < width) {
        w_out = 0.f;
        if (r.flags & 1) {
          const int64_t phys = (r.k - gp(c.level_k)) / dk;
          w_out = gp(c.level_w)[phys];
        }
      } else if (s < width + alpha_count) {
        w_out = (r.flags & 1) ? 1.f : 0.f;
      }
      const int64_t o = static_cast<int64_t>(lane) * p.out_cap + s;
      gp(p.out_w)[o] = w_out;
      if (p.out_valid) gp(p.out_valid)[o] = static_cast<uint8_t>(r.flags & 1);
    }
  }
  __syncthreads();
  const int units = p.dim / 4;   // per K row and per V row
  const int half = c.rope_n / 2;
  // Vector loads of 4 features and 4 table entries need 4-aligned rows and
  // contiguous tables with 4-aligned position strides (the usual layout).
  const bool vec = c.cos_s1 == 1 && c.sin_s1 == 1 && c.cos_s0 % 4 == 0 && c.sin_s0 % 4 == 0 && c.rope_n % 8 == 0 &&
                   reinterpret_cast<uintptr_t>(c.cos) % 16 == 0 && reinterpret_cast<uintptr_t>(c.sin) % 16 == 0;
  if (vec) {
    if (c.table_bf16) pack_units_vec<true>(c, p, src, first + i0, lane, units, half);
    else pack_units_vec<false>(c, p, src, first + i0, lane, units, half);
    return;
  }
  for (int it = tid; it < kPackRows * 2 * units; it += blockDim.x) {
    const int rr = it / (2 * units), u = it % (2 * units);
    const PackSrc r = src[rr];
    if (!(r.flags & 4)) continue;
    const int s = first + i0 + rr;
    const bool valid = r.flags & 1;
    float o[4];
    if (u < units) {
      const int d0 = 4 * u;
      if (d0 >= dk) {
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = d0 + q == dk ? r.bias : 0.f;
      } else {
        const int64_t pos = r.pos < 0 ? 0 : (r.pos >= c.rope_rows ? c.rope_rows - 1 : r.pos);
        float x[4], other[4], cs[4], sn[4];
        // Unconditional scalar loads at clamped indices, selected afterwards.
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int d = d0 + q, dd = d < dk ? d : dk - 1;
          const int pd = d < half ? d + half : d - half;
          const int pc = pd < 0 ? 0 : (pd < dk ? pd : dk - 1);
          const int rd = d < c.rope_n ? d : 0;
          x[q] = bf16_to_f32(r.k[dd]);
          other[q] = bf16_to_f32(r.k[pc]);
          cs[q] = table_at(c.cos, pos * c.cos_s0 + rd * c.cos_s1, c.table_bf16);
          sn[q] = table_at(c.sin, pos * c.sin_s0 + rd * c.sin_s1, c.table_bf16);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = rope_out(c, r, d0 + q, x[q], other[q], cs[q], sn[q], half, valid);
      }
    } else {
      const int d0 = 4 * (u - units);
      if (d0 < dv) {   // dv is a multiple of 4: the unit is whole
        const uint2 vu = *reinterpret_cast<const LOGKV_G uint2*>(r.v + d0);
        o[0] = valid ? lo_bf16(vu.x) : 0.f;
        o[1] = valid ? hi_bf16(vu.x) : 0.f;
        o[2] = valid ? lo_bf16(vu.y) : 0.f;
        o[3] = valid ? hi_bf16(vu.y) : 0.f;
      } else {
        o[0] = o[1] = o[2] = o[3] = 0.f;
      }
    }
    const int64_t orow = (static_cast<int64_t>(lane) * p.out_cap + s) * p.dim;
    store_bf16x4(u < units ? gp(p.out_k) + orow + 4 * u : gp(p.out_v) + orow + 4 * (u - units), o);
  }
}

// Split attention: partial (max, sum, acc) per (split, lane, query).
__global__ __launch_bounds__(256) void decode_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr,
                                                     float* __restrict__ part) {
  __shared__ float q_s[kMaxQ * kMaxPacked];
  __shared__ __align__(16) uint16_t kv_s[kTile * kMaxPacked];
  __shared__ float p_s[kMaxQ * kTile];
  __shared__ float m_s[kMaxQ], l_s[kMaxQ], corr_s[kMaxQ];
  const int lane = blockIdx.y;
  const int G = a.n_groups;
  const int b = lane / G, g = lane % G;
  const int rep = a.n_heads / G;
  const int nq = rep * a.tq;
  const int dim = a.dim;
  const int total = min(*width_ptr + a.tail + (a.alpha_count_dev ? *a.alpha_count_dev : 0), a.cap);
  const int r_begin = blockIdx.x * kSplitRows;
  const int r_end = min(r_begin + kSplitRows, total);
  float* out = part + (static_cast<int64_t>(lane) * gridDim.x + blockIdx.x) * nq * (a.dv + 2);
  // Queries [q, 1/scale (bf16), 0...] as float; query qi = head (g*rep + qi / tq), row qi % tq.
  for (int i = threadIdx.x; i < nq * dim; i += blockDim.x) {
    const int qi = i / dim, d = i % dim;
    const int h = g * rep + qi / a.tq, t = qi % a.tq;
    float x = 0.f;
    if (d < a.dk) x = bf16_to_f32(gp(a.q)[b * a.q_sb + h * a.q_sh + t * a.q_st + d]);
    else if (d == a.dk) x = a.inv_scale_bf16;
    q_s[qi * kMaxPacked + d] = x;
  }
  for (int qi = threadIdx.x; qi < nq; qi += blockDim.x) {
    m_s[qi] = -__builtin_inff();
    l_s[qi] = 0.f;
  }
  const int w = wave_id(), l = lane_id(), nw = blockDim.x / kWave;
  float acc[kAccPerThread];
#pragma unroll
  for (int i = 0; i < kAccPerThread; ++i) acc[i] = 0.f;
  const int n_out = nq * a.dv;
  const int per = (n_out + blockDim.x - 1) / blockDim.x;
  const LOGKV_G uint16_t* kbase = gp(a.k) + static_cast<int64_t>(lane) * a.cap * dim;
  const LOGKV_G uint16_t* vbase = gp(a.v) + static_cast<int64_t>(lane) * a.cap * dim;
  const int units = dim / 8;   // 16-byte units per packed row
  const int tail0 = total - a.causal_tail;
  for (int t0 = r_begin; t0 < r_end; t0 += kTile) {
    const int rows = min(kTile, r_end - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < rows * units; i += blockDim.x) {
      const int r = i / units, u = i % units;
      *reinterpret_cast<uint4*>(kv_s + r * dim + 8 * u) =
          *(const LOGKV_G uint4*)(kbase + (static_cast<int64_t>(t0) + r) * dim + 8 * u);
    }
    __syncthreads();
    // Scores and online softmax: the wave owning query qi has one row per lane.
    for (int qi = w; qi < nq; qi += nw) {
      const int r = l;
      float sc = -__builtin_inff();
      if (r < rows) {
        float dot = 0.f;
        const float* qv = q_s + qi * kMaxPacked;
        const uint16_t* kr = kv_s + r * dim;
        for (int d = 0; d < dim; d += 2) {
          const uint32_t pair = *reinterpret_cast<const uint32_t*>(kr + d);
          dot = __builtin_fmaf(qv[d], __uint_as_float(pair << 16), dot);
          dot = __builtin_fmaf(qv[d + 1], __uint_as_float(pair & 0xffff0000u), dot);
        }
        sc = a.scale * dot;
        const int row = t0 + r;
        if (a.causal_tail && row >= tail0 && row - tail0 > qi % a.tq) sc = -__builtin_inff();
      }
      float mx = sc;
      for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
      const float m_old = m_s[qi];
      const float m_new = fmaxf(m_old, mx);
      const float corr = m_new == -__builtin_inff() ? 1.f : __expf(m_old - m_new);
      const float pr = sc == -__builtin_inff() ? 0.f : __expf(sc - m_new);
      float sum = pr;
      for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, kWave);
      p_s[qi * kTile + r] = pr;
      if (l == 0) {
        l_s[qi] = l_s[qi] * corr + sum;
        m_s[qi] = m_new;
        corr_s[qi] = corr;
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < rows * units; i += blockDim.x) {
      const int r = i / units, u = i % units;
      *reinterpret_cast<uint4*>(kv_s + r * dim + 8 * u) =
          *(const LOGKV_G uint4*)(vbase + (static_cast<int64_t>(t0) + r) * dim + 8 * u);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kAccPerThread; ++k) {
      const int o = threadIdx.x + k * blockDim.x;
      if (k < per && o < n_out) {
        const int qi = o / a.dv, d = o % a.dv;
        float s = acc[k] * corr_s[qi];
        const float* pq = p_s + qi * kTile;
        for (int r = 0; r < rows; ++r) s = __builtin_fmaf(pq[r], bf16_to_f32(kv_s[r * dim + d]), s);
        acc[k] = s;
      }
    }
  }
  __syncthreads();
  // Partials: [m, l, acc[dv]] per query.
  for (int qi = threadIdx.x; qi < nq; qi += blockDim.x) {
    out[qi * (a.dv + 2)] = m_s[qi];
    out[qi * (a.dv + 2) + 1] = l_s[qi];
  }
#pragma unroll
  for (int k = 0; k < kAccPerThread; ++k) {
    const int o = threadIdx.x + k * blockDim.x;
    if (k < per && o < n_out) out[(o / a.dv) * (a.dv + 2) + 2 + o % a.dv] = acc[k];
  }
}

// Streaming decode for at most 4 queries per KV group (a decode step of GQA
// heads): no staging of K / V in LDS. A block is 16 row groups of 16 lanes; a
// group reads one packed row at a time (its 16-byte units spread over the 16
// lanes: [q, 1/scale] . [k, bias] folded over the group), keeps its own online
// softmax per query and accumulates its lanes' 8-wide slices of V, rows
// 4 at a time with all loads issued first; 512-row splits. At the end of the split the 16
// groups are combined in LDS in group order and the split's partials go to
// the workspace in the layout the split combine reads.
//
// SPLIT (dk a multiple of 8): the key's bias column dk starts a unit of its
// own, so the 16-byte units cover only the dk features and the bias is one
// 2-byte load per row, added after the group fold as q[dk] * bias; UJ then
// counts units of the dk features only (8 registers per row and query fewer).
template <int NQ, int UJ, bool SPLIT>
__global__ __launch_bounds__(256) void stream_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr,
                                                     float* __restrict__ part) {
  constexpr int kGroups = 16, kGl = 16, kRows = 4;
  __shared__ float m_s[kGroups][NQ], l_s[kGroups][NQ];
  __shared__ float acc_s[kGroups][NQ][128];
  const int lane = blockIdx.y, G = a.n_groups;
  const int b = lane / G, g = lane % G;
  const int rep = a.n_heads / G, nq = rep * a.tq;
  const int grp = threadIdx.x / kGl, gl = threadIdx.x % kGl;
  const int dim = a.dim, units = SPLIT ? a.dk / 8 : dim / 8, vunits = (a.dv + 7) / 8;   // the last unit may run into the zero pad (dim >= 8 * vunits)
  const float q_bias = a.inv_scale_bf16;
  const int total = min(*width_ptr + a.tail + (a.alpha_count_dev ? *a.alpha_count_dev : 0), a.cap);
  const int tail0 = total - a.causal_tail;
  // The lane's rows in gridDim.x equal shares, multiples of 64 (a pass of the
  // 16 row groups x 4 rows); splits past the rows write empty partials.
  const int share = max(64, (total + 64 * static_cast<int>(gridDim.x) - 1) / (64 * static_cast<int>(gridDim.x)) * 64);
  const int r_begin = blockIdx.x * share, r_end = min(r_begin + share, total);
  float* out = part + (static_cast<int64_t>(lane) * gridDim.x + blockIdx.x) * nq * (a.dv + 2);
  // This lane's slices of the queries [q, 1/scale (bf16), 0...]: units gl + 16 j,
  // as bf16 pairs (features 2e, 2e + 1 of a unit) for the packed dot products.
  uint32_t qp[NQ][UJ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int qq = q < nq ? q : nq - 1;
    const int h = g * rep + qq / a.tq, t = qq % a.tq;
#pragma unroll
    for (int j = 0; j < UJ; ++j) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        uint32_t pair = 0u;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int d = 8 * (gl + kGl * j) + e + hf;
          uint32_t x = 0u;
          if (d < a.dk) x = gp(a.q)[b * a.q_sb + h * a.q_sh + t * a.q_st + d];
          else if (!SPLIT && d == a.dk) x = f32_to_bf16(a.inv_scale_bf16);
          pair |= (q < nq ? x : 0u) << (16 * hf);
        }
        qp[q][j][e / 2] = pair;
      }
    }
  }
  float m[NQ], l[NQ], acc[NQ][8];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    m[q] = -__builtin_inff();
    l[q] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[q][e] = 0.f;
  }
  const LOGKV_G uint16_t* kbase = gp(a.k) + static_cast<int64_t>(lane) * a.cap * dim;
  const LOGKV_G uint16_t* vbase = gp(a.v) + static_cast<int64_t>(lane) * a.cap * dim;
  const bool v_on = gl < vunits;
  for (int r0 = r_begin + grp; r0 < r_end; r0 += kGroups * kRows) {
    uint4 kx[kRows][UJ], vx[kRows];
    uint16_t kb[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int row = min(r0 + kGroups * i, r_end - 1);
#pragma unroll
      for (int j = 0; j < UJ; ++j) {
        const int u = min(gl + kGl * j, units - 1);
        kx[i][j] = *(const LOGKV_G uint4*)(kbase + static_cast<int64_t>(row) * dim + 8 * u);
      }
      if (SPLIT) kb[i] = kbase[static_cast<int64_t>(row) * dim + a.dk];
      vx[i] = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(row) * dim + 8 * (v_on ? gl : 0));
    }
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int row = r0 + kGroups * i;
      if (row >= r_end) break;
      float dot[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) dot[q] = 0.f;
#pragma unroll
      for (int j = 0; j < UJ; ++j) {
        if (gl + kGl * j < units) {
          const uint32_t w4[4] = {kx[i][j].x, kx[i][j].y, kx[i][j].z, kx[i][j].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int q = 0; q < NQ; ++q)
              dot[q] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(rd_bf16x2, w4[e]),
                                                       __builtin_bit_cast(rd_bf16x2, qp[q][j][e]), dot[q], false);
          }
        }
      }
      const uint32_t v4[4] = {vx[i].x, vx[i].y, vx[i].z, vx[i].w};
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
#pragma unroll
        for (int off = kGl / 2; off >= 1; off >>= 1) dot[q] += __shfl_xor(dot[q], off, kGl);
        if (SPLIT) dot[q] = __builtin_fmaf(q_bias, bf16_to_f32(kb[i]), dot[q]);
        float sc = a.scale * dot[q];
        const int t = (q < nq ? q : nq - 1) % a.tq;
        if (q >= nq || (a.causal_tail && row >= tail0 && row - tail0 > t)) sc = -__builtin_inff();
        const float m_new = fmaxf(m[q], sc);
        const float p = sc == -__builtin_inff() ? 0.f : __expf(sc - m_new);
        // A new maximum rescales the sums; otherwise the factor is exactly 1
        // (2^0) and the products by it change nothing, so a wave whose lanes
        // all kept their maximum skips them.
        if (__ballot(m_new != m[q])) {
          const float corr = m_new == -__builtin_inff() ? 1.f : __expf(m[q] - m_new);
          l[q] = l[q] * corr;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[q][e] = acc[q][e] * corr;
        }
        l[q] = l[q] + p;
        m[q] = m_new;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[q][2 * e] = __builtin_fmaf(p, __uint_as_float(v4[e] << 16), acc[q][2 * e]);
          acc[q][2 * e + 1] = __builtin_fmaf(p, __uint_as_float(v4[e] & 0xffff0000u), acc[q][2 * e + 1]);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    if (gl == 0) {
      m_s[grp][q] = m[q];
      l_s[grp][q] = l[q];
    }
    if (v_on) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc_s[grp][q][8 * gl + e] = acc[q][e];
    }
  }
  __syncthreads();
  // Groups combined in group order: [m, l, acc[dv]] per query of this split.
  for (int o = threadIdx.x; o < nq * (a.dv + 2); o += blockDim.x) {
    const int q = o / (a.dv + 2), c = o % (a.dv + 2);
    float mx = -__builtin_inff();
    for (int gg = 0; gg < kGroups; ++gg) mx = fmaxf(mx, m_s[gg][q]);
    float val;
    if (c == 0) {
      val = mx;
    } else {
      val = 0.f;
      for (int gg = 0; gg < kGroups; ++gg) {
        if (m_s[gg][q] == -__builtin_inff()) continue;
        const float f = __expf(m_s[gg][q] - mx);
        val += (c == 1 ? l_s[gg][q] : acc_s[gg][q][c - 2]) * f;
      }
    }
    out[o] = val;
  }
}

// Combine the splits of each (lane, query) in split order: one block per
// (lane, query), one output feature per thread. An empty split carries
// m = -inf with zero sums, so it adds exp(-inf) * 0 = 0 and needs no test.
__global__ __launch_bounds__(256) void combine_kernel(logkv_attention_args a, const float* __restrict__ part,
                                                      int n_split) {
  const int lane = blockIdx.x, qi = blockIdx.y;
  const int G = a.n_groups, rep = a.n_heads / G, nq = rep * a.tq;
  const int b = lane / G, g = lane % G;
  const int stride = a.dv + 2;
  const float* base = part + (static_cast<int64_t>(lane) * n_split * nq + qi) * stride;
  const int64_t step = static_cast<int64_t>(nq) * stride;
  for (int d = threadIdx.x; d < a.dv; d += blockDim.x) {
    float m = -__builtin_inff();
#pragma unroll 8
    for (int sp = 0; sp < n_split; ++sp) m = fmaxf(m, base[sp * step]);
    float lsum = 0.f, acc = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < n_split; ++sp) {
      const float* pp = base + sp * step;
      const float f = __expf(pp[0] - m);
      lsum += pp[1] * f;
      acc += pp[2 + d] * f;
    }
    const int h = g * rep + qi / a.tq, t = qi % a.tq;
    gp(a.out)[b * a.o_sb + h * a.o_sh + t * a.o_st + d] = f32_to_bf16(acc / lsum);
  }
}

// Packed rows [B, G, S, dim] of unpacked attention slots (log_kv_slot_attention's
// inputs, litgpt/log_kv_cache.py:6439-6464): keys and values copied (bf16 bits),
// column dk the mass bias lam * log(w) - or, for the first s_m slots when
// anchor counts are given, -log(max(M, 1)) + lam * log(max(w, 1))
// (litgpt/log_kv_position.py:128-133) - rounded to bf16; the first s_valid
// slots with a false valid flag become all-zero rows with bias -10000. One
// thread per (row, 4-feature unit) of K, then of V.
__global__ __launch_bounds__(256) void slot_pack_kernel(logkv_slot_pack_args a) {
  const int units = a.dim / 4;
  const int64_t lane = blockIdx.y;
  const int b = static_cast<int>(lane / a.n_groups), g = static_cast<int>(lane % a.n_groups);
  const int64_t items = static_cast<int64_t>(a.slots) * 2 * units;
  for (int64_t it = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; it < items;
       it += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int s = static_cast<int>(it / (2 * units)), u = static_cast<int>(it % (2 * units));
    const bool valid = s >= a.s_valid || gp(a.valid)[b * a.valid_sb + g * a.valid_sg + s] != 0;
    uint32_t o[4] = {0u, 0u, 0u, 0u};
    if (u < units) {
      const int d0 = 4 * u;
      const LOGKV_G uint16_t* row = gp(a.k) + b * a.k_sb + g * a.k_sg + static_cast<int64_t>(s) * a.k_st;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = d0 + q;
        if (d < a.dk) {
          o[q] = valid ? row[d] : 0u;
        } else if (d == a.dk) {
          float bias = -10000.f;
          if (valid) {
            const float w = gp(a.w)[b * a.w_sb + g * a.w_sg + s];
            if (s < a.s_m) {
              const float m = static_cast<float>(gp(a.m)[b * a.m_sb + g * a.m_sg + s]);
              bias = -logf(m > 1.f ? m : 1.f);
              if (a.lam != 0.f) bias = bias + a.lam * logf(w > 1.f ? w : 1.f);
            } else {
              bias = a.lam != 0.f ? a.lam * logf(w) : 0.f;
            }
          }
          o[q] = f32_to_bf16(bias);
        }
      }
      const int64_t orow = (lane * a.out_cap + s) * a.dim;
      *reinterpret_cast<LOGKV_G uint2*>(gp(a.out_k) + orow + d0) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
    } else {
      const int d0 = 4 * (u - units);
      const LOGKV_G uint16_t* row = gp(a.v) + b * a.v_sb + g * a.v_sg + static_cast<int64_t>(s) * a.v_st;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = d0 + q;
        o[q] = valid && d < a.dv ? row[d] : 0u;
      }
      const int64_t orow = (lane * a.out_cap + s) * a.dim;
      *reinterpret_cast<LOGKV_G uint2*>(gp(a.out_v) + orow + d0) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
    }
  }
}

}  // namespace

int launch_slot_pack(const logkv_slot_pack_args& a, hipStream_t stream) {
  const int64_t items = static_cast<int64_t>(a.slots) * 2 * (a.dim / 4);
  if (items == 0) return LOGKV_OK;
  const int64_t blocks = std::min<int64_t>((items + 255) / 256, 4096);
  hipLaunchKernelGGL(slot_pack_kernel, dim3(static_cast<unsigned>(blocks), a.n_batch * a.n_groups), dim3(256), 0,
                     stream, a);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_plan(const logkv_readout_view& c, int32_t* table, hipStream_t stream) {
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, c, table);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_pack(const logkv_readout_view& c, const logkv_pack_args& p, const int32_t* table, hipStream_t stream) {
  // With skip_pooled the rows past the recent window's first new row (at most
  // the whole recent window and current rows; blocks past the end exit).
  const int rows = p.skip_pooled ? c.recent_count + p.cur_len - p.recent_start : p.out_cap;
  if (rows <= 0) return LOGKV_OK;
  // Tiles past the packed rows (known on the device only) exit at once.
  hipLaunchKernelGGL(pack_kernel, dim3((rows + kPackRows - 1) / kPackRows, c.n_batch * c.n_groups), dim3(256), 0,
                     stream, c, p, table);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

// 16-byte key units per row group lane of the streaming kernel (the bias
// column excluded when it starts a unit of its own).
int stream_key_units(const logkv_attention_args& a) {
  const int units = a.dk % 8 == 0 ? a.dk / 8 : a.dim / 8;
  return (units + 15) / 16;
}

bool use_stream(const logkv_attention_args& a) {
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  return nq <= 4 && a.dv <= 128 && a.dk >= 8 && stream_key_units(a) <= 3;
}

// Splits per lane: the staged kernel takes kSplitRows rows each; the streaming
// kernel takes up to kStreamRows each, but no more splits than keep every block
// of the launch resident at once (its splits then share the rows equally).
int attention_splits(const logkv_attention_args& a) {
  if (!use_stream(a)) return (a.cap + kSplitRows - 1) / kSplitRows;
  const int lanes = a.n_batch * a.n_groups;
  return std::max(1, std::min((a.cap + kStreamRows - 1) / kStreamRows, kStreamBlocks / std::max(1, lanes)));
}

int64_t attention_workspace_floats(const logkv_attention_args& a) {
  const int n_split = attention_splits(a);
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  return static_cast<int64_t>(a.n_batch) * a.n_groups * n_split * nq * (a.dv + 2);
}

int launch_combine(const logkv_attention_args& a, const float* part, int n_split, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(a.n_batch * a.n_groups, (a.n_heads / a.n_groups) * a.tq),
                     dim3(a.dv <= 64 ? 64 : 128), 0, stream, a, part, n_split);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_attention(const logkv_attention_args& a, const int32_t* width, float* part, hipStream_t stream) {
  const int n_split = attention_splits(a);
  const int lanes = a.n_batch * a.n_groups;
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  const int uj = stream_key_units(a);
  const dim3 grid(n_split, lanes);
  auto stream_launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, a, width, part);
  };
  auto by_units = [&](auto one, auto two, auto three) {
    if (uj == 1) stream_launch(one);
    else if (uj == 2) stream_launch(two);
    else stream_launch(three);
  };
  if (use_stream(a)) {
    if (a.dk % 8 == 0) {
      if (nq == 1) by_units(stream_kernel<1, 1, true>, stream_kernel<1, 2, true>, stream_kernel<1, 3, true>);
      else if (nq == 2) by_units(stream_kernel<2, 1, true>, stream_kernel<2, 2, true>, stream_kernel<2, 3, true>);
      else by_units(stream_kernel<4, 1, true>, stream_kernel<4, 2, true>, stream_kernel<4, 3, true>);
    } else {
      if (nq == 1) by_units(stream_kernel<1, 1, false>, stream_kernel<1, 2, false>, stream_kernel<1, 3, false>);
      else if (nq == 2) by_units(stream_kernel<2, 1, false>, stream_kernel<2, 2, false>, stream_kernel<2, 3, false>);
      else by_units(stream_kernel<4, 1, false>, stream_kernel<4, 2, false>, stream_kernel<4, 3, false>);
    }
  } else {
    hipLaunchKernelGGL(decode_kernel, grid, dim3(256), 0, stream, a, width, part);
  }
  hipLaunchKernelGGL(combine_kernel, dim3(lanes, nq), dim3(a.dv <= 64 ? 64 : 128), 0, stream, a, part, n_split);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
