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
#include "route.hpp"

namespace logkv {

namespace {

constexpr int kPlanThreads = 256;
constexpr int kTile = 64;          // rows per staged K/V tile
constexpr int kSplitRows = 512;    // rows per attention split
constexpr int kMaxQ = 16;          // queries per KV group (heads per group x query rows)
constexpr int kMaxPacked = 264;    // packed row width limit (dk + 1 rounded to 8, dv)
constexpr int kAccPerThread = kMaxQ * kMaxDim / 256;   // outputs per thread of a 256-thread split block

struct PlanCtx {
  const LOGKV_G int16_t* count;    // [lanes, K, L]
  int K, L;
};

// Lane pooled-row prefix over (cluster, level top-down) blocks -> plan table
// [lanes, K*L + 1] (offsets), plus the maximum lane count at table[lanes*(K*L+1)].
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(logkv_readout_view c, int32_t* __restrict__ table) {
  __shared__ int lane_max[kPlanThreads];
  const int lanes = c.n_batch * c.n_groups;
  const int KL = c.k_max * c.levels;
  int best = 0;
  for (int lane = threadIdx.x; lane < lanes; lane += kPlanThreads) {
    const LOGKV_G int16_t* cnt = gp(c.level_count) + static_cast<int64_t>(lane) * KL;
    LOGKV_G int32_t* row = gp(table) + static_cast<int64_t>(lane) * (KL + 1);
    int acc = 0;
    for (int cc = 0; cc < c.k_max; ++cc) {
      for (int e = c.levels - 1; e >= 0; --e) {
        row[cc * c.levels + (c.levels - 1 - e)] = acc;
        acc += cnt[cc * c.levels + e];
      }
    }
    row[KL] = acc;
    best = acc > best ? acc : best;
  }
  lane_max[threadIdx.x] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    int m = 0;
    for (int i = 0; i < kPlanThreads; ++i) m = lane_max[i] > m ? lane_max[i] : m;
    table[static_cast<int64_t>(lanes) * (KL + 1)] = m;
  }
}

__device__ __forceinline__ float table_at(const void* t, int64_t i, int bf16) {
  return bf16 ? bf16_to_f32(gp(static_cast<const uint16_t*>(t))[i]) : gp(static_cast<const float*>(t))[i];
}

// RoPE of element d of a bf16 row at `pos` (rotate-half over the first rope_n dims).
__device__ __forceinline__ float rope_at(const LOGKV_G uint16_t* row, int d, int64_t pos, const logkv_readout_view& c) {
  const float x = bf16_to_f32(row[d]);
  if (d >= c.rope_n) return x;
  pos = pos < 0 ? 0 : (pos >= c.rope_rows ? c.rope_rows - 1 : pos);
  const int half = c.rope_n / 2;
  const float other = bf16_to_f32(row[d < half ? d + half : d - half]);
  const float rot = d < half ? -other : other;
  const float cs = table_at(c.cos, pos * c.cos_s0 + d * c.cos_s1, c.table_bf16);
  const float sn = table_at(c.sin, pos * c.sin_s0 + d * c.sin_s1, c.table_bf16);
  float a = x * cs, b = rot * sn;
  if (c.table_bf16) {
    a = round_bf16(a);
    b = round_bf16(b);
  }
  return round_bf16(a + b);
}

// One wave per packed row; grid (row tiles, lanes).
__global__ __launch_bounds__(256) void pack_kernel(logkv_readout_view c, logkv_pack_args p,
                                                   const int32_t* __restrict__ table) {
  const int lanes = c.n_batch * c.n_groups;
  const int lane = blockIdx.y;
  const int b = lane / c.n_groups, g = lane % c.n_groups;
  const int KL = c.k_max * c.levels;
  const int width = table[static_cast<int64_t>(lanes) * (KL + 1)];
  const int alpha_count = c.alpha_count_dev ? *c.alpha_count_dev : c.alpha_count;
  const int tail_rows = alpha_count + c.recent_count + p.cur_len;
  const int i0 = blockIdx.x * (blockDim.x / kWave) + wave_id();
  int s;
  if (p.skip_pooled) {
    const int tail_start = alpha_count + p.recent_start;
    if (tail_start + i0 >= tail_rows) return;
    s = width + tail_start + i0;
  } else {
    if (i0 >= width + tail_rows) return;
    s = i0;
  }
  if (s >= p.out_cap) return;
  const int l = lane_id();
  LOGKV_G uint16_t* ok = gp(p.out_k) + (static_cast<int64_t>(lane) * p.out_cap + s) * p.dim;
  LOGKV_G uint16_t* ov = gp(p.out_v) + (static_cast<int64_t>(lane) * p.out_cap + s) * p.dim;
  const int dk = c.dk, dv = c.dv;
  const LOGKV_G uint16_t* kr = nullptr;
  const LOGKV_G uint16_t* vr = nullptr;
  bool rotate = false, valid = true;
  int64_t pos = 0;
  float bias = 0.f;
  if (s < width) {
    const LOGKV_G int32_t* row = gp(table) + static_cast<int64_t>(lane) * (KL + 1);
    const int n_lane = row[KL];
    valid = s < n_lane;
    if (valid) {
      // Block (cluster, level) holding pooled row s: largest prefix <= s.
      int lo = 0, hi = KL - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (row[mid] <= s) lo = mid;
        else hi = mid - 1;
      }
      // Skip empty blocks that share the prefix: the last block with prefix == row[lo].
      const int cc = lo / c.levels, e = c.levels - 1 - lo % c.levels;
      const int slot = s - row[lo];
      const int64_t phys = ((static_cast<int64_t>(lane) * c.k_max + cc) * c.levels + e) * c.slots + slot;
      const float w = gp(c.level_w)[phys];
      valid = w > 0.f;
      if (valid) {
        const int64_t wi = static_cast<int64_t>(w) > 1 ? static_cast<int64_t>(w) : 1;
        const int64_t swp = gp(c.level_sum_wp)[phys];
        int64_t num = 2 * swp + wi, den = 2 * wi;
        pos = num >= 0 ? num / den : -((-num + den - 1) / den);
        kr = gp(c.level_k) + phys * dk;
        vr = gp(c.level_v) + phys * dv;
        rotate = true;
        bias = round_bf16(logf(w > 1.f ? w : 1.f));
      }
    }
  } else if (s < width + alpha_count) {
    const int i = s - width;
    valid = gp(c.alpha_valid)[static_cast<int64_t>(b) * c.alpha_cap + i] != 0;
    if (valid) {
      pos = gp(c.alpha_pos)[static_cast<int64_t>(b) * c.alpha_cap + i];
      kr = gp(c.alpha_k) + (static_cast<int64_t>(lane) * c.alpha_cap + i) * dk;
      vr = gp(c.alpha_v) + (static_cast<int64_t>(lane) * c.alpha_cap + i) * dv;
      rotate = true;
    }
  } else if (s < width + alpha_count + c.recent_count) {
    const int i = s - width - alpha_count;
    kr = gp(c.recent_k) + (static_cast<int64_t>(lane) * c.recent_cap + i) * dk;
    vr = gp(c.recent_v) + (static_cast<int64_t>(lane) * c.recent_cap + i) * dv;
  } else {
    const int i = s - width - alpha_count - c.recent_count;
    kr = gp(p.cur_k) + b * p.ck_sb + g * p.ck_sg + static_cast<int64_t>(i) * p.ck_st;
    vr = gp(p.cur_v) + b * p.cv_sb + g * p.cv_sg + static_cast<int64_t>(i) * p.cv_st;
  }
  for (int d = l; d < p.dim; d += kWave) {
    float kx = 0.f, vx = 0.f;
    if (valid) {
      if (d < dk) kx = rotate ? rope_at(kr, d, pos, c) : bf16_to_f32(kr[d]);
      if (d < dv) vx = bf16_to_f32(vr[d]);
    }
    if (d == dk) kx = valid ? bias : -10000.0f;
    ok[d] = f32_to_bf16(kx);
    ov[d] = f32_to_bf16(vx);
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

// Combine the splits of each (lane, query) in split order.
__global__ __launch_bounds__(256) void combine_kernel(logkv_attention_args a, const float* __restrict__ part,
                                                      int n_split) {
  const int lane = blockIdx.x;
  const int G = a.n_groups, rep = a.n_heads / G, nq = rep * a.tq;
  const int b = lane / G, g = lane % G;
  for (int o = threadIdx.x; o < nq * a.dv; o += blockDim.x) {
    const int qi = o / a.dv, d = o % a.dv;
    float m = -__builtin_inff();
    for (int sp = 0; sp < n_split; ++sp)
      m = fmaxf(m, part[((static_cast<int64_t>(lane) * n_split + sp) * nq + qi) * (a.dv + 2)]);
    float lsum = 0.f, acc = 0.f;
    for (int sp = 0; sp < n_split; ++sp) {
      const float* pp = part + ((static_cast<int64_t>(lane) * n_split + sp) * nq + qi) * (a.dv + 2);
      if (pp[0] == -__builtin_inff()) continue;
      const float f = __expf(pp[0] - m);
      lsum += pp[1] * f;
      acc += pp[2 + d] * f;
    }
    const int h = g * rep + qi / a.tq, t = qi % a.tq;
    gp(a.out)[b * a.o_sb + h * a.o_sh + t * a.o_st + d] = f32_to_bf16(acc / lsum);
  }
}

}  // namespace

int launch_plan(const logkv_readout_view& c, int32_t* table, hipStream_t stream) {
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, c, table);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_pack(const logkv_readout_view& c, const logkv_pack_args& p, const int32_t* table, hipStream_t stream) {
  // With skip_pooled the rows past the recent window's first new row (at most
  // the whole recent window and current rows; blocks past the end exit).
  const int rows = p.skip_pooled ? c.recent_count + p.cur_len - p.recent_start : p.out_cap;
  if (rows <= 0) return LOGKV_OK;
  const int per_block = 256 / kWave;
  hipLaunchKernelGGL(pack_kernel, dim3((rows + per_block - 1) / per_block, c.n_batch * c.n_groups), dim3(256), 0,
                     stream, c, p, table);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int64_t attention_workspace_floats(const logkv_attention_args& a) {
  const int n_split = (a.cap + kSplitRows - 1) / kSplitRows;
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  return static_cast<int64_t>(a.n_batch) * a.n_groups * n_split * nq * (a.dv + 2);
}

int launch_attention(const logkv_attention_args& a, const int32_t* width, float* part, hipStream_t stream) {
  const int n_split = (a.cap + kSplitRows - 1) / kSplitRows;
  const int lanes = a.n_batch * a.n_groups;
  hipLaunchKernelGGL(decode_kernel, dim3(n_split, lanes), dim3(256), 0, stream, a, width, part);
  hipLaunchKernelGGL(combine_kernel, dim3(lanes), dim3(256), 0, stream, a, part, n_split);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
