// Alpha exact spans on the device: span scoring (with Beta novelty) and the
// exact-pool / archive partition.
//
// Scoring restates litgpt/alpha_log_kv.py:125-174: per span and KV group,
// mu_X = mean over tokens, E_X = mean over tokens of mean_d X^2,
// R_X = max(E_X - mean_d mu_X^2, 0) / max(E_X, 1e-12); Alpha q = mean_g R_K +
// mean_g R_V; Beta q_g = (R_K + R_V)/2 + N/(1+N) with
// N = min over live centers (mean_d mu_K^2 + mean_d c^2 - 2 mean_d mu_K c)_+ /
// max(E_K, 1e-12) (0 without live centers), q = mean of the two largest q_g.
// One wave per (span, group): lane l holds features l, l+64, ...; token sums
// run in span order, feature sums use the canonical butterfly, group sums run
// in group order.
//
// The partition restates litgpt/log_kv_updates_triton.py:285-328: kept rows go
// to the exact pool, archived rows to archive buffers, -1 slots are zero rows.
// Sources are the virtual rows [old pool (old_width rows) | flush].
#include "route.hpp"

namespace logkv {

namespace {

constexpr int kMaxGroups = 16;

struct Rows2 {
  const LOGKV_G uint16_t* pool;
  int64_t p_sb, p_sg, p_st;
  const LOGKV_G uint16_t* flush;
  int64_t f_sb, f_sg, f_st;
  int32_t width;
  __device__ __forceinline__ const LOGKV_G uint16_t* row(int b, int g, int t) const {
    return t < width ? pool + b * p_sb + g * p_sg + static_cast<int64_t>(t) * p_st
                     : flush + b * f_sb + g * f_sg + static_cast<int64_t>(t - width) * f_st;
  }
};

// Canonical feature sum: lane l adds its features l, l + 64, ... in order,
// then the wave adds the lanes (wave_sum0). NJ = features per lane.
template <int NJ>
__device__ __forceinline__ float canon_sum(const float* t) {
  float s = t[0];
#pragma unroll
  for (int j = 1; j < NJ; ++j) s = s + t[j];
  return wave_sum0(s);
}

constexpr int kTokBatch = 8;   // span rows whose loads are issued together

// x / d rounded as the division: a product with the reciprocal when d is a
// power of two (the reciprocal is exact, so the product's one rounding is the
// quotient's).
struct DimDiv {
  float d, inv;
  bool pow2;
  __device__ __forceinline__ explicit DimDiv(int D)
      : d(static_cast<float>(D)), inv(1.0f / static_cast<float>(D)), pow2(D > 0 && (D & (D - 1)) == 0) {}
  __device__ __forceinline__ float operator()(float x) const { return pow2 ? x * inv : x / d; }
};

// Running token statistics of one component over a span.
template <int NJ>
struct SpanAcc {
  float acc[NJ];
  float e;
};

// Folds kTokBatch held rows (those of them before `rows`) into a component's
// statistics: token sums and the rows' mean squares (canonical sums of
// squares, four rows per fold, divided by D lane-parallel), in span order.
template <int NJ>
__device__ __forceinline__ void span_fold(const float (&x)[kTokBatch][NJ], int i0, int rows, const DimDiv& dd,
                                          SpanAcc<NJ>& s) {
  const int l = lane_id();
  float ss[kTokBatch];
#pragma unroll
  for (int t = 0; t < kTokBatch; t += 4) {
    float part[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      part[k] = x[t + k][0] * x[t + k][0];
#pragma unroll
      for (int j = 1; j < NJ; ++j) part[k] = part[k] + x[t + k][j] * x[t + k][j];
    }
    wave_sum4(part[0], part[1], part[2], part[3], ss[t], ss[t + 1], ss[t + 2], ss[t + 3]);
  }
  float num = 0.f;
#pragma unroll
  for (int t = 0; t < kTokBatch; ++t) num = l == t ? ss[t] : num;
  const float msl = dd(num);
#pragma unroll
  for (int t = 0; t < kTokBatch; ++t) {
    if (t >= rows) break;
    const int i = i0 + t;
#pragma unroll
    for (int j = 0; j < NJ; ++j) s.acc[j] = i == 0 ? x[t][j] : s.acc[j] + x[t][j];
    const float ms = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(msl), t));
    s.e = i == 0 ? ms : s.e + ms;
  }
}

// A component's means (per lane features), energy E and mean square of the
// means; returns R = residual / energy.
template <int NJ, bool FULL>
__device__ __forceinline__ float span_finish(const SpanAcc<NJ>& s, int n, int D, const DimDiv& dd, float* mean,
                                             float& energy, float& msq) {
  const int l = lane_id();
  const float cnt = static_cast<float>(n);
  float m2[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    mean[j] = s.acc[j] / cnt;
    m2[j] = (FULL || l + j * kWave < D) ? mean[j] * mean[j] : 0.f;
  }
  energy = s.e / cnt;
  msq = dd(canon_sum<NJ>(m2));
  return fmaxf(energy - msq, 0.f) / fmaxf(energy, 1e-12f);
}

// Token statistics of both components over a span in one pass: the span's row
// indices are read a lane each, 64 at a time, and kTokBatch K and V rows are
// loaded together per step.
// FULL: dk = dv = 64 NJ, every lane's features are in the row (no masking).
template <int NJ, bool FULL>
__device__ __forceinline__ void span_components(const Rows2& ks, const Rows2& vs, int b, int g,
                                                const LOGKV_G int32_t* tok, int n, int dk, int dv, float* mean_k,
                                                float& e_k, float& msq_k, float& rk, float& rv) {
  const int l = lane_id();
  const DimDiv dk_div(FULL ? kWave * NJ : dk), dv_div(FULL ? kWave * NJ : dv);
  SpanAcc<NJ> sk{}, sv{};
  for (int c0 = 0; c0 < n; c0 += kWave) {
    const int cn = min(kWave, n - c0);
    const int tl = l < cn ? tok[c0 + l] : 0;
    for (int i0 = 0; i0 < cn; i0 += kTokBatch) {
      float xk[kTokBatch][NJ], xv[kTokBatch][NJ];
#pragma unroll
      for (int t = 0; t < kTokBatch; ++t) {
        const int tt = __builtin_amdgcn_readlane(tl, min(i0 + t, cn - 1));
        const LOGKV_G uint16_t* rowk = ks.row(b, g, tt);
        const LOGKV_G uint16_t* rowv = vs.row(b, g, tt);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          xk[t][j] = FULL ? bf16_to_f32(rowk[l + j * kWave]) : feat_or_zero(rowk, l + j * kWave, dk);
          xv[t][j] = FULL ? bf16_to_f32(rowv[l + j * kWave]) : feat_or_zero(rowv, l + j * kWave, dv);
        }
      }
      span_fold<NJ>(xk, c0 + i0, cn - i0, dk_div, sk);
      span_fold<NJ>(xv, c0 + i0, cn - i0, dv_div, sv);
    }
  }
  float mean_v[NJ], e_v, msq_v;
  rk = span_finish<NJ, FULL>(sk, n, dk, dk_div, mean_k, e_k, msq_k);
  rv = span_finish<NJ, FULL>(sv, n, dv, dv_div, mean_v, e_v, msq_v);
}

// Candidate slots of the select path: row b owns slots [b * slots, (b + 1) *
// slots), of which the first row_count[b] are candidates. NULL row_count: the
// spans are numbered densely (the first *n_spans_dev of n_spans if given).
struct SpanSlots {
  const int32_t* row_count;
  int32_t slots;
};

__device__ __forceinline__ bool span_live(const logkv_span_args& a, const SpanSlots& sl, int s) {
  return !a.n_spans_dev || s < *a.n_spans_dev;
}

template <int NJ, bool FULL>
__device__ __forceinline__ void score_span(const logkv_span_args& a, int s, float* part_k, float* part_v, float* q_s,
                                           float* __restrict__ out) {
  const int g = wave_id();
  const int G = a.n_groups;
  const LOGKV_G int32_t* offs = gp(a.span_offsets);
  const int start = offs[s], n = offs[s + 1] - start;
  const int b = a.span_rows[s];
  const LOGKV_G int32_t* tok = gp(a.tokens) + start;
  if (g < G && n > 0) {
    Rows2 ks{gp(a.pool_k), a.pk_sb, a.pk_sg, a.pk_st, gp(a.flush_k), a.fk_sb, a.fk_sg, a.fk_st, a.old_width};
    Rows2 vs{gp(a.pool_v), a.pv_sb, a.pv_sg, a.pv_st, gp(a.flush_v), a.fv_sb, a.fv_sg, a.fv_st, a.old_width};
    float mean_k[NJ], e_k, msq_k, rk, rv;
    span_components<NJ, FULL>(ks, vs, b, g, tok, n, a.dk, a.dv, mean_k, e_k, msq_k, rk, rv);
    float q = 0.f;
    if (a.beta_novelty) {
      const int l = lane_id();
      const LOGKV_G float* mu = gp(a.centroids) + (static_cast<int64_t>(b) * G + g) * a.k_max * a.dk;
      const LOGKV_G uint8_t* valid = gp(a.centroid_valid) + (static_cast<int64_t>(b) * G + g) * a.k_max;
      const DimDiv dk_div(FULL ? kWave * NJ : a.dk);
      float nearest = __builtin_inff();
      bool any = false;
      // Four centers at a time: their dot and square sums, each one canonical sum (wave_sum4).
      for (int c0 = 0; c0 < a.k_max; c0 += 4) {
        float pd[4], pc[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int c = min(c0 + k, a.k_max - 1);
          float m[NJ];
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            m[j] = FULL ? mu[c * a.dk + l + j * kWave] : feat_or_zero(mu + c * a.dk, l + j * kWave, a.dk);
          pd[k] = mean_k[0] * m[0];
          pc[k] = m[0] * m[0];
#pragma unroll
          for (int j = 1; j < NJ; ++j) {
            pd[k] = pd[k] + mean_k[j] * m[j];
            pc[k] = pc[k] + m[j] * m[j];
          }
        }
        float sd[4], sc[4];
        wave_sum4(pd[0], pd[1], pd[2], pd[3], sd[0], sd[1], sd[2], sd[3]);
        wave_sum4(pc[0], pc[1], pc[2], pc[3], sc[0], sc[1], sc[2], sc[3]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int c = c0 + k;
          if (c >= a.k_max) break;
          const float dist = fmaxf((msq_k + dk_div(sc[k])) - 2.0f * dk_div(sd[k]), 0.f);
          if (valid[c]) {
            any = true;
            nearest = fminf(nearest, dist);
          }
        }
      }
      if (!any) nearest = 0.f;
      const float nov = nearest / fmaxf(e_k, 1e-12f);
      q = (rk + rv) * 0.5f + nov / (1.0f + nov);
    }
    if (lane_id() == 0) {
      part_k[g] = rk;
      part_v[g] = rv;
      q_s[g] = q;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float score = 0.f;
    if (n > 0) {
      if (a.beta_novelty) {
        float t0 = -__builtin_inff(), t1 = -__builtin_inff();
        for (int gg = 0; gg < G; ++gg) {
          const float v = q_s[gg];
          if (v > t0) {
            t1 = t0;
            t0 = v;
          } else if (v > t1) {
            t1 = v;
          }
        }
        score = G >= 2 ? (t0 + t1) / 2.0f : t0;
      } else {
        float sk = part_k[0], sv = part_v[0];
        for (int gg = 1; gg < G; ++gg) {
          sk = sk + part_k[gg];
          sv = sv + part_v[gg];
        }
        score = (0.0f + sk / static_cast<float>(G)) + sv / static_cast<float>(G);
      }
    }
    out[s] = score;
  }
  __syncthreads();   // part_k / part_v / q_s are rewritten by the block's next span
}

// One span per block iteration (grid-stride over the span slots), one wave
// per KV group.
template <int NJ, bool FULL>
__global__ __launch_bounds__(kMaxGroups * kWave) void score_kernel(logkv_span_args a, SpanSlots sl,
                                                                   float* __restrict__ out) {
  __shared__ float part_k[kMaxGroups], part_v[kMaxGroups], q_s[kMaxGroups];
  if (sl.row_count) {   // grid (x, batch row): row b's candidates x, x + gridDim.x, ...
    const int b = blockIdx.y, n = sl.row_count[b];
    for (int i = blockIdx.x; i < n; i += gridDim.x)
      score_span<NJ, FULL>(a, b * sl.slots + i, part_k, part_v, q_s, out);
    return;
  }
  for (int s = blockIdx.x; s < a.n_spans; s += gridDim.x) {
    if (!span_live(a, sl, s)) continue;
    score_span<NJ, FULL>(a, s, part_k, part_v, q_s, out);
  }
}

// Destination rows [exact pool rows 0..P | archive rows] of one lane, a tile
// of kPartRows per block: the tile's source indices are read into LDS, then
// every thread copies kPartBatch 8-byte units of K|V, all loads issued before
// the stores (a source of -1 writes zeros).
constexpr int kPartRows = 32;
constexpr int kPartBatch = 8;

__global__ __launch_bounds__(256) void partition_kernel(logkv_partition_args a) {
  __shared__ int src_s[kPartRows];
  const int G = a.n_groups;
  const int lane_bg = blockIdx.y;
  const int b = lane_bg / G, g = lane_bg % G;
  const int r0 = blockIdx.x * kPartRows;
  const int rows = min(kPartRows, a.P + a.A - r0);
  if (rows <= 0) return;
  const int tid = static_cast<int>(threadIdx.x), nthr = static_cast<int>(blockDim.x);
  if (tid < rows) {
    const int r = r0 + tid;
    const bool to_pool = r < a.P;
    const int src = to_pool ? a.keep[static_cast<int64_t>(b) * a.P + r]
                            : a.archive[static_cast<int64_t>(b) * a.A + r - a.P];
    src_s[tid] = src;
    if (g == 0) {
      int64_t pos = 0;
      if (src >= 0)
        pos = src < a.old_width ? a.pool_pos[b * a.pp_sb + src] : a.flush_pos[b * a.fp_sb + src - a.old_width];
      if (to_pool) {
        a.out_pool_pos[static_cast<int64_t>(b) * a.P + r] = pos;
        a.out_pool_valid[static_cast<int64_t>(b) * a.P + r] = src >= 0 ? 1 : 0;
      } else {
        a.arch_pos[static_cast<int64_t>(b) * a.A + r - a.P] = pos;
      }
    }
  }
  __syncthreads();
  Rows2 ks{gp(a.pool_k), a.pk_sb, a.pk_sg, a.pk_st, gp(a.flush_k), a.fk_sb, a.fk_sg, a.fk_st, a.old_width};
  Rows2 vs{gp(a.pool_v), a.pv_sb, a.pv_sg, a.pv_st, gp(a.flush_v), a.fv_sb, a.fv_sg, a.fv_st, a.old_width};
  const int ku = a.dk / 4, units = (a.dk + a.dv) / 4, total = rows * units;
  const int64_t lane_row0 = (static_cast<int64_t>(b) * G + g);
  for (int i0 = tid; i0 < total; i0 += kPartBatch * nthr) {
    uint2 x[kPartBatch];
#pragma unroll
    for (int q = 0; q < kPartBatch; ++q) {
      const int i = min(i0 + q * nthr, total - 1);
      const int t = i / units, u = i % units;
      const int src = src_s[t];
      const int sr = src >= 0 ? src : 0;
      const LOGKV_G uint16_t* p = u < ku ? ks.row(b, g, sr) + 4 * u : vs.row(b, g, sr) + 4 * (u - ku);
      const uint2 v = *(const LOGKV_G uint2*)p;
      x[q] = src >= 0 ? v : make_uint2(0u, 0u);
    }
#pragma unroll
    for (int q = 0; q < kPartBatch; ++q) {
      const int i = i0 + q * nthr;
      if (i < total) {
        const int t = i / units, u = i % units, r = r0 + t;
        LOGKV_G uint16_t* dst;
        if (r < a.P) dst = u < ku ? gp(a.out_pool_k) + (lane_row0 * a.P + r) * a.dk + 4 * u
                                  : gp(a.out_pool_v) + (lane_row0 * a.P + r) * a.dv + 4 * (u - ku);
        else dst = u < ku ? gp(a.arch_k) + (lane_row0 * a.A + (r - a.P)) * a.dk + 4 * u
                          : gp(a.arch_v) + (lane_row0 * a.A + (r - a.P)) * a.dv + 4 * (u - ku);
        *(LOGKV_G uint2*)dst = x[q];
      }
    }
  }
}

// ---- Span selection on the device ------------------------------------------
//
// Candidates (litgpt/alpha_log_kv.py:84-122): per batch row, the closed spans
// of the current selection (old), the unfinished old span when a position
// jump closes it, then the runs of the new rows; a run closes after a
// boundary row, at max_span rows (the unfinished old span counts toward the
// first run, which it prefixes) and before a position jump. Token indices
// address [pool (P rows) | flush]. Choice (litgpt/alpha_log_kv.py:177-226):
// unfinished spans are mandatory, old closed spans are kept first at density
// 1.1 * score and evicted lowest density first (later span first on ties) to
// fit the budget, then the other spans by decreasing density (earlier first)
// take free room or replace the lowest-density kept spans whose summed
// density * length is strictly lower. Densities and losses are doubles, as
// the reference's Python floats.

struct SelectWs {
  int32_t* cand_row;     // [C] batch row of candidate slot i
  uint8_t* cand_flags;   // [C] bit 0 old, bit 1 closed
  int32_t* row_count;    // [n_batch] candidates of each row
  int32_t* offsets;      // [C] candidate i's tokens: tokens[offsets[i], offsets[i + 1])
  int32_t* tokens;       // [n_batch * (P + T)]
  float* scores;         // [C]
};

constexpr int kSelectThreads = 256;
constexpr int kCutBatch = 8;   // boundary rows per thread in flight in the cut

// Candidate slots of one batch row: at most P + T + 1 candidates plus the end
// offset of the last one. Row b owns slots [b * R, (b + 1) * R) and tokens
// [b * (P + T), (b + 1) * (P + T)).
__host__ __device__ inline int select_row_slots(int P, int T) { return P + T + 2; }

__host__ __device__ inline int64_t select_candidates(int n_batch, int P, int T) {
  return static_cast<int64_t>(n_batch) * select_row_slots(P, T);
}

// Inclusive wave scan by DPP: shifts 1, 2, 4, 8 within each row of 16 lanes,
// then lane 15 of each row into the next row, lane 31 into rows 2 and 3
// (lanes without a source add 0).
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);   // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);   // row_bcast:31
  return v;
}

// Lane l receives lane l - 1's value (DPP wave_shr:1; lane 0 keeps its own).
__device__ __forceinline__ int wave_shr1(int v) { return __builtin_amdgcn_update_dpp(v, v, 0x138, 0xf, 0xf, false); }
__device__ __forceinline__ double wave_shr1(double v) {
  const long long bits = __double_as_longlong(v);
  const int lo = wave_shr1(static_cast<int>(bits)), hi = wave_shr1(static_cast<int>(bits >> 32));
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<uint32_t>(lo));
}

// Exclusive block-wide scan of one int per thread (every thread of the block
// calls it: it holds barriers); `total` receives the block's sum.
__device__ __forceinline__ int block_excl_scan(int v, int* wave_tmp, int& total) {
  const int w = wave_id(), nw = static_cast<int>(blockDim.x) / kWave;
  const int incl = wave_incl_scan(v);
  if (lane_id() == kWave - 1) wave_tmp[w] = incl;
  __syncthreads();
  int before = 0, tot = 0;
  for (int q = 0; q < nw; ++q) {
    const int x = wave_tmp[q];
    before += q < w ? x : 0;
    tot += x;
  }
  __syncthreads();   // wave_tmp is free for the next scan
  total = tot;
  return before + incl - v;
}


// One block per batch row (litgpt/alpha_log_kv.py:16-53, :84-122). Closed old
// spans become candidates in order; the last open old span is pending: closed
// by a position jump before the first new row, else carried into the first
// run. New rows split into hard segments (first row, after a boundary, at a
// jump) and each segment into pieces of at most max_span rows (the carried
// rows count toward the first piece; a carry of max_span or more does not
// split its segment). Candidate numbers and token offsets come from block
// scans over old spans and over segments.
__global__ __launch_bounds__(kSelectThreads) void cut_kernel(logkv_alpha_select_args a, SelectWs w) {
  extern __shared__ __align__(16) uint8_t dyn[];
  const int b = blockIdx.x;
  const int T = a.tokens, P = a.budget, maxc = P + T + 1, ms = a.max_span;
  const int tid = static_cast<int>(threadIdx.x), nthr = static_cast<int>(blockDim.x);
  int32_t* seg = reinterpret_cast<int32_t*>(dyn);                            // [T + 1] segment starts
  int32_t* olen = seg + T + 1;                                               // [P]
  int32_t* c_first = olen + P;                                               // [maxc] first token of the range
  int32_t* c_len = c_first + maxc;                                           // [maxc] range length
  int32_t* c_pend = c_len + maxc;                                            // [maxc] prefixed pending rows
  int32_t* c_off = c_pend + maxc;                                            // [maxc] token offset in the row
  uint8_t* c_flags = reinterpret_cast<uint8_t*>(c_off + maxc);               // [maxc]
  uint8_t* flags = c_flags + maxc;                                           // [T] bit 0 boundary, 1 segment start
  uint8_t* oclosed = flags + T;                                              // [P]
  __shared__ int wave_tmp[kSelectThreads / kWave];
  __shared__ int pend_idx_s, pend_off_s, pend_len_s, carry_s, nc_s, nt_s;
  // One count per group of count_rows batch rows (0: one group); its first row's block clears it.
  const int count_rows = a.count_rows > 0 ? a.count_rows : a.n_batch;
  if (b % count_rows == 0 && tid == 0) a.alpha_count[b / count_rows] = 0;
  const LOGKV_G int64_t* pos = gp(a.new_pos + b * a.np_sb);
  const LOGKV_G uint8_t* ends = gp(a.ends + b * a.ends_sb);
  const int n_old = min(a.span_count[b], P);
  if (tid == 0) pend_idx_s = -1;
  for (int i = tid; i < n_old; i += nthr) {
    olen[i] = a.span_len[static_cast<int64_t>(b) * P + i];
    oclosed[i] = a.span_closed[static_cast<int64_t>(b) * P + i];
  }
  // Boundary flags, kCutBatch rows per thread loaded (clamped, unconditionally)
  // before any flag is written.
  for (int j0 = 0; j0 < T; j0 += kCutBatch * nthr) {
    int64_t pc[kCutBatch], pp[kCutBatch];
    uint8_t ec[kCutBatch], ep[kCutBatch];
#pragma unroll
    for (int q = 0; q < kCutBatch; ++q) {
      const int j = min(j0 + q * nthr + tid, T - 1);
      const int jp = j > 0 ? j - 1 : 0;
      pc[q] = pos[j];
      pp[q] = pos[jp];
      ec[q] = ends[j];
      ep[q] = ends[jp];
    }
#pragma unroll
    for (int q = 0; q < kCutBatch; ++q) {
      const int j = j0 + q * nthr + tid;
      if (j < T) {
        const bool end = ec[q] != 0;
        const bool jump = j > 0 && pc[q] != pp[q] + 1;
        const bool start = j == 0 || jump || (j > 0 && ep[q] != 0);
        flags[j] = static_cast<uint8_t>((end ? 1 : 0) | (start ? 2 : 0));
      }
    }
  }
  __syncthreads();
  // Segment starts in order (ballot compaction).
  int n_seg = 0;
  for (int j0 = 0; j0 < T; j0 += nthr) {
    const int j = j0 + tid;
    const bool mine = j < T && (flags[j] & 2);
    int tot;
    const int at = block_excl_scan(mine ? 1 : 0, wave_tmp, tot);
    if (mine) seg[n_seg + at] = j;
    n_seg += tot;
  }
  if (tid == 0) seg[n_seg] = T;
  // Closed old spans -> candidates 0.. in order; the last open one is pending.
  int n_closed = 0, closed_tok = 0, off_base = 0;
  for (int i0 = 0; i0 < n_old; i0 += nthr) {
    const int i = i0 + tid;
    const bool in = i < n_old;
    const int len = in ? olen[i] : 0;
    const bool cl = in && oclosed[i];
    int tot_len, tot_c, tot_t;
    const int off = off_base + block_excl_scan(len, wave_tmp, tot_len);
    const int ci = n_closed + block_excl_scan(cl ? 1 : 0, wave_tmp, tot_c);
    const int ti = closed_tok + block_excl_scan(cl ? len : 0, wave_tmp, tot_t);
    if (cl) {
      c_first[ci] = off;
      c_len[ci] = len;
      c_pend[ci] = 0;
      c_off[ci] = ti;
      c_flags[ci] = 3;   // old, closed
    }
    if (in && !cl) atomicMax(&pend_idx_s, i);
    __syncthreads();
    if (in && !cl && i == pend_idx_s) {   // this chunk's last open span (a later chunk may replace it)
      pend_off_s = off;
      pend_len_s = len;
    }
    off_base += tot_len;
    n_closed += tot_c;
    closed_tok += tot_t;
  }
  __syncthreads();
  if (tid == 0) {
    const bool has_pend = pend_idx_s >= 0 && pend_len_s > 0;
    const int pend_off = has_pend ? pend_off_s : 0, pend_len = has_pend ? pend_len_s : 0;
    int nc = n_closed, nt = closed_tok, carry = 0;
    if (T == 0) {
      if (pend_len) {
        c_first[nc] = pend_off;
        c_len[nc] = pend_len;
        c_pend[nc] = 0;
        c_off[nc] = nt;
        c_flags[nc] = 0;   // open
        ++nc;
        nt += pend_len;
      }
    } else if (pend_len) {
      const int64_t last = a.pool_pos[static_cast<int64_t>(b) * P + min(pend_off + pend_len, P) - 1];
      if (pos[0] != last + 1) {   // closed by the jump before the first new row
        c_first[nc] = pend_off;
        c_len[nc] = pend_len;
        c_pend[nc] = 0;
        c_off[nc] = nt;
        c_flags[nc] = 2;   // new, closed
        ++nc;
        nt += pend_len;
      } else {
        carry = pend_len;
      }
    }
    pend_off_s = pend_off;
    carry_s = carry;
    nc_s = nc;
    nt_s = nt;
  }
  __syncthreads();
  const int pend_off = pend_off_s, carry0 = carry_s;
  int nc = nc_s, nt = nt_s;
  // New segments -> pieces, numbered by block scans over the segments.
  for (int s0 = 0; s0 < n_seg; s0 += nthr) {
    const int sg = s0 + tid;
    const bool in = sg < n_seg;
    const int st = in ? seg[sg] : 0, e = in ? seg[sg + 1] : 0, len = e - st;
    const int carry = sg == 0 ? carry0 : 0;
    int pieces = 0;
    if (in) {
      if (carry >= ms) pieces = 1;
      else if (carry > 0) pieces = 1 + (max(len - (ms - carry), 0) + ms - 1) / ms;
      else pieces = (len + ms - 1) / ms;
    }
    int tot_p, tot_t;
    const int pbase = nc + block_excl_scan(pieces, wave_tmp, tot_p);
    const int tbase = nt + block_excl_scan(in ? len + carry : 0, wave_tmp, tot_t);
    if (in) {
      int p = st, cr = carry, t = tbase;
      for (int k = 0; k < pieces; ++k) {
        const int room = ms - cr;
        const int take = cr >= ms ? e - p : min(room, e - p);
        const bool closed = (cr < ms && take == room) || p + take < e || e < T || (flags[e - 1] & 1);
        c_first[pbase + k] = P + p;
        c_len[pbase + k] = take;
        c_pend[pbase + k] = cr;
        c_off[pbase + k] = t;
        c_flags[pbase + k] = closed ? 2 : 0;
        t += cr + take;
        p += take;
        cr = 0;
      }
    }
    nc += tot_p;
    nt += tot_t;
  }
  // Old spans claiming more than P rows are not a valid selection: the row
  // then has no candidates (its token lists would leave the row's region).
  if (nt > P + T) nc = nt = 0;
  __syncthreads();
  // Candidate table and token lists of this row's region.
  const int64_t cbase = static_cast<int64_t>(b) * select_row_slots(P, T);
  const int64_t tbase = static_cast<int64_t>(b) * (P + T);
  LOGKV_G int32_t* tok = gp(w.tokens) + tbase;
  for (int c = tid; c < nc; c += nthr) {
    w.offsets[cbase + c] = static_cast<int32_t>(tbase + c_off[c]);
    w.cand_row[cbase + c] = b;
    w.cand_flags[cbase + c] = c_flags[c];
    LOGKV_G int32_t* dst = tok + c_off[c];
    const int pend = c_pend[c];
    for (int t = 0; t < pend; ++t) dst[t] = pend_off + t;
    for (int t = 0; t < c_len[c]; ++t) dst[pend + t] = c_first[c] + t;
  }
  if (tid == 0) {
    w.offsets[cbase + nc] = static_cast<int32_t>(tbase + nt);
    w.row_count[b] = nc;
  }
}

// Strict weak order of the eviction list: ascending density, later candidate first.
__device__ __forceinline__ bool evict_before(double da, int ia, double db, int ib) {
  return da < db || (da == db && ia > ib);
}

// Sort key of a density: NaN as +inf, so that every order below is total.
__device__ __forceinline__ double sort_key(double d) { return d != d ? __builtin_inf() : d; }

constexpr int kCopyBatch = 8;       // token loads per thread in flight in the keep / archive copy
constexpr int kRankSortMax = 512;   // candidates sorted by counting ranks; more use a bitonic sort

// Value at list position p (uniform) of a per-lane slot array: slot p / 64 of lane p % 64.
template <int S>
__device__ __forceinline__ int slot_lane(const int (&x)[S], int p) {
  const int a = __builtin_amdgcn_readlane(x[0], p & (kWave - 1));
  if (S == 1) return a;
  const int b = __builtin_amdgcn_readlane(x[S - 1], p & (kWave - 1));
  return p < kWave ? a : b;
}
template <int S>
__device__ __forceinline__ double slot_lane(const double (&x)[S], int p) {
  const double a = readlane_f64(x[0], p & (kWave - 1));
  if (S == 1) return a;
  const double b = readlane_f64(x[S - 1], p & (kWave - 1));
  return p < kWave ? a : b;
}

// Eviction list held by one wave: list position p = 64 s + l is slot s of lane l (S <= 2).
template <int S>
struct EvictList {
  int id[S], sz[S];
  double dn[S];

  // Insert (i, d, s) at position q; positions q.. move up by one.
  __device__ __forceinline__ void insert(int q, int i, double d, int s) {
    const int l = lane_id();
#pragma unroll
    for (int k = S - 1; k >= 0; --k) {
      const int p = k * kWave + l;
      const int up_id = wave_shr1(id[k]), up_sz = wave_shr1(sz[k]);
      const double up_dn = wave_shr1(dn[k]);
      // Lane 0 of slot k takes lane 63 of slot k - 1.
      const int lo_id = k ? __builtin_amdgcn_readlane(id[k ? k - 1 : 0], kWave - 1) : 0;
      const int lo_sz = k ? __builtin_amdgcn_readlane(sz[k ? k - 1 : 0], kWave - 1) : 0;
      const double lo_dn = k ? readlane_f64(dn[k ? k - 1 : 0], kWave - 1) : 0.0;
      const bool from_prev = l == 0;
      const int pid = from_prev ? lo_id : up_id, psz = from_prev ? lo_sz : up_sz;
      const double pdn = from_prev ? lo_dn : up_dn;
      id[k] = p > q ? pid : (p == q ? i : id[k]);
      sz[k] = p > q ? psz : (p == q ? s : sz[k]);
      dn[k] = p > q ? pdn : (p == q ? d : dn[k]);
    }
  }
};

// The greedy over the ranked candidates (litgpt/alpha_log_kv.py:177-238) by one
// wave, the eviction list (at most 64 S positions) in registers. Each step:
// free room, else the shortest head of the list whose rows make room (from
// inclusive prefix sums of list sizes, rebuilt only when the list changes),
// its loss summed in list order; an accepted closed span is inserted at its
// place (a ballot counts the entries that stay before it). State bits in LDS
// follow every eviction and acceptance.
template <int S>
__device__ void greedy_wave(const int32_t* vict, int vh, int nv, int room, const int32_t* rank, int n_rank,
                            const int32_t* size, const double* dens, uint8_t* state) {
  const int l = lane_id();
  EvictList<S> V;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int p = s * kWave + l;
    int j = 0, sz = 0;
    double d = 0.0;
    if (p < nv) {
      j = vict[p];
      sz = size[j];
      d = dens[j];
    }
    V.id[s] = j;
    V.sz[s] = sz;
    V.dn[s] = d;
  }
  int cum[S];
  bool live[S];
  auto rescan = [&]() {
    int carry = 0;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int p = s * kWave + l;
      live[s] = p >= vh && p < nv;
      cum[s] = wave_incl_scan(live[s] ? V.sz[s] : 0) + carry;
      carry = __builtin_amdgcn_readlane(cum[s], kWave - 1);
    }
  };
  rescan();
  int ri = 0, rsz = 0, rfl = 0;
  double rdn = 0.0;
  for (int r = 0; r < n_rank; ++r) {
    const int k = r & (kWave - 1);
    if (k == 0 && r + l < n_rank) {
      ri = rank[r + l];
      rsz = size[ri];
      rdn = dens[ri];
      rfl = state[ri];
    }
    const int i = __builtin_amdgcn_readlane(ri, k), need = __builtin_amdgcn_readlane(rsz, k);
    const double di = readlane_f64(rdn, k);
    const bool closed = (__builtin_amdgcn_readlane(rfl, k) & 2) != 0;
    bool ok = room >= need;
    int last = -1, avail = room;
    if (!ok) {
#pragma unroll
      for (int s = S - 1; s >= 0; --s) {
        const uint64_t hit = __ballot(live[s] && cum[s] >= need - room);
        if (hit) last = s * kWave + __builtin_ctzll(hit);
      }
      if (last >= 0) {
        avail = room + slot_lane<S>(cum, last);
        double loss = 0.0;
        for (int t = vh; t <= last; ++t) loss += slot_lane<S>(V.dn, t) * static_cast<double>(slot_lane<S>(V.sz, t));
        ok = di * static_cast<double>(need) > loss;
      }
    }
    if (!ok) continue;
    if (last >= 0) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int p = s * kWave + l;
        if (p >= vh && p <= last) state[V.id[s]] &= ~4;
      }
      vh = last + 1;
    }
    if (l == 0) state[i] |= 4;
    room = avail - need;
    if (closed) {
      int before = 0;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int p = s * kWave + l;
        before += __popcll(__ballot(p >= vh && p < nv && !evict_before(di, i, V.dn[s], V.id[s])));
      }
      V.insert(vh + before, i, di, need);
      ++nv;
    }
    if (last >= 0 || closed) rescan();
  }
}

// The same greedy by one thread over the list in LDS (any list length).
__device__ void greedy_serial(int32_t* vict, int vh, int nv, int room, const int32_t* rank, int n_rank,
                              const int32_t* size, const double* dens, uint8_t* state) {
  for (int r = 0; r < n_rank; ++r) {
    const int i = rank[r];
    const int need = size[i];
    int avail = room, n_taken = 0;
    double loss = 0.0;
    if (avail < need) {
      for (int q = vh; q < nv; ++q) {
        const int j = vict[q];
        ++n_taken;
        avail += size[j];
        loss += dens[j] * static_cast<double>(size[j]);
        if (avail >= need) break;
      }
    }
    if (avail >= need && (n_taken == 0 || dens[i] * static_cast<double>(need) > loss)) {
      for (int t = 0; t < n_taken; ++t) state[vict[vh + t]] &= ~4;
      vh += n_taken;
      state[i] |= 4;
      room = avail - need;
      if (state[i] & 2) {   // a closed span joins the evictable list at its place
        int q = nv;
        while (q > vh && evict_before(dens[i], i, dens[vict[q - 1]], vict[q - 1])) {
          vict[q] = vict[q - 1];
          --q;
        }
        vict[q] = i;
        ++nv;
      }
    }
  }
}

// One block per batch row (litgpt/alpha_log_kv.py:177-238): candidates sorted
// into eviction order (ascending density, later first; its reverse is the
// ranking order), open and old spans taken first, the lowest-density chosen
// spans evicted while the budget is exceeded, then the greedy over the rest in
// ranking order; kept / archived rows and the new span list written by the
// block. Every phase but the greedy is block-parallel.
__global__ __launch_bounds__(kSelectThreads) void choose_kernel(logkv_alpha_select_args a, SelectWs w) {
  extern __shared__ __align__(16) uint8_t dyn[];
  const int b = blockIdx.x;
  const int P = a.budget, T = a.tokens;
  const int c0 = b * select_row_slots(P, T), n = w.row_count[b];
  const bool bitonic = n > kRankSortMax;
  int width = 1;
  while (bitonic && width < n) width <<= 1;
  double* key = reinterpret_cast<double*>(dyn);                      // [width] bitonic sort keys
  double* dens = key + width;                                        // [n] density by candidate
  int32_t* idx = reinterpret_cast<int32_t*>(dens + n);               // [max(width, n)] eviction order
  int32_t* size = idx + (width > n ? width : n);                     // [n]
  int32_t* koff = size + n;                                          // [n] keep / archive offsets
  int32_t* rank = koff + n;                                          // [n] candidates to rank
  // Evictable spans in eviction order. Entries are dropped from the head and
  // inserted once per acceptance, so the list spans at most 2n positions.
  int32_t* vict = rank + n;                                          // [2n]
  int32_t* cstart = vict + 2 * n;                                    // [n] token offset in the row
  uint8_t* state = reinterpret_cast<uint8_t*>(cstart + n);           // [n] bit 0 old, 1 closed, 2 chosen
  __shared__ int wave_tmp[kSelectThreads / kWave];
  __shared__ int vh_s, room_s;
  const int tid = static_cast<int>(threadIdx.x), nthr = static_cast<int>(blockDim.x);
  const int o0 = w.offsets[c0];
  // Densities (old spans x 1.1), sizes, token offsets; open and old spans are
  // chosen up front.
  int pre = 0;   // low 16 bits: rows chosen up front; high: closed candidates
  for (int i = tid; i < n; i += nthr) {
    const uint8_t f = w.cand_flags[c0 + i];
    const double d = static_cast<double>(w.scores[c0 + i]) * ((f & 1) ? 1.1 : 1.0);
    const int o = w.offsets[c0 + i];
    const int sz = w.offsets[c0 + i + 1] - o;
    const bool first = !(f & 2) || (f & 1);
    dens[i] = d;
    size[i] = sz;
    cstart[i] = o - o0;
    state[i] = static_cast<uint8_t>(f | (first ? 4 : 0));
    pre += (first ? sz : 0) + ((f & 2) ? 1 << 16 : 0);
  }
  int pre_total;
  block_excl_scan(pre, wave_tmp, pre_total);   // also the barrier after the loads
  int room = P - (pre_total & 0xffff);
  const int n_closed = pre_total >> 16;
  if (!bitonic) {
    // Counting sort: a candidate's place is the number of candidates before
    // it (a total order: NaN keys sort as +inf, ties by index).
    for (int i = tid; i < n; i += nthr) {
      const double di = sort_key(dens[i]);
      int at = 0;
#pragma unroll 8
      for (int j = 0; j < n; ++j) at += evict_before(sort_key(dens[j]), j, di, i) ? 1 : 0;
      idx[at] = i;
    }
  } else {
    for (int i = tid; i < width; i += nthr) {
      key[i] = i < n ? sort_key(dens[i]) : __builtin_inf();
      idx[i] = i < n ? i : 0x7fffffff;
    }
    __syncthreads();
    for (int sz = 2; sz <= width; sz <<= 1) {
      for (int stride = sz >> 1; stride > 0; stride >>= 1) {
        for (int t = tid; t < width; t += nthr) {
          const int partner = t ^ stride;
          if (partner > t) {
            const bool up = (t & sz) == 0;
            const double ka = key[t], kb = key[partner];
            const int ia = idx[t], ib = idx[partner];
            const bool pa = ia == 0x7fffffff, pb = ib == 0x7fffffff;
            const bool a_after = pa != pb ? pa : (!pa && evict_before(kb, ib, ka, ia));
            if (a_after == up) {
              key[t] = kb;
              key[partner] = ka;
              idx[t] = ib;
              idx[partner] = ia;
            }
          }
        }
        __syncthreads();
      }
    }
  }
  __syncthreads();
  // Evictable spans (chosen and closed) in eviction order.
  int nv = 0;
  for (int q0 = 0; q0 < n; q0 += nthr) {
    const int q = q0 + tid;
    const int i = q < n ? idx[q] : 0;
    const bool ev = q < n && (state[i] & 6) == 6;
    int tot;
    const int at = block_excl_scan(ev ? 1 : 0, wave_tmp, tot);
    if (ev) vict[nv + at] = i;
    nv += tot;
  }
  // Over budget: evict from the head of the list until the budget holds.
  if (tid == 0) {
    vh_s = room < 0 ? nv : 0;
    room_s = room;
  }
  __syncthreads();
  if (room < 0) {
    int cum = 0;
    for (int q0 = 0; q0 < nv; q0 += nthr) {
      const int q = q0 + tid;
      const int sz = q < nv ? size[vict[q]] : 0;
      int tot;
      const int before = cum + block_excl_scan(sz, wave_tmp, tot);
      if (q < nv && room + before < 0 && room + before + sz >= 0) {
        vh_s = q + 1;
        room_s = room + before + sz;
      }
      cum += tot;
    }
    __syncthreads();
    if (vh_s == nv && tid == 0) room_s = room + cum;
    __syncthreads();
    for (int q = tid; q < vh_s; q += nthr) state[vict[q]] &= ~4;
    __syncthreads();
  }
  const int vh = vh_s;
  room = room_s;
  // Candidates to rank: the unchosen ones, decreasing density, earlier first.
  int n_rank = 0;
  for (int r0 = 0; r0 < n; r0 += nthr) {
    const int q = n - 1 - (r0 + tid);
    const int i = q >= 0 ? idx[q] : 0;
    const bool rk = q >= 0 && !(state[i] & 4);
    int tot;
    const int at = block_excl_scan(rk ? 1 : 0, wave_tmp, tot);
    if (rk) rank[n_rank + at] = i;
    n_rank += tot;
  }
  // The list holds at most nv + (closed candidates ranked) <= n_closed + vh positions.
  const int list_cap = n_closed + vh;
  if (list_cap <= kWave) {
    if (wave_id() == 0) greedy_wave<1>(vict, vh, nv, room, rank, n_rank, size, dens, state);
  } else if (list_cap <= 2 * kWave) {
    if (wave_id() == 0) greedy_wave<2>(vict, vh, nv, room, rank, n_rank, size, dens, state);
  } else if (tid == 0) {
    greedy_serial(vict, vh, nv, room, rank, n_rank, size, dens, state);
  }
  __syncthreads();
  // Keep / archive offsets and the new span list, in candidate order.
  LOGKV_G int32_t* keep = gp(a.keep + static_cast<int64_t>(b) * P);
  int kept = 0, spans = 0;
  for (int i0 = 0; i0 < n; i0 += nthr) {
    const int i = i0 + tid;
    const bool kp = i < n && (state[i] & 4);
    const int sz = kp ? size[i] : 0;
    int tot;
    const int x = block_excl_scan(sz | (kp ? 1 << 16 : 0), wave_tmp, tot);
    if (i < n) {
      const int kept_before = kept + (x & 0xffff), spans_before = spans + (x >> 16);
      koff[i] = kp ? kept_before : cstart[i] - kept_before;
      if (kp) {
        a.new_span_len[static_cast<int64_t>(b) * P + spans_before] = sz;
        a.new_span_closed[static_cast<int64_t>(b) * P + spans_before] = (state[i] & 2) ? 1 : 0;
      }
    }
    kept += tot & 0xffff;
    spans += tot >> 16;
  }
  const int n_tok = w.offsets[c0 + n] - o0;
  const int arch = n_tok - kept;
  if (tid == 0) {
    a.new_span_count[b] = spans;
    a.archive_count[b] = arch;
    atomicMax(a.alpha_count + b / (a.count_rows > 0 ? a.count_rows : a.n_batch), kept);
  }
  __syncthreads();
  const int A = P + T;
  LOGKV_G int32_t* archive = gp(a.archive + static_cast<int64_t>(b) * A);
  // One thread per token of the row (its candidate by binary search over the
  // candidates' token offsets), so the token loads are all in flight.
  for (int g0 = 0; g0 < n_tok; g0 += kCopyBatch * nthr) {
    int32_t v[kCopyBatch];
#pragma unroll
    for (int q = 0; q < kCopyBatch; ++q) v[q] = w.tokens[o0 + min(g0 + q * nthr + tid, n_tok - 1)];
    // The token's candidate: the largest c with cstart[c] <= g, kCopyBatch
    // branch-free binary searches (uniform lengths, unconditional LDS loads)
    // advanced in lockstep.
    int lo[kCopyBatch];
#pragma unroll
    for (int q = 0; q < kCopyBatch; ++q) lo[q] = 0;
    for (int len = n; len > 1;) {
      const int half = len >> 1;
#pragma unroll
      for (int q = 0; q < kCopyBatch; ++q) {
        const int g = g0 + q * nthr + tid;
        lo[q] = cstart[lo[q] + half] <= g ? lo[q] + half : lo[q];
      }
      len -= half;
    }
#pragma unroll
    for (int q = 0; q < kCopyBatch; ++q) {
      const int g = g0 + q * nthr + tid;
      if (g < n_tok) {
        const int c = lo[q], t = g - cstart[c];
        const bool kept_i = (state[c] & 4) != 0;
        const int cap = kept_i ? P - koff[c] : A - koff[c];   // the greedy keeps at most P rows
        if (t < cap) (kept_i ? keep : archive)[koff[c] + t] = v[q];
      }
    }
  }
  for (int i = kept + tid; i < P; i += nthr) keep[i] = -1;
  for (int i = arch + tid; i < A; i += nthr) archive[i] = -1;
  if (a.scores) {
    // Scores out densely: row b's candidates follow those of rows 0..b-1.
    int dense = 0;
    for (int r = 0; r < b; ++r) dense += w.row_count[r];
    for (int i = tid; i < n; i += nthr) a.scores[dense + i] = w.scores[c0 + i];
  }
}

}  // namespace

constexpr int kScoreBlocks = 2048;   // most blocks of a score launch (each strides over span slots)

int launch_score_slots(const logkv_span_args& a, const SpanSlots& sl, float* out, int n_rows, hipStream_t stream) {
  if (a.n_spans <= 0) return LOGKV_OK;
  // Per-row slots: kScoreBlocks spread over the rows, at least 32 per row and
  // no more than a row's slots.
  const dim3 grid = sl.row_count
                        ? dim3(static_cast<unsigned>(std::min(sl.slots, std::max(32, kScoreBlocks / n_rows))),
                               static_cast<unsigned>(n_rows))
                        : dim3(static_cast<unsigned>(std::min(a.n_spans, kScoreBlocks)));
  if (a.dk == 2 * kWave && a.dv == 2 * kWave)
    hipLaunchKernelGGL((score_kernel<2, true>), grid, dim3(a.n_groups * kWave), 0, stream, a, sl, out);
  else if (a.dk <= 2 * kWave && a.dv <= 2 * kWave)
    hipLaunchKernelGGL((score_kernel<2, false>), grid, dim3(a.n_groups * kWave), 0, stream, a, sl, out);
  else
    hipLaunchKernelGGL((score_kernel<4, false>), grid, dim3(a.n_groups * kWave), 0, stream, a, sl, out);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_score(const logkv_span_args& a, float* out, hipStream_t stream) {
  return launch_score_slots(a, SpanSlots{nullptr, 0}, out, 1, stream);
}

int64_t select_workspace_bytes(const logkv_alpha_select_args& a) {
  const int64_t C = select_candidates(a.n_batch, a.budget, a.tokens);
  auto al = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  return al(C * 4) + al(C) + al(static_cast<int64_t>(a.n_batch) * 4) + al(C * 4) +
         al(static_cast<int64_t>(a.n_batch) * (a.budget + a.tokens) * 4) + al(C * 4);
}

int launch_select(const logkv_alpha_select_args& a, void* ws, hipStream_t stream) {
  const int64_t C = select_candidates(a.n_batch, a.budget, a.tokens);
  auto al = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  uint8_t* p = static_cast<uint8_t*>(ws);
  SelectWs w;
  w.cand_row = reinterpret_cast<int32_t*>(p);
  p += al(C * 4);
  w.cand_flags = p;
  p += al(C);
  w.row_count = reinterpret_cast<int32_t*>(p);
  p += al(static_cast<int64_t>(a.n_batch) * 4);
  w.offsets = reinterpret_cast<int32_t*>(p);
  p += al(C * 4);
  w.tokens = reinterpret_cast<int32_t*>(p);
  p += al(static_cast<int64_t>(a.n_batch) * (a.budget + a.tokens) * 4);
  w.scores = reinterpret_cast<float*>(p);
  const size_t cut_c = static_cast<size_t>(a.budget) + a.tokens + 1;
  const size_t cut_shmem = 4 * (static_cast<size_t>(a.tokens) + 1) + 5 * static_cast<size_t>(a.budget) +
                           17 * cut_c + static_cast<size_t>(a.tokens) + 16;
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&cut_kernel), cut_shmem)) return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(cut_kernel, dim3(a.n_batch), dim3(kSelectThreads), cut_shmem, stream, a, w);
  logkv_span_args sa = a.rows;
  sa.old_width = a.budget;
  sa.tokens = w.tokens;
  sa.span_offsets = w.offsets;
  sa.span_rows = w.cand_row;
  sa.n_spans = static_cast<int32_t>(C);
  sa.n_spans_dev = nullptr;
  int rc = launch_score_slots(sa, SpanSlots{w.row_count, select_row_slots(a.budget, a.tokens)}, w.scores, a.n_batch,
                              stream);
  if (rc) return rc;
  const int maxc = a.budget + a.tokens + 1;
  int width = 1;
  while (width < maxc) width <<= 1;
  const size_t choose_shmem = static_cast<size_t>(width) * (8 + 4) + static_cast<size_t>(maxc) * (8 + 6 * 4 + 1) + 16;
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&choose_kernel), choose_shmem)) return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(choose_kernel, dim3(a.n_batch), dim3(kSelectThreads), choose_shmem, stream, a, w);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_partition(const logkv_partition_args& a, hipStream_t stream) {
  const int rows = a.P + a.A;
  if (rows <= 0) return LOGKV_OK;
  hipLaunchKernelGGL(partition_kernel, dim3((rows + kPartRows - 1) / kPartRows, a.n_batch * a.n_groups), dim3(256), 0,
                     stream, a);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
