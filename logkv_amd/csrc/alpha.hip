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

// Token statistics of one component over a span: means (per lane features),
// energy E and mean square of the means; returns R = residual / energy. Rows
// are loaded kTokBatch at a time and then added in span order.
template <int NJ>
__device__ __forceinline__ float span_component(const Rows2& src, int b, int g, const LOGKV_G int32_t* tok, int n,
                                                int D, float* mean, float& energy, float& msq) {
  const int l = lane_id();
  float acc[NJ], e = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = 0.f;
  const float d_f = static_cast<float>(D);
  for (int i0 = 0; i0 < n; i0 += kTokBatch) {
    float xb[kTokBatch][NJ];
#pragma unroll
    for (int t = 0; t < kTokBatch; ++t) {
      const int i = i0 + t < n ? i0 + t : n - 1;
      const LOGKV_G uint16_t* row = src.row(b, g, tok[i]);
#pragma unroll
      for (int j = 0; j < NJ; ++j) xb[t][j] = feat_or_zero(row, l + j * kWave, D);
    }
#pragma unroll
    for (int t = 0; t < kTokBatch; ++t) {
      const int i = i0 + t;
      if (i >= n) break;
      float sq[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        sq[j] = xb[t][j] * xb[t][j];
        acc[j] = i == 0 ? xb[t][j] : acc[j] + xb[t][j];
      }
      const float ms = canon_sum<NJ>(sq) / d_f;
      e = i == 0 ? ms : e + ms;
    }
  }
  const float cnt = static_cast<float>(n);
  float m2[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    mean[j] = acc[j] / cnt;
    m2[j] = (l + j * kWave < D) ? mean[j] * mean[j] : 0.f;
  }
  energy = e / cnt;
  msq = canon_sum<NJ>(m2) / d_f;
  return fmaxf(energy - msq, 0.f) / fmaxf(energy, 1e-12f);
}

template <int NJ>
__global__ __launch_bounds__(kMaxGroups * kWave) void score_kernel(logkv_span_args a, float* __restrict__ out) {
  __shared__ float part_k[kMaxGroups], part_v[kMaxGroups], q_s[kMaxGroups];
  const int s = blockIdx.x;
  const int g = wave_id();
  const int G = a.n_groups;
  const LOGKV_G int32_t* offs = gp(a.span_offsets);
  const int start = offs[s], n = offs[s + 1] - start;
  const int b = a.span_rows[s];
  const LOGKV_G int32_t* tok = gp(a.tokens) + start;
  if (g < G && n > 0) {
    Rows2 ks{gp(a.pool_k), a.pk_sb, a.pk_sg, a.pk_st, gp(a.flush_k), a.fk_sb, a.fk_sg, a.fk_st, a.old_width};
    Rows2 vs{gp(a.pool_v), a.pv_sb, a.pv_sg, a.pv_st, gp(a.flush_v), a.fv_sb, a.fv_sg, a.fv_st, a.old_width};
    float mean_k[NJ], mean_v[NJ], e_k, e_v, msq_k, msq_v;
    const float rk = span_component<NJ>(ks, b, g, tok, n, a.dk, mean_k, e_k, msq_k);
    const float rv = span_component<NJ>(vs, b, g, tok, n, a.dv, mean_v, e_v, msq_v);
    float q = 0.f;
    if (a.beta_novelty) {
      const int l = lane_id();
      const LOGKV_G float* mu = gp(a.centroids) + (static_cast<int64_t>(b) * G + g) * a.k_max * a.dk;
      const LOGKV_G uint8_t* valid = gp(a.centroid_valid) + (static_cast<int64_t>(b) * G + g) * a.k_max;
      float nearest = __builtin_inff();
      bool any = false;
      for (int c = 0; c < a.k_max; ++c) {
        float dt[NJ], cc[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const float m = feat_or_zero(mu + c * a.dk, l + j * kWave, a.dk);
          dt[j] = mean_k[j] * m;
          cc[j] = m * m;
        }
        const float dot = canon_sum<NJ>(dt) / static_cast<float>(a.dk);
        const float cms = canon_sum<NJ>(cc) / static_cast<float>(a.dk);
        const float dist = fmaxf((msq_k + cms) - 2.0f * dot, 0.f);
        if (valid[c]) {
          any = true;
          nearest = fminf(nearest, dist);
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
}

// One wave per destination row (exact pool rows [0, P), then archive rows).
__global__ __launch_bounds__(256) void partition_kernel(logkv_partition_args a) {
  const int G = a.n_groups;
  const int lane_bg = blockIdx.y;
  const int b = lane_bg / G, g = lane_bg % G;
  const int r = blockIdx.x * (blockDim.x / kWave) + wave_id();
  if (r >= a.P + a.A) return;
  const bool to_pool = r < a.P;
  const int src = to_pool ? a.keep[static_cast<int64_t>(b) * a.P + r] : a.archive[static_cast<int64_t>(b) * a.A + r - a.P];
  Rows2 ks{gp(a.pool_k), a.pk_sb, a.pk_sg, a.pk_st, gp(a.flush_k), a.fk_sb, a.fk_sg, a.fk_st, a.old_width};
  Rows2 vs{gp(a.pool_v), a.pv_sb, a.pv_sg, a.pv_st, gp(a.flush_v), a.fv_sb, a.fv_sg, a.fv_st, a.old_width};
  LOGKV_G uint16_t* dk_row;
  LOGKV_G uint16_t* dv_row;
  if (to_pool) {
    dk_row = gp(a.out_pool_k) + ((static_cast<int64_t>(b) * G + g) * a.P + r) * a.dk;
    dv_row = gp(a.out_pool_v) + ((static_cast<int64_t>(b) * G + g) * a.P + r) * a.dv;
  } else {
    dk_row = gp(a.arch_k) + ((static_cast<int64_t>(b) * G + g) * a.A + (r - a.P)) * a.dk;
    dv_row = gp(a.arch_v) + ((static_cast<int64_t>(b) * G + g) * a.A + (r - a.P)) * a.dv;
  }
  const int ku = a.dk / 4, units = (a.dk + a.dv) / 4;
  const LOGKV_G uint16_t* sk = src >= 0 ? ks.row(b, g, src) : nullptr;
  const LOGKV_G uint16_t* sv = src >= 0 ? vs.row(b, g, src) : nullptr;
  for (int u = lane_id(); u < units; u += kWave) {
    uint2 x = make_uint2(0u, 0u);
    if (src >= 0) x = *(const LOGKV_G uint2*)(u < ku ? sk + 4 * u : sv + 4 * (u - ku));
    *(LOGKV_G uint2*)(u < ku ? dk_row + 4 * u : dv_row + 4 * (u - ku)) = x;
  }
  if (g == 0 && lane_id() == 0) {
    int64_t pos = 0;
    if (src >= 0) pos = src < a.old_width ? a.pool_pos[b * a.pp_sb + src] : a.flush_pos[b * a.fp_sb + src - a.old_width];
    if (to_pool) {
      a.out_pool_pos[static_cast<int64_t>(b) * a.P + r] = pos;
      a.out_pool_valid[static_cast<int64_t>(b) * a.P + r] = src >= 0 ? 1 : 0;
    } else {
      a.arch_pos[static_cast<int64_t>(b) * a.A + r - a.P] = pos;
    }
  }
}

}  // namespace

int launch_score(const logkv_span_args& a, float* out, hipStream_t stream) {
  if (a.n_spans <= 0) return LOGKV_OK;
  if (a.dk <= 2 * kWave && a.dv <= 2 * kWave)
    hipLaunchKernelGGL(score_kernel<2>, dim3(a.n_spans), dim3(a.n_groups * kWave), 0, stream, a, out);
  else
    hipLaunchKernelGGL(score_kernel<4>, dim3(a.n_spans), dim3(a.n_groups * kWave), 0, stream, a, out);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_partition(const logkv_partition_args& a, hipStream_t stream) {
  const int rows = a.P + a.A;
  if (rows <= 0) return LOGKV_OK;
  const int per_block = 256 / kWave;
  hipLaunchKernelGGL(partition_kernel, dim3((rows + per_block - 1) / per_block, a.n_batch * a.n_groups), dim3(256), 0,
                     stream, a);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
