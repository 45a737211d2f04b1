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
  if (a.n_spans_dev && s >= *a.n_spans_dev) return;
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
  int32_t* cand_row;     // [C] batch row of candidate i
  uint8_t* cand_flags;   // [C] bit 0 old, bit 1 closed
  int32_t* row_cand;     // [n_batch + 1] first candidate of each row
  int32_t* offsets;      // [C + 1] candidate i's tokens: tokens[offsets[i], offsets[i + 1])
  int32_t* tokens;       // [n_batch * (P + T)]
  int32_t* n_spans;      // [1]
  float* scores;         // [C]
};

constexpr int kSelectThreads = 256;

__host__ __device__ inline int64_t select_candidates(int n_batch, int P, int T) {
  return static_cast<int64_t>(n_batch) * (P + T + 1);
}

// One block: rows in order. The block finds segment starts (first row, after
// a boundary, at a jump); thread 0 turns segments into candidate descriptors
// in LDS; the block writes the candidate table and token lists.
__global__ __launch_bounds__(kSelectThreads) void cut_kernel(logkv_alpha_select_args a, SelectWs w) {
  extern __shared__ __align__(16) uint8_t dyn[];
  const int T = a.tokens, P = a.budget, maxc = P + T + 1;
  int32_t* seg = reinterpret_cast<int32_t*>(dyn);                            // [T + 1] segment starts
  int32_t* olen = seg + T + 1;                                               // [P]
  int32_t* c_first = olen + P;                                               // [maxc] first token of the range
  int32_t* c_len = c_first + maxc;                                           // [maxc] range length
  int32_t* c_pend = c_len + maxc;                                            // [maxc] prefixed pending rows
  int32_t* c_off = c_pend + maxc;                                            // [maxc] token offset in the row
  uint8_t* c_flags = reinterpret_cast<uint8_t*>(c_off + maxc);               // [maxc]
  uint8_t* flags = c_flags + maxc;                                           // [T]
  uint8_t* oclosed = flags + T;                                              // [P]
  __shared__ int wave_cnt[kSelectThreads / kWave];
  __shared__ int n_seg_s, nc_s, nt_s, row_nc_s, row_nt_s, pend_off_s;
  if (threadIdx.x == 0) {
    nc_s = 0;
    nt_s = 0;
    *a.alpha_count = 0;
  }
  for (int b = 0; b < a.n_batch; ++b) {
    const LOGKV_G int64_t* pos = gp(a.new_pos + b * a.np_sb);
    const LOGKV_G uint8_t* ends = gp(a.ends + b * a.ends_sb);
    const int n_old = a.span_count[b];
    for (int i = threadIdx.x; i < n_old; i += blockDim.x) {
      olen[i] = a.span_len[static_cast<int64_t>(b) * P + i];
      oclosed[i] = a.span_closed[static_cast<int64_t>(b) * P + i];
    }
    for (int j = threadIdx.x; j < T; j += blockDim.x) {
      const bool end = ends[j] != 0;
      const bool jump = j > 0 && pos[j] != pos[j - 1] + 1;
      const bool start = j == 0 || jump || ends[j > 0 ? j - 1 : 0] != 0;
      flags[j] = static_cast<uint8_t>((end ? 1 : 0) | (start ? 2 : 0));
    }
    if (threadIdx.x == 0) n_seg_s = 0;
    __syncthreads();
    for (int j0 = 0; j0 < T; j0 += blockDim.x) {
      const int j = j0 + threadIdx.x;
      const bool mine = j < T && (flags[j] & 2);
      const uint64_t ballot = __ballot(mine);
      const int l = lane_id(), wv = wave_id();
      const int before = __popcll(ballot & ((l == 0) ? 0ull : (~0ull >> (kWave - l))));
      if (l == 0) wave_cnt[wv] = __popcll(ballot);
      __syncthreads();
      int base = n_seg_s;
      for (int q = 0; q < wv; ++q) base += wave_cnt[q];
      if (mine) seg[base + before] = j;
      __syncthreads();
      if (threadIdx.x == 0) {
        int add = 0;
        for (int q = 0; q < static_cast<int>(blockDim.x) / kWave; ++q) add += wave_cnt[q];
        n_seg_s += add;
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      int nc = 0, nt = 0;
      const int n_seg = n_seg_s;
      seg[n_seg] = T;
      auto emit = [&](int first, int len, int pend, bool old, bool closed) {
        c_first[nc] = first;
        c_len[nc] = len;
        c_pend[nc] = pend;
        c_off[nc] = nt;
        c_flags[nc] = static_cast<uint8_t>((old ? 1 : 0) | (closed ? 2 : 0));
        nt += pend + len;
        ++nc;
      };
      int off = 0, pend_off = 0, pend_len = 0;
      for (int i = 0; i < n_old; ++i) {
        if (oclosed[i]) emit(off, olen[i], 0, true, true);
        else {
          pend_off = off;
          pend_len = olen[i];
        }
        off += olen[i];
      }
      if (T == 0) {
        if (pend_len) emit(pend_off, pend_len, 0, false, false);
      } else {
        const bool pend_closed =
            pend_len > 0 && pos[0] != a.pool_pos[static_cast<int64_t>(b) * P + pend_off + pend_len - 1] + 1;
        if (pend_closed) emit(pend_off, pend_len, 0, false, true);
        int carry = pend_closed ? 0 : pend_len;
        for (int sg = 0; sg < n_seg; ++sg) {
          const int e = seg[sg + 1];
          for (int p = seg[sg]; p < e;) {
            const int room = a.max_span - carry;
            const int take = min(room, e - p);
            const bool closed = take == room || p + take < e || e < T || (flags[e - 1] & 1);
            emit(P + p, take, carry, false, closed);
            carry = 0;
            p += take;
          }
        }
      }
      row_nc_s = nc;
      row_nt_s = nt;
      pend_off_s = pend_off;
      w.row_cand[b] = nc_s;
    }
    __syncthreads();
    const int nc = row_nc_s, cbase = nc_s, tbase = nt_s, pend_off = pend_off_s;
    LOGKV_G int32_t* tok = gp(w.tokens) + tbase;
    for (int c = threadIdx.x; c < nc; c += blockDim.x) {
      w.offsets[cbase + c] = tbase + c_off[c];
      w.cand_row[cbase + c] = b;
      w.cand_flags[cbase + c] = c_flags[c];
      LOGKV_G int32_t* dst = tok + c_off[c];
      const int pend = c_pend[c];
      for (int t = 0; t < pend; ++t) dst[t] = pend_off + t;
      for (int t = 0; t < c_len[c]; ++t) dst[pend + t] = c_first[c] + t;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      nc_s += nc;
      nt_s += row_nt_s;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    w.row_cand[a.n_batch] = nc_s;
    w.offsets[nc_s] = nt_s;
    *w.n_spans = nc_s;
  }
}

// Strict weak order of the eviction list: ascending density, later candidate first.
__device__ __forceinline__ bool evict_before(double da, int ia, double db, int ib) {
  return da < db || (da == db && ia > ib);
}

// One block per batch row: densities sorted by the block, the greedy run by
// thread 0 over a compact sorted list of evictable spans, kept / archived rows
// written by the block.
__global__ __launch_bounds__(kSelectThreads) void choose_kernel(logkv_alpha_select_args a, SelectWs w) {
  extern __shared__ __align__(16) uint8_t dyn[];
  const int b = blockIdx.x;
  const int P = a.budget, T = a.tokens;
  const int c0 = w.row_cand[b], n = w.row_cand[b + 1] - c0;
  int width = 1;
  while (width < n) width <<= 1;
  double* key = reinterpret_cast<double*>(dyn);                      // [width] sort keys
  double* dens = key + width;                                        // [n] density by candidate
  int32_t* idx = reinterpret_cast<int32_t*>(dens + n);               // [width] sorted candidates
  int32_t* size = idx + width;                                       // [n]
  int32_t* koff = size + n;                                          // [n] keep / archive offsets
  int32_t* rank = koff + n;                                          // [n] candidates to rank
  int32_t* vict = rank + n;                                          // [n] evictable spans, eviction order
  uint8_t* state = reinterpret_cast<uint8_t*>(vict + n);             // [n] bit 0 old, 1 closed, 2 chosen
  __shared__ int kept_s, arch_s;
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    if (i < n) {
      const uint8_t f = w.cand_flags[c0 + i];
      const double d = static_cast<double>(w.scores[c0 + i]) * ((f & 1) ? 1.1 : 1.0);
      dens[i] = d;
      key[i] = d;
      idx[i] = i;
      size[i] = w.offsets[c0 + i + 1] - w.offsets[c0 + i];
      state[i] = f;
    } else {
      key[i] = __builtin_inf();
      idx[i] = 0x7fffffff;
    }
  }
  __syncthreads();
  // Eviction order (its reverse is the ranking order: decreasing density,
  // earlier first); padding sorts last.
  for (int sz = 2; sz <= width; sz <<= 1) {
    for (int stride = sz >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < width; t += blockDim.x) {
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
  if (threadIdx.x == 0) {
    int room = P;
    for (int i = 0; i < n; ++i) {
      if (!(state[i] & 2) || (state[i] & 1)) {
        state[i] |= 4;
        room -= size[i];
      }
    }
    // Evictable spans (chosen and closed) in eviction order, from vict[vh].
    int nv = 0;
    for (int q = 0; q < n; ++q) {
      const int i = idx[q];
      if ((state[i] & 4) && (state[i] & 2)) vict[nv++] = i;
    }
    int vh = 0;
    while (room < 0 && vh < nv) {
      const int i = vict[vh++];
      state[i] &= ~4;
      room += size[i];
    }
    int n_rank = 0;
    for (int q = n - 1; q >= 0; --q)
      if (!(state[idx[q]] & 4)) rank[n_rank++] = idx[q];
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
    int kept = 0, arch = 0, spans = 0;
    for (int i = 0; i < n; ++i) {
      if (state[i] & 4) {
        koff[i] = kept;
        kept += size[i];
        ++spans;
      } else {
        koff[i] = arch;
        arch += size[i];
      }
    }
    kept_s = kept;
    arch_s = arch;
    a.new_span_count[b] = spans;
    a.archive_count[b] = arch;
    atomicMax(a.alpha_count, kept);
  }
  __syncthreads();
  const int A = P + T;
  const int kept = kept_s, arch = arch_s;
  LOGKV_G int32_t* keep = gp(a.keep + static_cast<int64_t>(b) * P);
  LOGKV_G int32_t* archive = gp(a.archive + static_cast<int64_t>(b) * A);
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int o = w.offsets[c0 + i];
    const bool kept_i = (state[i] & 4) != 0;
    LOGKV_G int32_t* dst = kept_i ? keep + koff[i] : archive + koff[i];
    const int cap = kept_i ? P - koff[i] : A - koff[i];   // the greedy keeps at most P rows
    for (int t = 0; t < size[i] && t < cap; ++t) dst[t] = w.tokens[o + t];
  }
  // The new selection's spans, in candidate order.
  if (threadIdx.x == 0) {
    int sp = 0;
    for (int i = 0; i < n; ++i) {
      if (state[i] & 4) {
        a.new_span_len[static_cast<int64_t>(b) * P + sp] = size[i];
        a.new_span_closed[static_cast<int64_t>(b) * P + sp] = (state[i] & 2) ? 1 : 0;
        ++sp;
      }
    }
  }
  for (int i = kept + threadIdx.x; i < P; i += blockDim.x) keep[i] = -1;
  for (int i = arch + threadIdx.x; i < A; i += blockDim.x) archive[i] = -1;
  if (a.scores) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) a.scores[c0 + i] = w.scores[c0 + i];
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

int64_t select_workspace_bytes(const logkv_alpha_select_args& a) {
  const int64_t C = select_candidates(a.n_batch, a.budget, a.tokens);
  auto al = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  return al(C * 4) + al(C) + al((a.n_batch + 1) * 4) + al((C + 1) * 4) +
         al(static_cast<int64_t>(a.n_batch) * (a.budget + a.tokens) * 4) + al(4) + al(C * 4);
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
  w.row_cand = reinterpret_cast<int32_t*>(p);
  p += al((a.n_batch + 1) * 4);
  w.offsets = reinterpret_cast<int32_t*>(p);
  p += al((C + 1) * 4);
  w.tokens = reinterpret_cast<int32_t*>(p);
  p += al(static_cast<int64_t>(a.n_batch) * (a.budget + a.tokens) * 4);
  w.n_spans = reinterpret_cast<int32_t*>(p);
  p += al(4);
  w.scores = reinterpret_cast<float*>(p);
  const size_t cut_c = static_cast<size_t>(a.budget) + a.tokens + 1;
  const size_t cut_shmem = 4 * (static_cast<size_t>(a.tokens) + 1) + 5 * static_cast<size_t>(a.budget) +
                           17 * cut_c + static_cast<size_t>(a.tokens) + 16;
  if (cut_shmem > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&cut_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(cut_shmem)) != hipSuccess)
    return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(cut_kernel, dim3(1), dim3(kSelectThreads), cut_shmem, stream, a, w);
  logkv_span_args sa = a.rows;
  sa.old_width = a.budget;
  sa.tokens = w.tokens;
  sa.span_offsets = w.offsets;
  sa.span_rows = w.cand_row;
  sa.n_spans = static_cast<int32_t>(C);
  sa.n_spans_dev = w.n_spans;
  int rc = launch_score(sa, w.scores, stream);
  if (rc) return rc;
  const int maxc = a.budget + a.tokens + 1;
  int width = 1;
  while (width < maxc) width <<= 1;
  const size_t choose_shmem = static_cast<size_t>(width) * (8 + 4) + static_cast<size_t>(maxc) * (8 + 4 * 4 + 1) + 16;
  if (choose_shmem > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&choose_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(choose_shmem)) != hipSuccess)
    return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(choose_kernel, dim3(a.n_batch), dim3(kSelectThreads), choose_shmem, stream, a, w);
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
