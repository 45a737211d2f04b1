// Beta 4->2 compaction of a group of four ordered entries (litgpt/beta_log_kv.py:29-105):
// the cut of minimum normalised distortion and the two weighted-mean outputs with their
// anchor metadata. Shared by the ladder's carries and the standalone merge kernel, so
// both evaluate the same float operations in the same order. One wave per group:
// features l + 64 j (j < NJ) of every row live in lane l, lane i < 4 holds row i's
// metadata; every lane of the wave must be active.
#pragma once

#include "common.hpp"

namespace logkv {

// One ladder entry's scalar fields: mass, position range, sum of w * position,
// arrival order and the padding flag.
struct Meta {
  float w;
  int64_t lo, hi, swp, ord;
  uint8_t pad;
};

// Sum over j (in order) of the squares of row i's features l + 64 j held in lane l.
template <int NJ>
__device__ __forceinline__ float lane_sq(const float (&x)[NJ]) {
  float s = x[0] * x[0];
#pragma unroll
  for (int j = 1; j < NJ; ++j) s = s + x[j] * x[j];
  return s;
}

// Side mass ((w0 + w1) + w2) + w3 (zero weights outside the side).
__device__ __forceinline__ float side_mass(const float* wt) { return ((wt[0] + wt[1]) + wt[2]) + wt[3]; }

// Products of one component's rows with their weights (p = x w) and with a
// zero weight (z = x * 0, which carries x's sign and turns inf / NaN into NaN).
template <int NJ>
struct RowProducts {
  float p[4][NJ], z[4][NJ];
  __device__ __forceinline__ RowProducts(const float (&x)[4][NJ], const float* w) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        p[i][j] = x[i][j] * w[i];
        z[i][j] = x[i][j] * 0.f;
      }
  }
};

// Weighted mean of a side: sum_i x_i w_i (row order, rows outside the side
// with weight 0) / max(mass, 1e-12), the division through the side's double
// reciprocal `rcp` (div_by_rcp).
template <int NJ>
__device__ __forceinline__ void side_mean(const RowProducts<NJ>& pr, unsigned member, double rcp, float* mean) {
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    float acc = (member & 1u) ? pr.p[0][j] : pr.z[0][j];
    acc = acc + ((member & 2u) ? pr.p[1][j] : pr.z[1][j]);
    acc = acc + ((member & 4u) ? pr.p[2][j] : pr.z[2][j]);
    acc = acc + ((member & 8u) ? pr.p[3][j] : pr.z[3][j]);
    mean[j] = div_by_rcp(acc, rcp);
  }
}

// Split weights of cut c: left rows i < c, right rows i >= c.
__device__ __forceinline__ void cut_weights(const float* wr, int c, float* wl, float* wrt) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wl[i] = i < c ? wr[i] : 0.f;
    wrt[i] = i < c ? 0.f : wr[i];
  }
}

// Double reciprocals of max(mass, 1e-12) of the six sides of the cuts
// (2, 1, 3), left then right, from one lane-parallel division.
__device__ __forceinline__ void side_rcps(const float* wr, double* rcp) {
  const int l = lane_id();
  float mine = 1.f;
#pragma unroll
  for (int opt = 0; opt < 3; ++opt) {
    const int c = opt == 0 ? 2 : (opt == 1 ? 1 : 3);
    float wl[4], wrt[4];
    cut_weights(wr, c, wl, wrt);
    mine = l == 2 * opt ? side_mass(wl) : mine;
    mine = l == 2 * opt + 1 ? side_mass(wrt) : mine;
  }
  const double r = 1.0 / static_cast<double>(fmaxf(mine, 1e-12f));
#pragma unroll
  for (int k = 0; k < 6; ++k) rcp[k] = readlane_f64(r, k);
}

// One component's row energies sum_d x_id^2 -> e = sum_i sq_i w_i (row order),
// and for the cuts (2, 1, 3) the losses sum_i w_i |x_i - mean_side|^2 of the
// left and right sides (row order; rows of the other side add w = 0 times
// their distance to the other side's mean). Feature sums are canonical; the
// four rows of a cut are folded together (wave_sum4).
template <int NJ>
__device__ __forceinline__ void beta_component_losses(const float (&x)[4][NJ], const float* wr, const double* rcp,
                                                      float& e, float* loss) {
  const RowProducts<NJ> pr(x, wr);
  float sq[4];
  wave_sum4(lane_sq<NJ>(x[0]), lane_sq<NJ>(x[1]), lane_sq<NJ>(x[2]), lane_sq<NJ>(x[3]), sq[0], sq[1], sq[2], sq[3]);
  e = sq[0] * wr[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) e = e + sq[i] * wr[i];
#pragma unroll
  for (int opt = 0; opt < 3; ++opt) {
    const int c = opt == 0 ? 2 : (opt == 1 ? 1 : 3);
    float wl[4], wrt[4], ml[NJ], mr[NJ];
    cut_weights(wr, c, wl, wrt);
    const unsigned left_rows = (1u << c) - 1u;
    side_mean<NJ>(pr, left_rows, rcp[2 * opt], ml);
    side_mean<NJ>(pr, 0xfu & ~left_rows, rcp[2 * opt + 1], mr);
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float d[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) d[j] = x[i][j] - (i < c ? ml[j] : mr[j]);
      t[i] = lane_sq<NJ>(d);
    }
    float per[4];
    wave_sum4(t[0], t[1], t[2], t[3], per[0], per[1], per[2], per[3]);
    float left = per[0] * wl[0], right = per[0] * wrt[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      left = left + per[i] * wl[i];
      right = right + per[i] * wrt[i];
    }
    loss[2 * opt] = left;
    loss[2 * opt + 1] = right;
  }
}

// Cut of a full group (litgpt/beta_log_kv.py:29-85): costs of (2, 1, 3) summed
// over K then V, left side then right, of loss / energy with energy =
// max(e / total, 1e-12); the smallest cost wins (first on ties). The 2 + 12
// uniform divisions run as two lane-parallel divisions.
template <int NJ>
__device__ __forceinline__ int beta_cut(const float (&xk)[4][NJ], const float (&xv)[4][NJ], const float* wr,
                                        const double* rcp) {
  const int l = lane_id();
  const float total = fmaxf(((wr[0] + wr[1]) + wr[2]) + wr[3], 1e-12f);
  float ek, ev, lk[6], lv[6];
  beta_component_losses<NJ>(xk, wr, rcp, ek, lk);
  beta_component_losses<NJ>(xv, wr, rcp, ev, lv);
  const float en = (l == 0 ? ek : ev) / total;
  const float energy_k = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(en), 0)), 1e-12f);
  const float energy_v = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(en), 1)), 1e-12f);
  float num = 0.f;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    num = l == k ? lk[k] : num;
    num = l == 6 + k ? lv[k] : num;
  }
  const float q = num / (l < 6 ? energy_k : energy_v);
  float costs[3] = {0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 12; ++k)
    costs[(k % 6) / 2] = costs[(k % 6) / 2] + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q), k));
  int best = 0;
  if (costs[1] < costs[best]) best = 1;
  if (costs[2] < costs[best]) best = 2;
  return best == 0 ? 2 : (best == 1 ? 1 : 3);
}

// Quad (4-lane) butterfly exchanges: lane i reads lane i ^ 1 / i ^ 2 of its quad.
constexpr int kQuadXor1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4E;   // quad_perm [2, 3, 0, 1]

template <int CTRL>
__device__ __forceinline__ int64_t quad_xor64(int64_t x) {
  const int lo = __builtin_amdgcn_mov_dpp(static_cast<int>(x & 0xffffffff), CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_mov_dpp(static_cast<int>(x >> 32), CTRL, 0xf, 0xf, false);
  return (static_cast<int64_t>(hi) << 32) | static_cast<int64_t>(static_cast<uint32_t>(lo));
}

template <int CTRL>
__device__ __forceinline__ int quad_xor32(int x) {
  return __builtin_amdgcn_mov_dpp(x, CTRL, 0xf, 0xf, false);
}

// Metadata of a merged side from lanes 0..3 of the wave, lane i holding row i
// of the group (litgpt/beta_log_kv.py:86-105, litgpt/log_kv_position.py:13-30):
// p_lo / p_hi over rows with w > 0, sums of w*p, smallest order, all-padding.
// Integer reductions, so the lane order does not matter. Valid in lane 0.
__device__ __forceinline__ Meta side_meta(const Meta& mine, bool member, float mass) {
  const bool live = member && mine.w > 0.f;
  int64_t lo = live ? mine.lo : INT64_MAX;
  int64_t hi = live ? mine.hi : INT64_MIN;
  int64_t swp = member ? mine.swp : 0;
  int64_t ord = member ? mine.ord : INT64_MAX;
  int pad = member ? mine.pad : 1;
  lo = imin64(lo, quad_xor64<kQuadXor1>(lo));
  hi = imax64(hi, quad_xor64<kQuadXor1>(hi));
  swp = swp + quad_xor64<kQuadXor1>(swp);
  ord = imin64(ord, quad_xor64<kQuadXor1>(ord));
  pad = pad & quad_xor32<kQuadXor1>(pad);
  lo = imin64(lo, quad_xor64<kQuadXor2>(lo));
  hi = imax64(hi, quad_xor64<kQuadXor2>(hi));
  swp = swp + quad_xor64<kQuadXor2>(swp);
  ord = imin64(ord, quad_xor64<kQuadXor2>(ord));
  pad = pad & quad_xor32<kQuadXor2>(pad);
  Meta r;
  r.w = mass;
  r.lo = mass > 0.f ? lo : 0;
  r.hi = mass > 0.f ? hi : 0;
  r.swp = swp;
  r.ord = ord;
  r.pad = static_cast<uint8_t>(pad);
  return r;
}

}  // namespace logkv
