// Standalone Beta 4->2 compaction of a block of entries (the reference's
// beta_log_kv.select_cuts / apply_cuts / merge_blocks, litgpt/beta_log_kv.py:29-105).
//
// One wave per layout row (start, width, out_start): width 4 groups choose the
// cut of (2, 1, 3) with the smallest normalised distortion (or apply a recorded
// one) and emit two weighted means at out_start, out_start + 1; width 2 groups
// (a lane's two-row tail) merge into one row at out_start and record the
// sentinel cut 1. Means are float32 (the reference returns float32 K / V); the
// metadata follows the pair-merge rules. The arithmetic is beta.hpp's, shared
// with the ladder's carries.
#include "beta.hpp"
#include "route.hpp"

namespace logkv {

namespace {

constexpr int kBetaThreads = 256;   // four groups per block

template <bool F32>
__device__ __forceinline__ float feat(const void* base, int64_t row, int64_t st, int d, int D) {
  if (F32) return feat_or_zero(gp(static_cast<const float*>(base)) + row * st, d, D);
  return feat_or_zero(gp(static_cast<const uint16_t*>(base)) + row * st, d, D);
}

template <int NJ, bool KF32, bool VF32>
__global__ __launch_bounds__(kBetaThreads) void beta_merge_kernel(logkv_beta_args a, int32_t* status) {
  const int64_t gi = static_cast<int64_t>(blockIdx.x) * (kBetaThreads / kWave) + wave_id();
  if (gi >= a.n_groups) return;   // whole waves exit together
  const int l = lane_id();
  const int64_t start = a.layout[3 * gi], out0 = a.layout[3 * gi + 2];
  const int64_t width = a.layout[3 * gi + 1];
  const int64_t n_out = a.n_rows / 2;
  int cut = 2;
  bool ok = (width == 4 || width == 2) && start >= 0 && start + width <= a.n_rows && out0 >= 0 &&
            out0 + (width == 4 ? 2 : 1) <= n_out;
  if (ok && a.apply && width == 4) {
    cut = a.cuts[gi];
    ok = cut >= 1 && cut <= 3;
  }
  if (!ok) {
    if (l == 0 && status) atomicOr(status, 1);
    return;
  }
  float xk[4][NJ], xv[4][NJ], wr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool valid = i < width;
    const int64_t row = start + (valid ? i : 0);
    wr[i] = valid ? a.w[row] : 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = l + j * kWave;
      const float x = feat<KF32>(a.k, row, a.k_st, d, a.dk), y = feat<VF32>(a.v, row, a.v_st, d, a.dv);
      xk[i][j] = valid ? x : 0.f;
      xv[i][j] = valid ? y : 0.f;
    }
  }
  Meta mine{};
  if (l < width) {
    const int64_t row = start + l;
    mine.w = a.w[row];
    mine.lo = a.p_lo ? a.p_lo[row] : 0;
    mine.hi = a.p_hi ? a.p_hi[row] : 0;
    mine.swp = a.sum_wp ? a.sum_wp[row] : 0;
    mine.ord = a.order ? a.order[row] : 0;
    mine.pad = a.pad ? a.pad[row] : 0;
  }
  double rcp[6];
  side_rcps(wr, rcp);
  if (width == 4 && !a.apply) cut = beta_cut<NJ>(xk, xv, wr, rcp);
  if (!a.apply && l == 0) a.cuts[gi] = static_cast<uint8_t>(width == 4 ? cut : 1);
  if (!a.out_k) return;   // cuts only (select_cuts)
  const int c = width == 4 ? cut : 2;   // a two-row tail is the left side of cut 2
  const int opt = c == 2 ? 0 : (c == 1 ? 1 : 2);
  for (int side = 0; side < (width == 4 ? 2 : 1); ++side) {
    const unsigned member = side == 0 ? ((1u << c) - 1u) : (0xfu & ~((1u << c) - 1u));
    float wt[4], mk[NJ], mv[NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i) wt[i] = ((member >> i) & 1u) ? wr[i] : 0.f;
    const float mass = side_mass(wt);
    const RowProducts<NJ> pk(xk, wr), pv(xv, wr);
    const double left = opt == 0 ? rcp[0] : (opt == 1 ? rcp[2] : rcp[4]);
    const double right = opt == 0 ? rcp[1] : (opt == 1 ? rcp[3] : rcp[5]);
    side_mean<NJ>(pk, member, side == 0 ? left : right, mk);
    side_mean<NJ>(pv, member, side == 0 ? left : right, mv);
    const int64_t o = out0 + side;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = l + j * kWave;
      if (d < a.dk) gp(a.out_k)[o * a.dk + d] = mk[j];
      if (d < a.dv) gp(a.out_v)[o * a.dv + d] = mv[j];
    }
    const bool in_side = l < width && ((member >> (l & 3)) & 1u);
    const Meta r = side_meta(mine, in_side, mass);
    if (l == 0) {
      a.out_w[o] = r.w;
      if (a.out_p_lo) a.out_p_lo[o] = r.lo;
      if (a.out_p_hi) a.out_p_hi[o] = r.hi;
      if (a.out_sum_wp) a.out_sum_wp[o] = r.swp;
      if (a.out_order) a.out_order[o] = r.ord;
      if (a.out_pad) a.out_pad[o] = r.pad;
    }
  }
}

template <int NJ>
int launch_nj(const logkv_beta_args& a, int32_t* status, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.n_groups + kBetaThreads / kWave - 1) / (kBetaThreads / kWave)));
  if (a.k_f32 && a.v_f32) hipLaunchKernelGGL((beta_merge_kernel<NJ, true, true>), grid, dim3(kBetaThreads), 0, stream, a, status);
  else if (a.k_f32) hipLaunchKernelGGL((beta_merge_kernel<NJ, true, false>), grid, dim3(kBetaThreads), 0, stream, a, status);
  else if (a.v_f32) hipLaunchKernelGGL((beta_merge_kernel<NJ, false, true>), grid, dim3(kBetaThreads), 0, stream, a, status);
  else hipLaunchKernelGGL((beta_merge_kernel<NJ, false, false>), grid, dim3(kBetaThreads), 0, stream, a, status);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace

int launch_beta_merge(const logkv_beta_args& a, int32_t* status, hipStream_t stream) {
  if (a.n_groups == 0) return LOGKV_OK;
  const int nj = (std::max(a.dk, a.dv) + kWave - 1) / kWave;
  if (nj == 1) return launch_nj<1>(a, status, stream);
  if (nj == 2) return launch_nj<2>(a, status, stream);
  if (nj == 3) return launch_nj<3>(a, status, stream);
  return launch_nj<4>(a, status, stream);
}

}  // namespace logkv
