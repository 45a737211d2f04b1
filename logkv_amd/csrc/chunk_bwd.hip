// Backward of the packed chunk attention on the matrix cores (training: the
// gradient of one streaming block, litgpt/log_kv_cache.py:6867-7098, whose
// per-block autograd.grad this replaces; slot attention's gradient,
// litgpt/log_kv_cache.py:6501-6630).
//
// Forward: o_i = sum_j p_ij v_j, p_ij = softmax_j(scale * [q_i, 1/scale] . [k_j, bias_j])
// over the packed rows, the last causal_tail rows causal. With D_i = dO_i . o_i
// (= sum_j p_ij dO_i . v_j, formed in float32 here) and dS_ij = p_ij (dO_i . v_j - D_i):
//   dq_i = scale * sum_j dS_ij k_j      (key features only; the bias coordinate has no gradient)
//   dk_j = scale * sum_i dS_ij q_i,  dv_j = sum_i p_ij dO_i
// for the last `grad_rows` packed rows (the in-flight chunk; every row for slot attention).
//
// Two launches, both v_mfma_f32_32x32x16_bf16 with the forward's fragment layout:
//  * dq_kernel: a block owns 128 query rows of one KV group (4 waves x 32, a query per
//    lane column) and walks the key tiles twice: first the row maximum and sum (the
//    log-sum-exp) and D, then S^T = K Q^T, dP^T = V dO^T, dS^T and dQ^T += K^T dS^T. It
//    writes each query's log-sum-exp and D for the second launch.
//  * dkv_kernel: a block owns 128 gradient rows (a key per lane column) and walks the
//    query tiles: S = Q K^T, dP = dO V^T, P and dS from the stored statistics, then
//    dV^T += dO^T P and dK^T += Q^T dS.
// The P / dS operands are the lanes' own accumulator registers (the k-index permutation of
// the forward's P^T operand), each as a high and a low bf16 part; accumulation is float32.
#include <algorithm>

#include "route.hpp"

namespace logkv {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kRows = 128;       // query rows (dq) / gradient rows (dkv) per block
constexpr int kTile = 64;        // key rows (dq) / query rows (dkv) per staged tile
constexpr int kMaxSteps = 9;     // 16-wide steps of the packed width (<= 144)
constexpr int kLdK = 152;        // row stride of row-major Q / K tiles (bf16)
constexpr int kLdD = 136;        // row stride of row-major dO / V tiles (dv <= 128)
constexpr int kLdT = kTile + 8;  // row stride of transposed tiles
constexpr int kMaxBlk = 4;       // 32-row blocks of dk / dv (<= 128)
constexpr float kLog2e = 1.44269504088896341f;

__device__ __forceinline__ bf16x8 load8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }

// A operand of a transposed tile (rows x tile columns), columns in the
// permuted order 16 st + 8 (j / 4) + 4 h + j % 4 of step st.
__device__ __forceinline__ bf16x8 load_t(const uint16_t* base, int row, int st, int h) {
  const uint16_t* r = base + row * kLdT + 16 * st + 4 * h;
  const uint2 x0 = *reinterpret_cast<const uint2*>(r);
  const uint2 x1 = *reinterpret_cast<const uint2*>(r + 8);
  return __builtin_bit_cast(bf16x8, make_uint4(x0.x, x0.y, x1.x, x1.y));
}

// B operand of step st from accumulator blocks acc[2] (elements 8 (st % 2) .. + 8 of block
// st / 2) as two bf16 parts: the truncated high half and the rounded remainder, so the two
// products keep about 16 significant bits (the softmax backward sums dS terms that cancel).
__device__ __forceinline__ void regs_b(const f32x16 (&acc)[2], int st, bf16x8& hi, bf16x8& lo) {
  uint32_t hw[4], lw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x0 = acc[st / 2][8 * (st % 2) + 2 * j], x1 = acc[st / 2][8 * (st % 2) + 2 * j + 1];
    const uint32_t u0 = __float_as_uint(x0), u1 = __float_as_uint(x1);
    hw[j] = __builtin_amdgcn_perm(u1, u0, 0x07060302u);
    const float r0 = x0 - __uint_as_float(u0 & 0xffff0000u), r1 = x1 - __uint_as_float(u1 & 0xffff0000u);
    lw[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{r0, r1}, bf16x2));
  }
  hi = __builtin_bit_cast(bf16x8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
  lo = __builtin_bit_cast(bf16x8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
}

__device__ __forceinline__ int packed_total(const logkv_attention_args& a, const int32_t* width_ptr) {
  return min(*width_ptr + a.tail + (a.alpha_count_dev ? *a.alpha_count_dev : 0), a.cap);
}

}  // namespace

__global__ __launch_bounds__(256, 1) void dq_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr,
                                                    logkv_attention_grad_args gr, float* __restrict__ stats) {
  __shared__ __align__(16) uint16_t q_s[kRows * kLdK];
  __shared__ __align__(16) uint16_t do_s[kRows * kLdD];
  __shared__ __align__(16) uint16_t k_s[kTile * kLdK];
  __shared__ __align__(16) uint16_t kt_s[kMaxBlk * 32 * kLdT];
  __shared__ __align__(16) uint16_t v_s[kTile * kLdD];
  const int lane_ix = blockIdx.y, G = a.n_groups;
  const int b = lane_ix / G, g = lane_ix % G;
  const int rep = a.n_heads / G, nq = rep * a.tq;
  const int w = wave_id(), l = lane_id(), h = l >> 5, col = l & 31;
  const int dim = a.dim, nks = (dim + 15) / 16, nvs = a.dv / 16, ndk = (a.dk + 31) / 32;
  const int qi = blockIdx.x * kRows + w * 32 + col;
  const bool q_ok = qi < nq;
  const int qc = q_ok ? qi : nq - 1;
  const int head = g * rep + qc / a.tq, t = qc % a.tq;
  const int total = packed_total(a, width_ptr);
  const int tail0 = total - a.causal_tail;
  const int q_first = blockIdx.x * kRows, q_last = min(q_first + kRows, nq) - 1;
  const int t_max = q_first / a.tq == q_last / a.tq ? q_last % a.tq : a.tq - 1;
  const int key_end = a.causal_tail ? min(total, tail0 + t_max + 1) : total;
  const float c2 = a.scale * kLog2e;

  for (int i = threadIdx.x; i < kRows * kLdK; i += blockDim.x) {
    const int r = i / kLdK, d = i - r * kLdK;
    const int qr = min(q_first + r, nq - 1);
    const int hr = g * rep + qr / a.tq, tr = qr % a.tq;
    const float x = d < a.dk ? bf16_to_f32(gp(a.q)[b * a.q_sb + hr * a.q_sh + tr * a.q_st + (d < a.dk ? d : 0)])
                             : (d == a.dk ? a.inv_scale_bf16 : 0.f);
    q_s[i] = f32_to_bf16(x);
  }
  for (int i = threadIdx.x; i < kRows * kLdD; i += blockDim.x) {
    const int r = i / kLdD, d = i - r * kLdD;
    const int qr = min(q_first + r, nq - 1);
    const int hr = g * rep + qr / a.tq, tr = qr % a.tq;
    do_s[i] = d < a.dv ? gp(gr.dout)[b * gr.do_sb + hr * gr.do_sh + tr * gr.do_st + (d < a.dv ? d : 0)] : 0;
  }
  for (int i = threadIdx.x; i < kTile * (kLdK - dim); i += blockDim.x) {
    const int r = i / (kLdK - dim), c = dim + i % (kLdK - dim);
    k_s[r * kLdK + c] = 0;
  }
  const LOGKV_G uint16_t* kbase = gp(a.k) + static_cast<int64_t>(lane_ix) * a.cap * dim;
  const LOGKV_G uint16_t* vbase = gp(a.v) + static_cast<int64_t>(lane_ix) * a.cap * dim;
  const int units = dim / 8, vunits = a.dv / 8;

  auto scores = [&](f32x16 (&s)[2]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb][i] = 0.f;
#pragma unroll
      for (int ks = 0; ks < kMaxSteps; ++ks)
        if (ks < nks)
          s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(load8(k_s + (32 * kb + col) * kLdK + 16 * ks + 8 * h),
                                                          load8(q_s + (32 * w + col) * kLdK + 16 * ks + 8 * h),
                                                          s[kb], 0, 0, 0);
    }
  };
  auto mask = [&](f32x16 (&s)[2], int t0, int rows) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = t0 + 32 * kb + 8 * (i / 4) + 4 * h + (i % 4);
        const bool masked = key >= t0 + rows || (a.causal_tail && key >= tail0 && key - tail0 > t);
        s[kb][i] = masked ? -__builtin_inff() : s[kb][i];
      }
  };
  auto stage_k = [&](int t0, int rows) {
    for (int i = threadIdx.x; i < kTile * units; i += blockDim.x) {
      const int r = i / units, u = i - r * units;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (r < rows) x = *(const LOGKV_G uint4*)(kbase + static_cast<int64_t>(t0 + r) * dim + 8 * u);
      *reinterpret_cast<uint4*>(k_s + r * kLdK + 8 * u) = x;
    }
  };
  auto stage_v = [&](int t0, int rows) {
    for (int i = threadIdx.x; i < kTile * vunits; i += blockDim.x) {
      const int r = i / vunits, u = i - r * vunits;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (r < rows) x = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(t0 + r) * dim + 8 * u);
      *reinterpret_cast<uint4*>(v_s + r * kLdD + 8 * u) = x;
    }
  };
  // dP^T = V dO^T for the staged tile (keys x this lane's query).
  auto dscores = [&](f32x16 (&dp)[2]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) dp[kb][i] = 0.f;
      for (int st = 0; st < nvs; ++st)
        dp[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(load8(v_s + (32 * kb + col) * kLdD + 16 * st + 8 * h),
                                                         load8(do_s + (32 * w + col) * kLdD + 16 * st + 8 * h),
                                                         dp[kb], 0, 0, 0);
    }
  };

  // Pass 1: the log-sum-exp of this lane's query (base 2, scaled by c2) and
  // D = dO . o = sum_j p_j dP_j, accumulated with the same online rescaling in
  // float32 (the rounded forward output would lose the bits that cancel in dS).
  float m = -__builtin_inff(), lsum = 0.f, dacc = 0.f;
  for (int t0 = 0; t0 < key_end; t0 += kTile) {
    const int rows = min(kTile, key_end - t0);
    __syncthreads();
    stage_k(t0, rows);
    stage_v(t0, rows);
    __syncthreads();
    f32x16 s[2], dp[2];
    scores(s);
    dscores(dp);
    mask(s, t0, rows);
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m, mx * c2);
    const float mb = m_new == -__builtin_inff() ? 0.f : m_new;
    float sum = 0.f, dsum_t = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], c2, -mb));
        sum += p;
        dsum_t += p * dp[kb][i];
      }
    sum += __shfl_xor(sum, 32, kWave);
    dsum_t += __shfl_xor(dsum_t, 32, kWave);
    const float corr = __builtin_amdgcn_exp2f(m - mb);
    lsum = lsum * corr + sum;
    dacc = dacc * corr + dsum_t;
    m = m_new;
  }
  const float lse = lsum > 0.f ? m + __log2f(lsum) : 0.f;
  const float dsum = lsum > 0.f ? dacc / lsum : 0.f;
  if (q_ok && h == 0) {
    stats[(static_cast<int64_t>(lane_ix) * nq + qi) * 2] = lse;
    stats[(static_cast<int64_t>(lane_ix) * nq + qi) * 2 + 1] = dsum;
  }

  // Pass 2: dQ^T += K^T dS^T.
  f32x16 dq[kMaxBlk];
#pragma unroll
  for (int blk = 0; blk < kMaxBlk; ++blk)
#pragma unroll
    for (int i = 0; i < 16; ++i) dq[blk][i] = 0.f;
  for (int t0 = 0; t0 < key_end; t0 += kTile) {
    const int rows = min(kTile, key_end - t0);
    __syncthreads();
    stage_k(t0, rows);
    // K^T (key features only) and V, row-major.
    for (int i = threadIdx.x; i < kTile * (a.dk / 2); i += blockDim.x) {
      const int r = i % kTile, d2 = i / kTile;
      uint32_t x = 0;
      if (r < rows) x = *(const LOGKV_G uint32_t*)(kbase + static_cast<int64_t>(t0 + r) * dim + 2 * d2);
      kt_s[(2 * d2) * kLdT + r] = static_cast<uint16_t>(x);
      kt_s[(2 * d2 + 1) * kLdT + r] = static_cast<uint16_t>(x >> 16);
    }
    stage_v(t0, rows);
    __syncthreads();
    f32x16 s[2], dp[2];
    scores(s);
    mask(s, t0, rows);
    dscores(dp);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], c2, -lse));
        dp[kb][i] = p * (dp[kb][i] - dsum);
      }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      bf16x8 dh, dl;
      regs_b(dp, st, dh, dl);
#pragma unroll
      for (int blk = 0; blk < kMaxBlk; ++blk)
        if (blk < ndk) {
          const bf16x8 kf = load_t(kt_s, 32 * blk + col, st, h);
          dq[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, dh, dq[blk], 0, 0, 0);
          dq[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, dl, dq[blk], 0, 0, 0);
        }
    }
  }
  if (!q_ok) return;
  LOGKV_G uint16_t* drow = gp(gr.dq) + b * gr.dq_sb + head * gr.dq_sh + t * gr.dq_st;
#pragma unroll
  for (int blk = 0; blk < kMaxBlk; ++blk)
    if (blk < ndk)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = 32 * blk + 8 * (i / 4) + 4 * h + (i % 4);
        if (d < a.dk) drow[d] = f32_to_bf16(dq[blk][i] * a.scale);
      }
}

__global__ __launch_bounds__(256, 1) void dkv_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr,
                                                     logkv_attention_grad_args gr, const float* __restrict__ stats) {
  __shared__ __align__(16) uint16_t ks_s[kRows * kLdK];
  __shared__ __align__(16) uint16_t vs_s[kRows * kLdD];
  __shared__ __align__(16) uint16_t q_t[kTile * kLdK];
  __shared__ __align__(16) uint16_t qt_t[kMaxBlk * 32 * kLdT];
  __shared__ __align__(16) uint16_t do_t[kTile * kLdD];
  __shared__ __align__(16) uint16_t dot_t[kMaxBlk * 32 * kLdT];
  __shared__ float st_s[kTile][2];
  const int lane_ix = blockIdx.y, G = a.n_groups;
  const int b = lane_ix / G, g = lane_ix % G;
  const int rep = a.n_heads / G, nq = rep * a.tq;
  const int w = wave_id(), l = lane_id(), h = l >> 5, col = l & 31;
  const int dim = a.dim, nks = (dim + 15) / 16, ndv = a.dv / 32, nvs = a.dv / 16, ndk = (a.dk + 31) / 32;
  const int total = packed_total(a, width_ptr);
  const int tail0 = total - a.causal_tail;
  const int first = total - gr.grad_rows;                // first gradient row
  const int r_first = first + blockIdx.x * kRows;
  const int key = r_first + w * 32 + col;                  // this lane's key row
  const bool key_ok = key < total && key >= 0;
  const float c2 = a.scale * kLog2e;
  const LOGKV_G uint16_t* kbase = gp(a.k) + static_cast<int64_t>(lane_ix) * a.cap * dim;
  const LOGKV_G uint16_t* vbase = gp(a.v) + static_cast<int64_t>(lane_ix) * a.cap * dim;
  const int units = dim / 8, vunits = a.dv / 8;
  for (int i = threadIdx.x; i < kRows * units; i += blockDim.x) {
    const int r = i / units, u = i - r * units;
    const int kr = r_first + r;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (kr < total && kr >= 0) x = *(const LOGKV_G uint4*)(kbase + static_cast<int64_t>(kr) * dim + 8 * u);
    *reinterpret_cast<uint4*>(ks_s + r * kLdK + 8 * u) = x;
  }
  for (int i = threadIdx.x; i < kRows * (kLdK - dim); i += blockDim.x) {
    const int r = i / (kLdK - dim), c = dim + i % (kLdK - dim);
    ks_s[r * kLdK + c] = 0;
  }
  for (int i = threadIdx.x; i < kRows * vunits; i += blockDim.x) {
    const int r = i / vunits, u = i - r * vunits;
    const int kr = r_first + r;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (kr < total && kr >= 0) x = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(kr) * dim + 8 * u);
    *reinterpret_cast<uint4*>(vs_s + r * kLdD + 8 * u) = x;
  }
  for (int i = threadIdx.x; i < kTile * (kLdK - dim); i += blockDim.x) {
    const int r = i / (kLdK - dim), c = dim + i % (kLdK - dim);
    q_t[r * kLdK + c] = 0;
  }
  // The smallest causal index of this block's rows: query tiles whose every t is
  // below it see none of them.
  const int block_min_t = a.causal_tail ? max(0, r_first - tail0) : 0;
  f32x16 dk[kMaxBlk], dv[kMaxBlk];
#pragma unroll
  for (int blk = 0; blk < kMaxBlk; ++blk)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      dk[blk][i] = 0.f;
      dv[blk][i] = 0.f;
    }
  for (int q0 = 0; q0 < nq; q0 += kTile) {
    const int qn = min(kTile, nq - q0);
    const int t_hi = q0 / a.tq == (q0 + qn - 1) / a.tq ? (q0 + qn - 1) % a.tq : a.tq - 1;
    if (a.causal_tail && r_first >= tail0 && t_hi < block_min_t) continue;   // uniform over the block
    __syncthreads();
    for (int i = threadIdx.x; i < kTile * dim; i += blockDim.x) {
      const int r = i / dim, d = i - r * dim;
      const int qr = min(q0 + r, nq - 1);
      const int hr = g * rep + qr / a.tq, tr = qr % a.tq;
      const float x = r >= qn ? 0.f
                      : (d < a.dk ? bf16_to_f32(gp(a.q)[b * a.q_sb + hr * a.q_sh + tr * a.q_st + (d < a.dk ? d : 0)])
                                  : (d == a.dk ? a.inv_scale_bf16 : 0.f));
      const uint16_t xb = f32_to_bf16(x);
      q_t[r * kLdK + d] = xb;
      if (d < a.dk) qt_t[d * kLdT + r] = xb;
    }
    for (int i = threadIdx.x; i < kTile * a.dv; i += blockDim.x) {
      const int r = i / a.dv, d = i - r * a.dv;
      const int qr = min(q0 + r, nq - 1);
      const int hr = g * rep + qr / a.tq, tr = qr % a.tq;
      const uint16_t x = r >= qn ? 0 : gp(gr.dout)[b * gr.do_sb + hr * gr.do_sh + tr * gr.do_st + d];
      do_t[r * kLdD + d] = x;
      dot_t[d * kLdT + r] = x;
    }
    for (int i = threadIdx.x; i < kTile * 2; i += blockDim.x) {
      const int r = i / 2, c = i % 2;
      st_s[r][c] = r < qn ? stats[(static_cast<int64_t>(lane_ix) * nq + q0 + r) * 2 + c] : 0.f;
    }
    __syncthreads();
    f32x16 s[2], dp[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[qb][i] = 0.f;
        dp[qb][i] = 0.f;
      }
#pragma unroll
      for (int ks = 0; ks < kMaxSteps; ++ks)
        if (ks < nks)
          s[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(load8(q_t + (32 * qb + col) * kLdK + 16 * ks + 8 * h),
                                                          load8(ks_s + (32 * w + col) * kLdK + 16 * ks + 8 * h),
                                                          s[qb], 0, 0, 0);
      for (int st = 0; st < nvs; ++st)
        dp[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(load8(do_t + (32 * qb + col) * kLdD + 16 * st + 8 * h),
                                                         load8(vs_s + (32 * w + col) * kLdD + 16 * st + 8 * h),
                                                         dp[qb], 0, 0, 0);
    }
    // P and dS of this lane's key against the tile's queries (row i of block qb is query
    // q0 + 32 qb + 8 (i / 4) + 4 h + i % 4).
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 32 * qb + 8 * (i / 4) + 4 * h + (i % 4);
        const int qr = q0 + r;
        const int tq_r = qr % a.tq;
        const bool vis = r < qn && key_ok && !(a.causal_tail && key >= tail0 && key - tail0 > tq_r);
        const float p = vis ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][i], c2, -st_s[r][0])) : 0.f;
        s[qb][i] = p;
        dp[qb][i] = p * (dp[qb][i] - st_s[r][1]);
      }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      bf16x8 ph, pl, dh, dl;
      regs_b(s, st, ph, pl);
      regs_b(dp, st, dh, dl);
#pragma unroll
      for (int blk = 0; blk < kMaxBlk; ++blk) {
        if (blk < ndv) {
          const bf16x8 of = load_t(dot_t, 32 * blk + col, st, h);
          dv[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(of, ph, dv[blk], 0, 0, 0);
          dv[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(of, pl, dv[blk], 0, 0, 0);
        }
        if (blk < ndk) {
          const bf16x8 qf = load_t(qt_t, 32 * blk + col, st, h);
          dk[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf, dh, dk[blk], 0, 0, 0);
          dk[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf, dl, dk[blk], 0, 0, 0);
        }
      }
    }
  }
  if (!key_ok || key < first) return;
  const int64_t row = static_cast<int64_t>(lane_ix) * gr.grad_rows + (key - first);
#pragma unroll
  for (int blk = 0; blk < kMaxBlk; ++blk)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 32 * blk + 8 * (i / 4) + 4 * h + (i % 4);
      if (blk < ndk && d < a.dk) gp(gr.dk)[row * a.dk + d] = f32_to_bf16(dk[blk][i] * a.scale);
      if (blk < ndv && d < a.dv) gp(gr.dv)[row * a.dv + d] = f32_to_bf16(dv[blk][i]);
    }
}

int64_t chunk_backward_workspace_floats(const logkv_attention_args& a) {
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  return static_cast<int64_t>(a.n_batch) * a.n_groups * nq * 2;
}

int launch_chunk_backward(const logkv_attention_args& a, const int32_t* width, const logkv_attention_grad_args& g,
                          float* stats, hipStream_t stream) {
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  const int lanes = a.n_batch * a.n_groups;
  hipLaunchKernelGGL(dq_kernel, dim3((nq + kRows - 1) / kRows, lanes), dim3(256), 0, stream, a, width, g, stats);
  if (g.grad_rows > 0)
    hipLaunchKernelGGL(dkv_kernel, dim3((g.grad_rows + kRows - 1) / kRows, lanes), dim3(256), 0, stream, a, width, g,
                       stats);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
