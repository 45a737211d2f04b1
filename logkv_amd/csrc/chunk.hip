// Chunk attention on the matrix cores: many query rows per KV group (a prefill
// or training chunk) over the packed rows [pooled | exact | recent | current].
//
// Same math as the decode kernel (litgpt/log_kv_cache.py:6428-6464, :6751-6758):
// softmax(scale * [q, 1/scale] . [k, bias]) v, the last `causal_tail` rows
// causal against the query rows. Flash attention with gfx950's
// v_mfma_f32_32x32x16_bf16: a block of 4 waves owns 128 query rows of one KV
// group, a wave 32 of them (one per lane column). Per 64-row key tile, staged
// in LDS (K row-major, V transposed):
//   S^T = K Q^T   (keys x queries; each lane holds 16 keys of its own query),
//   online softmax per lane (its query's max and sum, the other 16 keys of the
//   32-key block in lane ^ 32),
//   O^T += V^T P^T (dv x queries), P split into bf16 high and low parts so the
//   product keeps ~16 significant bits of P (two MFMAs per step).
// The P^T operand is the lane's own score registers: MFMA B operand element j
// of a 16-key step s is key 16s + 8(j/4) + 4(lane/32) + j%4, which is exactly
// accumulator element 8(s%2) + j of S^T block s/2, so V^T is read with the same
// key order and no data moves between lanes.
#include "route.hpp"

namespace logkv {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kQRows = 128;      // query rows per block (4 waves x 32)
constexpr int kKeys = 64;        // key rows per staged tile
constexpr int kMaxSteps = 9;     // 16-wide steps of the packed width (<= 144)
constexpr int kLdK = 152;        // K tile row stride in LDS (bf16)
constexpr int kLdV = kKeys + 8;  // V^T row stride in LDS (bf16)
constexpr int kMaxDvBlocks = 4;  // dv <= 128

__device__ __forceinline__ __bf16 to_bf16(float x) { return static_cast<__bf16>(x); }

}  // namespace

__global__ __launch_bounds__(256) void chunk_kernel(logkv_attention_args a, const int32_t* __restrict__ width_ptr) {
  __shared__ __align__(16) uint16_t k_s[kKeys * kLdK];
  __shared__ __align__(16) uint16_t vt_s[kMaxDvBlocks * 32 * kLdV];
  const int lane_ix = blockIdx.y, G = a.n_groups;
  const int b = lane_ix / G, g = lane_ix % G;
  const int rep = a.n_heads / G, nq = rep * a.tq;
  const int w = wave_id(), l = lane_id(), h = l >> 5, col = l & 31;
  const int dim = a.dim, nks = (dim + 15) / 16, ndv = a.dv / 32;
  const int qi = blockIdx.x * kQRows + w * 32 + col;
  const bool q_ok = qi < nq;
  const int qc = q_ok ? qi : nq - 1;
  const int head = g * rep + qc / a.tq, t = qc % a.tq;
  const int total = min(*width_ptr + a.tail + (a.alpha_count_dev ? *a.alpha_count_dev : 0), a.cap);
  const int tail0 = total - a.causal_tail;
  // Last key row any query of the block can see.
  const int q_first = blockIdx.x * kQRows, q_last = min(q_first + kQRows, nq) - 1;
  const int t_max = q_first / a.tq == q_last / a.tq ? q_last % a.tq : a.tq - 1;
  const int key_end = a.causal_tail ? min(total, tail0 + t_max + 1) : total;

  // Query fragments [q, 1/scale, 0...] (B operand: dims 16 ks + 8 h + j of this lane's query).
  bf16x8 qf[kMaxSteps];
  const LOGKV_G uint16_t* qrow = gp(a.q) + b * a.q_sb + head * a.q_sh + t * a.q_st;
#pragma unroll
  for (int ks = 0; ks < kMaxSteps; ++ks) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = 16 * ks + 8 * h + j;
      const float x = d < a.dk ? bf16_to_f32(qrow[d < a.dk ? d : 0]) : (d == a.dk ? a.inv_scale_bf16 : 0.f);
      qf[ks][j] = to_bf16(x);
    }
  }
  // Columns past the packed width stay zero in every tile.
  for (int i = threadIdx.x; i < kKeys * (kLdK - dim); i += blockDim.x) {
    const int r = i / (kLdK - dim), c = dim + i % (kLdK - dim);
    k_s[r * kLdK + c] = 0;
  }
  f32x16 o[kMaxDvBlocks];
#pragma unroll
  for (int blk = 0; blk < kMaxDvBlocks; ++blk)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[blk][i] = 0.f;
  float m = -__builtin_inff(), lsum = 0.f;
  const LOGKV_G uint16_t* kbase = gp(a.k) + static_cast<int64_t>(lane_ix) * a.cap * dim;
  const LOGKV_G uint16_t* vbase = gp(a.v) + static_cast<int64_t>(lane_ix) * a.cap * dim;
  const int units = dim / 8;
  const int vunits = a.dv / 8;

  for (int t0 = 0; t0 < key_end; t0 += kKeys) {
    const int rows = min(kKeys, key_end - t0);
    __syncthreads();
    // K rows (16-byte units), zero rows past the end.
    for (int i = threadIdx.x; i < kKeys * units; i += blockDim.x) {
      const int r = i / units, u = i - r * units;
      const int src = t0 + min(r, rows - 1);
      uint4 x = *(const LOGKV_G uint4*)(kbase + static_cast<int64_t>(src) * dim + 8 * u);
      if (r >= rows) x = make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(k_s + r * kLdK + 8 * u) = x;
    }
    // V^T: each task takes two consecutive key rows of one 8-wide dv unit and
    // writes 8 dwords (key pairs), zero rows past the end.
    for (int i = threadIdx.x; i < (kKeys / 2) * vunits; i += blockDim.x) {
      const int kp = i % (kKeys / 2), u = i / (kKeys / 2);
      const int r0 = 2 * kp, r1 = 2 * kp + 1;
      uint4 x0 = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(t0 + min(r0, rows - 1)) * dim + 8 * u);
      uint4 x1 = *(const LOGKV_G uint4*)(vbase + static_cast<int64_t>(t0 + min(r1, rows - 1)) * dim + 8 * u);
      if (r0 >= rows) x0 = make_uint4(0, 0, 0, 0);
      if (r1 >= rows) x1 = make_uint4(0, 0, 0, 0);
      const uint32_t a0[4] = {x0.x, x0.y, x0.z, x0.w}, a1[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = (a0[j] & 0xffffu) | (a1[j] << 16);
        const uint32_t hi = (a0[j] >> 16) | (a1[j] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(vt_s + (8 * u + 2 * j) * kLdV + r0) = lo;
        *reinterpret_cast<uint32_t*>(vt_s + (8 * u + 2 * j + 1) * kLdV + r0) = hi;
      }
    }
    __syncthreads();
    // S^T = K Q^T over the packed width.
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb][i] = 0.f;
#pragma unroll
      for (int ks = 0; ks < kMaxSteps; ++ks) {
        if (ks < nks) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(k_s + (32 * kb + col) * kLdK + 16 * ks + 8 * h);
          s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb], 0, 0, 0);
        }
      }
    }
    // Scores, masks, online softmax of this lane's query.
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = t0 + 32 * kb + 8 * (i / 4) + 4 * h + (i % 4);
        float sc = a.scale * s[kb][i];
        const bool masked = !q_ok || key >= t0 + rows || (a.causal_tail && key >= tail0 && key - tail0 > t);
        sc = masked ? -__builtin_inff() : sc;
        s[kb][i] = sc;
        mx = fmaxf(mx, sc);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m, mx);
    const float corr = m_new == -__builtin_inff() ? 1.f : __expf(m - m_new);
    float sum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = s[kb][i] == -__builtin_inff() ? 0.f : __expf(s[kb][i] - m_new);
        s[kb][i] = p;
        sum += p;
      }
    }
    sum += __shfl_xor(sum, 32, kWave);
    lsum = lsum * corr + sum;
    m = m_new;
#pragma unroll
    for (int blk = 0; blk < kMaxDvBlocks; ++blk)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[blk][i] *= corr;
    // O^T += V^T P^T, four 16-key steps, P as high + low bf16 parts.
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      bf16x8 ph, pl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = s[st / 2][8 * (st % 2) + j];
        const __bf16 hi = to_bf16(p);
        ph[j] = hi;
        pl[j] = to_bf16(p - static_cast<float>(hi));
      }
#pragma unroll
      for (int blk = 0; blk < kMaxDvBlocks; ++blk) {
        if (blk < ndv) {
          const uint16_t* vr = vt_s + (32 * blk + col) * kLdV + 16 * st + 4 * h;
          const uint2 v0 = *reinterpret_cast<const uint2*>(vr);
          const uint2 v1 = *reinterpret_cast<const uint2*>(vr + 8);
          bf16x8 vf;
          const uint32_t wv[4] = {v0.x, v0.y, v1.x, v1.y};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            vf[2 * j] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(wv[j] & 0xffffu));
            vf[2 * j + 1] = __builtin_bit_cast(__bf16, static_cast<uint16_t>(wv[j] >> 16));
          }
          o[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, ph, o[blk], 0, 0, 0);
          o[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pl, o[blk], 0, 0, 0);
        }
      }
    }
  }
  if (!q_ok) return;
  LOGKV_G uint16_t* orow = gp(a.out) + b * a.o_sb + head * a.o_sh + t * a.o_st;
#pragma unroll
  for (int blk = 0; blk < kMaxDvBlocks; ++blk) {
    if (blk < ndv) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d = 32 * blk + 8 * i4 + 4 * h;
        const uint32_t lo = static_cast<uint32_t>(f32_to_bf16(o[blk][4 * i4] / lsum)) |
                            (static_cast<uint32_t>(f32_to_bf16(o[blk][4 * i4 + 1] / lsum)) << 16);
        const uint32_t hi = static_cast<uint32_t>(f32_to_bf16(o[blk][4 * i4 + 2] / lsum)) |
                            (static_cast<uint32_t>(f32_to_bf16(o[blk][4 * i4 + 3] / lsum)) << 16);
        *(LOGKV_G uint2*)(orow + d) = make_uint2(lo, hi);
      }
    }
  }
}

int launch_chunk_attention(const logkv_attention_args& a, const int32_t* width, hipStream_t stream) {
  const int nq = (a.n_heads / a.n_groups) * a.tq;
  hipLaunchKernelGGL(chunk_kernel, dim3((nq + kQRows - 1) / kQRows, a.n_batch * a.n_groups), dim3(256), 0, stream, a,
                     width);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
