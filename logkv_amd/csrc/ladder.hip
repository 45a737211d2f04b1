// One flush committed into the ladders: one block per (lane, cluster) ladder.
//
// A block gathers its cluster's rows from the attach decisions (position
// order), opens a dead cluster with its earliest row, and Fenwick-appends the
// rest through every level itself: fill free slots; pair (or Beta 4->2) the
// oldest 2*ceil(m/2) rows of [stored | staged] into carries for the next level;
// move survivors to the front; fold a saturated top level. Carries are kept as
// bf16 in per-ladder scratch (the reference keeps them in fp32 but rounds them
// to the storage dtype on every read, litgpt/log_kv_updates_triton.py:16-23,
// so the values are identical). The center update sums the new keys in
// position order. Rules: litgpt/log_kv_cache.py:1756-1929 (append), :1670-1728
// (top fold), :5217-5312 + litgpt/log_kv_position.py:13-30 (pair merge),
// litgpt/beta_log_kv.py:29-105 (Beta), :2268-2298 (new cluster),
// :4116-4175 + :4326-4359 (joins and centers), :3690-3788 (delayed archive).
#include "route.hpp"

namespace logkv {

namespace {

constexpr int kThreads = 256;
constexpr int kChunkRows = 64;   // survivor rows moved per barrier

struct Soa {
  uint16_t* k;
  uint16_t* v;
  float* w;
  int64_t* lo;
  int64_t* hi;
  int64_t* swp;
  int64_t* ord;
  uint8_t* pad;
};

__host__ __device__ inline int64_t align16(int64_t x) { return (x + 15) & ~int64_t(15); }

__host__ __device__ inline int64_t soa_bytes(int64_t cap, int dk, int dv) {
  return align16(cap * dk * 2) + align16(cap * dv * 2) + align16(cap * 4) + 4 * align16(cap * 8) + align16(cap);
}

__device__ inline Soa soa_at(uint8_t* base, int64_t cap, int dk, int dv) {
  Soa s;
  s.k = reinterpret_cast<uint16_t*>(base);
  base += align16(cap * dk * 2);
  s.v = reinterpret_cast<uint16_t*>(base);
  base += align16(cap * dv * 2);
  s.w = reinterpret_cast<float*>(base);
  base += align16(cap * 4);
  s.lo = reinterpret_cast<int64_t*>(base);
  base += align16(cap * 8);
  s.hi = reinterpret_cast<int64_t*>(base);
  base += align16(cap * 8);
  s.swp = reinterpret_cast<int64_t*>(base);
  base += align16(cap * 8);
  s.ord = reinterpret_cast<int64_t*>(base);
  base += align16(cap * 8);
  s.pad = base;
  return s;
}

struct Meta {
  float w;
  int64_t lo, hi, swp, ord;
  uint8_t pad;
};

// Where the staged rows of the current level come from.
//  kind 0: flush rows tok[r] of the lane (w=1, anchors = position, order = base + r)
//  kind 1: a scratch SoA buffer
//  kind 2: delayed archive, row r = perm[r] over [existing entries in S0 | flush rows tok[]]
struct Src {
  int kind;
  const uint16_t* tok;
  int64_t order_base;
  const uint16_t* kb;
  const uint16_t* vb;
  int64_t k_st, v_st;
  const int64_t* posb;
  Soa buf;
  const uint16_t* perm;
  int n_exist;
};

struct Ladder {
  uint16_t* k;
  uint16_t* v;
  float* w;
  int64_t* lo;
  int64_t* hi;
  int64_t* swp;
  int64_t* ord;
  uint8_t* pad;
  int dk, dv, B;
};

__device__ __forceinline__ const uint16_t* src_k(const Src& s, int r, int dk) {
  if (s.kind == 1) return s.buf.k + static_cast<int64_t>(r) * dk;
  if (s.kind == 2) {
    const int q = s.perm[r];
    if (q < s.n_exist) return s.buf.k + static_cast<int64_t>(q) * dk;
    return s.kb + static_cast<int64_t>(s.tok[q - s.n_exist]) * s.k_st;
  }
  return s.kb + static_cast<int64_t>(s.tok[r]) * s.k_st;
}

__device__ __forceinline__ const uint16_t* src_v(const Src& s, int r, int dv) {
  if (s.kind == 1) return s.buf.v + static_cast<int64_t>(r) * dv;
  if (s.kind == 2) {
    const int q = s.perm[r];
    if (q < s.n_exist) return s.buf.v + static_cast<int64_t>(q) * dv;
    return s.vb + static_cast<int64_t>(s.tok[q - s.n_exist]) * s.v_st;
  }
  return s.vb + static_cast<int64_t>(s.tok[r]) * s.v_st;
}

__device__ __forceinline__ Meta soa_meta(const Soa& b, int64_t i) {
  return Meta{b.w[i], b.lo[i], b.hi[i], b.swp[i], b.ord[i], b.pad[i]};
}

__device__ __forceinline__ Meta src_meta(const Src& s, int r) {
  if (s.kind == 1) return soa_meta(s.buf, r);
  int t;
  if (s.kind == 2) {
    const int q = s.perm[r];
    if (q < s.n_exist) {
      Meta m = soa_meta(s.buf, q);
      m.ord = r;
      return m;
    }
    t = s.tok[q - s.n_exist];
    const int64_t p = s.posb[t];
    return Meta{1.0f, p, p, p, static_cast<int64_t>(r), 0};
  }
  t = s.tok[r];
  const int64_t p = s.posb[t];
  return Meta{1.0f, p, p, p, s.order_base + r, 0};
}

__device__ __forceinline__ Meta slot_meta(const Ladder& L, int64_t i) {
  return Meta{L.w[i], L.lo[i], L.hi[i], L.swp[i], L.ord[i], L.pad[i]};
}

__device__ __forceinline__ void put_slot_meta(const Ladder& L, int64_t i, const Meta& m) {
  L.w[i] = m.w;
  L.lo[i] = m.lo;
  L.hi[i] = m.hi;
  L.swp[i] = m.swp;
  L.ord[i] = m.ord;
  L.pad[i] = m.pad;
}

__device__ __forceinline__ void put_soa_meta(const Soa& b, int64_t i, const Meta& m) {
  b.w[i] = m.w;
  b.lo[i] = m.lo;
  b.hi[i] = m.hi;
  b.swp[i] = m.swp;
  b.ord[i] = m.ord;
  b.pad[i] = m.pad;
}

// Pair merge metadata (litgpt/log_kv_position.py:13-30, litgpt/log_kv_updates_triton.py:37-57).
__device__ __forceinline__ Meta merge_meta(const Meta& a, const Meta& b) {
  const bool ra = a.w > 0.f, rb = b.w > 0.f;
  Meta m;
  m.w = a.w + b.w;
  m.lo = (ra && rb) ? imin64(a.lo, b.lo) : (ra ? a.lo : b.lo);
  m.hi = (ra && rb) ? imax64(a.hi, b.hi) : (ra ? a.hi : b.hi);
  m.swp = a.swp + b.swp;
  m.ord = imin64(a.ord, b.ord);
  m.pad = a.pad & b.pad;
  return m;
}

// Pool row p of a level: storage slot p (p < B) or staged row take + p - B.
struct Pool {
  const Ladder* L;
  int64_t level_base;  // row index of slot 0 of this level
  const Src* src;
  int take;
  __device__ __forceinline__ bool stored(int p) const { return p < L->B; }
  __device__ __forceinline__ const uint16_t* k(int p) const {
    return stored(p) ? L->k + (level_base + p) * L->dk : src_k(*src, take + p - L->B, L->dk);
  }
  __device__ __forceinline__ const uint16_t* v(int p) const {
    return stored(p) ? L->v + (level_base + p) * L->dv : src_v(*src, take + p - L->B, L->dv);
  }
  __device__ __forceinline__ Meta meta(int p) const {
    return stored(p) ? slot_meta(*L, level_base + p) : src_meta(*src, take + p - L->B);
  }
};

// Copy 4 bf16 (8 bytes) units of a K|V row; unit u < dk/4 is K, the rest V.
__device__ __forceinline__ uint2 load_unit(const uint16_t* k, const uint16_t* v, int u, int ku) {
  return u < ku ? *reinterpret_cast<const uint2*>(k + 4 * u) : *reinterpret_cast<const uint2*>(v + 4 * (u - ku));
}

__device__ __forceinline__ void store_unit(uint16_t* k, uint16_t* v, int u, int ku, uint2 x) {
  if (u < ku) *reinterpret_cast<uint2*>(k + 4 * u) = x;
  else *reinterpret_cast<uint2*>(v + 4 * (u - ku)) = x;
}

__device__ __forceinline__ float lo_half(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float hi_half(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// alpha*a + (1-alpha)*b on 4 bf16, rounded back to bf16.
__device__ __forceinline__ uint2 blend_unit(uint2 a, uint2 b, float alpha) {
  const float beta = 1.0f - alpha;
  uint2 o;
  o.x = pack2(alpha * lo_half(a.x) + beta * lo_half(b.x), alpha * hi_half(a.x) + beta * hi_half(b.x));
  o.y = pack2(alpha * lo_half(a.y) + beta * lo_half(b.y), alpha * hi_half(a.y) + beta * hi_half(b.y));
  return o;
}

// Rows [0, n) of `src` to storage slots [dst0, dst0 + n) (no overlap with the source).
__device__ void copy_src_to_slots(const Ladder& L, int64_t level_base, const Src& src, int src0, int dst0, int n) {
  const int ku = L.dk / 4, units = (L.dk + L.dv) / 4;
  for (int i = threadIdx.x; i < n * units; i += kThreads) {
    const int r = i / units, u = i % units;
    const int64_t slot = level_base + dst0 + r;
    store_unit(L.k + slot * L.dk, L.v + slot * L.dv, u, ku, load_unit(src_k(src, src0 + r, L.dk), src_v(src, src0 + r, L.dv), u, ku));
  }
  for (int r = threadIdx.x; r < n; r += kThreads) put_slot_meta(L, level_base + dst0 + r, src_meta(src, src0 + r));
}

// Storage slots [from, from + n) -> [to, to + n) with to <= from, overlap allowed.
// Each chunk is loaded whole before any of it is stored; later chunks never
// read what earlier chunks wrote because the destination trails the source.
__device__ void shift_slots_down(const Ladder& L, int64_t level_base, int from, int to, int n) {
  if (n <= 0 || from == to) return;
  const int ku = L.dk / 4, units = (L.dk + L.dv) / 4;
  constexpr int kMaxUnitsPerThread = kChunkRows * (2 * kMaxDim / 4) / kThreads;
  for (int c0 = 0; c0 < n; c0 += kChunkRows) {
    const int rows = min(kChunkRows, n - c0);
    uint2 buf[kMaxUnitsPerThread];
    Meta m{};
    const int total = rows * units;
#pragma unroll
    for (int q = 0; q < kMaxUnitsPerThread; ++q) {
      const int i = threadIdx.x + q * kThreads;
      if (i < total) {
        const int r = i / units, u = i % units;
        const int64_t s = level_base + from + c0 + r;
        buf[q] = load_unit(L.k + s * L.dk, L.v + s * L.dv, u, ku);
      }
    }
    if (threadIdx.x < rows) m = slot_meta(L, level_base + from + c0 + threadIdx.x);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kMaxUnitsPerThread; ++q) {
      const int i = threadIdx.x + q * kThreads;
      if (i < total) {
        const int r = i / units, u = i % units;
        const int64_t d = level_base + to + c0 + r;
        store_unit(L.k + d * L.dk, L.v + d * L.dv, u, ku, buf[q]);
      }
    }
    if (threadIdx.x < rows) put_slot_meta(L, level_base + to + c0 + threadIdx.x, m);
  }
}

__device__ void clear_slots(const Ladder& L, int64_t first, int64_t n) {
  const int ku = L.dk / 4, units = (L.dk + L.dv) / 4;
  const uint2 z = make_uint2(0u, 0u);
  for (int64_t i = threadIdx.x; i < n * units; i += kThreads) {
    const int64_t s = first + i / units;
    store_unit(L.k + s * L.dk, L.v + s * L.dv, static_cast<int>(i % units), ku, z);
  }
  for (int64_t r = threadIdx.x; r < n; r += kThreads) put_slot_meta(L, first + r, Meta{0.f, 0, 0, 0, 0, 0});
}

// Carries j in [0, n_carry): pool rows (2j, 2j+1), one wave per carry.
__device__ void pair_carries(const Pool& pool, const Soa& out, int n_carry, int dk, int dv) {
  const int ku = dk / 4, units = (dk + dv) / 4;
  const int l = lane_id(), w = wave_id(), nw = kThreads / kWave;
  for (int j = w; j < n_carry; j += nw) {
    const Meta a = pool.meta(2 * j), b = pool.meta(2 * j + 1);
    const float alpha = a.w / fmaxf(a.w + b.w, 1e-8f);
    const uint16_t *ak = pool.k(2 * j), *av = pool.v(2 * j), *bk = pool.k(2 * j + 1), *bv = pool.v(2 * j + 1);
    for (int u = l; u < units; u += kWave)
      store_unit(out.k + static_cast<int64_t>(j) * dk, out.v + static_cast<int64_t>(j) * dv, u, ku,
                 blend_unit(load_unit(ak, av, u, ku), load_unit(bk, bv, u, ku), alpha));
    if (l == 0) put_soa_meta(out, j, merge_meta(a, b));
  }
}

// ---- Beta 4->2 -------------------------------------------------------------
constexpr int kJ = kMaxDim / kWave;

// Canonical sum over the features held as x[j] (feature l + 64 j) in every lane.
__device__ __forceinline__ float feat_sum(const float* t, int J) {
  float s = t[0];
#pragma unroll
  for (int j = 1; j < kJ; ++j)
    if (j < J) s = s + t[j];
  return wave_tree(s);
}

// Loss sum_i w_i |x_i - mean|^2 of one side; rows outside the side contribute +0.
__device__ float side_loss(const float (*x)[kJ], const float* wt, const float* mean, int J, int D, unsigned member) {
  float loss = 0.f;
  const int l = lane_id();
  for (int i = 0; i < 4; ++i) {
    float per = 0.f;
    if ((member >> i) & 1u) {
      float t[kJ];
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const float d = (l + j * kWave < D) ? x[i][j] - mean[j] : 0.f;
        t[j] = d * d;
      }
      per = feat_sum(t, J);
    }
    const float term = per * wt[i];
    loss = i == 0 ? term : loss + term;
  }
  return loss;
}

__device__ __forceinline__ void side_mean(const float (*x)[kJ], const float* wt, float* mean, float& mass, int J) {
  mass = ((wt[0] + wt[1]) + wt[2]) + wt[3];
  const float den = fmaxf(mass, 1e-12f);
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    if (j < J) {
      float acc = x[0][j] * wt[0];
      acc = acc + x[1][j] * wt[1];
      acc = acc + x[2][j] * wt[2];
      acc = acc + x[3][j] * wt[3];
      mean[j] = acc / den;
    }
  }
}

__device__ void beta_carries(const Pool& pool, const Soa& out, int n_pair, int dk, int dv) {
  const int l = lane_id(), w = wave_id(), nw = kThreads / kWave;
  const int Jk = (dk + kWave - 1) / kWave, Jv = (dv + kWave - 1) / kWave;
  const int n_groups = (n_pair + 3) / 4;
  for (int gi = w; gi < n_groups; gi += nw) {
    const int start = 4 * gi;
    const int width = min(4, n_pair - start);
    float xk[4][kJ], xv[4][kJ], wr[4];
    Meta m[4];
    for (int i = 0; i < 4; ++i) {
      const bool valid = i < width;
      m[i] = valid ? pool.meta(start + i) : Meta{0.f, 0, 0, 0, 0, 0};
      wr[i] = valid ? m[i].w : 0.f;
      const uint16_t* kr = valid ? pool.k(start + i) : nullptr;
      const uint16_t* vr = valid ? pool.v(start + i) : nullptr;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int d = l + j * kWave;
        xk[i][j] = (valid && j < Jk && d < dk) ? bf16_to_f32(kr[d]) : 0.f;
        xv[i][j] = (valid && j < Jv && d < dv) ? bf16_to_f32(vr[d]) : 0.f;
      }
    }
    int cut = 1;
    if (width == 4) {
      const float total = fmaxf(((wr[0] + wr[1]) + wr[2]) + wr[3], 1e-12f);
      float costs[3] = {0.f, 0.f, 0.f};
      for (int comp = 0; comp < 2; ++comp) {
        const float(*x)[kJ] = comp == 0 ? xk : xv;
        const int J = comp == 0 ? Jk : Jv, D = comp == 0 ? dk : dv;
        float e = 0.f;
        for (int i = 0; i < 4; ++i) {
          float t[kJ];
#pragma unroll
          for (int j = 0; j < kJ; ++j) t[j] = x[i][j] * x[i][j];
          const float term = feat_sum(t, J) * wr[i];
          e = i == 0 ? term : e + term;
        }
        const float energy = fmaxf(e / total, 1e-12f);
        for (int opt = 0; opt < 3; ++opt) {
          const int c = opt == 0 ? 2 : (opt == 1 ? 1 : 3);
          for (int side = 0; side < 2; ++side) {
            const unsigned member = side == 0 ? ((1u << c) - 1u) : (0xfu & ~((1u << c) - 1u));
            float wt[4], mean[kJ], mass;
            for (int i = 0; i < 4; ++i) wt[i] = ((member >> i) & 1u) ? wr[i] : 0.f;
            side_mean(x, wt, mean, mass, J);
            costs[opt] = costs[opt] + side_loss(x, wt, mean, J, D, member) / energy;
          }
        }
      }
      int best = 0;
      if (costs[1] < costs[best]) best = 1;
      if (costs[2] < costs[best]) best = 2;
      cut = best == 0 ? 2 : (best == 1 ? 1 : 3);
    }
    const int dest = start / 2;
    for (int side = 0; side < (width == 4 ? 2 : 1); ++side) {
      unsigned member;
      if (width == 2) member = 0x3u;
      else member = side == 0 ? ((1u << cut) - 1u) : (0xfu & ~((1u << cut) - 1u));
      float wt[4], mk[kJ], mv[kJ], mass;
      for (int i = 0; i < 4; ++i) wt[i] = ((member >> i) & 1u) ? wr[i] : 0.f;
      side_mean(xk, wt, mk, mass, Jk);
      side_mean(xv, wt, mv, mass, Jv);
      const int64_t o = dest + side;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int d = l + j * kWave;
        if (j < Jk && d < dk) out.k[o * dk + d] = f32_to_bf16(mk[j]);
        if (j < Jv && d < dv) out.v[o * dv + d] = f32_to_bf16(mv[j]);
      }
      if (l == 0) {
        Meta r;
        r.w = mass;
        int64_t lo = INT64_MAX, hi = INT64_MIN, swp = 0, ord = INT64_MAX;
        uint8_t pad = 1;
        for (int i = 0; i < 4; ++i) {
          if (!((member >> i) & 1u)) continue;
          if (m[i].w > 0.f) {
            lo = imin64(lo, m[i].lo);
            hi = imax64(hi, m[i].hi);
          }
          swp += m[i].swp;
          ord = imin64(ord, m[i].ord);
          pad &= m[i].pad;
        }
        r.lo = mass > 0.f ? lo : 0;
        r.hi = mass > 0.f ? hi : 0;
        r.swp = swp;
        r.ord = ord;
        r.pad = pad;
        put_soa_meta(out, o, r);
      }
    }
  }
}

// ---- top-level fold --------------------------------------------------------
// Slot 0 <- left fold of pool[0..mr] (rounded to bf16 after each merge),
// slots 1..B-1 <- pool[mr+1 .. mr+B-1].
__device__ void fold_top(const Ladder& L, int64_t level_base, const Src& src, int take, int mr) {
  const int B = L.B;
  const int ku = L.dk / 4, units = (L.dk + L.dv) / 4;
  Pool pool{&L, level_base, &src, take};
  constexpr int kMaxUnitsPerLane = (2 * kMaxDim / 4) / kWave;
  uint2 acc[kMaxUnitsPerLane];
  Meta am{};
  if (wave_id() == 0) {
    const int l = lane_id();
    am = pool.meta(0);
#pragma unroll
    for (int q = 0; q < kMaxUnitsPerLane; ++q) {
      const int u = l + q * kWave;
      if (u < units) acc[q] = load_unit(pool.k(0), pool.v(0), u, ku);
    }
    for (int t = 1; t <= mr; ++t) {
      const Meta b = pool.meta(t);
      const float alpha = am.w / fmaxf(am.w + b.w, 1e-8f);
      const uint16_t *bk = pool.k(t), *bv = pool.v(t);
#pragma unroll
      for (int q = 0; q < kMaxUnitsPerLane; ++q) {
        const int u = l + q * kWave;
        if (u < units) acc[q] = blend_unit(acc[q], load_unit(bk, bv, u, ku), alpha);
      }
      am = merge_meta(am, b);
    }
  }
  __syncthreads();
  // Stored part of the tail shifts down by mr; staged part follows.
  const int stored_from = mr + 1;
  const int n_stored = stored_from < B ? B - stored_from : 0;
  shift_slots_down(L, level_base, stored_from, 1, n_stored);
  __syncthreads();
  const int first_staged = stored_from > B ? stored_from : B;   // pool index
  const int n_staged = (mr + B - 1) - first_staged + 1;
  if (n_staged > 0) copy_src_to_slots(L, level_base, src, take + first_staged - B, first_staged - mr, n_staged);
  if (wave_id() == 0) {
    const int l = lane_id();
#pragma unroll
    for (int q = 0; q < kMaxUnitsPerLane; ++q) {
      const int u = l + q * kWave;
      if (u < units) store_unit(L.k + level_base * L.dk, L.v + level_base * L.dv, u, ku, acc[q]);
    }
    if (l == 0) put_slot_meta(L, level_base, am);
  }
  __syncthreads();
}

// Fenwick append of m0 staged rows from `src0` into one ladder.
__device__ void fenwick_append(const Ladder& L, int16_t* counts_s, int levels, Src src0, int m0, Soa bufA, Soa bufB,
                               bool beta) {
  const int B = L.B;
  Src cur = src0;
  int m = m0;
  for (int ell = 0; ell < levels && m > 0; ++ell) {
    const int64_t level_base = static_cast<int64_t>(ell) * B;
    const bool top = ell == levels - 1;
    const int cnt = counts_s[ell];
    const int take = min(B - cnt, m);
    if (take > 0) copy_src_to_slots(L, level_base, cur, 0, cnt, take);
    __syncthreads();
    const int mr = m - take;
    if (mr == 0) {
      if (threadIdx.x == 0) counts_s[ell] = static_cast<int16_t>(cnt + take);
      __syncthreads();
      break;
    }
    if (top) {
      fold_top(L, level_base, cur, take, mr);
      if (threadIdx.x == 0) counts_s[ell] = static_cast<int16_t>(B);
      __syncthreads();
      break;
    }
    const int n_carry = (mr + 1) / 2, n_pair = 2 * n_carry;
    const Soa out = (ell & 1) ? bufB : bufA;
    Pool pool{&L, level_base, &cur, take};
    if (beta) beta_carries(pool, out, n_pair, L.dk, L.dv);
    else pair_carries(pool, out, n_carry, L.dk, L.dv);
    __syncthreads();
    const int n_surv = B + mr - n_pair;
    if (n_pair < B) {
      shift_slots_down(L, level_base, n_pair, 0, B - n_pair);
      __syncthreads();
      copy_src_to_slots(L, level_base, cur, take, B - n_pair, mr);
    } else {
      copy_src_to_slots(L, level_base, cur, take + n_pair - B, 0, n_surv);
    }
    clear_slots(L, level_base + n_surv, B - n_surv);
    __syncthreads();
    if (threadIdx.x == 0) counts_s[ell] = static_cast<int16_t>(n_surv);
    __syncthreads();
    Src next{};
    next.kind = 1;
    next.buf = out;
    cur = next;
    m = n_carry;
  }
}

}  // namespace

int64_t row_bytes(int dk, int dv) { return 2 * (dk + dv) + 4 + 32 + 1; }

int64_t ladder_scratch_rows(int64_t m0, int64_t slots, int64_t& s0, int64_t& ca, int64_t& cb, int64_t existing) {
  (void)slots;
  s0 = existing;
  ca = (m0 + 1) / 2 + 1;
  cb = (m0 + 3) / 4 + 2;
  return s0 + ca + cb;
}

int64_t ladder_scratch_bytes(const LadderArgs& c, int64_t s0, int64_t ca, int64_t cb) {
  return soa_bytes(s0, c.dk, c.dv) + soa_bytes(ca, c.dk, c.dv) + soa_bytes(cb, c.dk, c.dv);
}

__global__ __launch_bounds__(kThreads) void commit_kernel(LadderArgs c, RowsArgs r, RouteParams prm, Workspace ws) {
  extern __shared__ __align__(16) uint8_t dyn[];
  __shared__ int wave_sum[kThreads / kWave];
  __shared__ int16_t counts_s[64];
  __shared__ int m_s;
  const int K = c.k_max, L = c.levels, B = c.slots, dk = c.dk, dv = c.dv;
  const int ladder = blockIdx.x;
  const int lane_ix = ladder / K, cc = ladder % K;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  const int n = valid_rows(r, b);
  uint16_t* tok = reinterpret_cast<uint16_t*>(dyn);
  const int8_t* as = ws.assign + static_cast<int64_t>(lane_ix) * r.tokens;
  const int32_t* ord = ws.order + static_cast<int64_t>(b) * r.tokens;

  // 1. This cluster's rows in position order (stable compaction).
  if (threadIdx.x == 0) m_s = 0;
  __syncthreads();
  for (int s0 = 0; s0 < n; s0 += kThreads) {
    const int s = s0 + threadIdx.x;
    const bool mine = s < n && as[s] == cc;
    const uint64_t ballot = __ballot(mine);
    const int l = lane_id(), w = wave_id();
    const int before = __popcll(ballot & ((l == 0) ? 0ull : (~0ull >> (kWave - l))));
    if (l == 0) wave_sum[w] = __popcll(ballot);
    __syncthreads();
    int base = m_s;
    for (int q = 0; q < w; ++q) base += wave_sum[q];
    if (mine) tok[base + before] = static_cast<uint16_t>(ord[s]);
    __syncthreads();
    if (threadIdx.x == 0) {
      int add = 0;
      for (int q = 0; q < kThreads / kWave; ++q) add += wave_sum[q];
      m_s = m_s + add;
    }
    __syncthreads();
  }
  const int m = m_s;
  if (m == 0) return;

  const int64_t cl = static_cast<int64_t>(lane_ix) * K + cc;
  const int64_t row0 = cl * L * B;
  Ladder lad{c.level_k + row0 * dk, c.level_v + row0 * dv, c.level_w + row0, c.level_p_lo + row0,
             c.level_p_hi + row0, c.level_sum_wp + row0, c.level_order + row0, c.pad_mask + row0, dk, dv, B};
  const uint16_t* kb = r.k + b * r.k_sb + g * r.k_sg;
  const uint16_t* vb = r.v + b * r.v_sb + g * r.v_sg;
  const int64_t* posb = r.pos + b * r.pos_sb;
  float* mu = c.centroid + cl * dk;
  uint8_t* scratch = ws.ladder + ladder * ws.ladder_stride;
  const Soa S0 = soa_at(scratch, ws.s0_rows, dk, dv);
  scratch += soa_bytes(ws.s0_rows, dk, dv);
  const Soa bufA = soa_at(scratch, ws.carry_a_rows, dk, dv);
  scratch += soa_bytes(ws.carry_a_rows, dk, dv);
  const Soa bufB = soa_at(scratch, ws.carry_b_rows, dk, dv);

  for (int e = threadIdx.x; e < L; e += kThreads) counts_s[e] = c.level_count[cl * L + e];
  bool alive = c.alive[cl] != 0;
  float n_eff = c.n_eff[cl];
  int32_t n_total = c.n_total[cl];
  int64_t p_hi = c.p_hi_c[cl];
  int32_t phase = c.level0_phase[cl];
  __syncthreads();

  int first = 0;
  if (!alive) {
    // 2. A dead cluster opens with its earliest row (clears every slot first).
    clear_slots(lad, 0, static_cast<int64_t>(L) * B);
    for (int e = threadIdx.x; e < L; e += kThreads) counts_s[e] = 0;
    const int t0 = tok[0];
    for (int d = threadIdx.x; d < dk; d += kThreads) mu[d] = bf16_to_f32(kb[static_cast<int64_t>(t0) * r.k_st + d]);
    __syncthreads();
    Src one{};
    one.kind = 0;
    one.tok = tok;
    one.order_base = 0;
    one.kb = kb;
    one.vb = vb;
    one.k_st = r.k_st;
    one.v_st = r.v_st;
    one.posb = posb;
    fenwick_append(lad, counts_s, L, one, 1, bufA, bufB, prm.beta_merge != 0);
    alive = true;
    n_eff = 1.0f;
    n_total = 1;
    p_hi = posb[t0];
    phase = 1;
    first = 1;
  }
  const int nn = m - first;
  if (nn > 0) {
    const int64_t first_pos = posb[tok[first]];
    const bool late = prm.late_joins && first_pos < p_hi;
    // 3. Center update over the new rows, summed in position order
    //    (mu = (pre*mu + sum)/(pre + n), pre = n_eff).
    int64_t last_pos = posb[tok[m - 1]];
    for (int d = threadIdx.x; d < dk; d += kThreads) {
      float acc = bf16_to_f32(kb[static_cast<int64_t>(tok[first]) * r.k_st + d]);
      for (int i = first + 1; i < m; ++i) acc = acc + bf16_to_f32(kb[static_cast<int64_t>(tok[i]) * r.k_st + d]);
      const float pre = n_eff;
      const float den = pre + static_cast<float>(nn);
      mu[d] = pre > 0.f ? (pre * mu[d] + acc) / den : acc / static_cast<float>(nn);
    }
    Src src{};
    src.tok = tok + first;
    src.kb = kb;
    src.vb = vb;
    src.k_st = r.k_st;
    src.v_st = r.v_st;
    src.posb = posb;
    int m0 = nn;
    if (!late) {
      src.kind = 0;
      src.order_base = phase;
      phase += nn;
      p_hi = last_pos;
    } else {
      // 4. Delayed archive: existing entries (level by level, slots in order)
      //    and the new rows, stably sorted by p_lo, re-appended from level 0.
      int n_exist = 0;
      for (int e = 0; e < L; ++e) n_exist += counts_s[e];
      uint64_t* keys = reinterpret_cast<uint64_t*>(dyn + ((2 * r.tokens + 15) & ~15));
      uint16_t* perm = reinterpret_cast<uint16_t*>(keys + ws.sort_width);
      int base = 0;
      for (int e = 0; e < L; ++e) {
        const int ce = counts_s[e];
        const int ku = dk / 4, units = (dk + dv) / 4;
        for (int i = threadIdx.x; i < ce * units; i += kThreads) {
          const int rr = i / units, u = i % units;
          const int64_t slot = static_cast<int64_t>(e) * B + rr;
          store_unit(S0.k + static_cast<int64_t>(base + rr) * dk, S0.v + static_cast<int64_t>(base + rr) * dv, u, ku,
                     load_unit(lad.k + slot * dk, lad.v + slot * dv, u, ku));
        }
        for (int rr = threadIdx.x; rr < ce; rr += kThreads) {
          const Meta mt = slot_meta(lad, static_cast<int64_t>(e) * B + rr);
          put_soa_meta(S0, base + rr, mt);
          keys[base + rr] = (static_cast<uint64_t>(mt.lo) << kOrderIndexBits) | static_cast<uint64_t>(base + rr);
        }
        base += ce;
      }
      const int total = n_exist + nn;
      for (int i = threadIdx.x; i < nn; i += kThreads)
        keys[n_exist + i] = (static_cast<uint64_t>(posb[tok[first + i]]) << kOrderIndexBits) |
                            static_cast<uint64_t>(n_exist + i);
      int width = 1;
      while (width < total) width <<= 1;
      for (int i = total + threadIdx.x; i < width; i += kThreads) keys[i] = ~0ull;
      __syncthreads();
      for (int size = 2; size <= width; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          for (int t = threadIdx.x; t < width; t += kThreads) {
            const int partner = t ^ stride;
            if (partner > t) {
              const bool up = (t & size) == 0;
              const uint64_t a = keys[t], bk = keys[partner];
              if ((a > bk) == up) {
                keys[t] = bk;
                keys[partner] = a;
              }
            }
          }
          __syncthreads();
        }
      }
      for (int i = threadIdx.x; i < total; i += kThreads) perm[i] = static_cast<uint16_t>(keys[i] & kOrderIndexMask);
      int64_t hi = p_hi;
      for (int i = first; i < m; ++i) hi = imax64(hi, posb[tok[i]]);
      p_hi = hi;
      phase = total;
      __syncthreads();
      clear_slots(lad, 0, static_cast<int64_t>(L) * B);
      for (int e = threadIdx.x; e < L; e += kThreads) counts_s[e] = 0;
      __syncthreads();
      src.kind = 2;
      src.buf = S0;
      src.perm = perm;
      src.n_exist = n_exist;
      m0 = total;
    }
    n_eff = n_eff + static_cast<float>(nn);
    n_total += nn;
    __syncthreads();
    fenwick_append(lad, counts_s, L, src, m0, bufA, bufB, prm.beta_merge != 0);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < L; e += kThreads) c.level_count[cl * L + e] = counts_s[e];
  if (threadIdx.x == 0) {
    c.alive[cl] = 1;
    c.n_eff[cl] = n_eff;
    c.n_total[cl] = n_total;
    c.p_hi_c[cl] = p_hi;
    c.level0_phase[cl] = phase;
  }
}

int launch_commit(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                  hipStream_t stream) {
  const int ladders = c.n_batch * c.n_groups * c.k_max;
  size_t shmem = ((2 * static_cast<size_t>(r.tokens) + 15) & ~size_t(15));
  if (p.late_joins) shmem += static_cast<size_t>(ws.sort_width) * 8 + static_cast<size_t>(ws.sort_width) * 2;
  if (shmem > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&commit_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(shmem)) != hipSuccess)
    return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(commit_kernel, dim3(ladders), dim3(kThreads), shmem, stream, c, r, p, ws);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
