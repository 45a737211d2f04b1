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
#include <algorithm>

#include "beta.hpp"
#include "route.hpp"
#include "unified.hpp"

namespace logkv {

namespace {

constexpr int kThreads = 512;
constexpr int kMoveUnits = 8;    // 8-byte units per thread staged in registers per move chunk

struct Soa {
  LOGKV_G uint16_t* k;
  LOGKV_G uint16_t* v;
  LOGKV_G float* w;
  LOGKV_G int64_t* lo;
  LOGKV_G int64_t* hi;
  LOGKV_G int64_t* swp;
  LOGKV_G int64_t* ord;
  LOGKV_G uint8_t* pad;
};

__host__ __device__ inline int64_t align16(int64_t x) { return (x + 15) & ~int64_t(15); }

__host__ __device__ inline int64_t soa_bytes(int64_t cap, int dk, int dv) {
  return align16(cap * dk * 2) + align16(cap * dv * 2) + align16(cap * 4) + 4 * align16(cap * 8) + align16(cap);
}

__device__ inline Soa soa_at(uint8_t* base, int64_t cap, int dk, int dv) {
  Soa s;
  s.k = gp(reinterpret_cast<uint16_t*>(base));
  base += align16(cap * dk * 2);
  s.v = gp(reinterpret_cast<uint16_t*>(base));
  base += align16(cap * dv * 2);
  s.w = gp(reinterpret_cast<float*>(base));
  base += align16(cap * 4);
  s.lo = gp(reinterpret_cast<int64_t*>(base));
  base += align16(cap * 8);
  s.hi = gp(reinterpret_cast<int64_t*>(base));
  base += align16(cap * 8);
  s.swp = gp(reinterpret_cast<int64_t*>(base));
  base += align16(cap * 8);
  s.ord = gp(reinterpret_cast<int64_t*>(base));
  base += align16(cap * 8);
  s.pad = gp(base);
  return s;
}

// Where the staged rows of the current level come from.
//  kind 0: flush rows tok[r] of the lane (w=1, anchors = position, order = base + r)
//  kind 1: a scratch SoA buffer
//  kind 2: as kind 0 with the row list read from global memory
struct Src {
  int kind;
  const LOGKV_S uint16_t* tok;     // kind 0: row list in LDS
  const LOGKV_G uint16_t* gtok;    // kind 2: row list in global memory
  int64_t order_base;
  const LOGKV_G uint16_t* kb;
  const LOGKV_G uint16_t* vb;
  int64_t k_st, v_st;
  const LOGKV_G int64_t* posb;
  Soa buf;
};

struct Ladder {
  LOGKV_G uint16_t* k;
  LOGKV_G uint16_t* v;
  LOGKV_G float* w;
  LOGKV_G int64_t* lo;
  LOGKV_G int64_t* hi;
  LOGKV_G int64_t* swp;
  LOGKV_G int64_t* ord;
  LOGKV_G uint8_t* pad;
  int dk, dv, B;
};

__device__ __forceinline__ Meta soa_meta(const Soa& b, int64_t i) {
  return Meta{b.w[i], b.lo[i], b.hi[i], b.swp[i], b.ord[i], b.pad[i]};
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

// Virtual pool of one level: [stored slots 0..cnt | staged rows 0..m]. Filling
// the free slots and then pairing the oldest rows of [stored | rest of staged]
// (litgpt/log_kv_cache.py:1815-1853) only ever reads this sequence, so a level
// step is a function of it and needs no barrier between fill and pairing.
// KIND is the staged source (0 flush rows, 1 scratch rows); row addresses are
// resolved with selects so the copy loops stay branch-free.
template <int KIND>
struct PoolT {
  Ladder L;
  int64_t base;  // row index of slot 0 of this level
  int cnt;       // rows stored before this step
  Src src;
  __device__ __forceinline__ int64_t staged_row(int q) const {
    if (KIND == 1) return static_cast<int64_t>(q);
    return KIND == 2 ? static_cast<int64_t>(src.gtok[q]) : static_cast<int64_t>(src.tok[q]);
  }
  __device__ __forceinline__ const LOGKV_G uint16_t* k(int p) const {
    const bool st = p < cnt;
    const int q = st ? 0 : p - cnt;
    const LOGKV_G uint16_t* staged =
        KIND == 1 ? src.buf.k + staged_row(q) * L.dk : src.kb + staged_row(q) * src.k_st;
    return st ? L.k + (base + p) * L.dk : staged;
  }
  __device__ __forceinline__ const LOGKV_G uint16_t* v(int p) const {
    const bool st = p < cnt;
    const int q = st ? 0 : p - cnt;
    const LOGKV_G uint16_t* staged =
        KIND == 1 ? src.buf.v + staged_row(q) * L.dv : src.vb + staged_row(q) * src.v_st;
    return st ? L.v + (base + p) * L.dv : staged;
  }
  // Branch-free: every load is issued (a stored slot index clamps to slot 0,
  // a staged index to row 0) and the value is selected afterwards.
  __device__ __forceinline__ float w(int p) const {
    const bool st = p < cnt;
    if (KIND != 1) {
      const float stored = L.w[base + (st ? p : 0)];
      return st ? stored : 1.0f;
    }
    const LOGKV_G float* wp = st ? L.w + base + p : src.buf.w + (p - cnt);
    return *wp;
  }
  // Row pointers and metadata of pool row p whose staged row index t is
  // already known (KIND 2: a flush row list read ahead).
  __device__ __forceinline__ const LOGKV_G uint16_t* k_at(int p, int64_t t) const {
    return p < cnt ? L.k + (base + p) * L.dk : src.kb + t * src.k_st;
  }
  __device__ __forceinline__ const LOGKV_G uint16_t* v_at(int p, int64_t t) const {
    return p < cnt ? L.v + (base + p) * L.dv : src.vb + t * src.v_st;
  }
  __device__ __forceinline__ Meta meta_at(int p, int64_t t) const {
    const bool st = p < cnt;
    const int64_t pos = src.posb[t];
    const Meta stored = slot_meta(L, st ? base + p : base);
    return st ? stored : Meta{1.0f, pos, pos, pos, src.order_base + (p - cnt), 0};
  }
  __device__ __forceinline__ Meta meta(int p) const {
    const bool st = p < cnt;
    const int64_t i = st ? base + p : 0;
    if (KIND == 1) {
      const int64_t j = st ? 0 : p - cnt;
      return Meta{*(st ? L.w + i : src.buf.w + j), *(st ? L.lo + i : src.buf.lo + j),
                  *(st ? L.hi + i : src.buf.hi + j), *(st ? L.swp + i : src.buf.swp + j),
                  *(st ? L.ord + i : src.buf.ord + j), *(st ? L.pad + i : src.buf.pad + j)};
    }
    const int q = st ? 0 : p - cnt;
    const int64_t pos = src.posb[staged_row(q)];
    const Meta stored = slot_meta(L, st ? i : base);
    return st ? stored : Meta{1.0f, pos, pos, pos, src.order_base + q, 0};
  }
};

// Thread -> (row, unit) decomposition of a row-major K|V copy: thread t owns
// unit t % units of rows t / units, t / units + rows_per_pass, ...
struct RowUnits {
  int ku, units, u, r0, step;
  __device__ __forceinline__ RowUnits(int dk, int dv) {
    ku = dk / 4;
    units = (dk + dv) / 4;
    u = static_cast<int>(threadIdx.x) % units;
    r0 = static_cast<int>(threadIdx.x) / units;
    step = static_cast<int>(blockDim.x) / units;
    if (r0 >= step) r0 = 1 << 30;  // threads past the last full pass stay idle
  }
};

// Copy 4 bf16 (8 bytes) units of a K|V row; unit u < dk/4 is K, the rest V.
__device__ __forceinline__ uint2 load_unit(const LOGKV_G uint16_t* k, const LOGKV_G uint16_t* v, int u, int ku) {
  const LOGKV_G uint16_t* p = u < ku ? k + 4 * u : v + 4 * (u - ku);
  return *(const LOGKV_G uint2*)p;
}

__device__ __forceinline__ void store_unit(LOGKV_G uint16_t* k, LOGKV_G uint16_t* v, int u, int ku, uint2 x) {
  LOGKV_G uint16_t* p = u < ku ? k + 4 * u : v + 4 * (u - ku);
  *(LOGKV_G uint2*)p = x;
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

// Pool rows [p0, p0 + n) -> slots [d0, d0 + n) of the level, d0 <= p0. Each chunk
// is loaded whole into registers, then a barrier, then stored: a chunk's
// stores never reach a later chunk's sources because the destination trails
// the source, and every earlier load of the step precedes the first barrier.
template <int KIND>
__device__ __forceinline__ void move_rows(const PoolT<KIND>& pool, int p0, int d0, int n) {
  const Ladder& L = pool.L;
  const RowUnits ru(L.dk, L.dv);
  const int per_chunk = kMoveUnits * ru.step;
  for (int c0 = 0; c0 < n; c0 += per_chunk) {
    const int rows = min(per_chunk, n - c0);
    uint2 buf[kMoveUnits];
#pragma unroll
    for (int q = 0; q < kMoveUnits; ++q) {
      // Unconditional loads (a row past the chunk re-reads its last row) keep
      // every load of the chunk in flight at once.
      const int r = min(ru.r0 + q * ru.step, rows - 1);
      buf[q] = load_unit(pool.k(p0 + c0 + r), pool.v(p0 + c0 + r), ru.u, ru.ku);
    }
    Meta m{};
    if (static_cast<int>(threadIdx.x) < rows) m = pool.meta(p0 + c0 + threadIdx.x);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kMoveUnits; ++q) {
      const int r = ru.r0 + q * ru.step;
      if (r < rows) {
        const int64_t d = pool.base + d0 + c0 + r;
        store_unit(L.k + d * L.dk, L.v + d * L.dv, ru.u, ru.ku, buf[q]);
      }
    }
    if (static_cast<int>(threadIdx.x) < rows) put_slot_meta(L, pool.base + d0 + c0 + threadIdx.x, m);
  }
}

constexpr int kBatch = 4;   // rows per thread whose loads are issued before any of their stores

// Staged rows [s0, s0 + n) -> slots [d0, d0 + n); the staged rows never alias the level.
template <int KIND>
__device__ __forceinline__ void copy_staged(const Ladder& L, int64_t base, const Src& src, int s0, int d0, int n) {
  const RowUnits ru(L.dk, L.dv);
  const PoolT<KIND> pool{L, base, 0, src};
  for (int r0 = ru.r0; r0 < n; r0 += kBatch * ru.step) {
    uint2 x[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int r = min(r0 + q * ru.step, n - 1);
      x[q] = load_unit(pool.k(s0 + r), pool.v(s0 + r), ru.u, ru.ku);
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int r = r0 + q * ru.step;
      if (r < n) {
        const int64_t slot = base + d0 + r;
        store_unit(L.k + slot * L.dk, L.v + slot * L.dv, ru.u, ru.ku, x[q]);
      }
    }
  }
  for (int r = threadIdx.x; r < n; r += blockDim.x) put_slot_meta(L, base + d0 + r, pool.meta(s0 + r));
}

__device__ __forceinline__ void clear_slots(const Ladder& L, int64_t first, int64_t n) {
  const RowUnits ru(L.dk, L.dv);
  const uint2 z = make_uint2(0u, 0u);
  for (int64_t r = ru.r0; r < n; r += ru.step) {
    const int64_t s = first + r;
    store_unit(L.k + s * L.dk, L.v + s * L.dv, ru.u, ru.ku, z);
  }
  for (int64_t r = threadIdx.x; r < n; r += blockDim.x) put_slot_meta(L, first + r, Meta{0.f, 0, 0, 0, 0, 0});
}


constexpr int kCarryThreads = 256;   // block size of the carries launches

// Saturated top level: slot 0 <- left fold of P[0..mr] (bf16 after every
// merge), slots 1..B'-1 <- P[mr+1..]. The fold is sequential in its rows and
// parallel in its features: wave 0 holds two 8-byte units of every lane,
// prefetches 8 rows ahead and reads row weights from the lane that loaded
// them. The folded metadata is an order-free reduction except for the mass,
// which follows the fold's left-to-right sums: lo / hi are the min / max over
// rows of positive mass (the last row's if none), sum(w*p) the sum, order the
// min and the pad flag the AND (merge_meta applied left to right).
__device__ __forceinline__ int64_t shfl_xor64(int64_t x, int mask) {
  const int lo = __shfl_xor(static_cast<int>(x), mask, kWave);
  const int hi = __shfl_xor(static_cast<int>(x >> 32), mask, kWave);
  return (static_cast<int64_t>(hi) << 32) | static_cast<uint32_t>(lo);
}

constexpr int kFoldAhead = 8;   // rows of the top fold in flight

template <int KIND>
__device__ __forceinline__ void fold_top(const PoolT<KIND> pool, int mr) {
  const Ladder& L = pool.L;
  const int B = L.B, ku = L.dk / 4, units = (L.dk + L.dv) / 4;   // units <= 2 * kWave
  const int64_t base = pool.base;
  uint2 acc0{}, acc1{};
  Meta am{};
  if (wave_id() == 0) {
    const int l = lane_id();
    const int c0 = min(l, units - 1), c1 = min(l + kWave, units - 1);
    acc0 = load_unit(pool.k(0), pool.v(0), c0, ku);
    acc1 = load_unit(pool.k(0), pool.v(0), c1, ku);
    float mass = pool.w(0);
    for (int t0 = 1; t0 <= mr; t0 += kWave) {
      const int nb = min(kWave, mr + 1 - t0);
      const float wl = pool.w(t0 + min(l, nb - 1));
      for (int i0 = 0; i0 < nb; i0 += kFoldAhead) {
        uint2 x0[kFoldAhead], x1[kFoldAhead];
#pragma unroll
        for (int q = 0; q < kFoldAhead; ++q) {
          const int t = t0 + min(i0 + q, nb - 1);
          x0[q] = load_unit(pool.k(t), pool.v(t), c0, ku);
          x1[q] = load_unit(pool.k(t), pool.v(t), c1, ku);
        }
#pragma unroll
        for (int q = 0; q < kFoldAhead; ++q) {
          if (i0 + q < nb) {
            const float bw = __shfl(wl, i0 + q, kWave);
            const float alpha = mass / fmaxf(mass + bw, 1e-8f);
            acc0 = blend_unit(acc0, x0[q], alpha);
            acc1 = blend_unit(acc1, x1[q], alpha);
            mass = mass + bw;
          }
        }
      }
    }
    // Metadata of rows 0..mr, lane l taking rows l, l + 64, ...
    bool real = false;
    int64_t lo = INT64_MAX, hi = INT64_MIN, swp = 0, ord = INT64_MAX;
    int pad = 1;
    for (int t = l; t <= mr; t += kWave) {
      const Meta m = pool.meta(t);
      const bool rt = m.w > 0.f;
      real = real || rt;
      lo = rt ? imin64(lo, m.lo) : lo;
      hi = rt ? imax64(hi, m.hi) : hi;
      swp += m.swp;
      ord = imin64(ord, m.ord);
      pad &= m.pad;
    }
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      lo = imin64(lo, shfl_xor64(lo, d));
      hi = imax64(hi, shfl_xor64(hi, d));
      swp += shfl_xor64(swp, d);
      ord = imin64(ord, shfl_xor64(ord, d));
      pad &= __shfl_xor(pad, d, kWave);
    }
    const bool any_real = __any(real);
    const Meta last = pool.meta(mr);
    am = Meta{mass, any_real ? lo : last.lo, any_real ? hi : last.hi, swp, ord, static_cast<uint8_t>(pad)};
  }
  move_rows(pool, mr + 1, 1, B - 1);
  if (wave_id() == 0) {
    const int l = lane_id();
    if (l < units) store_unit(L.k + base * L.dk, L.v + base * L.dv, l, ku, acc0);
    if (l + kWave < units) store_unit(L.k + base * L.dk, L.v + base * L.dv, l + kWave, ku, acc1);
    if (l == 0) put_slot_meta(L, base, am);
  }
}

// ---- Flat carry work ---------------------------------------------------------
//
// A carries launch spreads one level's carry work over every wave of the GPU:
// a unit is one Beta group of four pair rows (two outputs) or one pair carry,
// units are numbered ladder after ladder (prefix sums over ladders), and each
// wave takes units by a grid stride. A unit's rows are loaded by its wave
// directly, every load issued before its arithmetic.

// One Beta group (litgpt/beta_log_kv.py:29-105): rows [4 gi, 4 gi + width) of
// the level's pool into outputs 2 gi, 2 gi + 1. Features l + 64 j (j < NJ) of
// every row live in lane l; lane i < 4 also holds row i's metadata. The whole
// wave must be active.
template <int NJ, int KIND>
__device__ __forceinline__ void beta_group(const PoolT<KIND>& pool, const Soa& out, int n_pair, int gi, int dk,
                                           int dv) {
  const int l = lane_id();
  const int start = 4 * gi;
  const int width = min(4, n_pair - start);
  float xk[4][NJ], xv[4][NJ], wr[4];
  const Meta ml = pool.meta(l < width ? start + l : start);
  const Meta mine = l < width ? ml : Meta{};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool valid = i < width;
    const int p = valid ? start + i : start;
    const float wp = pool.w(p);
    wr[i] = valid ? wp : 0.f;
    const LOGKV_G uint16_t* kr = pool.k(p);
    const LOGKV_G uint16_t* vr = pool.v(p);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = l + j * kWave;
      const float a = feat_or_zero(kr, d, dk), b = feat_or_zero(vr, d, dv);
      xk[i][j] = valid ? a : 0.f;
      xv[i][j] = valid ? b : 0.f;
    }
  }
  // Side reciprocals of the cuts (2, 1, 3); a 2-row tail group (rows 2, 3 of
  // weight 0) is the left side of cut 2.
  double rcp[6];
  side_rcps(wr, rcp);
  const int cut = width == 4 ? beta_cut<NJ>(xk, xv, wr, rcp) : 2;
  const int opt = cut == 2 ? 0 : (cut == 1 ? 1 : 2);
  const int dest = start / 2;
  for (int side = 0; side < (width == 4 ? 2 : 1); ++side) {
    const unsigned member = side == 0 ? ((1u << cut) - 1u) : (0xfu & ~((1u << cut) - 1u));
    float wt[4], mk[NJ], mv[NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i) wt[i] = ((member >> i) & 1u) ? wr[i] : 0.f;
    const float mass = side_mass(wt);
    const RowProducts<NJ> pk(xk, wr), pv(xv, wr);
    // Selected without indexing the array by a run-time value (which would place it in scratch).
    const double left = opt == 0 ? rcp[0] : (opt == 1 ? rcp[2] : rcp[4]);
    const double right = opt == 0 ? rcp[1] : (opt == 1 ? rcp[3] : rcp[5]);
    const double side_rcp = side == 0 ? left : right;
    side_mean<NJ>(pk, member, side_rcp, mk);
    side_mean<NJ>(pv, member, side_rcp, mv);
    const int64_t o = dest + side;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = l + j * kWave;
      if (d < dk) out.k[o * dk + d] = f32_to_bf16(mk[j]);
      if (d < dv) out.v[o * dv + d] = f32_to_bf16(mv[j]);
    }
    const bool in_side = l < width && ((member >> (l & 3)) & 1u);
    const Meta r = side_meta(mine, in_side, mass);
    if (l == 0) put_soa_meta(out, o, r);
  }
}

// One pair carry j (pool rows 2j, 2j + 1), one wave.
template <int KIND>
__device__ __forceinline__ void pair_carry(const PoolT<KIND>& pool, const Soa& out, int j, int dk, int dv) {
  const int ku = dk / 4, units = (dk + dv) / 4;
  const float wa = pool.w(2 * j), wb = pool.w(2 * j + 1);
  const float alpha = wa / fmaxf(wa + wb, 1e-8f);
  const LOGKV_G uint16_t *ak = pool.k(2 * j), *av = pool.v(2 * j), *bk = pool.k(2 * j + 1), *bv = pool.v(2 * j + 1);
  for (int u = lane_id(); u < units; u += kWave)
    store_unit(out.k + static_cast<int64_t>(j) * dk, out.v + static_cast<int64_t>(j) * dv, u, ku,
               blend_unit(load_unit(ak, av, u, ku), load_unit(bk, bv, u, ku), alpha));
  if (lane_id() == 0) put_soa_meta(out, j, merge_meta(pool.meta(2 * j), pool.meta(2 * j + 1)));
}

// One level of a Fenwick append. With the virtual pool P = [stored 0..cnt |
// staged 0..m] of n_pool = cnt + m rows:
//  * n_pool <= B': the staged rows fill slots [cnt, n_pool);
//  * otherwise, below the top: the oldest n_pair = 2*ceil((n_pool-B')/2) rows
//    pair into carries, P[n_pair..) moves to slots [0, n_surv), the rest clears;
//  * at the top: slot 0 = left fold of P[0..mr] (bf16 after every merge) and
//    slots 1..B'-1 = P[mr+1..n_pool), mr = n_pool - B'.
// The carries are computed by the level's carries launch (spread over the
// grid); the slot writes (fill, move, clear, fold) by one block in the finish
// launch, after every carry of every level has read the stored slots.
__host__ __device__ inline int carries_of(int cnt, int m, int B, bool top) {
  const int n_pool = cnt + m;
  if (m == 0 || n_pool <= B || top) return 0;
  return (n_pool - B + 1) / 2;
}

// Slot writes of one level step; returns the level's new count.
template <int KIND, bool TOP>
__device__ __forceinline__ int level_finish(const Ladder& L, int ell, int cnt, const Src& cur, int m) {
  const int B = L.B;
  const int64_t base = static_cast<int64_t>(ell) * B;
  const int n_pool = cnt + m;
  const PoolT<KIND> pool{L, base, cnt, cur};
  if (n_pool <= B) {
    copy_staged<KIND>(L, base, cur, 0, cnt, m);
    return n_pool;
  }
  const int mr = n_pool - B;
  if (TOP) {
    fold_top<KIND>(pool, mr);
    return B;
  }
  const int n_pair = 2 * ((mr + 1) / 2);
  const int n_surv = n_pool - n_pair;   // >= B' - 1 >= 1, so move_rows always runs its barrier
  move_rows<KIND>(pool, n_pair, 0, n_surv);
  clear_slots(L, base + n_surv, B - n_surv);
  return n_surv;
}

}  // namespace


// Carries of level l (at most ceil(m0 / 2^(l+1)): level l stages at most
// ceil(m0 / 2^l) rows) get a buffer of their own, so every level's slot
// writes can run after all carries, in one launch.
__host__ __device__ inline int64_t carry_cap(int64_t m0, int ell) {
  return ((m0 + (int64_t(1) << (ell + 1)) - 1) >> (ell + 1)) + 1;
}

int64_t ladder_scratch_bytes(const LadderArgs& c, int64_t s0, int64_t m0) {
  int64_t bytes = soa_bytes(s0, c.dk, c.dv);
  for (int ell = 0; ell + 1 < c.levels; ++ell) bytes += soa_bytes(carry_cap(m0, ell), c.dk, c.dv);
  return bytes;
}

namespace {

__device__ inline Soa s0_of(const Workspace& ws, int ladder, int dk, int dv) {
  return soa_at(ws.ladder + ladder * ws.ladder_stride, ws.s0_rows, dk, dv);
}

__device__ inline Soa carry_of(const Workspace& ws, int ladder, int ell, int dk, int dv) {
  int64_t off = soa_bytes(ws.s0_rows, dk, dv);
  for (int e = 0; e < ell; ++e) off += soa_bytes(carry_cap(ws.m0_cap, e), dk, dv);
  return soa_at(ws.ladder + ladder * ws.ladder_stride + off, carry_cap(ws.m0_cap, ell), dk, dv);
}

// Staged rows of level ell: S0 (delayed archive) at level 0, else level ell - 1's carries.
__device__ inline Src staged_of(const Workspace& ws, int ladder, int ell, int dk, int dv) {
  Src s{};
  s.kind = 1;
  s.buf = ell == 0 ? s0_of(ws, ladder, dk, dv) : carry_of(ws, ladder, ell - 1, dk, dv);
  return s;
}

// The ladder's flush rows as a level-0 source; the tok list is copied to LDS.
__device__ inline Src flush_rows_of(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, const LadderPlan* pl,
                                    int ladder, uint16_t* tok) {
  const int lane_ix = ladder / c.k_max;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  const LOGKV_G uint16_t* src = gp(ws.tok + static_cast<int64_t>(ladder) * r.tokens);
  stage_copy<uint16_t>(tok, src, pl->m_tok, threadIdx.x, blockDim.x);
  __syncthreads();
  Src s{};
  s.kind = 0;
  s.tok = (const LOGKV_S uint16_t*)tok + pl->first;
  s.order_base = pl->order_base;
  s.kb = gp(r.k + b * r.k_sb + g * r.k_sg);
  s.vb = gp(r.v + b * r.v_sb + g * r.v_sg);
  s.k_st = r.k_st;
  s.v_st = r.v_st;
  s.posb = gp(r.pos + b * r.pos_sb);
  return s;
}

__device__ inline Ladder ladder_of(const LadderArgs& c, int ladder) {
  const int64_t row0 = static_cast<int64_t>(ladder) * c.levels * c.slots;
  return Ladder{gp(c.level_k + row0 * c.dk), gp(c.level_v + row0 * c.dv), gp(c.level_w + row0),
                gp(c.level_p_lo + row0), gp(c.level_p_hi + row0), gp(c.level_sum_wp + row0),
                gp(c.level_order + row0), gp(c.pad_mask + row0), c.dk, c.dv, c.slots};
}

}  // namespace

constexpr int kBucketThreads = 1024;

// Each lane's flush rows bucketed by cluster, stably in position order: one
// block per lane, 1024 positions at a time, one ballot per cluster and wave.
// Cluster cc's rows (indices into the flush) go to the ladder's row list
// ws.tok[(lane K + cc) T ..] and their count to plans[lane K + cc].m_tok, which
// commit_kernel reads.
__global__ __launch_bounds__(kBucketThreads) void bucket_kernel(LadderArgs c, RowsArgs r, Workspace ws) {
  __shared__ int wave_cnt[kBucketThreads / kWave][kMaxClusters];
  __shared__ int base_s[kMaxClusters];
  const int K = c.k_max, T = r.tokens;
  const int lane_ix = blockIdx.x, b = lane_ix / c.n_groups;
  const int n = valid_rows(r, b);
  const int tid = static_cast<int>(threadIdx.x), l = lane_id(), w = wave_id();
  const LOGKV_G int8_t* as = gp(ws.assign + static_cast<int64_t>(lane_ix) * T);
  const LOGKV_G int32_t* ord = gp(ws.order + static_cast<int64_t>(b) * T);
  LOGKV_G uint16_t* tok = gp(ws.tok + static_cast<int64_t>(lane_ix) * K * T);
  if (tid < K) base_s[tid] = 0;
  __syncthreads();
  const uint64_t below = l == 0 ? 0ull : (~0ull >> (kWave - l));
  for (int g0 = 0; g0 < n; g0 += kBucketThreads) {
    const int s = g0 + tid;
    const int a = s < n ? as[s] : -1;
    const int o = s < n ? ord[s] : 0;
    int before = 0;
    for (int cc = 0; cc < K; ++cc) {
      const uint64_t bal = __ballot(a == cc);
      if (a == cc) before = __popcll(bal & below);
      if (l == 0) wave_cnt[w][cc] = __popcll(bal);
    }
    __syncthreads();
    if (a >= 0 && a < K) {
      int off = base_s[a] + before;
      for (int q = 0; q < w; ++q) off += wave_cnt[q][a];
      tok[static_cast<int64_t>(a) * T + off] = static_cast<uint16_t>(o);
    }
    __syncthreads();
    if (tid < K) {
      int add = 0;
      for (int q = 0; q < kBucketThreads / kWave; ++q) add += wave_cnt[q][tid];
      base_s[tid] += add;
    }
    __syncthreads();
  }
  if (tid < K) {
    const int64_t cl = static_cast<int64_t>(lane_ix) * K + tid;
    ws.plans[cl].m_tok = base_s[tid];
    // The alive flags as they were before the flush (the commit launches read
    // this snapshot; the op-log record keeps it).
    ws.snap_alive[cl] = c.alive[cl] ? 1 : 0;
  }
}

// Center updates of the commit: mu <- (pre*mu + sum k) / (pre + n), pre =
// n_eff, the new rows' keys summed in position order
// (litgpt/log_kv_cache.py:4344-4359), one at a time (a left fold) or in tiles
// of kCenterTile rows from the first new row, each tile summed by a halving
// tree with zeros past the last row and the tiles folded in order
// (prm.center_tile, the centroid backend); a new cluster starts from its first
// row's key with n_eff = 1 (litgpt/log_kv_cache.py:2276-2278).
//
// Every feature is its own fold, so a ladder takes two waves and a lane folds
// features 64 w + l + 128 j. The ladder's row list is staged in LDS; rows come
// in batches of kCenterTile whose loads are issued a batch ahead of the fold
// (two register sets), since one cluster can hold most of a flush's rows. Runs
// on a side stream beside the commit and level launches, which neither read
// the centers nor write what this launch reads (the row lists, m_tok and the
// alive snapshot are bucket_kernel's); the caller's stream waits for it.
constexpr int kCenterWaves = 2;

template <int NJ>
__device__ __forceinline__ void center_batch_load(const LOGKV_G uint16_t* kb, const uint16_t* tok, int64_t k_st,
                                                  int r0, int m, int f0, int dk, float (&x)[kCenterTile][NJ]) {
#pragma unroll
  for (int q = 0; q < kCenterTile; ++q) {
    const int64_t base = static_cast<int64_t>(tok[min(r0 + q, m - 1)]) * k_st;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int f = f0 + 2 * kWave * j;
      x[q][j] = bf16_to_f32(kb[base + (f < dk ? f : 0)]);
    }
  }
}

// Folds one batch (rows r0 .. r0 + rows - 1) into acc: a left fold, or a tile's
// halving tree (zeros past the last row) added to acc. `start`: the batch
// begins the sum.
template <int NJ>
__device__ __forceinline__ void center_batch_fold(float (&x)[kCenterTile][NJ], int rows, bool start, bool tiles,
                                                  float (&acc)[NJ]) {
  if (tiles) {
#pragma unroll
    for (int q = 0; q < kCenterTile; ++q)
#pragma unroll
      for (int j = 0; j < NJ; ++j) x[q][j] = q < rows ? x[q][j] : 0.f;
#pragma unroll
    for (int h = kCenterTile / 2; h >= 1; h /= 2)
#pragma unroll
      for (int q = 0; q < h; ++q)
#pragma unroll
        for (int j = 0; j < NJ; ++j) x[q][j] = x[q][j] + x[q + h][j];
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] = start ? x[0][j] : acc[j] + x[0][j];
  } else {
#pragma unroll
    for (int q = 0; q < kCenterTile; ++q)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (q < rows) acc[j] = (start && q == 0) ? x[q][j] : acc[j] + x[q][j];
  }
}

// One ladder's center update by a block of at least kCenterWaves waves (the
// others leave once the row list is staged in `ctok`, 2 * T bytes of LDS).
template <int NJ>
__device__ __forceinline__ void center_block(const LadderArgs& c, const RowsArgs& r, const RouteParams& prm,
                                             const Workspace& ws, int ladder, uint16_t* ctok) {
  if (ws.abort && *ws.abort) return;   // a failed replay check: nothing written
  const int m = ws.plans[ladder].m_tok;
  if (m == 0) return;
  const int K = c.k_max, dk = c.dk;
  const int lane_ix = ladder / K;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  const int64_t cl = ladder;
  const bool was_alive = ws.snap_alive[cl] != 0;   // the top-level finish may rewrite `alive` meanwhile
  const int first = was_alive ? 0 : 1;            // a dead cluster opens with its earliest row
  const int nn = m - first;
  {
    const LOGKV_G uint16_t* list = gp(ws.tok + cl * r.tokens);
    stage_copy<uint16_t>(ctok, list, m, threadIdx.x, blockDim.x);
  }
  __syncthreads();
  if (wave_id() >= kCenterWaves) return;
  const LOGKV_G uint16_t* kb = gp(r.k + b * r.k_sb + g * r.k_sg);
  LOGKV_G float* mu = gp(c.centroid + cl * dk);
  const int f0 = wave_id() * kWave + lane_id();
  float n_eff = was_alive ? c.n_eff[cl] : 1.0f;
  float mu_d[NJ];
  {
    const int64_t t0 = static_cast<int64_t>(ctok[0]) * r.k_st;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int f = f0 + 2 * kWave * j;
      mu_d[j] = 0.f;
      if (f < dk) mu_d[j] = was_alive ? mu[f] : bf16_to_f32(kb[t0 + f]);
    }
  }
  if (nn > 0) {
    const bool tiles = prm.center_tile == kCenterTile;
    float acc[NJ], xa[kCenterTile][NJ], xb[kCenterTile][NJ];
    center_batch_load<NJ>(kb, ctok, r.k_st, first, m, f0, dk, xa);
    for (int r0 = first; r0 < m; r0 += 2 * kCenterTile) {
      const int r1 = r0 + kCenterTile;
      if (r1 < m) center_batch_load<NJ>(kb, ctok, r.k_st, r1, m, f0, dk, xb);
      center_batch_fold<NJ>(xa, min(kCenterTile, m - r0), r0 == first, tiles, acc);
      if (r1 >= m) break;
      const int r2 = r1 + kCenterTile;
      if (r2 < m) center_batch_load<NJ>(kb, ctok, r.k_st, r2, m, f0, dk, xa);
      center_batch_fold<NJ>(xb, min(kCenterTile, m - r1), false, tiles, acc);
    }
    const float pre = n_eff;
    const float den = pre + static_cast<float>(nn);
#pragma unroll
    for (int j = 0; j < NJ; ++j) mu_d[j] = pre > 0.f ? (pre * mu_d[j] + acc[j]) / den : acc[j] / static_cast<float>(nn);
    n_eff = den;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int f = f0 + 2 * kWave * j;
    if (f < dk) mu[f] = mu_d[j];
  }
  if (threadIdx.x == 0) c.n_eff[cl] = n_eff;
}

template <int NJ>
__global__ __launch_bounds__(kCenterWaves* kWave) void center_kernel(LadderArgs c, RowsArgs r, RouteParams prm,
                                                                    Workspace ws) {
  extern __shared__ __align__(16) uint16_t ctok[];
  center_block<NJ>(c, r, prm, ws, static_cast<int>(blockIdx.x), ctok);
}

// The ladder plans of the commit (y = 0) and, when the call has no side stream
// for center_kernel and keys of at most 128 features, the center updates
// beside them (y = 1, CENTERS).
template <bool CENTERS>
__global__ __launch_bounds__(kThreads) void commit_kernel(LadderArgs c, RowsArgs r, RouteParams prm, Workspace ws) {
  extern __shared__ __align__(16) uint8_t dyn[];
  __shared__ int16_t counts_s[64];
  __shared__ int level_start_s[64];
  const int K = c.k_max, L = c.levels, B = c.slots, dk = c.dk, dv = c.dv;
  const int ladder = blockIdx.x;
  const int lane_ix = ladder / K;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  uint16_t* tok = reinterpret_cast<uint16_t*>(dyn);
  const int keys_off = (2 * r.tokens + 15) & ~15;
  if constexpr (CENTERS) {
    if (blockIdx.y == 1) {   // keys of at most 128 features
      center_block<1>(c, r, prm, ws, ladder, tok);
      return;
    }
  }

  if (ws.abort && *ws.abort) {
    // A failed replay check: no rows, nothing written (the later launches read the plan).
    if (threadIdx.x == 0) {
      ws.plans[ladder].active = 0;
      ws.plans[ladder].m_tok = 0;
    }
    return;
  }

  // 1. This cluster's rows in position order, bucketed by bucket_kernel.
  const int m = ws.plans[ladder].m_tok;
  {
    const LOGKV_G uint16_t* list = gp(ws.tok + static_cast<int64_t>(ladder) * r.tokens);
    stage_copy<uint16_t>(tok, list, m, threadIdx.x, kThreads);
  }
  __syncthreads();
  if (m == 0) {
    if (threadIdx.x == 0) ws.plans[ladder].active = 0;   // m_tok is already 0
    return;
  }

  const int64_t cl = ladder;   // lane_ix * K + cluster
  const int64_t row0 = cl * L * B;
  Ladder lad{gp(c.level_k + row0 * dk), gp(c.level_v + row0 * dv), gp(c.level_w + row0), gp(c.level_p_lo + row0),
             gp(c.level_p_hi + row0), gp(c.level_sum_wp + row0), gp(c.level_order + row0), gp(c.pad_mask + row0),
             dk, dv, B};
  const LOGKV_G uint16_t* kb = gp(r.k + b * r.k_sb + g * r.k_sg);
  const LOGKV_G uint16_t* vb = gp(r.v + b * r.v_sb + g * r.v_sg);
  const LOGKV_G int64_t* posb = gp(r.pos + b * r.pos_sb);
  const LOGKV_S uint16_t* tok_s = (const LOGKV_S uint16_t*)tok;
  const Soa S0 = s0_of(ws, ladder, dk, dv);

  const bool was_alive = ws.snap_alive[cl] != 0;   // written by bucket_kernel
  const int first = was_alive ? 0 : 1;   // a dead cluster opens with its earliest row
  const int nn = m - first;

  // Ladder role.
  for (int e = threadIdx.x; e < L; e += kThreads) counts_s[e] = c.level_count[cl * L + e];
  int32_t n_total = c.n_total[cl];
  int64_t p_hi = c.p_hi_c[cl];
  int32_t phase = c.level0_phase[cl];
  __syncthreads();

  if (!was_alive) {
    // 2. A dead cluster: clear every slot, its earliest row takes level 0 slot 0.
    clear_slots(lad, 0, static_cast<int64_t>(L) * B);
    for (int e = threadIdx.x; e < L; e += kThreads) counts_s[e] = 0;
    const int t0 = tok[0];
    Src one{};
    one.kind = 0;
    one.tok = tok_s;
    one.order_base = 0;
    one.kb = kb;
    one.vb = vb;
    one.k_st = r.k_st;
    one.v_st = r.v_st;
    one.posb = posb;
    __syncthreads();
    copy_staged<0>(lad, 0, one, 0, 0, 1);
    if (threadIdx.x == 0) counts_s[0] = 1;
    __syncthreads();
    n_total = 1;
    p_hi = posb[t0];
    phase = 1;
  }
  int kind0 = 0, m0 = 0;
  int64_t order_base = 0;
  if (nn > 0) {
    const int64_t first_pos = posb[tok[first]];
    const bool late = prm.late_joins && first_pos < p_hi;
    const int64_t last_pos = posb[tok[m - 1]];
    m0 = nn;
    if (!late) {
      order_base = phase;
      phase += nn;
      p_hi = last_pos;
    } else {
      // 4. Delayed archive: existing entries (level by level, slots in order)
      //    and the new rows, stably sorted by p_lo (key = p_lo << 13 | index),
      //    gathered into S0 in that order with order = rank, re-appended from
      //    level 0 of the cleared ladder.
      int n_exist = 0;
      int* level_start = level_start_s;
      for (int e = 0; e < L; ++e) n_exist += counts_s[e];
      if (threadIdx.x == 0) {
        int acc = 0;
        for (int e = 0; e < L; ++e) {
          level_start[e] = acc;
          acc += counts_s[e];
        }
      }
      __syncthreads();
      uint64_t* keys = reinterpret_cast<uint64_t*>(dyn + keys_off);
      const int total = n_exist + nn;
      int width = 1;
      while (width < total) width <<= 1;
      for (int i = threadIdx.x; i < width; i += kThreads) {
        uint64_t key = ~0ull;
        if (i < n_exist) {
          int e = 0;
          while (e + 1 < L && level_start[e + 1] <= i) ++e;
          const int64_t slot = static_cast<int64_t>(e) * B + (i - level_start[e]);
          key = (static_cast<uint64_t>(lad.lo[slot]) << kOrderIndexBits) | static_cast<uint64_t>(i);
        } else if (i < total) {
          key = (static_cast<uint64_t>(posb[tok[first + i - n_exist]]) << kOrderIndexBits) | static_cast<uint64_t>(i);
        }
        keys[i] = key;
      }
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
      // Gather row rank -> S0[rank], kBatch rows per thread loaded before any store.
      {
        const RowUnits ru(dk, dv);
        for (int r0 = ru.r0; r0 < total; r0 += kBatch * ru.step) {
          uint2 x[kBatch];
#pragma unroll
          for (int qb = 0; qb < kBatch; ++qb) {
            // Addresses by selects and an unconditional load (a rank past the
            // end re-reads the last one), so all kBatch loads are in flight.
            const int rank = min(r0 + qb * ru.step, total - 1);
            const int q = static_cast<int>(keys[rank] & kOrderIndexMask);
            const bool ex = q < n_exist;
            int e = 0;
            while (e + 1 < L && level_start[e + 1] <= q) ++e;
            const int64_t slot = static_cast<int64_t>(e) * B + (q - level_start[e]);
            const int t = tok[first + max(q - n_exist, 0)];   // the flush rows start at tok[first]
            const LOGKV_G uint16_t* ks = ex ? lad.k + slot * dk : kb + static_cast<int64_t>(t) * r.k_st;
            const LOGKV_G uint16_t* vs = ex ? lad.v + slot * dv : vb + static_cast<int64_t>(t) * r.v_st;
            x[qb] = load_unit(ks, vs, ru.u, ru.ku);
          }
#pragma unroll
          for (int qb = 0; qb < kBatch; ++qb) {
            const int rank = r0 + qb * ru.step;
            if (rank < total)
              store_unit(S0.k + static_cast<int64_t>(rank) * dk, S0.v + static_cast<int64_t>(rank) * dv, ru.u, ru.ku,
                         x[qb]);
          }
        }
      }
      for (int rank = threadIdx.x; rank < total; rank += kThreads) {
        const int q = static_cast<int>(keys[rank] & kOrderIndexMask);
        Meta mt;
        if (q < n_exist) {
          int e = 0;
          while (e + 1 < L && level_start[e + 1] <= q) ++e;
          mt = slot_meta(lad, static_cast<int64_t>(e) * B + (q - level_start[e]));
        } else {
          const int64_t p = posb[tok[first + q - n_exist]];
          mt = Meta{1.0f, p, p, p, 0, 0};
        }
        mt.ord = rank;
        put_soa_meta(S0, rank, mt);
      }
      p_hi = imax64(p_hi, last_pos);   // rows are in position order
      phase = total;
      __syncthreads();
      clear_slots(lad, 0, static_cast<int64_t>(L) * B);
      for (int e = threadIdx.x; e < L; e += kThreads) counts_s[e] = 0;
      __syncthreads();
      kind0 = 1;
      m0 = total;
    }
    n_total += nn;
  }
  // Hand-off to the level launches (the rows in position order are already in
  // ws.tok): the counts before the append (the level launches rewrite the
  // levels they touch) and the per-level plan of the cascade.
  __syncthreads();
  for (int e = threadIdx.x; e < L; e += kThreads) c.level_count[cl * L + e] = counts_s[e];
  if (threadIdx.x == 0) {
    LadderPlan pl;
    pl.active = nn > 0 ? 1 : 0;
    pl.kind0 = kind0;
    pl.first = first;
    pl.order_base = order_base;
    int mm = m0;
    for (int e = 0; e < kMaxLevels; ++e) {
      const bool used = e < L;
      pl.cnt[e] = used ? counts_s[e] : 0;
      pl.m[e] = used ? mm : 0;
      mm = used ? carries_of(counts_s[e], mm, B, e == L - 1) : 0;
    }
    // Every field but m_tok (bucket_kernel's count, which the center launch
    // may be reading concurrently).
    LadderPlan* dst = ws.plans + ladder;
    dst->active = pl.active;
    dst->kind0 = pl.kind0;
    dst->first = pl.first;
    dst->order_base = pl.order_base;
    for (int e = 0; e < kMaxLevels; ++e) {
      dst->cnt[e] = pl.cnt[e];
      dst->m[e] = pl.m[e];
    }
    c.n_total[cl] = n_total;
    c.p_hi_c[cl] = p_hi;
    c.level0_phase[cl] = phase;
  }
}

// Carry work of every level: block ell writes units[ell][i] = work units of
// ladders 0..i-1 at level ell (a unit is one Beta group of two carries, or one
// pair carry), i = 0..ladders.
constexpr int kUnitsThreads = 1024;
constexpr int kUnitsPer = kMaxLadders / kUnitsThreads;   // consecutive ladders per thread at most

// One block per level: thread t owns ladders [t per, (t + 1) per) (per = the
// ladder count over 1024, rounded up), loads all their plans first, then one
// block scan of the threads' totals gives every prefix.
__global__ __launch_bounds__(kUnitsThreads) void units_kernel(LadderArgs c, RouteParams prm, Workspace ws) {
  __shared__ int wave_total[kUnitsThreads / kWave];
  const int ell = blockIdx.x;
  const int ladders = c.n_batch * c.n_groups * c.k_max;
  const int per = (ladders + kUnitsThreads - 1) / kUnitsThreads;
  int32_t* out = ws.units + static_cast<int64_t>(ell) * (ladders + 1);
  const int l = lane_id(), w = wave_id();
  const int i0 = static_cast<int>(threadIdx.x) * per;
  int n[kUnitsPer];
  int mine = 0;
#pragma unroll
  for (int q = 0; q < kUnitsPer; ++q) {
    n[q] = 0;
    const int i = i0 + q;
    if (q < per && i < ladders) {
      const LadderPlan* pl = ws.plans + i;
      const int nc = pl->active ? carries_of(pl->cnt[ell], pl->m[ell], c.slots, ell == c.levels - 1) : 0;
      n[q] = prm.beta_merge ? (nc + 1) / 2 : nc;
    }
    mine += n[q];
  }
  int incl = mine;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int t = __shfl_up(incl, d, kWave);
    if (l >= d) incl += t;
  }
  if (l == kWave - 1) wave_total[w] = incl;
  __syncthreads();
  int acc = incl - mine;
  for (int q = 0; q < w; ++q) acc += wave_total[q];
  if (threadIdx.x == 0) out[0] = 0;
#pragma unroll
  for (int q = 0; q < kUnitsPer; ++q) {
    const int i = i0 + q;
    if (q < per && i < ladders) {
      acc += n[q];
      out[i + 1] = acc;
    }
  }
}

// The ladder's flush rows as a level-0 source, row list read from global memory.
__device__ inline Src flush_rows_global(const LadderArgs& c, const RowsArgs& r, const Workspace& ws,
                                        const LadderPlan* pl, int ladder) {
  const int lane_ix = ladder / c.k_max;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  Src s{};
  s.kind = 2;
  s.gtok = gp(ws.tok + static_cast<int64_t>(ladder) * r.tokens + pl->first);
  s.order_base = pl->order_base;
  s.kb = gp(r.k + b * r.k_sb + g * r.k_sg);
  s.vb = gp(r.v + b * r.v_sb + g * r.v_sg);
  s.k_st = r.k_st;
  s.v_st = r.v_st;
  s.posb = gp(r.pos + b * r.pos_sb);
  return s;
}

// Units [u, u_end) of one ladder at level ell (lu = u - first unit of the ladder).
template <int NJ, int KIND>
__device__ __forceinline__ void ladder_units(const PoolT<KIND>& pool, const Soa& out, int n_carry, bool beta, int lu0,
                                             int lu1, int dk, int dv) {
  for (int lu = lu0; lu < lu1; ++lu) {
    if (beta) beta_group<NJ, KIND>(pool, out, 2 * n_carry, lu, dk, dv);
    else pair_carry<KIND>(pool, out, lu, dk, dv);
  }
}

// ---------------------------------------------------------------------------
// Beta carries four groups to a wave. A 16-lane row of the wave takes one Beta
// group; lane l of the row holds features l + 16 k (k < 4 NJ) of the group's
// rows. That places leaves l, l + 16, l + 32, l + 48 of the 64-leaf canonical
// order in the lane (leaf a of the lane sums features l + 16 a + 64 j over j in
// order), so the first two tree levels add inside the lane and the last four
// (partners 8, 4, 2, 1 lanes away) are row rotations: every lane of the row
// ends with the canonical sum, and each float operation of beta_group (the
// cut costs, the side means, the outputs) is evaluated on the same operands
// in the same order. Row-level scalars (side reciprocals, energies, the 12
// cost quotients) are computed lane-parallel inside the row and exchanged by
// lane permutes.

template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}

// Value of lane `k` of this lane's 16-lane row.
__device__ __forceinline__ float row_lane(float x, int k) {
  return __int_as_float(__shfl(__float_as_int(x), (lane_id() & ~15) + k, kWave));
}
__device__ __forceinline__ int row_lane_i(int x, int k) { return __shfl(x, (lane_id() & ~15) + k, kWave); }
__device__ __forceinline__ double row_lane_d(double x, int k) {
  const long long b = __double_as_longlong(x);
  const int lo = __shfl(static_cast<int>(b), (lane_id() & ~15) + k, kWave);
  const int hi = __shfl(static_cast<int>(b >> 32), (lane_id() & ~15) + k, kWave);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<uint32_t>(lo));
}

// Features l16 + 16 k of one bf16 row (0 past D): one base address per row and
// compile-time offsets; a lane past the row's end loads nothing.
template <int F>
__device__ __forceinline__ void load_row16(const LOGKV_G uint16_t* row, int l16, int D, bool valid, float (&x)[F]) {
  const LOGKV_G uint16_t* at = row + l16;
#pragma unroll
  for (int k = 0; k < F; ++k) {
    float a = 0.f;
    if (l16 + 16 * k < D) a = bf16_to_f32(at[16 * k]);
    x[k] = valid ? a : 0.f;
  }
}

// beta_component_losses on the row layout. Side sums of the cuts, feature by
// feature: a side's sum in row order is its member rows' products x w with
// the other rows' x * 0 between them; those zero-weight terms are +-0 or NaN,
// and a run of them added to a partial sum gives the same result however the
// run is grouped (NaN if any is NaN, -0 only if the partial sum and every
// term are -0, else the partial sum). So the left side of cut c is the prefix
// p0 + .. + p(c-1) plus the grouped zero-weight terms of rows c..3, and the
// right side the zero-weight prefix of rows 0..c-1 followed by pc, .., p3 in
// order: the term-by-term sums' values from shared partial sums. The
// features are visited leaf by leaf (leaves a and a + 2 of the lane, then
// a + 1 and a + 3), so only the pending level-32 nodes of the 12 (cut, row)
// distance sums stay live between the passes.
template <int NJ>
__device__ __forceinline__ void row_component_losses(const float (&x)[4][4 * NJ], const float* wr, double rl, float& e,
                                                     float* loss) {
  float sq[4];
  {
    float n32[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float lf[2][4];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int a = h + 2 * half;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int k = a + 4 * j;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float v = x[i][k] * x[i][k];
            lf[half][i] = j == 0 ? v : lf[half][i] + v;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) n32[h][i] = lf[0][i] + lf[1][i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s16 = n32[0][i] + n32[1][i];
      s16 = s16 + row_ror<8>(s16);
      s16 = s16 + row_ror<4>(s16);
      s16 = s16 + row_ror<2>(s16);
      sq[i] = s16 + row_ror<1>(s16);
    }
  }
  e = sq[0] * wr[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) e = e + sq[i] * wr[i];
  // The side reciprocals of the cuts (2, 1, 3), left then right, from the
  // row's lanes 0..5.
  double rcp[6];
#pragma unroll
  for (int q = 0; q < 6; ++q) rcp[q] = row_lane_d(rl, q);
  float n32[2][3][4];   // [h][opt][row]
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float lf[2][3][4];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int a = h + 2 * half;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int k = a + 4 * j;
        const float p0 = x[0][k] * wr[0], p1 = x[1][k] * wr[1], p2 = x[2][k] * wr[2], p3 = x[3][k] * wr[3];
        const float z0 = x[0][k] * 0.f, z1 = x[1][k] * 0.f, z2 = x[2][k] * 0.f, z3 = x[3][k] * 0.f;
        const float l2 = p0 + p1, l3 = l2 + p2;            // left prefixes of cuts 2, 3 (cut 1: p0)
        const float s2 = z2 + z3, s1 = z1 + s2;            // zero-weight runs of rows c..3 (cut 3: z3)
        const float zp2 = z0 + z1, zp3 = zp2 + z2;         // zero-weight prefixes of rows 0..c-1
        float mean[3][2];                                  // [opt][side]
        mean[1][0] = div_by_rcp(p0 + s1, rcp[2]);
        mean[0][0] = div_by_rcp(l2 + s2, rcp[0]);
        mean[2][0] = div_by_rcp(l3 + z3, rcp[4]);
        mean[1][1] = div_by_rcp(((z0 + p1) + p2) + p3, rcp[3]);
        mean[0][1] = div_by_rcp((zp2 + p2) + p3, rcp[1]);
        mean[2][1] = div_by_rcp(zp3 + p3, rcp[5]);
#pragma unroll
        for (int opt = 0; opt < 3; ++opt) {
          const int c = opt == 0 ? 2 : (opt == 1 ? 1 : 3);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float d = x[i][k] - mean[opt][i < c ? 0 : 1];
            const float v = d * d;
            lf[half][opt][i] = j == 0 ? v : lf[half][opt][i] + v;
          }
        }
      }
    }
#pragma unroll
    for (int opt = 0; opt < 3; ++opt)
#pragma unroll
      for (int i = 0; i < 4; ++i) n32[h][opt][i] = lf[0][opt][i] + lf[1][opt][i];
  }
#pragma unroll
  for (int opt = 0; opt < 3; ++opt) {
    const int c = opt == 0 ? 2 : (opt == 1 ? 1 : 3);
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s16 = n32[0][opt][i] + n32[1][opt][i];
      s16 = s16 + row_ror<8>(s16);
      s16 = s16 + row_ror<4>(s16);
      s16 = s16 + row_ror<2>(s16);
      t[i] = s16 + row_ror<1>(s16);
    }
    float left = t[0] * (0 < c ? wr[0] : 0.f), right = t[0] * (0 < c ? 0.f : wr[0]);
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      left = left + t[i] * (i < c ? wr[i] : 0.f);
      right = right + t[i] * (i < c ? 0.f : wr[i]);
    }
    loss[2 * opt] = left;
    loss[2 * opt + 1] = right;
  }
}

// Rows of one Beta group as seen by a lane: the pool is per lane (its row's
// ladder), the staged source by kind.
struct GroupRows {
  const LOGKV_G uint16_t* k[4];
  const LOGKV_G uint16_t* v[4];
  float w[4];
};

// Group rows of a flush-sourced pool whose four staged row indices (for rows
// start .. start + 3) were read ahead.
__device__ __forceinline__ void group_rows_at(const PoolT<2>& pool, int start, int width, const uint32_t (&t)[4],
                                              GroupRows& g) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = i < width ? start + i : start;
    const int64_t ti = i < width ? t[i] : t[0];
    g.k[i] = pool.k_at(p, ti);
    g.v[i] = pool.v_at(p, ti);
    const float wp = pool.w(p);
    g.w[i] = i < width ? wp : 0.f;
  }
}

template <int KIND>
__device__ __forceinline__ void group_rows(const PoolT<KIND>& pool, int start, int width, GroupRows& g) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = i < width ? start + i : start;
    g.k[i] = pool.k(p);
    g.v[i] = pool.v(p);
    const float wp = pool.w(p);
    g.w[i] = i < width ? wp : 0.f;
  }
}

// Screened cut decision of a full group (rows in the row layout). The loss of a
// side S is sum_{i<j in S} w_i w_j |x_i - x_j|^2 / m_S (the weighted spread
// about the side's mean), so the three cuts' costs need only the squared
// distances d01, d02, d12, d13, d23 and the four squared norms (the energy):
// 14 operations per feature and component instead of the canonical
// evaluation's ~76, with every term non-negative, so the costs' relative
// error stays a few tens of ulps. `screen_sums` leaves in every lane of the
// row the component's sums [n0, n1, n2, n3, d01, d02, d12, d13, d23], in any
// order (fused multiply-adds).
template <int F>
__device__ __forceinline__ void screen_sums(const float (&x)[4][F], float* s9) {
#pragma unroll
  for (int q = 0; q < 9; ++q) s9[q] = 0.f;
#pragma unroll
  for (int k = 0; k < F; ++k) {
#pragma unroll
    for (int i = 0; i < 4; ++i) s9[i] = __builtin_fmaf(x[i][k], x[i][k], s9[i]);
    const float t01 = x[0][k] - x[1][k], t02 = x[0][k] - x[2][k], t12 = x[1][k] - x[2][k];
    const float t13 = x[1][k] - x[3][k], t23 = x[2][k] - x[3][k];
    s9[4] = __builtin_fmaf(t01, t01, s9[4]);
    s9[5] = __builtin_fmaf(t02, t02, s9[5]);
    s9[6] = __builtin_fmaf(t12, t12, s9[6]);
    s9[7] = __builtin_fmaf(t13, t13, s9[7]);
    s9[8] = __builtin_fmaf(t23, t23, s9[8]);
  }
#pragma unroll
  for (int q = 0; q < 9; ++q) {
    float v = s9[q];
    v = v + row_ror<8>(v);
    v = v + row_ror<4>(v);
    v = v + row_ror<2>(v);
    s9[q] = v + row_ror<1>(v);
  }
}

// Reciprocals a group's screened costs divide by: the total mass and the
// masses of the four sides the cuts (2, 1, 3) form (shared by K and V).
struct ScreenRcp {
  float total, s01, s23, s123, s012;
};

__device__ __forceinline__ ScreenRcp screen_rcp(const float* w, float total) {
  return ScreenRcp{1.0f / total, 1.0f / fmaxf(w[0] + w[1], 1e-12f), 1.0f / fmaxf(w[2] + w[3], 1e-12f),
                   1.0f / fmaxf((w[1] + w[2]) + w[3], 1e-12f), 1.0f / fmaxf((w[0] + w[1]) + w[2], 1e-12f)};
}

// Adds one component's screened costs of the cuts (2, 1, 3) to `cost`; each
// quotient is a product with a rounded reciprocal (one more half ulp).
__device__ __forceinline__ void screen_costs(const float* s9, const float* w, const ScreenRcp& rc, float* cost) {
  const float e = ((s9[0] * w[0] + s9[1] * w[1]) + s9[2] * w[2]) + s9[3] * w[3];
  const float re = 1.0f / fmaxf(e * rc.total, 1e-12f);
  const float p01 = (w[0] * w[1]) * s9[4], p02 = (w[0] * w[2]) * s9[5], p12 = (w[1] * w[2]) * s9[6];
  const float p13 = (w[1] * w[3]) * s9[7], p23 = (w[2] * w[3]) * s9[8];
  const float c2 = p01 * rc.s01 + p23 * rc.s23;
  const float c1 = ((p12 + p13) + p23) * rc.s123;
  const float c3 = ((p01 + p02) + p12) * rc.s012;
  cost[0] += c2 * re;
  cost[1] += c1 * re;
  cost[2] += c3 * re;
}

// The cut the canonical evaluation chooses, when the screened costs settle it:
// its costs and the screen's both err by at most ~95 ulps relative (sums of
// non-negative terms of depth <= 16, a handful of products and quotients; the
// canonical side means' rounding adds at most 25 eps^2 of the side's energy
// per side, covered by the absolute term), so a runner-up more than 2^-13
// relative above the smallest screened cost (and 2^-36 of the group's mass)
// cannot be the canonical minimum. Returns 0 when it is not settled: near ties
// (exact ties, duplicate rows), non-finite costs, masses in (0, 2^-20) whose
// clamped side means the pairwise form does not model.
__device__ __forceinline__ int screened_cut(const float* ck, const float* cv, const float* w, float total) {
  float cost[3] = {0.f, 0.f, 0.f};
  const ScreenRcp rc = screen_rcp(w, total);
  screen_costs(ck, w, rc, cost);
  screen_costs(cv, w, rc, cost);
  int best = 0;
  if (cost[1] < cost[best]) best = 1;
  if (cost[2] < cost[best]) best = 2;
  const float second = fminf(cost[(best + 1) % 3], cost[(best + 2) % 3]);
  bool ok = __builtin_isfinite(cost[0]) && __builtin_isfinite(cost[1]) && __builtin_isfinite(cost[2]) &&
            __builtin_isfinite(total);
#pragma unroll
  for (int i = 0; i < 4; ++i) ok = ok && (w[i] == 0.f || w[i] >= 0x1p-20f);
  ok = ok && second - cost[best] > 0x1p-13f * second + 0x1p-36f * total;
  return ok ? (best == 0 ? 2 : (best == 1 ? 1 : 3)) : 0;
}

// Raw bf16 rows held 8 contiguous features to a lane (lane l16 of the row:
// features 8 l16 .. 8 l16 + 7 of a 128-feature row, two 8-byte loads), the
// layout of the screen and of the outputs, whose sums are order-free.
struct Rows8 {
  uint2 k[4][2], v[4][2];
};

// Rows past the group's width are zeros (their x * 0 terms are +0, as the
// reference's zero-filled rows give); every load is issued, then selected.
__device__ __forceinline__ void load_rows8(const GroupRows& g, int l16, int width, Rows8& x) {
  const uint2 zero = make_uint2(0u, 0u);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const LOGKV_G uint2* pk = reinterpret_cast<const LOGKV_G uint2*>(g.k[i] + 8 * l16);
    const LOGKV_G uint2* pv = reinterpret_cast<const LOGKV_G uint2*>(g.v[i] + 8 * l16);
    const uint2 k0 = pk[0], k1 = pk[1], v0 = pv[0], v1 = pv[1];
    x.k[i][0] = i < width ? k0 : zero;
    x.k[i][1] = i < width ? k1 : zero;
    x.v[i][0] = i < width ? v0 : zero;
    x.v[i][1] = i < width ? v1 : zero;
  }
}

// Feature f (0..7) of a lane's 8 contiguous bf16 features as float.
__device__ __forceinline__ float feat8(const uint2 (&u)[2], int f) {
  const uint32_t w = f < 4 ? (f < 2 ? u[0].x : u[0].y) : (f < 6 ? u[1].x : u[1].y);
  return (f & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
}

__device__ __forceinline__ void screen_sums8(const uint2 (&x)[4][2], float* s9) {
  float f[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) f[i][k] = feat8(x[i], k);
  screen_sums<8>(f, s9);
}

// Two floats to packed bf16, round to nearest even (the hardware conversion;
// f32_to_bf16 agrees on every non-NaN float, and a settled group's means are
// never NaN: its costs are finite, so are its rows and their weighted sums).
__device__ __forceinline__ uint32_t pack_bf16_finite(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// One side's output means of a 128-feature group from the held rows: per
// feature beta_group's row-order sum (member rows x w, the others x * 0) over
// the side's double reciprocal, 8 features to a lane, two 8-byte stores.
__device__ __forceinline__ void side_out8(const uint2 (&x)[4][2], const float* w, unsigned member, double rcp,
                                          LOGKV_G uint16_t* at) {
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float h[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int f = 2 * q + e;
      float acc = (member & 1u) ? feat8(x[0], f) * w[0] : feat8(x[0], f) * 0.f;
#pragma unroll
      for (int i = 1; i < 4; ++i) acc = acc + (((member >> i) & 1u) ? feat8(x[i], f) * w[i] : feat8(x[i], f) * 0.f);
      h[e] = div_by_rcp(acc, rcp);
    }
    o[q] = pack_bf16_finite(h[0], h[1]);
  }
  LOGKV_G uint2* dst = reinterpret_cast<LOGKV_G uint2*>(at);
  dst[0] = make_uint2(o[0], o[1]);
  dst[1] = make_uint2(o[2], o[3]);
}

// One Beta group per 16-lane row: rows [4 gi, 4 gi + width) of the lane's
// ladder pool at level ell into its carries 2 gi, 2 gi + 1 (beta_group's
// arithmetic), rows of fewer than 128 features (lane l holding features
// l + 16 k, masked past the width). `live` false: the row only takes part in
// the row exchanges.
template <int NJ>
__device__ __forceinline__ void beta_row_group(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, int ladder,
                                               int ell, int gi, bool live) {
  constexpr int F = 4 * NJ;
  const int l16 = lane_id() & 15;
  const LadderPlan* pl = ws.plans + ladder;
  const int cnt = pl->cnt[ell], m = pl->m[ell];
  const int n_pair = 2 * carries_of(cnt, m, c.slots, false);
  const int start = 4 * gi;
  const int width = max(0, min(4, n_pair - start));
  const bool flush_src = ell == 0 && pl->kind0 == 0;
  const Ladder lad = ladder_of(c, ladder);
  const int64_t base = static_cast<int64_t>(ell) * c.slots;
  const int dk = c.dk, dv = c.dv;
  GroupRows g;
  if (flush_src) group_rows<2>(PoolT<2>{lad, base, cnt, flush_rows_global(c, r, ws, pl, ladder)}, start, width, g);
  else group_rows<1>(PoolT<1>{lad, base, cnt, staged_of(ws, ladder, ell, dk, dv)}, start, width, g);
  // A full group's cut is evaluated; a partial group is the left side of cut 2.
  int cut = 2;
  const bool settled = width != 4;
  if (__ballot(!settled)) {
    float xk[4][F];
#pragma unroll
    for (int i = 0; i < 4; ++i) load_row16<F>(g.k[i], l16, dk, i < width, xk[i]);
    // Side reciprocals of the cuts (2, 1, 3): lane l16 < 6 of the row divides
    // (left, right of cut 2, of cut 1, of cut 3).
    double rl;
    {
      float mass = 1.f;
#pragma unroll
      for (int opt = 0; opt < 3; ++opt) {
        const int cc = opt == 0 ? 2 : (opt == 1 ? 1 : 3);
        float wl[4], wrt[4];
        cut_weights(g.w, cc, wl, wrt);
        mass = l16 == 2 * opt ? side_mass(wl) : mass;
        mass = l16 == 2 * opt + 1 ? side_mass(wrt) : mass;
      }
      rl = 1.0 / static_cast<double>(fmaxf(mass, 1e-12f));
    }
    {
      float ek, ev, lk[6], lv[6];
      row_component_losses<NJ>(xk, g.w, rl, ek, lk);
      asm volatile("" ::: "memory");   // V's loads after K's costs: one component's rows live at a time
      float xv[4][F];
#pragma unroll
      for (int i = 0; i < 4; ++i) load_row16<F>(g.v[i], l16, dv, i < width, xv[i]);
      row_component_losses<NJ>(xv, g.w, rl, ev, lv);
      // beta_cut's decision: energies and the 12 quotients lane-parallel in the
      // row, the costs summed in lane 0 in beta_cut's order.
      const float total = fmaxf(((g.w[0] + g.w[1]) + g.w[2]) + g.w[3], 1e-12f);
      const float en = (l16 == 0 ? ek : ev) / total;
      const float energy_k = fmaxf(row_lane(en, 0), 1e-12f);
      const float energy_v = fmaxf(row_lane(en, 1), 1e-12f);
      float num = 0.f;
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        num = l16 == k ? lk[k] : num;
        num = l16 == 6 + k ? lv[k] : num;
      }
      const float q = num / (l16 < 6 ? energy_k : energy_v);
      float costs[3] = {0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 12; ++k) costs[(k % 6) / 2] = costs[(k % 6) / 2] + row_lane(q, k);
      int best = 0;
      if (costs[1] < costs[best]) best = 1;
      if (costs[2] < costs[best]) best = 2;
      if (!settled) cut = best == 0 ? 2 : (best == 1 ? 1 : 3);
    }
  }
  // Outputs (beta_group's side means), K then V; the rows are loaded again
  // (the barrier keeps the compiler from holding the first loads live).
  asm volatile("" ::: "memory");
  // The side reciprocals of the chosen cut (lane 0: left, 1: right).
  double rl;
  {
    float wl[4], wrt[4];
    cut_weights(g.w, cut, wl, wrt);
    rl = 1.0 / static_cast<double>(fmaxf(l16 == 0 ? side_mass(wl) : side_mass(wrt), 1e-12f));
  }
  const int dest = start / 2;
  const Soa out = carry_of(ws, ladder, ell, dk, dv);
  const double left_rcp = row_lane_d(rl, 0), right_rcp = row_lane_d(rl, 1);
  const unsigned left_rows = (1u << cut) - 1u;
#pragma unroll
  for (int comp = 0; comp < 2; ++comp) {
    const int D = comp == 0 ? dk : dv;
    float x[4][F];
#pragma unroll
    for (int i = 0; i < 4; ++i) load_row16<F>(comp == 0 ? g.k[i] : g.v[i], l16, D, i < width, x[i]);
    LOGKV_G uint16_t* dst = comp == 0 ? out.k : out.v;
#pragma unroll
    for (int side = 0; side < 2; ++side) {
      const unsigned member = side == 0 ? left_rows : (0xfu & ~left_rows);
      const double srcp = side == 0 ? left_rcp : right_rcp;
      LOGKV_G uint16_t* at = dst + static_cast<int64_t>(dest + side) * D + l16;
      const bool write = live && (side == 0 || width == 4);
#pragma unroll
      for (int k = 0; k < F; ++k) {
        float acc = (member & 1u) ? x[0][k] * g.w[0] : x[0][k] * 0.f;
#pragma unroll
        for (int i = 1; i < 4; ++i) acc = acc + (((member >> i) & 1u) ? x[i][k] * g.w[i] : x[i][k] * 0.f);
        if (write && l16 + 16 * k < D) at[16 * k] = f32_to_bf16(div_by_rcp(acc, srcp));
      }
    }
  }
  // Metadata of both outputs: lanes 0-3 of the row hold rows 0-3 for the left
  // side, lanes 4-7 the same rows for the right side (quads of side_meta).
  {
    Meta mine{};
    const int mi = l16 & 3;
    if (l16 < 8 && mi < width) {
      if (flush_src) mine = PoolT<2>{lad, base, cnt, flush_rows_global(c, r, ws, pl, ladder)}.meta(start + mi);
      else mine = PoolT<1>{lad, base, cnt, staged_of(ws, ladder, ell, dk, dv)}.meta(start + mi);
    }
    const int side = (l16 >> 2) & 1;
    const unsigned member = side == 0 ? left_rows : (0xfu & ~left_rows);
    float wt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wt[i] = ((member >> i) & 1u) ? g.w[i] : 0.f;
    const float mass = side_mass(wt);
    const bool in_side = mi < width && ((member >> mi) & 1u);
    const Meta res = side_meta(mine, in_side, mass);
    if (live && l16 < 8 && (l16 & 3) == 0 && (side == 0 || width == 4)) put_soa_meta(out, dest + side, res);
  }
}

// Plan values of a lane's ladder at one level, kept while the lane's
// consecutive quads stay on that ladder.
struct RowPlan {
  int ladder;
  int cnt, m;
  bool flush_src;
  int first;
  int64_t order_base;
};

__device__ __forceinline__ void load_row_plan(const Workspace& ws, int ladder, int ell, RowPlan& pp) {
  const LadderPlan* pl = ws.plans + ladder;
  pp.ladder = ladder;
  pp.cnt = pl->cnt[ell];
  pp.m = pl->m[ell];
  pp.flush_src = ell == 0 && pl->kind0 == 0;
  pp.first = pl->first;
  pp.order_base = pl->order_base;
}

// The ladder's flush rows as a level-0 source from a lane's plan values.
__device__ inline Src flush_rows_planned(const LadderArgs& c, const RowsArgs& r, const Workspace& ws,
                                         const RowPlan& pp) {
  const int lane_ix = pp.ladder / c.k_max;
  const int b = lane_ix / c.n_groups, g = lane_ix % c.n_groups;
  Src s{};
  s.kind = 2;
  s.gtok = gp(ws.tok + static_cast<int64_t>(pp.ladder) * r.tokens + pp.first);
  s.order_base = pp.order_base;
  s.kb = gp(r.k + b * r.k_sb + g * r.k_sg);
  s.vb = gp(r.v + b * r.v_sb + g * r.v_sg);
  s.k_st = r.k_st;
  s.v_st = r.v_st;
  s.posb = gp(r.pos + b * r.pos_sb);
  return s;
}

// One Beta group of 128-feature rows per 16-lane row, one load batch: the
// group's rows, weights and metadata are loaded together, the screened cut
// decides from the held rows and the side means are written from them.
// Returns false (nothing written) when the screen does not settle the cut.
__device__ __forceinline__ bool beta_row_group_held(const LadderArgs& c, const RowsArgs& r, const Workspace& ws,
                                                    const RowPlan& pp, int ell, int gi, bool live,
                                                    const uint32_t (&pre)[4], bool have_pre) {
  const int l16 = lane_id() & 15, mi = l16 & 3;
  const int n_pair = 2 * carries_of(pp.cnt, pp.m, c.slots, false);
  const int start = 4 * gi;
  const int width = max(0, min(4, n_pair - start));
  const Ladder lad = ladder_of(c, pp.ladder);
  const int64_t base = static_cast<int64_t>(ell) * c.slots;
  GroupRows g;
  Meta mine{};
  if (pp.flush_src) {
    const PoolT<2> pool{lad, base, pp.cnt, flush_rows_planned(c, r, ws, pp)};
    if (have_pre) {
      group_rows_at(pool, start, width, pre, g);
      if (l16 < 8 && mi < width) mine = pool.meta_at(start + mi, pre[mi]);
    } else {
      group_rows<2>(pool, start, width, g);
      if (l16 < 8 && mi < width) mine = pool.meta(start + mi);
    }
  } else {
    const PoolT<1> pool{lad, base, pp.cnt, staged_of(ws, pp.ladder, ell, c.dk, c.dv)};
    group_rows<1>(pool, start, width, g);
    if (l16 < 8 && mi < width) mine = pool.meta(start + mi);
  }
  Rows8 held;
  load_rows8(g, l16, width, held);
  int cut = 2;
  if (width == 4) {
    const float total = fmaxf(((g.w[0] + g.w[1]) + g.w[2]) + g.w[3], 1e-12f);
    float sk[9], sv[9];
    screen_sums8(held.k, sk);
    screen_sums8(held.v, sv);
    cut = screened_cut(sk, sv, g.w, total);
  }
  const bool settled = cut != 0;
  cut = settled ? cut : 2;
  const bool emit = live && settled;
  // The held rows count as rewritten here, so the output means unpack them
  // again instead of keeping the screen's 64 unpacked features live.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
      asm volatile("" : "+v"(held.k[i][h2].x), "+v"(held.k[i][h2].y), "+v"(held.v[i][h2].x), "+v"(held.v[i][h2].y));
  double rl;
  {
    float wl[4], wrt[4];
    cut_weights(g.w, cut, wl, wrt);
    rl = 1.0 / static_cast<double>(fmaxf(l16 == 0 ? side_mass(wl) : side_mass(wrt), 1e-12f));
  }
  const int dest = start / 2;
  const Soa out = carry_of(ws, pp.ladder, ell, c.dk, c.dv);
  const double left_rcp = row_lane_d(rl, 0), right_rcp = row_lane_d(rl, 1);
  const unsigned left_rows = (1u << cut) - 1u;
#pragma unroll
  for (int comp = 0; comp < 2; ++comp) {
    LOGKV_G uint16_t* dst = comp == 0 ? out.k : out.v;
#pragma unroll
    for (int side = 0; side < 2; ++side) {
      if (emit && (side == 0 || width == 4))
        side_out8(comp == 0 ? held.k : held.v, g.w, side == 0 ? left_rows : (0xfu & ~left_rows),
                  side == 0 ? left_rcp : right_rcp, dst + static_cast<int64_t>(dest + side) * 128 + 8 * l16);
    }
  }
  {
    const int side = (l16 >> 2) & 1;
    const unsigned member = side == 0 ? left_rows : (0xfu & ~left_rows);
    float wt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wt[i] = ((member >> i) & 1u) ? g.w[i] : 0.f;
    const float mass = side_mass(wt);
    const bool in_side = mi < width && ((member >> mi) & 1u);
    const Meta res = side_meta(mine, in_side, mass);
    if (emit && l16 < 8 && (l16 & 3) == 0 && (side == 0 || width == 4)) put_soa_meta(out, dest + side, res);
  }
  return settled;
}

// Beta carries launch `ell`: the level's units in consecutive quads, one quad
// per wave step (a wave's quads are contiguous); each lane finds its row's
// ladder by binary search once, then walks forward. FULL (128-feature rows):
// a lane keeps its ladder's plan values while its quads stay on that ladder,
// a group is one load batch (rows, weights, metadata) decided by the screen
// and written from the held rows, and the groups the screen leaves open are
// evaluated canonically by beta_group, one at a time on the whole wave (so
// the rare path's registers stay out of the screened one's).
template <int NJ, bool FULL>
__global__ __launch_bounds__(kCarryThreads, 3) void beta_carries_kernel(LadderArgs c, RowsArgs r, Workspace ws, int ell) {
  extern __shared__ __align__(16) int32_t prefix_s[];
  const int ladders = c.n_batch * c.n_groups * c.k_max;
  const LOGKV_G int32_t* pre = gp(ws.units + static_cast<int64_t>(ell) * (ladders + 1));
  // The level's unit count first: a block without quads leaves before it stages the table.
  const int total = pre[ladders];
  if (total == 0) return;
  const int quads = (total + 3) / 4;
  const int wpb = static_cast<int>(blockDim.x) / kWave;
  const int n_waves = static_cast<int>(gridDim.x) * wpb;
  const int per = (quads + n_waves - 1) / n_waves;
  if (static_cast<int>(blockIdx.x) * wpb * per >= quads) return;
  stage_copy<int32_t>(prefix_s, pre, ladders + 1, threadIdx.x, blockDim.x);
  __syncthreads();
  int qd = (static_cast<int>(blockIdx.x) * wpb + wave_id()) * per;
  const int qd_end = min(quads, qd + per);
  if (qd >= qd_end) return;
  const int row = lane_id() >> 4;
  int ladder = 0;   // prefix_s[ladder] <= unit < prefix_s[ladder + 1]
  {
    const int u0 = min(4 * qd + row, total - 1);
    for (int len = ladders; len > 1;) {
      const int half = len >> 1;
      ladder = prefix_s[ladder + half] <= u0 ? ladder + half : ladder;
      len -= half;
    }
  }
  if constexpr (FULL) {
    RowPlan pp;
    pp.ladder = -1;
    // The next group's flush row indices, read a group ahead when it is on the
    // same flush-sourced ladder (its loads precede this group's row loads).
    uint32_t pre[4] = {0u, 0u, 0u, 0u};
    int pre_ladder = -1, pre_gi = -1;
    for (; qd < qd_end; ++qd) {
      const int unit = 4 * qd + row;
      const bool live = unit < total;
      const int uu = live ? unit : total - 1;
      while (prefix_s[ladder + 1] <= uu) ++ladder;
      if (ladder != pp.ladder) load_row_plan(ws, ladder, ell, pp);
      const int gi = uu - prefix_s[ladder];
      const bool have_pre = pre_ladder == ladder && pre_gi == gi;
      uint32_t cur[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) cur[i] = pre[i];
      const int nx = uu + 4;
      if (pp.flush_src && qd + 1 < qd_end && nx < total && nx < prefix_s[ladder + 1]) {
        const LOGKV_G uint16_t* gtok = gp(ws.tok + static_cast<int64_t>(ladder) * r.tokens + pp.first);
        const int n_rows = pp.cnt + pp.m;   // pool rows: stored, then staged
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int p = 4 * (gi + 4) + i;
          pre[i] = (p >= pp.cnt && p < n_rows) ? gtok[p - pp.cnt] : 0u;
        }
        pre_ladder = ladder;
        pre_gi = gi + 4;
      } else {
        pre_ladder = -1;
      }
      const bool settled = beta_row_group_held(c, r, ws, pp, ell, gi, live, cur, have_pre);
      // Groups the screen leaves open (near ties, non-finite costs, tiny
      // masses): the canonical evaluation, one group at a time on the whole wave.
      uint64_t open = __ballot(live && !settled && (lane_id() & 15) == 0);
      while (open) {
        const int src = __builtin_ctzll(open);
        open &= open - 1;
        RowPlan q;
        q.ladder = __shfl(pp.ladder, src, kWave);
        q.cnt = __shfl(pp.cnt, src, kWave);
        q.m = __shfl(pp.m, src, kWave);
        q.flush_src = __shfl(static_cast<int>(pp.flush_src), src, kWave) != 0;
        q.first = __shfl(pp.first, src, kWave);
        q.order_base = __shfl(pp.order_base, src, kWave);
        const int qgi = __shfl(gi, src, kWave);
        const int n_pair = 2 * carries_of(q.cnt, q.m, c.slots, false);
        const Ladder lad = ladder_of(c, q.ladder);
        const int64_t base = static_cast<int64_t>(ell) * c.slots;
        const Soa out = carry_of(ws, q.ladder, ell, c.dk, c.dv);
        if (q.flush_src)
          beta_group<NJ, 2>(PoolT<2>{lad, base, q.cnt, flush_rows_planned(c, r, ws, q)}, out, n_pair, qgi, c.dk, c.dv);
        else
          beta_group<NJ, 1>(PoolT<1>{lad, base, q.cnt, staged_of(ws, q.ladder, ell, c.dk, c.dv)}, out, n_pair, qgi,
                            c.dk, c.dv);
      }
    }
  } else {
    for (; qd < qd_end; ++qd) {
      const int unit = 4 * qd + row;
      const bool live = unit < total;
      const int uu = live ? unit : total - 1;
      while (prefix_s[ladder + 1] <= uu) ++ladder;
      beta_row_group<NJ>(c, r, ws, ladder, ell, uu - prefix_s[ladder], live);
    }
  }
}

// Carries launch `ell`: the level's work units (numbered ladder after ladder
// by units_kernel) are split into contiguous ranges, one per wave, so a wave
// resolves a ladder's plan and sources once for all its units there and reads
// the ladder's rows in order. A wave finds its first ladder by binary search
// over the unit prefix table staged in LDS. Launches ell = 0..L-2 run in
// stream order (level ell stages level ell - 1's carries); slots are not
// written here.
template <int NJ>
__global__ __launch_bounds__(kCarryThreads) void carries_kernel(LadderArgs c, RowsArgs r, RouteParams prm,
                                                                Workspace ws, int ell) {
  extern __shared__ __align__(16) int32_t prefix_s[];
  const int ladders = c.n_batch * c.n_groups * c.k_max;
  const LOGKV_G int32_t* pre = gp(ws.units + static_cast<int64_t>(ell) * (ladders + 1));
  // The level's unit count first: a block without units leaves before it stages the table.
  const int total = pre[ladders];
  const int wpb = static_cast<int>(blockDim.x) / kWave;
  const int n_waves = static_cast<int>(gridDim.x) * wpb;
  const int per = (total + n_waves - 1) / n_waves;
  if (total == 0 || static_cast<int>(blockIdx.x) * wpb * per >= total) return;
  stage_copy<int32_t>(prefix_s, pre, ladders + 1, threadIdx.x, blockDim.x);
  __syncthreads();
  int u = (static_cast<int>(blockIdx.x) * wpb + wave_id()) * per;
  const int u_end = min(total, u + per);
  if (u >= u_end) return;
  int ladder = 0;   // the ladder of unit u: prefix_s[ladder] <= u < prefix_s[ladder + 1]
  for (int len = ladders; len > 1;) {
    const int half = len >> 1;
    ladder = prefix_s[ladder + half] <= u ? ladder + half : ladder;
    len -= half;
  }
  ladder = __builtin_amdgcn_readfirstlane(ladder);
  const bool beta = prm.beta_merge != 0;
  const int64_t base = static_cast<int64_t>(ell) * c.slots;
  while (u < u_end) {
    const int first = prefix_s[ladder], last = min(prefix_s[ladder + 1], u_end);
    if (last > u) {
      const LadderPlan* pl = ws.plans + ladder;
      const int cnt = pl->cnt[ell], m = pl->m[ell];
      const int n_carry = carries_of(cnt, m, c.slots, false);
      const Ladder lad = ladder_of(c, ladder);
      const Soa out = carry_of(ws, ladder, ell, c.dk, c.dv);
      if (ell == 0 && pl->kind0 == 0)
        ladder_units<NJ, 2>(PoolT<2>{lad, base, cnt, flush_rows_global(c, r, ws, pl, ladder)}, out, n_carry, beta,
                            u - first, last - first, c.dk, c.dv);
      else
        ladder_units<NJ, 1>(PoolT<1>{lad, base, cnt, staged_of(ws, ladder, ell, c.dk, c.dv)}, out, n_carry, beta,
                            u - first, last - first, c.dk, c.dv);
      u = last;
    }
    ++ladder;
  }
}

// Slot writes of every level (block (ladder, level)): fill, move and clear, or
// top fold. A level's writes read only its own stored slots and its staged
// rows (the previous level's carries), so the levels run side by side.
// TOP = false: levels 0..L-2 (grid y = L - 1); TOP = true: the top level
// (grid y = 1), whose saturated fold keeps its registers out of the other
// levels' launch.
// Slot writes of levels ell0 .. ell0 + gridDim.y - 1 (blockIdx.y), one block per
// (ladder, level). TOP launches end at the top level and put it at y = 0, so the
// top folds (sequential in their rows, the slowest blocks) are dispatched first.
template <bool TOP>
__global__ __launch_bounds__(kThreads) void finish_kernel(LadderArgs c, RowsArgs r, Workspace ws, int ell0) {
  extern __shared__ __align__(16) uint8_t dyn[];
  const int y = static_cast<int>(blockIdx.y);
  const bool top = TOP && y == 0;
  const int ladder = blockIdx.x, ell = top ? c.levels - 1 : ell0 + y - (TOP ? 1 : 0);
  const LadderPlan* pl = ws.plans + ladder;
  // The last launch of a commit marks every cluster that took rows as live.
  if (top && threadIdx.x == 0 && pl->m_tok > 0) c.alive[ladder] = 1;
  if (!pl->active) return;
  const int cnt = pl->cnt[ell], m = pl->m[ell];
  if (m == 0) return;
  const Ladder lad = ladder_of(c, ladder);
  int n;
  if (top)
    n = ell == 0 && pl->kind0 == 0
            ? level_finish<0, true>(lad, ell, cnt, flush_rows_of(c, r, ws, pl, ladder, reinterpret_cast<uint16_t*>(dyn)), m)
            : level_finish<1, true>(lad, ell, cnt, staged_of(ws, ladder, ell, c.dk, c.dv), m);
  else if (ell == 0 && pl->kind0 == 0)
    n = level_finish<0, false>(lad, ell, cnt, flush_rows_of(c, r, ws, pl, ladder, reinterpret_cast<uint16_t*>(dyn)), m);
  else
    n = level_finish<1, false>(lad, ell, cnt, staged_of(ws, ladder, ell, c.dk, c.dv), m);
  if (threadIdx.x == 0) c.level_count[static_cast<int64_t>(ladder) * c.levels + ell] = static_cast<int16_t>(n);
}

// Old-old merge of the unified route (litgpt/log_kv_cache.py:2517-2580), one
// block per lane: the lane's step-th merge (keep, retire), if it has one. The
// two ladders' entries are ordered by the reference's entry rule
// (litgpt/log_kv_cache.py:2395-2447): each side stably by order, an entry's
// key the p_lo of the next massive entry at or after it on its side (its own
// order if there is none), the sides merged keep-first on ties. They are
// gathered in that order into the keep ladder's level-0 staging with order =
// rank, both ladders are cleared, the keep cluster takes the n_total-weighted
// center, the summed n_eff and n_total, the larger p_hi and phase = entries,
// the retired cluster is emptied (its center is left as it was), and the level
// launches re-append the staged rows. Every other ladder of the lane gets an
// inactive plan.
__global__ __launch_bounds__(kThreads) void ward_kernel(LadderArgs c, Workspace ws, const int32_t* jobs,
                                                        const int32_t* n_jobs, int step) {
  extern __shared__ __align__(16) uint8_t dyn[];
  __shared__ int start_s[2 * kMaxLevels + 2];
  __shared__ int16_t cnt_s[2 * kMaxLevels];
  const int lane = blockIdx.x, K = c.k_max, L = c.levels, B = c.slots, dk = c.dk, dv = c.dv;
  for (int cc = threadIdx.x; cc < K; cc += kThreads) {
    ws.plans[static_cast<int64_t>(lane) * K + cc].active = 0;
    ws.plans[static_cast<int64_t>(lane) * K + cc].m_tok = 0;
  }
  if (step >= n_jobs[lane]) return;
  const int keep = jobs[(static_cast<int64_t>(lane) * kMaxClusters + step) * 2];
  const int retire = jobs[(static_cast<int64_t>(lane) * kMaxClusters + step) * 2 + 1];
  const int kl = lane * K + keep, fl = lane * K + retire;
  const Ladder side[2] = {ladder_of(c, kl), ladder_of(c, fl)};
  for (int e = threadIdx.x; e < L; e += kThreads) {
    cnt_s[e] = c.level_count[static_cast<int64_t>(kl) * L + e];
    cnt_s[L + e] = c.level_count[static_cast<int64_t>(fl) * L + e];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int e = 0; e < 2 * L; ++e) {
      start_s[e] = acc;
      acc += cnt_s[e];
    }
    start_s[2 * L] = acc;
  }
  __syncthreads();
  const int n_k = start_s[L], total = start_s[2 * L];
  // Entry i -> (side, slot): levels of the keep ladder, then of the retired one.
  auto where = [&](int i, int& sd, int64_t& slot) {
    int e = 0;
    while (e + 1 < 2 * L && start_s[e + 1] <= i) ++e;
    sd = e >= L ? 1 : 0;
    slot = static_cast<int64_t>(e - sd * L) * B + (i - start_s[e]);
  };
  int width = 1;
  while (width < total) width <<= 1;
  uint64_t* keys = reinterpret_cast<uint64_t*>(dyn);
  int64_t* eff = reinterpret_cast<int64_t*>(keys + width);
  int16_t* merged = reinterpret_cast<int16_t*>(eff + total);
  for (int i = threadIdx.x; i < width; i += kThreads) {
    uint64_t key = ~0ull;
    if (i < total) {
      int sd;
      int64_t slot;
      where(i, sd, slot);
      key = (static_cast<uint64_t>(sd) << 63) | (static_cast<uint64_t>(side[sd].ord[slot]) << kOrderIndexBits) |
            static_cast<uint64_t>(i);
    }
    keys[i] = key;
  }
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
  if (threadIdx.x == 0) {
    // Keys: the next massive entry's p_lo on the same side, else the entry's order.
    for (int sd = 0; sd < 2; ++sd) {
      const int lo = sd ? n_k : 0, hi = sd ? total : n_k;
      bool have = false;
      int64_t next = 0;
      for (int j = hi - 1; j >= lo; --j) {
        int s2;
        int64_t slot;
        where(static_cast<int>(keys[j] & kOrderIndexMask), s2, slot);
        if (side[s2].w[slot] > 0.f) {
          have = true;
          next = side[s2].lo[slot];
        }
        eff[j] = have ? next : side[s2].ord[slot];
      }
    }
    int i = 0, j = n_k, rank = 0;
    while (i < n_k && j < total) merged[rank++] = static_cast<int16_t>(eff[i] <= eff[j] ? i++ : j++);
    while (i < n_k) merged[rank++] = static_cast<int16_t>(i++);
    while (j < total) merged[rank++] = static_cast<int16_t>(j++);
  }
  __syncthreads();
  const Soa S0 = s0_of(ws, kl, dk, dv);
  {
    const RowUnits ru(dk, dv);
    for (int r0 = ru.r0; r0 < total; r0 += ru.step) {
      int sd;
      int64_t slot;
      where(static_cast<int>(keys[merged[r0]] & kOrderIndexMask), sd, slot);
      const uint2 x = load_unit(side[sd].k + slot * dk, side[sd].v + slot * dv, ru.u, ru.ku);
      store_unit(S0.k + static_cast<int64_t>(r0) * dk, S0.v + static_cast<int64_t>(r0) * dv, ru.u, ru.ku, x);
    }
  }
  for (int rank = threadIdx.x; rank < total; rank += kThreads) {
    int sd;
    int64_t slot;
    where(static_cast<int>(keys[merged[rank]] & kOrderIndexMask), sd, slot);
    Meta mt = slot_meta(side[sd], slot);
    mt.ord = rank;
    put_soa_meta(S0, rank, mt);
  }
  // Center and scalars (the reads precede every write of the same value).
  const int64_t ck = static_cast<int64_t>(kl), cf = static_cast<int64_t>(fl);
  const float nk = static_cast<float>(c.n_total[ck]), nf = static_cast<float>(c.n_total[cf]);
  for (int d = threadIdx.x; d < dk; d += kThreads) {
    const float mk = c.centroid[ck * dk + d], mf = c.centroid[cf * dk + d];
    const float den = nk + nf;
    c.centroid[ck * dk + d] = (nk * mk + nf * mf) / (den < 1.f ? 1.f : den);
  }
  __syncthreads();
  clear_slots(side[0], 0, static_cast<int64_t>(L) * B);
  clear_slots(side[1], 0, static_cast<int64_t>(L) * B);
  for (int e = threadIdx.x; e < L; e += kThreads) {
    c.level_count[ck * L + e] = 0;
    c.level_count[cf * L + e] = 0;
  }
  if (threadIdx.x == 0) {
    c.n_eff[ck] = c.n_eff[ck] + c.n_eff[cf];
    c.n_eff[cf] = 0.f;
    c.n_total[ck] = c.n_total[ck] + c.n_total[cf];
    c.n_total[cf] = 0;
    c.p_hi_c[ck] = imax64(c.p_hi_c[ck], c.p_hi_c[cf]);
    c.p_hi_c[cf] = -1;
    c.level0_phase[ck] = total;
    c.level0_phase[cf] = 0;
    c.alive[ck] = 1;
    c.alive[cf] = 0;
    LadderPlan pl;
    pl.active = total > 0 ? 1 : 0;
    pl.kind0 = 1;
    pl.m_tok = 0;
    pl.first = 0;
    pl.order_base = 0;
    int mm = total;
    for (int e = 0; e < kMaxLevels; ++e) {
      const bool used = e < L;
      pl.cnt[e] = 0;
      pl.m[e] = used ? mm : 0;
      mm = used ? carries_of(0, mm, B, e == L - 1) : 0;
    }
    ws.plans[ck] = pl;
  }
}

constexpr int kCarryBlocks = 2048;   // most blocks of a carries launch (8 per CU)

int launch_ward_step(const LadderArgs& c, const Workspace& ws, const int32_t* jobs, const int32_t* n_jobs, int step,
                     hipStream_t stream) {
  const int lanes = c.n_batch * c.n_groups;
  int width = 1;
  while (width < 2 * c.levels * c.slots) width <<= 1;
  const size_t shmem = static_cast<size_t>(width) * 8 + static_cast<size_t>(2 * c.levels * c.slots) * 10 + 16;
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&ward_kernel), shmem)) return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(ward_kernel, dim3(lanes), dim3(kThreads), shmem, stream, c, ws, jobs, n_jobs, step);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

// A side stream and its fork / join events per (device, caller stream),
// created on first use and kept for the process (default priority,
// non-blocking). Returned locked: the caller unlocks once its join is
// enqueued, so two host threads on one stream never share the events
// mid-sequence. Null when none can be made (the work then stays on the
// caller's stream).
struct SideStream {
  int dev = -1;
  hipStream_t main = nullptr, side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  hipEvent_t level[kMaxLevels] = {};   // level ell's carries enqueued on the caller's stream
  std::mutex mu;
};

constexpr int kSideLadders = 1024;
constexpr int kSideFinishLevels = 3;   // lowest levels whose finishes run on the side stream

static SideStream* side_stream_for(hipStream_t main) {
  constexpr int kSlots = 64;
  static SideStream slots[kSlots];
  static std::mutex table_mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  SideStream* hit = nullptr;
  {
    std::lock_guard<std::mutex> lock(table_mu);
    for (SideStream& e : slots)
      if (e.side && e.dev == dev && e.main == main) hit = &e;
    if (!hit) {
      for (SideStream& e : slots)
        if (!e.side) {
          hipStream_t s = nullptr;
          hipEvent_t f = nullptr, j = nullptr;
          if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
          if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
              hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess)
            return nullptr;
          for (hipEvent_t& ev : e.level)
            if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return nullptr;
          e.dev = dev;
          e.main = main;
          e.fork = f;
          e.join = j;
          e.side = s;
          hit = &e;
          break;
        }
    }
  }
  if (hit) hit->mu.lock();
  return hit;
}

int launch_commit(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                  hipStream_t stream) {
  const int ladders = c.n_batch * c.n_groups * c.k_max;
  const size_t tok_bytes = (2 * static_cast<size_t>(r.tokens) + 15) & ~size_t(15);
  const size_t shmem = tok_bytes + (p.late_joins ? static_cast<size_t>(ws.sort_width) * 8 : 0);
  if (!allow_dynamic_lds(reinterpret_cast<const void*>(&commit_kernel<false>), shmem) ||
      !allow_dynamic_lds(reinterpret_cast<const void*>(&commit_kernel<true>), shmem))
    return LOGKV_ERUNTIME;
  hipLaunchKernelGGL(bucket_kernel, dim3(c.n_batch * c.n_groups), dim3(kBucketThreads), 0, stream, c, r, ws);
  // The center updates run beside the ladder launches (a few clusters can hold
  // most of a flush's rows, and each center is a fold over its rows in order),
  // for calls of at least kSideLadders ladders: every cross-queue event costs
  // the queue a few microseconds, and small calls from several streams would
  // share the device's few hardware queues with their side streams.
  SideStream* side = ladders >= kSideLadders ? side_stream_for(stream) : nullptr;
  hipStream_t cs = stream;
  if (side && hipEventRecord(side->fork, stream) == hipSuccess && hipStreamWaitEvent(side->side, side->fork, 0) == hipSuccess)
    cs = side->side;
  const bool forked = cs != stream;
  const int nj = (c.dk + kCenterWaves * kWave - 1) / (kCenterWaves * kWave);
  const bool inline_centers = !forked && nj == 1;   // commit_kernel's y = 1 blocks
  if (!inline_centers) {
    const size_t ctok_bytes = 2 * static_cast<size_t>(r.tokens);
    if (nj == 1)
      hipLaunchKernelGGL(center_kernel<1>, dim3(ladders), dim3(kCenterWaves * kWave), ctok_bytes, cs, c, r, p, ws);
    else
      hipLaunchKernelGGL(center_kernel<2>, dim3(ladders), dim3(kCenterWaves * kWave), ctok_bytes, cs, c, r, p, ws);
  }
  if (inline_centers)
    hipLaunchKernelGGL(commit_kernel<true>, dim3(ladders, 2), dim3(kThreads), shmem, stream, c, r, p, ws);
  else
    hipLaunchKernelGGL(commit_kernel<false>, dim3(ladders, 1), dim3(kThreads), shmem, stream, c, r, p, ws);
  const int rc = launch_levels(c, r, p, ws, stream, forked ? side : nullptr);
  if (forked && hipEventRecord(side->join, side->side) != hipSuccess) {
    side->mu.unlock();
    return LOGKV_ERUNTIME;
  }
  if (forked && hipStreamWaitEvent(stream, side->join, 0) != hipSuccess) {
    side->mu.unlock();
    return LOGKV_ERUNTIME;
  }
  if (side) side->mu.unlock();
  return rc;
}

// The level launches that follow a prepare step (commit_kernel or ward_kernel):
// carry work units, carries per level, then the slot writes of every level.
int launch_levels(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                  hipStream_t stream, SideStream* side) {
  const int ladders = c.n_batch * c.n_groups * c.k_max;
  const size_t tok_bytes = (2 * static_cast<size_t>(r.tokens) + 15) & ~size_t(15);
  const int side_levels = side ? std::min(kSideFinishLevels, c.levels - 1) : 0;
  if (c.levels > 1) {
    hipLaunchKernelGGL(units_kernel, dim3(c.levels - 1), dim3(kUnitsThreads), 0, stream, c, p, ws);
    const size_t carry_shmem = (static_cast<size_t>(ladders) + 1) * 4;
    const bool narrow = c.dk <= 2 * kWave && c.dv <= 2 * kWave;
    // Beta groups of rows up to 128 features: four groups to a wave.
    const bool rows16 = narrow && p.beta_merge != 0;
    const bool full = c.dk == 2 * kWave && c.dv == 2 * kWave;
    const void* carries = rows16   ? (full ? reinterpret_cast<const void*>(&beta_carries_kernel<2, true>)
                                           : reinterpret_cast<const void*>(&beta_carries_kernel<2, false>))
                          : narrow ? reinterpret_cast<const void*>(&carries_kernel<2>)
                                   : reinterpret_cast<const void*>(&carries_kernel<4>);
    if (!allow_dynamic_lds(carries, carry_shmem)) return LOGKV_ERUNTIME;
    const int units_per_block = (kCarryThreads / kWave) * (rows16 ? 4 : 1);
    for (int ell = 0; ell + 1 < c.levels; ++ell) {
      // Units at level ell: at most ceil(carries / 2) Beta groups (or carries) per ladder.
      const int64_t bound = static_cast<int64_t>(ladders) * carry_cap(ws.m0_cap, ell);
      const int64_t blocks = std::min<int64_t>(kCarryBlocks, std::max<int64_t>(1, bound / units_per_block));
      if (rows16 && full)
        hipLaunchKernelGGL((beta_carries_kernel<2, true>), dim3(blocks), dim3(kCarryThreads), carry_shmem, stream, c, r, ws,
                           ell);
      else if (rows16)
        hipLaunchKernelGGL((beta_carries_kernel<2, false>), dim3(blocks), dim3(kCarryThreads), carry_shmem, stream, c, r,
                           ws, ell);
      else if (narrow)
        hipLaunchKernelGGL(carries_kernel<2>, dim3(blocks), dim3(kCarryThreads), carry_shmem, stream, c, r, p, ws, ell);
      else
        hipLaunchKernelGGL(carries_kernel<4>, dim3(blocks), dim3(kCarryThreads), carry_shmem, stream, c, r, p, ws, ell);
      // With a side stream, the finishes of the lowest kSideFinishLevels levels (their slots:
      // staged rows in, survivors moved) run there once their carries launches are done: the
      // later carries launches read only higher levels' slots and the carry buffers, which no
      // finish writes. Every event costs each queue a few microseconds, so level 0's finish (the
      // largest) follows its own carries, levels 1 .. kSideFinishLevels - 1 share one launch after
      // the last of theirs, and the smaller finishes of the levels above wait for the last carries
      // launch and run with the top level's.
      if (side && ell < side_levels && (ell == 0 || ell == side_levels - 1)) {
        if (hipEventRecord(side->level[ell], stream) != hipSuccess ||
            hipStreamWaitEvent(side->side, side->level[ell], 0) != hipSuccess)
          return LOGKV_ERUNTIME;
        const int e0 = ell == 0 ? 0 : 1;
        hipLaunchKernelGGL(finish_kernel<false>, dim3(ladders, ell - e0 + 1), dim3(kThreads), tok_bytes, side->side, c,
                           r, ws, e0);
      }
    }
  }
  // Levels side_levels .. levels - 2, then the top level (y = 0).
  hipLaunchKernelGGL(finish_kernel<true>, dim3(ladders, c.levels - side_levels), dim3(kThreads), tok_bytes, stream, c,
                     r, ws, side_levels);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
