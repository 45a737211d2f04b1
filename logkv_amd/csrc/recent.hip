// The recent window's row moves on the device: one launch appends a block of
// rows to every recent buffer, one launch moves the rows left after a flush to
// the front and clears the vacated rows (litgpt/log_kv_cache.py:5668-5718,
// :5640-5659, there as separate tensor copies and fills per buffer).
//
// Bf16 rows move in 8-byte units of four features; positions and span flags
// one entry per thread.
#include "route.hpp"

namespace logkv {

namespace {

struct RecentBuf {
  uint16_t* base;
  int32_t d;   // features per row
};

__device__ __forceinline__ uint2* unit_at(uint16_t* base, int64_t row, int d, int u) {
  return reinterpret_cast<uint2*>(base + row * d + 4 * u);
}

}  // namespace

// Block rows [0, n) of each source into recent rows [at, at + n).
__global__ __launch_bounds__(256) void recent_append_kernel(logkv_recent_args a, int at, int n) {
  const int lanes = a.n_batch * a.n_groups;
  const int uk = a.dk / 4, ukr = a.dkr / 4, uv = a.dv / 4, per = uk + ukr + uv;
  const int64_t total = static_cast<int64_t>(lanes) * n * per;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int u = static_cast<int>(i % per);
    const int64_t rest = i / per;
    const int t = static_cast<int>(rest % n), lane = static_cast<int>(rest / n);
    const int b = lane / a.n_groups, g = lane % a.n_groups;
    const int64_t row = static_cast<int64_t>(lane) * a.cap + at + t;
    if (u < uk) {
      const uint2 x = *reinterpret_cast<const LOGKV_G uint2*>(gp(a.k) + b * a.k_sb + g * a.k_sg + t * a.k_st + 4 * u);
      *unit_at(a.recent_k, row, a.dk, u) = x;
    } else if (u < uk + ukr) {
      const int w = u - uk;
      const uint2 x =
          *reinterpret_cast<const LOGKV_G uint2*>(gp(a.k_raw) + b * a.kr_sb + g * a.kr_sg + t * a.kr_st + 4 * w);
      *unit_at(a.recent_k_raw, row, a.dkr, w) = x;
    } else {
      const int w = u - uk - ukr;
      const uint2 x = *reinterpret_cast<const LOGKV_G uint2*>(gp(a.v) + b * a.v_sb + g * a.v_sg + t * a.v_st + 4 * w);
      *unit_at(a.recent_v, row, a.dv, w) = x;
    }
  }
  const int64_t flags = static_cast<int64_t>(a.n_batch) * n;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < flags;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int b = static_cast<int>(i / n), t = static_cast<int>(i % n);
    a.recent_pos[static_cast<int64_t>(b) * a.cap + at + t] = a.pos[b * a.pos_sb + t * a.pos_st];
    if (a.recent_ends) a.recent_ends[static_cast<int64_t>(b) * a.cap + at + t] = a.ends[b * a.ends_sb + t];
  }
}

// Rows [take, count) move to [0, count - take) and rows [count - take, count)
// become zero. Needs count - take <= take: then every source row lies in the
// cleared range, and the thread that reads it clears it.
__global__ __launch_bounds__(256) void recent_shift_kernel(logkv_recent_args a, int take, int count) {
  const int lanes = a.n_batch * a.n_groups;
  const int remaining = count - take;
  const int uk = a.dk / 4, ukr = a.dkr / 4, uv = a.dv / 4, per = uk + ukr + uv;
  // Units of rows [0, take): row r < remaining receives row take + r (and clears
  // it); rows remaining <= r < take are cleared.
  const int64_t total = static_cast<int64_t>(lanes) * take * per;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int u = static_cast<int>(i % per);
    const int64_t rest = i / per;
    const int r = static_cast<int>(rest % take), lane = static_cast<int>(rest / take);
    RecentBuf buf;
    int w;
    if (u < uk) buf = {a.recent_k, a.dk}, w = u;
    else if (u < uk + ukr) buf = {a.recent_k_raw, a.dkr}, w = u - uk;
    else buf = {a.recent_v, a.dv}, w = u - uk - ukr;
    const int64_t row0 = static_cast<int64_t>(lane) * a.cap;
    uint2* dst = unit_at(buf.base, row0 + r, buf.d, w);
    if (r < remaining) {
      uint2* src = unit_at(buf.base, row0 + take + r, buf.d, w);
      const uint2 x = *src;
      *dst = x;
      *src = make_uint2(0u, 0u);
    } else {
      *dst = make_uint2(0u, 0u);
    }
  }
  const int64_t flags = static_cast<int64_t>(a.n_batch) * take;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < flags;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int b = static_cast<int>(i / take), r = static_cast<int>(i % take);
    const int64_t row0 = static_cast<int64_t>(b) * a.cap;
    if (r < remaining) {
      a.recent_pos[row0 + r] = a.recent_pos[row0 + take + r];
      a.recent_pos[row0 + take + r] = 0;
      if (a.recent_ends) {
        a.recent_ends[row0 + r] = a.recent_ends[row0 + take + r];
        a.recent_ends[row0 + take + r] = 0;
      }
    } else {
      a.recent_pos[row0 + r] = 0;
      if (a.recent_ends) a.recent_ends[row0 + r] = 0;
    }
  }
}

int launch_recent_append(const logkv_recent_args& a, int at, int n, hipStream_t stream) {
  const int64_t units = static_cast<int64_t>(a.n_batch) * a.n_groups * n * ((a.dk + a.dkr + a.dv) / 4);
  const int blocks = static_cast<int>(std::min<int64_t>(4096, std::max<int64_t>(1, (units + 255) / 256)));
  hipLaunchKernelGGL(recent_append_kernel, dim3(blocks), dim3(256), 0, stream, a, at, n);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_recent_shift(const logkv_recent_args& a, int take, int count, hipStream_t stream) {
  const int64_t units = static_cast<int64_t>(a.n_batch) * a.n_groups * take * ((a.dk + a.dkr + a.dv) / 4);
  const int blocks = static_cast<int>(std::min<int64_t>(4096, std::max<int64_t>(1, (units + 255) / 256)));
  hipLaunchKernelGGL(recent_shift_kernel, dim3(blocks), dim3(256), 0, stream, a, take, count);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
