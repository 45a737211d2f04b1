// Route op-log on the device: recording the decisions of a committed flush,
// and replaying a logged flush through the same commit without routing.
//
// The log format is the reference's (litgpt/log_kv_cache.py:90-94,
// :2006-2096): per lane (batch row, KV group) int32 rows (op, cluster, arg,
// position). The reference builds the rows on the host from its host plan and
// parses them on the host for replay (litgpt/log_kv_cache.py:4856-4926). Here
// the commit's per-ladder plans are already on the device, so one block per
// lane writes its rows straight from them, and replay turns the rows back
// into the attach decision array the commit kernels consume, so record and
// replay share every kernel that writes the cache.
#include "route.hpp"

namespace logkv {

namespace {

constexpr int kRecordThreads = 256;

__device__ __forceinline__ void put_row(int32_t* rows, int64_t at, int32_t op, int32_t cl, int64_t pos) {
  *reinterpret_cast<int4*>(rows + at * 4) = make_int4(op, cl, 0, static_cast<int32_t>(pos));
}

}  // namespace

// Rows of the flush just committed, per lane (litgpt/log_kv_cache.py:4682-4707
// fixes the order of the three record sites): NEW_CLUSTER of every opened
// cluster in ascending id with its earliest row's position
// (:2286-2297); JOIN of the other rows of ordinary joins, cluster ascending,
// rows in position order (:4153-4166); then, with delayed archival, JOIN of
// the delayed clusters' new rows in the same order (:3782-3788, "ordinary op
// rows still precede the delayed ones"). Each valid flush row gives one row.
__global__ __launch_bounds__(kRecordThreads) void record_kernel(LadderArgs c, RowsArgs r, Workspace ws,
                                                                logkv_op_log_view log) {
  __shared__ int new_at[kMaxClusters];    // section index of a cluster's NEW_CLUSTER row, -1 if none
  __shared__ int join_at[kMaxClusters];   // index of its first JOIN row
  __shared__ int joins[kMaxClusters];     // its JOIN rows
  __shared__ uint8_t late[kMaxClusters];  // delayed archive (re-sorted ladder)
  __shared__ int total_s;
  __shared__ int64_t len0_s;
  const int lane_ix = blockIdx.x, K = c.k_max;
  const int b = lane_ix / c.n_groups;
  const int64_t ladder0 = static_cast<int64_t>(lane_ix) * K;
  if (threadIdx.x == 0) {
    int n_new = 0, n_ord = 0, n_late = 0;
    for (int cc = 0; cc < K; ++cc) {
      const LadderPlan* pl = ws.plans + ladder0 + cc;
      const int m = pl->m_tok;
      const bool opened = m > 0 && !ws.snap_alive[ladder0 + cc];
      joins[cc] = m - (opened ? 1 : 0);
      late[cc] = pl->active && pl->kind0 == 1;
      new_at[cc] = opened ? n_new++ : -1;
      if (!late[cc]) n_ord += joins[cc];
      else n_late += joins[cc];
    }
    int ord = n_new, lat = n_new + n_ord;
    for (int cc = 0; cc < K; ++cc) {
      if (!late[cc]) {
        join_at[cc] = ord;
        ord += joins[cc];
      } else {
        join_at[cc] = lat;
        lat += joins[cc];
      }
    }
    total_s = n_new + n_ord + n_late;
    len0_s = log.lengths[lane_ix];
  }
  __syncthreads();
  const int64_t len0 = len0_s, cap = log.capacity;
  const int64_t* posb = r.pos + b * r.pos_sb;
  int32_t* rows = log.rows + static_cast<int64_t>(lane_ix) * cap * 4;
  for (int cc = 0; cc < K; ++cc) {
    const int m = ws.plans[ladder0 + cc].m_tok;
    if (m == 0) continue;
    const uint16_t* tok = ws.tok + (ladder0 + cc) * r.tokens;
    const int first = new_at[cc] >= 0 ? 1 : 0;
    const int64_t at0 = len0 + join_at[cc] - first;
    for (int i = first + static_cast<int>(threadIdx.x); i < m; i += kRecordThreads)
      if (at0 + i < cap) put_row(rows, at0 + i, LOGKV_OP_JOIN, cc, posb[tok[i]]);
    if (first && threadIdx.x == 0 && len0 + new_at[cc] < cap)
      put_row(rows, len0 + new_at[cc], LOGKV_OP_NEW_CLUSTER, cc, posb[tok[0]]);
  }
  if (threadIdx.x == 0) log.lengths[lane_ix] = static_cast<int32_t>(len0 + total_s);
}

// WARD_MERGE rows (keep, free, -1) of the unified route's old-old merges, per
// lane in merge order (litgpt/log_kv_cache.py:2597-2598): appended before the
// flush's NEW_CLUSTER / JOIN rows, as the reference's merge steps run before
// its new clusters and joins (:3661-3688). jobs [lanes, kMaxClusters, 2].
__global__ __launch_bounds__(kWave) void record_ward_kernel(const int32_t* __restrict__ jobs,
                                                            const int32_t* __restrict__ n_jobs, logkv_op_log_view log) {
  const int lane_ix = blockIdx.x, l = threadIdx.x;
  const int n = n_jobs[lane_ix];
  const int64_t len0 = log.lengths[lane_ix], cap = log.capacity;
  int32_t* rows = log.rows + static_cast<int64_t>(lane_ix) * cap * 4;
  const int32_t* jl = jobs + static_cast<int64_t>(lane_ix) * kMaxClusters * 2;
  for (int j = l; j < n; j += kWave)
    if (len0 + j < cap) *reinterpret_cast<int4*>(rows + (len0 + j) * 4) = make_int4(LOGKV_OP_WARD_MERGE, jl[2 * j], jl[2 * j + 1], -1);
  __syncthreads();
  if (l == 0) log.lengths[lane_ix] = static_cast<int32_t>(len0 + n);
}

// Replay parse, one wave per lane: the log rows [cursor, cursor + n) name the
// cluster of every valid flush row by position (litgpt/log_kv_cache.py:
// 4856-4904, one row per consumed token). Writes the decision array in
// position order (assign[lane, s] for the row order[b, s]) and checks what the reference's parse and commit
// would reject or could not reproduce: unknown ops, positions missing from or
// repeated in the flush, a short log, a NEW_CLUSTER of a live cluster or a
// JOIN into a dead one, a cluster's rows out of position order (the commit
// appends each cluster's rows in position order, and a dead cluster opens
// with its earliest row, as recorded).
//
// With `wards` (the unified route's logs), each lane has its own cursor and
// the lane's rows may open with WARD_MERGE rows (keep, free): they become the
// lane's merge list in the unified workspace layout, every merge between two
// distinct clusters live at that point (the free one dies), and the flush's
// NEW_CLUSTER / JOIN rows are checked against the clusters live after the
// merges. The rows a lane consumed and the most merges of any lane are
// reported for the host.
struct ReplayWards {
  const int64_t* cursors;   // [lanes] per-lane cursors
  int32_t* consumed;        // [lanes] rows consumed (merges + flush rows)
  int32_t* jobs;            // [lanes, kMaxClusters, 2] (keep, free) in log order
  int32_t* n_jobs;          // [lanes]
  int32_t* steps;           // most merges of a lane (atomic max; zeroed by the order launch)
};

__global__ __launch_bounds__(kWave) void replay_kernel(LadderArgs c, RowsArgs r, Workspace ws, logkv_op_log_view log,
                                                       int64_t cursor, int32_t* status, ReplayWards wards) {
  __shared__ int64_t last_pos[kMaxClusters];
  __shared__ int seen[kMaxClusters];
  __shared__ int chunk_c[kWave];
  __shared__ int64_t chunk_p[kWave];
  __shared__ int n_ward_s, ward_err_s;
  __shared__ uint32_t alive_s;
  const int lane_ix = blockIdx.x, K = c.k_max, l = threadIdx.x;
  const int b = lane_ix / c.n_groups;
  const int n = valid_rows(r, b), T = r.tokens;
  const int64_t ladder0 = static_cast<int64_t>(lane_ix) * K;
  const int64_t* posb = r.pos + b * r.pos_sb;
  const int32_t* ord = ws.order + static_cast<int64_t>(b) * T;
  int8_t* as = ws.assign + static_cast<int64_t>(lane_ix) * T;
  uint32_t alive = 0;
  for (int cc = 0; cc < K; ++cc) alive |= (c.alive[ladder0 + cc] ? 1u : 0u) << cc;
  if (l < K) {
    seen[l] = 0;
    last_pos[l] = 0;
  }
  for (int s = l; s < T; s += kWave) as[s] = -1;
  int err = 0;
  for (int s = l + 1; s < n; s += kWave)
    if (posb[ord[s]] == posb[ord[s - 1]]) err |= LOGKV_REPLAY_DUPLICATE_POSITION;
  const int64_t logged = min(static_cast<int64_t>(log.lengths[lane_ix]), log.capacity);
  const int32_t* rows = log.rows + static_cast<int64_t>(lane_ix) * log.capacity * 4;
  if (wards.jobs) {
    cursor = wards.cursors[lane_ix];
    if (l == 0) {
      int j = 0, werr = 0;
      uint32_t live = alive;
      int32_t* jl = wards.jobs + static_cast<int64_t>(lane_ix) * kMaxClusters * 2;
      while (cursor >= 0 && cursor + j < logged) {
        const int4 row = *reinterpret_cast<const int4*>(rows + (cursor + j) * 4);
        if (row.x != LOGKV_OP_WARD_MERGE) break;
        const int keep = row.y, fr = row.z;
        const bool ok = j < K - 1 && keep >= 0 && keep < K && fr >= 0 && fr < K && keep != fr &&
                        ((live >> keep) & 1u) && ((live >> fr) & 1u);
        if (!ok) {
          werr |= LOGKV_REPLAY_BAD_OP;
          break;
        }
        jl[2 * j] = keep;
        jl[2 * j + 1] = fr;
        live &= ~(1u << fr);
        ++j;
      }
      wards.n_jobs[lane_ix] = werr ? 0 : j;
      n_ward_s = j;
      ward_err_s = werr;
      alive_s = live;
    }
    __syncthreads();
    err |= ward_err_s;
    cursor += n_ward_s;
    alive = alive_s;
  }
  if (cursor < 0 || cursor + n > logged) err |= LOGKV_REPLAY_SHORT_LOG;
  __threadfence_block();
  __syncthreads();
  for (int i0 = 0; i0 < n; i0 += kWave) {
    const int i = i0 + l;
    const bool in = i < n && cursor >= 0 && cursor + i < logged;
    int4 row = make_int4(-1, -1, -1, 0);
    if (in) row = *reinterpret_cast<const int4*>(rows + (cursor + i) * 4);
    const int op = row.x, cl = row.y;
    const int64_t p = row.w;
    const bool ok = in && (op == LOGKV_OP_NEW_CLUSTER || op == LOGKV_OP_JOIN) && row.z == 0 && cl >= 0 && cl < K;
    if (in && !ok) err |= LOGKV_REPLAY_BAD_OP;
    int found = -1;
    if (ok) {
      // Lowest s in [0, n) with posb[ord[s]] >= p; the positions are sorted along s.
      int lo = 0, hi = n;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (posb[ord[mid]] < p) lo = mid + 1;
        else hi = mid;
      }
      if (lo < n && posb[ord[lo]] == p) found = lo;
      else err |= LOGKV_REPLAY_UNKNOWN_POSITION;
    }
    chunk_c[l] = found >= 0 ? cl : -1;
    chunk_p[l] = p;
    __syncthreads();
    bool last_of_cluster = false;
    if (found >= 0) {
      int j = l - 1;
      while (j >= 0 && chunk_c[j] != cl) --j;
      const bool has_prev = j >= 0 || seen[cl];
      const int64_t prev = j >= 0 ? chunk_p[j] : last_pos[cl];
      const bool was_alive = (alive >> cl) & 1u;
      if (op == LOGKV_OP_NEW_CLUSTER) {
        if (was_alive || has_prev) err |= LOGKV_REPLAY_BAD_CLUSTER;
      } else {
        if (!was_alive && !has_prev) err |= LOGKV_REPLAY_BAD_CLUSTER;
        if (has_prev && p <= prev) err |= LOGKV_REPLAY_BAD_ORDER;
      }
      as[found] = static_cast<int8_t>(cl);
      int k = l + 1;
      while (k < kWave && chunk_c[k] != cl) ++k;
      last_of_cluster = k == kWave;
    }
    __syncthreads();
    if (last_of_cluster) {
      seen[cl] = 1;
      last_pos[cl] = p;
    }
    __syncthreads();
  }
  // Every valid flush row named exactly once: n rows named n distinct rows.
  __threadfence_block();
  __syncthreads();
  for (int s = l; s < n; s += kWave)
    if (as[s] < 0) err |= LOGKV_REPLAY_UNCONSUMED;
  for (int d = 1; d < kWave; d <<= 1) err |= __shfl_xor(err, d, kWave);
  if (l == 0 && err) atomicOr(status, err);
  if (wards.jobs && l == 0) {
    wards.consumed[lane_ix] = n_ward_s + n;
    atomicMax(wards.steps, n_ward_s);
  }
}

int launch_record(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, const logkv_op_log_view& log,
                  hipStream_t stream) {
  const int lanes = c.n_batch * c.n_groups;
  hipLaunchKernelGGL(record_kernel, dim3(lanes), dim3(kRecordThreads), 0, stream, c, r, ws, log);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_replay(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, const logkv_op_log_view& log,
                  int64_t cursor, int32_t* status, hipStream_t stream) {
  const int lanes = c.n_batch * c.n_groups;
  int rc = launch_order(r, c.n_batch, ws.order, status, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(replay_kernel, dim3(lanes), dim3(kWave), 0, stream, c, r, ws, log, cursor, status, ReplayWards{});
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

int launch_record_wards(const LadderArgs& c, const int32_t* jobs, const int32_t* n_jobs, const logkv_op_log_view& log,
                        hipStream_t stream) {
  hipLaunchKernelGGL(record_ward_kernel, dim3(c.n_batch * c.n_groups), dim3(kWave), 0, stream, jobs, n_jobs, log);
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

// status[0]: the check bits, status[1]: the most merges of a lane (both
// cleared in stream order by the order launch's first block).
int launch_unified_replay(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, const logkv_op_log_view& log,
                          const int64_t* cursors, int32_t* consumed, int32_t* jobs, int32_t* n_jobs, int32_t* status,
                          hipStream_t stream) {
  const int lanes = c.n_batch * c.n_groups;
  int rc = launch_order(r, c.n_batch, ws.order, status, stream, 2);
  if (rc) return rc;
  hipLaunchKernelGGL(replay_kernel, dim3(lanes), dim3(kWave), 0, stream, c, r, ws, log, int64_t(0), status,
                     ReplayWards{cursors, consumed, jobs, n_jobs, status + 1});
  return hipGetLastError() == hipSuccess ? LOGKV_OK : LOGKV_ERUNTIME;
}

}  // namespace logkv
