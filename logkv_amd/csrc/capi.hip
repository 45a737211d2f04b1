// extern "C" entry points: argument validation, workspace carving, launches.
#include <cstdio>
#include <cstdarg>
#include <cstdint>
#include <cstring>
#include <cmath>

#include <algorithm>
#include <mutex>

#include "route.hpp"
#include "unified.hpp"

thread_local const char* logkv::g_refusal = nullptr;

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

// A launch function's failure: its refusal reason when it gave one, else the HIP error.
int launch_failed(int rc, const char* what) {
  const char* why = logkv::g_refusal;
  logkv::g_refusal = nullptr;
  return fail(rc, "%s launch failed: %s", what, why ? why : hipGetErrorString(hipGetLastError()));
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int check_ladder(const logkv_ladder_view* c) {
  if (!c) return fail(LOGKV_EINVAL, "ladder view is NULL");
  if (c->n_batch < 1 || c->n_groups < 1) return fail(LOGKV_EINVAL, "batch and groups must be >= 1");
  if (c->k_max < 1 || c->k_max > logkv::kMaxClusters)
    return fail(LOGKV_EINVAL, "cluster count %d outside [1, %d]", c->k_max, logkv::kMaxClusters);
  if (int64_t(c->n_batch) * c->n_groups * c->k_max > logkv::kMaxLadders)
    return fail(LOGKV_EINVAL, "batch * groups * clusters = %lld exceeds %d",
                (long long)(int64_t(c->n_batch) * c->n_groups * c->k_max), logkv::kMaxLadders);
  // level_count and the ladder plans hold per-level counts in int16.
  if (c->slots < 2 || c->slots > INT16_MAX)
    return fail(LOGKV_EINVAL, "slots per level must be in [2, %d], got %d", INT16_MAX, c->slots);
  if (c->levels < 1 || c->levels > logkv::kMaxLevels)
    return fail(LOGKV_EINVAL, "levels %d outside [1, %d]", c->levels, logkv::kMaxLevels);
  if (c->dk < 4 || c->dv < 4 || c->dk % 4 || c->dv % 4 || c->dk > logkv::kMaxDim || c->dv > logkv::kMaxDim)
    return fail(LOGKV_EINVAL, "key/value widths must be multiples of 4 in [4, %d], got %d/%d", logkv::kMaxDim,
                c->dk, c->dv);
  if (!c->level_k || !c->level_v || !c->level_w || !c->level_p_lo || !c->level_p_hi || !c->level_sum_wp ||
      !c->level_order || !c->pad_mask || !c->level_count || !c->centroid || !c->n_eff || !c->n_total ||
      !c->p_hi_c || !c->level0_phase || !c->alive || !c->s_h)
    return fail(LOGKV_EINVAL, "ladder view has a NULL buffer");
  if (reinterpret_cast<uintptr_t>(c->level_k) % 16 || reinterpret_cast<uintptr_t>(c->level_v) % 16 ||
      reinterpret_cast<uintptr_t>(c->centroid) % 16)
    return fail(LOGKV_EINVAL, "level_k, level_v and centroid must be 16-byte aligned");
  return LOGKV_OK;
}

int check_rows(const logkv_ladder_view* c, const logkv_rows_view* r) {
  if (!r) return fail(LOGKV_EINVAL, "rows view is NULL");
  if (r->tokens < 0 || r->tokens > logkv::kMaxOrderRows)
    return fail(LOGKV_EINVAL, "rows per flush %d outside [0, %d]", r->tokens, logkv::kMaxOrderRows);
  if (r->tokens && (!r->k || !r->v || !r->pos)) return fail(LOGKV_EINVAL, "rows view has a NULL buffer");
  if (reinterpret_cast<uintptr_t>(r->k) % 8 || reinterpret_cast<uintptr_t>(r->v) % 8 || r->k_st % 4 ||
      r->v_st % 4 || r->k_sb % 4 || r->k_sg % 4 || r->v_sb % 4 || r->v_sg % 4)
    return fail(LOGKV_EINVAL, "row tensors need 8-byte aligned rows (strides multiple of 4 elements)");
  (void)c;
  return LOGKV_OK;
}

struct Plan {
  int64_t order, assign, s_win, dist, snap, plans, tok, units, ladder, total;
  int64_t stride, s0, m0;
  int32_t sort_width;
};

// ward: the unified route's old-old merges stage both ladders' entries at level 0.
Plan plan_for(const logkv_ladder_view* c, int32_t tokens, int32_t late, int32_t ward = 0) {
  Plan p{};
  const int64_t lanes = int64_t(c->n_batch) * c->n_groups;
  const int64_t ladders = lanes * c->k_max;
  const int64_t existing = late ? int64_t(c->levels) * c->slots : 0;
  const int64_t m0 = std::max<int64_t>(tokens + existing, ward ? 2 * int64_t(c->levels) * c->slots : 0);
  p.s0 = late || ward ? m0 : 0;
  p.m0 = m0;
  p.stride = align256(logkv::ladder_scratch_bytes(*c, p.s0, p.m0));
  int64_t off = 0;
  p.order = off;
  off += align256(int64_t(c->n_batch) * tokens * 4);
  p.assign = off;
  off += align256(lanes * tokens);
  p.s_win = off;
  off += align256(lanes * tokens * 4);
  p.dist = off;
  off += align256(lanes * tokens * 4);
  p.snap = off;
  off += align256(ladders);
  p.plans = off;
  off += align256(ladders * int64_t(sizeof(logkv::LadderPlan)));
  p.tok = off;
  off += align256(ladders * tokens * 2);
  p.units = off;
  off += align256(int64_t(c->levels) * (ladders + 1) * 4);
  p.ladder = off;
  // A capped route's orphan distances live in the ladder scratch before the commit uses it.
  off += std::max(ladders * p.stride, align256(lanes * tokens * c->k_max * 4));
  p.total = off;
  int w = 1;
  while (late && w < m0) w <<= 1;
  p.sort_width = late ? w : 0;
  return p;
}

int carve(const logkv_ladder_view* c, const logkv_rows_view* r, const logkv_route_params* prm, void* workspace,
          int64_t bytes, int8_t* assign, int32_t* order, logkv::Workspace& ws, int ward = 0) {
  int rc = check_ladder(c);
  if (rc) return rc;
  if ((rc = check_rows(c, r))) return rc;
  if (!prm) return fail(LOGKV_EINVAL, "route params are NULL");
  if (prm->center_tile != 0 && prm->center_tile != 1 && prm->center_tile != logkv::kCenterTile)
    return fail(LOGKV_EINVAL, "center_tile must be 0, 1 or %d", logkv::kCenterTile);
  if (std::isnan(prm->hard_cap) || (prm->hard_cap > 0.f && prm->hard_cap_rows < 0))
    return fail(LOGKV_EINVAL, "hard_cap must not be NaN and hard_cap_rows must be >= 0");
  const int late = prm->late_joins ? 1 : 0;
  if (late && int64_t(c->levels) * c->slots + r->tokens > logkv::kMaxOrderRows)
    return fail(LOGKV_EINVAL, "delayed archive sort needs L*B' + T <= %d", logkv::kMaxOrderRows);
  if (ward && 2 * int64_t(c->levels) * c->slots > logkv::kMaxOrderRows)
    return fail(LOGKV_EINVAL, "old-old merges need 2*L*B' <= %d", logkv::kMaxOrderRows);
  const Plan p = plan_for(c, r->tokens, late, ward);
  if (!workspace || bytes < p.total)
    return fail(LOGKV_EINVAL, "workspace of %lld bytes is smaller than the %lld required", (long long)bytes,
                (long long)p.total);
  uint8_t* base = static_cast<uint8_t*>(workspace);
  ws.order = order ? order : reinterpret_cast<int32_t*>(base + p.order);
  ws.assign = assign ? assign : reinterpret_cast<int8_t*>(base + p.assign);
  ws.s_win = reinterpret_cast<float*>(base + p.s_win);
  ws.dist = reinterpret_cast<float*>(base + p.dist);
  ws.snap_alive = base + p.snap;
  ws.ladder = base + p.ladder;
  ws.cap_dist = reinterpret_cast<float*>(base + p.ladder);
  ws.ladder_stride = p.stride;
  ws.s0_rows = p.s0;
  ws.m0_cap = p.m0;
  ws.plans = reinterpret_cast<logkv::LadderPlan*>(base + p.plans);
  ws.tok = reinterpret_cast<uint16_t*>(base + p.tok);
  ws.units = reinterpret_cast<int32_t*>(base + p.units);
  ws.sort_width = p.sort_width;
  return LOGKV_OK;
}

// The unified route's region, after the route workspace sized for old-old
// merges. With base == NULL only the size is computed.
int64_t unified_layout(const logkv_ladder_view* c, int32_t tokens, int32_t late, uint8_t* base,
                       logkv::UnifiedBufs* u, int64_t* stats_offset = nullptr) {
  const int64_t lanes = int64_t(c->n_batch) * c->n_groups;
  const int64_t M = int64_t(tokens) + c->k_max, D = c->dk;
  int64_t off = align256(plan_for(c, tokens, late, 1).total);
  auto take = [&](int64_t bytes) {
    uint8_t* at = base ? base + off : nullptr;
    off += align256(bytes);
    return at;
  };
  logkv::UnifiedBufs b{};
  b.M = static_cast<int32_t>(M);
  b.D = static_cast<int32_t>(D);
  b.mu1 = reinterpret_cast<float*>(take(lanes * M * D * 4));
  b.mass1 = reinterpret_cast<float*>(take(lanes * M * 4));
  b.count1 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.mu2 = reinterpret_cast<float*>(take(lanes * M * D * 4));
  b.mass2 = reinterpret_cast<float*>(take(lanes * M * 4));
  b.count2 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.dist = reinterpret_cast<float*>(take(lanes * M * M * 4));
  b.bound = reinterpret_cast<float*>(take(lanes * M * 4));
  b.alive1 = take(lanes * M);
  b.alive2 = take(lanes * M);
  b.trace1 = reinterpret_cast<int32_t*>(take(lanes * M * 8));
  b.trace2 = reinterpret_cast<int32_t*>(take(lanes * M * 8));
  b.n_trace1 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.n_trace2 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.stuck1 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.stuck2 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.label1 = reinterpret_cast<int32_t*>(take(lanes * M * 4));
  b.label2 = reinterpret_cast<int32_t*>(take(lanes * M * 4));
  b.n_roots1 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.n_roots2 = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.n_old = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.old_ids = reinterpret_cast<int32_t*>(take(lanes * logkv::kMaxClusters * 4));
  b.jobs = reinterpret_cast<int32_t*>(take(lanes * logkv::kMaxClusters * 8));
  b.n_jobs = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.image_stride = logkv::unified_image_stride(static_cast<int>(M));
  b.image = take(lanes * b.image_stride);
  b.ctl = reinterpret_cast<logkv::LaneCtl*>(take(lanes * static_cast<int64_t>(sizeof(logkv::LaneCtl))));
  b.live = reinterpret_cast<int16_t*>(take(lanes * M * 6));
  if (stats_offset) *stats_offset = off;
  b.stats = reinterpret_cast<int32_t*>(take(lanes * 2 * logkv::kStatsInts * 4));
  b.restricted = reinterpret_cast<uint64_t*>(take(lanes * M * 8));
  for (int s = 0; s < 2; ++s) {
    b.cmu[s] = reinterpret_cast<float*>(take(lanes * M * D * 4));
    b.cmass[s] = reinterpret_cast<float*>(take(lanes * M * 4));
    b.crad[s] = reinterpret_cast<float*>(take(lanes * M * 4));
    b.croot[s] = reinterpret_cast<int32_t*>(take(lanes * M * 4));
  }
  b.n_cur = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.cbuf = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.dcount = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.rounds = reinterpret_cast<int32_t*>(take(lanes * 4));
  b.keys = reinterpret_cast<uint64_t*>(take(lanes * M * 16));
  if (u) *u = b;
  return off;
}

int check_unified(const logkv_ladder_view* c, const logkv_rows_view* r) {
  if (int64_t(r->tokens) + c->k_max > logkv::kMaxNodes)
    return fail(LOGKV_EINVAL, "the unified route takes at most %d rows + clusters per flush, got %d + %d",
                logkv::kMaxNodes, r->tokens, c->k_max);
  if (logkv::unified_reduce_lds(r->tokens + c->k_max) > 160 * 1024)
    return fail(LOGKV_EINVAL, "unified reducer state exceeds the LDS of a CU");
  return LOGKV_OK;
}

}  // namespace

namespace {

// Argument checks shared by the two decode entry points (workspace and static scratch).
int check_decode(const logkv_attention_args* a, const int32_t* table, int64_t table_ints) {
  if (!a || !table || table_ints < 1) return fail(LOGKV_EINVAL, "attention args or plan table are NULL");
  if (a->n_groups < 1 || a->n_heads % a->n_groups) return fail(LOGKV_EINVAL, "heads must be a multiple of groups");
  const int nq = (a->n_heads / a->n_groups) * a->tq;
  if (a->tq < 1 || nq > 16) return fail(LOGKV_EINVAL, "queries per KV group (%d) must be in [1, 16]", nq);
  if (a->dim % 8 || a->dim > 264 || a->dim <= a->dk || a->dim < a->dv || a->dv > logkv::kMaxDim)
    return fail(LOGKV_EINVAL, "bad packed width %d", a->dim);
  if (a->causal_tail < 0 || a->causal_tail > a->tail || (a->causal_tail && a->causal_tail != a->tq))
    return fail(LOGKV_EINVAL, "causal_tail must be 0 or the query length");
  if (a->n_batch < 1 || a->cap < 1 || a->tail < 0 || a->tail > a->cap)
    return fail(LOGKV_EINVAL, "attention needs n_batch >= 1 and 0 <= tail <= cap (cap >= 1)");
  if (!a->q || !a->k || !a->v || !a->out) return fail(LOGKV_EINVAL, "attention buffer is NULL");
  // The streaming and tiled kernels read packed rows in 16-byte units.
  if (reinterpret_cast<uintptr_t>(a->k) % 16 || reinterpret_cast<uintptr_t>(a->v) % 16)
    return fail(LOGKV_EINVAL, "packed K/V must be 16-byte aligned");
  return LOGKV_OK;
}

// Device-resident scratch of logkv_decode_attention_static: the split partials of one
// decode call, for callers that cannot allocate. Each GPU holds its own copy for the
// life of the process; in host code the array's name is not a device address, so its
// address is taken once per device with hipGetSymbolAddress and only that is used.
constexpr int64_t kStaticScratchBytes = int64_t(16) << 20;
constexpr int kMaxScratchDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
void* g_scratch_ptr[kMaxScratchDevices] = {};
std::mutex g_scratch_mutex;

int static_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail(LOGKV_ERUNTIME, "no current HIP device for the static scratch");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return fail(LOGKV_ERUNTIME, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(err));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LOGKV_OK;
}

}  // namespace

extern "C" {

const char* logkv_last_error(void) { return g_error; }

int64_t logkv_unified_workspace_bytes(const logkv_ladder_view* cache, int32_t tokens, int32_t late_joins) {
  if (check_ladder(cache) || tokens < 0) return -1;
  return unified_layout(cache, tokens, late_joins ? 1 : 0, nullptr, nullptr);
}

int64_t logkv_unified_stats_offset(const logkv_ladder_view* cache, int32_t tokens, int32_t late_joins) {
  if (check_ladder(cache) || tokens < 0) return -1;
  int64_t at = -1;
  unified_layout(cache, tokens, late_joins ? 1 : 0, nullptr, nullptr, &at);
  return at;
}

int logkv_unified_plan(const logkv_ladder_view* cache, const logkv_rows_view* rows, const logkv_route_params* params,
                       const float* limits, void* workspace, int64_t workspace_bytes, int32_t* summary, void* stream) {
  logkv::Workspace ws{};
  int rc = carve(cache, rows, params, workspace, workspace_bytes, nullptr, nullptr, ws, 1);
  if (rc) return rc;
  if ((rc = check_unified(cache, rows))) return rc;
  if (!limits || !summary) return fail(LOGKV_EINVAL, "radius limits or summary are NULL");
  const int64_t need = unified_layout(cache, rows->tokens, params->late_joins ? 1 : 0, nullptr, nullptr);
  if (workspace_bytes < need)
    return fail(LOGKV_EINVAL, "workspace of %lld bytes is smaller than the %lld required", (long long)workspace_bytes,
                (long long)need);
  if (params->merge_passes < 0) return fail(LOGKV_EINVAL, "merge_passes must be >= 0 (0 or 1: one matching pass)");
  logkv::UnifiedBufs u{};
  unified_layout(cache, rows->tokens, params->late_joins ? 1 : 0, static_cast<uint8_t*>(workspace), &u);
  u.limit = limits;
  u.passes = params->merge_passes > 1 ? params->merge_passes : 1;
  u.cap = params->hard_cap > 0.f ? params->hard_cap : 0.f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = rows->tokens ? logkv::launch_unified_plan(*cache, *rows, u, ws, s) : LOGKV_OK;
  if (!rc) rc = logkv::launch_unified_summary(*cache, u, summary, rows->tokens, s);
  if (rc) return launch_failed(rc, "unified plan");
  return LOGKV_OK;
}

int logkv_unified_commit(const logkv_ladder_view* cache, const logkv_rows_view* rows, const logkv_route_params* params,
                         void* workspace, int64_t workspace_bytes, int32_t merge_steps, void* stream) {
  logkv::Workspace ws{};
  int rc = carve(cache, rows, params, workspace, workspace_bytes, nullptr, nullptr, ws, 1);
  if (rc) return rc;
  if ((rc = check_unified(cache, rows))) return rc;
  if (merge_steps < 0 || merge_steps > cache->k_max) return fail(LOGKV_EINVAL, "merge steps outside [0, K]");
  if (!rows->tokens) return LOGKV_OK;
  logkv::UnifiedBufs u{};
  unified_layout(cache, rows->tokens, params->late_joins ? 1 : 0, static_cast<uint8_t*>(workspace), &u);
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int step = 0; step < merge_steps && !rc; ++step) {
    rc = logkv::launch_ward_step(*cache, ws, u.jobs, u.n_jobs, step, s);
    if (!rc) rc = logkv::launch_levels(*cache, *rows, *params, ws, s);
  }
  if (!rc) rc = logkv::launch_commit(*cache, *rows, *params, ws, s);
  if (rc) return launch_failed(rc, "unified commit");
  return LOGKV_OK;
}

int64_t logkv_route_workspace_bytes(const logkv_ladder_view* cache, int32_t tokens, int32_t late_joins) {
  if (check_ladder(cache) || tokens < 0) return -1;
  return plan_for(cache, tokens, late_joins ? 1 : 0).total;
}

int logkv_attach_assign(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                        const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                        int8_t* assign, int32_t* order, void* stream) {
  logkv::Workspace ws{};
  int rc = carve(cache, rows, params, workspace, workspace_bytes, assign, order, ws);
  if (rc) return rc;
  if (!rows->tokens) return LOGKV_OK;
  rc = logkv::launch_route(*cache, *rows, *params, ws, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "attach");
  return LOGKV_OK;
}

int logkv_route_commit(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                       const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                       int8_t* assign, int32_t* order, void* stream) {
  logkv::Workspace ws{};
  int rc = carve(cache, rows, params, workspace, workspace_bytes, assign, order, ws);
  if (rc) return rc;
  if (!rows->tokens) return LOGKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = logkv::launch_route(*cache, *rows, *params, ws, s);
  if (!rc) rc = logkv::launch_commit(*cache, *rows, *params, ws, s);
  if (rc) return launch_failed(rc, "route/commit");
  return LOGKV_OK;
}

int logkv_commit_only(const logkv_ladder_view* cache, const logkv_rows_view* rows, const logkv_route_params* params,
                      void* workspace, int64_t workspace_bytes, const int8_t* assign, const int32_t* order,
                      void* stream) {
  logkv::Workspace ws{};
  int rc = carve(cache, rows, params, workspace, workspace_bytes, const_cast<int8_t*>(assign),
                 const_cast<int32_t*>(order), ws);
  if (rc) return rc;
  if (!rows->tokens) return LOGKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = logkv::launch_commit(*cache, *rows, *params, ws, s);
  if (rc) return launch_failed(rc, "commit");
  return LOGKV_OK;
}

namespace {

int check_log(const logkv_ladder_view* c, const logkv_op_log_view* log) {
  if (!log || !log->rows || !log->lengths) return fail(LOGKV_EINVAL, "op-log view or its buffers are NULL");
  if (log->capacity < 1) return fail(LOGKV_EINVAL, "op-log capacity must be positive");
  if (reinterpret_cast<uintptr_t>(log->rows) % 16) return fail(LOGKV_EINVAL, "op-log rows must be 16-byte aligned");
  (void)c;
  return LOGKV_OK;
}

}  // namespace

int logkv_record_ops(const logkv_ladder_view* cache, const logkv_rows_view* rows, void* workspace,
                     int64_t workspace_bytes, const logkv_op_log_view* log, void* stream) {
  // The plan, row-list and alive-snapshot regions sit before the delayed-archive
  // staging, at offsets that do not depend on late joins.
  const logkv_route_params plain{1.f, 1.f, 1.f, 0, 0};
  logkv::Workspace ws{};
  int rc = carve(cache, rows, &plain, workspace, workspace_bytes, nullptr, nullptr, ws);
  if (rc) return rc;
  if ((rc = check_log(cache, log))) return rc;
  if (!rows->tokens) return LOGKV_OK;
  rc = logkv::launch_record(*cache, *rows, ws, *log, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "op-log record");
  return LOGKV_OK;
}

int logkv_replay_commit(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                        const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                        const logkv_op_log_view* log, int64_t cursor, int32_t* status, void* stream) {
  logkv::Workspace ws{};
  int rc = carve(cache, rows, params, workspace, workspace_bytes, nullptr, nullptr, ws);
  if (rc) return rc;
  if ((rc = check_log(cache, log))) return rc;
  if (!status) return fail(LOGKV_EINVAL, "replay status pointer is NULL");
  if (cursor < 0) return fail(LOGKV_EINVAL, "replay cursor must be >= 0");
  if (!rows->tokens) return LOGKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = logkv::launch_replay(*cache, *rows, ws, *log, cursor, status, s);
  ws.abort = status;
  if (!rc) rc = logkv::launch_commit(*cache, *rows, *params, ws, s);
  if (rc) return launch_failed(rc, "replay");
  return LOGKV_OK;
}

namespace {

// Carves the unified workspace as logkv_unified_plan / logkv_unified_commit do.
int unified_bufs(const logkv_ladder_view* cache, const logkv_rows_view* rows, const logkv_route_params* params,
                 void* workspace, int64_t workspace_bytes, logkv::Workspace& ws, logkv::UnifiedBufs& u) {
  int rc = carve(cache, rows, params, workspace, workspace_bytes, nullptr, nullptr, ws, 1);
  if (rc) return rc;
  if ((rc = check_unified(cache, rows))) return rc;
  const int late = params->late_joins ? 1 : 0;
  const int64_t need = unified_layout(cache, rows->tokens, late, nullptr, nullptr);
  if (workspace_bytes < need)
    return fail(LOGKV_EINVAL, "workspace of %lld bytes is smaller than the %lld required", (long long)workspace_bytes,
                (long long)need);
  unified_layout(cache, rows->tokens, late, static_cast<uint8_t*>(workspace), &u);
  return LOGKV_OK;
}

}  // namespace

int logkv_unified_record_ops(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                             const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                             const logkv_op_log_view* log, void* stream) {
  logkv::Workspace ws{};
  logkv::UnifiedBufs u{};
  int rc = unified_bufs(cache, rows, params, workspace, workspace_bytes, ws, u);
  if (rc) return rc;
  if ((rc = check_log(cache, log))) return rc;
  if (!rows->tokens) return LOGKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = logkv::launch_record_wards(*cache, u.jobs, u.n_jobs, *log, s);
  if (!rc) rc = logkv::launch_record(*cache, *rows, ws, *log, s);
  if (rc) return launch_failed(rc, "op-log record");
  return LOGKV_OK;
}

int logkv_unified_replay_plan(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                              const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                              const logkv_op_log_view* log, const int64_t* cursors, int32_t* consumed,
                              int32_t* status, void* stream) {
  logkv::Workspace ws{};
  logkv::UnifiedBufs u{};
  int rc = unified_bufs(cache, rows, params, workspace, workspace_bytes, ws, u);
  if (rc) return rc;
  if ((rc = check_log(cache, log))) return rc;
  if (!cursors || !consumed || !status) return fail(LOGKV_EINVAL, "replay cursors, consumed or status are NULL");
  if (!rows->tokens) return LOGKV_OK;
  rc = logkv::launch_unified_replay(*cache, *rows, ws, *log, cursors, consumed, u.jobs, u.n_jobs, status,
                                    static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "replay");
  return LOGKV_OK;
}

int logkv_unified_decisions(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                            const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                            int8_t* assign, int32_t* order, int32_t* jobs, int32_t* n_jobs, int32_t into_workspace,
                            void* stream) {
  logkv::Workspace ws{};
  logkv::UnifiedBufs u{};
  int rc = unified_bufs(cache, rows, params, workspace, workspace_bytes, ws, u);
  if (rc) return rc;
  if (!assign || !order || !jobs || !n_jobs) return fail(LOGKV_EINVAL, "decision buffers are NULL");
  const int64_t lanes = int64_t(cache->n_batch) * cache->n_groups;
  struct Region {
    void* ws;
    void* user;
    int64_t bytes;
  } const regions[4] = {{ws.assign, assign, lanes * rows->tokens},
                        {ws.order, order, int64_t(cache->n_batch) * rows->tokens * 4},
                        {u.jobs, jobs, lanes * logkv::kMaxClusters * 8},
                        {u.n_jobs, n_jobs, lanes * 4}};
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (const Region& g : regions) {
    const hipError_t e = into_workspace ? hipMemcpyAsync(g.ws, g.user, g.bytes, hipMemcpyDeviceToDevice, s)
                                        : hipMemcpyAsync(g.user, g.ws, g.bytes, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return fail(LOGKV_ERUNTIME, "decision copy failed: %s", hipGetErrorString(e));
  }
  return LOGKV_OK;
}

int logkv_score_spans(const logkv_span_args* a, float* scores, void* stream) {
  if (!a || !scores) return fail(LOGKV_EINVAL, "span args or output are NULL");
  if (a->n_spans < 0) return fail(LOGKV_EINVAL, "negative span count");
  if (a->n_groups < 1 || a->n_groups > 16)
    return fail(LOGKV_EINVAL, "span scoring supports 1..16 KV groups, got %d", a->n_groups);
  if (a->dk < 1 || a->dv < 1 || a->dk > logkv::kMaxDim || a->dv > logkv::kMaxDim)
    return fail(LOGKV_EINVAL, "span scoring widths must be in [1, %d]", logkv::kMaxDim);
  if (a->n_spans && (!a->tokens || !a->span_offsets || !a->span_rows || !a->flush_k || !a->flush_v))
    return fail(LOGKV_EINVAL, "span tables or rows are NULL");
  if (a->old_width > 0 && (!a->pool_k || !a->pool_v)) return fail(LOGKV_EINVAL, "pool rows are NULL");
  if (a->beta_novelty && (!a->centroids || !a->centroid_valid || a->k_max < 1))
    return fail(LOGKV_EINVAL, "Beta novelty needs centroids and their valid flags");
  const int rc = logkv::launch_score(*a, scores, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "score");
  return LOGKV_OK;
}

int logkv_alpha_partition(const logkv_partition_args* a, void* stream) {
  if (!a) return fail(LOGKV_EINVAL, "partition args are NULL");
  if (a->P < 0 || a->A < 0 || a->n_batch < 1 || a->n_groups < 1) return fail(LOGKV_EINVAL, "bad partition sizes");
  if (a->dk % 4 || a->dv % 4 || a->dk < 4 || a->dv < 4)
    return fail(LOGKV_EINVAL, "partition widths must be multiples of 4");
  if ((a->P && (!a->out_pool_k || !a->out_pool_v || !a->out_pool_pos || !a->out_pool_valid || !a->keep)) ||
      (a->A && (!a->arch_k || !a->arch_v || !a->arch_pos || !a->archive)))
    return fail(LOGKV_EINVAL, "partition outputs or index tables are NULL");
  const int rc = logkv::launch_partition(*a, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "partition");
  return LOGKV_OK;
}

static int check_select(const logkv_alpha_select_args* a) {
  if (!a) return fail(LOGKV_EINVAL, "select args are NULL");
  if (a->n_batch < 1 || a->budget < 1 || a->max_span < 1 || a->max_span > a->budget || a->tokens < 0)
    return fail(LOGKV_EINVAL, "bad selection sizes");
  if (int64_t(a->budget) + a->tokens + 1 > logkv::kMaxCandidates)
    return fail(LOGKV_EINVAL, "budget + rows + 1 = %d exceeds %d candidates per batch row",
                a->budget + a->tokens + 1, logkv::kMaxCandidates);
  if (!a->span_len || !a->span_closed || !a->span_count || !a->pool_pos || !a->keep || !a->archive ||
      !a->archive_count || !a->new_span_len || !a->new_span_closed || !a->new_span_count || !a->alpha_count)
    return fail(LOGKV_EINVAL, "selection buffer is NULL");
  if (a->tokens && (!a->new_pos || !a->ends)) return fail(LOGKV_EINVAL, "new positions or boundaries are NULL");
  if (a->count_rows < 0 || (a->count_rows && a->n_batch % a->count_rows))
    return fail(LOGKV_EINVAL, "count_rows %d must be 0 or divide the %d batch rows", a->count_rows, a->n_batch);
  const logkv_span_args& r = a->rows;
  if (r.n_groups < 1 || r.n_groups > 16 || r.dk < 1 || r.dv < 1 || r.dk > logkv::kMaxDim || r.dv > logkv::kMaxDim)
    return fail(LOGKV_EINVAL, "bad groups or widths");
  if (!r.pool_k || !r.pool_v || (a->tokens && (!r.flush_k || !r.flush_v)))
    return fail(LOGKV_EINVAL, "span row tensors are NULL");
  if (r.beta_novelty && (!r.centroids || !r.centroid_valid || r.k_max < 1))
    return fail(LOGKV_EINVAL, "Beta novelty needs centroids");
  if (a->span_len == a->new_span_len || a->span_closed == a->new_span_closed)
    return fail(LOGKV_EINVAL, "the new selection must not overwrite the current one");
  return LOGKV_OK;
}

int64_t logkv_alpha_select_workspace_bytes(const logkv_alpha_select_args* a) {
  if (check_select(a)) return -1;
  return logkv::select_workspace_bytes(*a);
}

int logkv_alpha_select(const logkv_alpha_select_args* a, void* ws, int64_t ws_bytes, void* stream) {
  int rc = check_select(a);
  if (rc) return rc;
  if (!ws || ws_bytes < logkv::select_workspace_bytes(*a)) return fail(LOGKV_EINVAL, "selection workspace too small");
  rc = logkv::launch_select(*a, ws, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "selection");
  return LOGKV_OK;
}

int64_t logkv_plan_table_ints(const logkv_readout_view* c) {
  if (!c) return -1;
  return int64_t(c->n_batch) * c->n_groups * (int64_t(c->k_max) * c->levels + 1) + 1;
}

static int check_readout(const logkv_readout_view* c) {
  if (!c) return fail(LOGKV_EINVAL, "readout view is NULL");
  if (c->n_batch < 1 || c->n_groups < 1 || c->k_max < 1 || c->levels < 1 || c->slots < 1)
    return fail(LOGKV_EINVAL, "bad readout sizes");
  if (c->dk < 1 || c->dv < 1 || c->dk > logkv::kMaxDim || c->dv > logkv::kMaxDim)
    return fail(LOGKV_EINVAL, "readout widths must be in [1, %d]", logkv::kMaxDim);
  if (!c->level_k || !c->level_v || !c->level_w || !c->level_sum_wp || !c->level_count)
    return fail(LOGKV_EINVAL, "readout ladder buffer is NULL");
  if (c->alpha_count < 0 || c->alpha_count > c->alpha_cap ||
      ((c->alpha_count || c->alpha_count_dev) && (!c->alpha_k || !c->alpha_v || !c->alpha_pos || !c->alpha_valid)))
    return fail(LOGKV_EINVAL, "bad exact pool view");
  if (c->recent_count < 0 || c->recent_count > c->recent_cap || (c->recent_count && (!c->recent_k || !c->recent_v)))
    return fail(LOGKV_EINVAL, "bad recent window view");
  if (!c->cos || !c->sin || c->rope_n < 0 || c->rope_n > c->dk || c->rope_n % 2 || c->rope_rows < 1)
    return fail(LOGKV_EINVAL, "bad RoPE tables");
  return LOGKV_OK;
}

int logkv_mid_plan(const logkv_readout_view* c, int32_t* table, void* stream) {
  int rc = check_readout(c);
  if (rc) return rc;
  if (!table) return fail(LOGKV_EINVAL, "plan table is NULL");
  rc = logkv::launch_plan(*c, table, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "plan");
  return LOGKV_OK;
}

int logkv_pack(const logkv_readout_view* c, const logkv_pack_args* p, const int32_t* table, void* stream) {
  int rc = check_readout(c);
  if (rc) return rc;
  if (!p || !table || !p->out_k || !p->out_v) return fail(LOGKV_EINVAL, "pack outputs or plan table are NULL");
  if (p->dim <= c->dk || p->dim < c->dv || p->dim % 8 || p->dim > 264)
    return fail(LOGKV_EINVAL, "packed width %d must exceed dk, hold dv, be a multiple of 8 and <= 264", p->dim);
  if (p->cur_len < 0 || (p->cur_len && (!p->cur_k || !p->cur_v)) || p->recent_start < 0 ||
      p->recent_start > c->recent_count || p->out_cap < 0)
    return fail(LOGKV_EINVAL, "bad current rows or output capacity");
  if (p->cur_len && (reinterpret_cast<uintptr_t>(p->cur_k) % 8 || reinterpret_cast<uintptr_t>(p->cur_v) % 8 ||
                     p->ck_sb % 4 || p->ck_sg % 4 || p->ck_st % 4 || p->cv_sb % 4 || p->cv_sg % 4 || p->cv_st % 4))
    return fail(LOGKV_EINVAL, "current rows must be 8-byte aligned (strides multiples of 4 elements)");
  rc = logkv::launch_pack(*c, *p, table, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "pack");
  return LOGKV_OK;
}

int64_t logkv_attention_workspace_bytes(const logkv_attention_args* a) {
  if (!a || a->n_groups < 1) return -1;
  return logkv::attention_workspace_floats(*a) * 4;
}

int logkv_decode_attention(const logkv_attention_args* a, const int32_t* table, int64_t table_ints, void* ws,
                           int64_t ws_bytes, void* stream) {
  int rc = check_decode(a, table, table_ints);
  if (rc) return rc;
  if (!ws || ws_bytes < logkv::attention_workspace_floats(*a) * 4)
    return fail(LOGKV_EINVAL, "attention workspace too small");
  rc = logkv::launch_attention(*a, table + table_ints - 1, static_cast<float*>(ws), static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "attention");
  return LOGKV_OK;
}

int logkv_decode_attention_static(const logkv_attention_args* a, const int32_t* table, int64_t table_ints,
                                  void* stream) {
  int rc = check_decode(a, table, table_ints);
  if (rc) return rc;
  const int64_t need = logkv::attention_workspace_floats(*a) * 4;
  if (need > kStaticScratchBytes)
    return fail(LOGKV_EINVAL, "decode partials need %lld bytes, above the static scratch of %lld bytes",
                (long long)need, (long long)kStaticScratchBytes);
  void* scratch_ptr = nullptr;
  rc = static_scratch(&scratch_ptr);
  if (rc) return rc;
  rc = logkv::launch_attention(*a, table + table_ints - 1, static_cast<float*>(scratch_ptr),
                               static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "attention");
  return LOGKV_OK;
}

int64_t logkv_chunk_workspace_bytes(const logkv_attention_args* a) {
  if (!a || a->n_groups < 1 || a->n_heads % a->n_groups || a->n_batch < 1 || a->cap < 1 || a->tq < 1 ||
      a->dv < 1 || a->dv > logkv::kMaxDim)
    return -1;
  return logkv::chunk_workspace_floats(*a) * 4;
}

int logkv_chunk_attention(const logkv_attention_args* a, const int32_t* table, int64_t table_ints, void* ws,
                          int64_t ws_bytes, void* stream) {
  if (!a || !table || table_ints < 1) return fail(LOGKV_EINVAL, "attention args or plan table are NULL");
  if (a->n_groups < 1 || a->n_heads % a->n_groups) return fail(LOGKV_EINVAL, "heads must be a multiple of groups");
  if (a->tq < 1) return fail(LOGKV_EINVAL, "query length must be >= 1");
  if (a->dim % 8 || a->dim > 144 || a->dim <= a->dk || a->dim < a->dv)
    return fail(LOGKV_EINVAL, "chunk attention takes packed widths up to 144 (multiples of 8), got %d", a->dim);
  if (a->dv % 32 || a->dv < 32 || a->dv > 128) return fail(LOGKV_EINVAL, "chunk attention takes dv in {32, 64, 96, 128}");
  if (a->causal_tail < 0 || a->causal_tail > a->tail || (a->causal_tail && a->causal_tail != a->tq))
    return fail(LOGKV_EINVAL, "causal_tail must be 0 or the query length");
  if (a->n_batch < 1 || a->cap < 1 || a->tail < 0 || a->tail > a->cap)
    return fail(LOGKV_EINVAL, "attention needs n_batch >= 1 and 0 <= tail <= cap (cap >= 1)");
  if (!a->q || !a->k || !a->v || !a->out) return fail(LOGKV_EINVAL, "attention buffer is NULL");
  if (reinterpret_cast<uintptr_t>(a->out) % 8 || a->o_st % 4 || a->o_sh % 4 || a->o_sb % 4)
    return fail(LOGKV_EINVAL, "chunk attention output rows must be 8-byte aligned");
  if (reinterpret_cast<uintptr_t>(a->k) % 16 || reinterpret_cast<uintptr_t>(a->v) % 16)
    return fail(LOGKV_EINVAL, "packed K/V must be 16-byte aligned");
  if (ws_bytes < logkv::chunk_workspace_floats(*a) * 4 || (logkv::chunk_workspace_floats(*a) && !ws))
    return fail(LOGKV_EINVAL, "chunk attention workspace too small");
  const int rc = logkv::launch_chunk_attention(*a, table + table_ints - 1, static_cast<float*>(ws),
                                               static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "chunk attention");
  return LOGKV_OK;
}

namespace {
int check_recent(const logkv_recent_args* a) {
  if (!a) return fail(LOGKV_EINVAL, "recent args are NULL");
  if (a->n_batch < 1 || a->n_groups < 1 || a->cap < 1)
    return fail(LOGKV_EINVAL, "recent window needs n_batch, n_groups, cap >= 1");
  for (int d : {a->dk, a->dkr, a->dv})
    if (d < 4 || d % 4 || d > logkv::kMaxDim)
      return fail(LOGKV_EINVAL, "recent feature counts must be multiples of 4 in [4, %d]", logkv::kMaxDim);
  if (!a->recent_k || !a->recent_k_raw || !a->recent_v || !a->recent_pos)
    return fail(LOGKV_EINVAL, "recent buffer is NULL");
  if (reinterpret_cast<uintptr_t>(a->recent_k) % 8 || reinterpret_cast<uintptr_t>(a->recent_k_raw) % 8 ||
      reinterpret_cast<uintptr_t>(a->recent_v) % 8)
    return fail(LOGKV_EINVAL, "recent buffers must be 8-byte aligned");
  return LOGKV_OK;
}
}  // namespace

int logkv_recent_append(const logkv_recent_args* a, int32_t at, int32_t n, void* stream) {
  int rc = check_recent(a);
  if (rc) return rc;
  if (at < 0 || n < 0 || int64_t(at) + n > a->cap)
    return fail(LOGKV_EINVAL, "append of %d rows at %d exceeds the recent capacity %d", n, at, a->cap);
  if (n == 0) return LOGKV_OK;
  if (!a->k || !a->k_raw || !a->v || !a->pos) return fail(LOGKV_EINVAL, "append source is NULL");
  if ((a->recent_ends == nullptr) != (a->ends == nullptr))
    return fail(LOGKV_EINVAL, "span flags must be given exactly when the window keeps them");
  if (reinterpret_cast<uintptr_t>(a->k) % 8 || reinterpret_cast<uintptr_t>(a->k_raw) % 8 ||
      reinterpret_cast<uintptr_t>(a->v) % 8 || a->k_sb % 4 || a->k_sg % 4 || a->k_st % 4 || a->kr_sb % 4 ||
      a->kr_sg % 4 || a->kr_st % 4 || a->v_sb % 4 || a->v_sg % 4 || a->v_st % 4)
    return fail(LOGKV_EINVAL, "append sources need 8-byte aligned rows (strides multiple of 4 elements)");
  rc = logkv::launch_recent_append(*a, at, n, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "recent append");
  return LOGKV_OK;
}

int logkv_recent_shift(const logkv_recent_args* a, int32_t take, int32_t count, void* stream) {
  int rc = check_recent(a);
  if (rc) return rc;
  if (take < 1 || take > count || count > a->cap || count - take > take)
    return fail(LOGKV_EINVAL, "shift of %d of %d rows needs 1 <= take <= count <= cap and count - take <= take",
                take, count);
  rc = logkv::launch_recent_shift(*a, take, count, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "recent shift");
  return LOGKV_OK;
}

int logkv_beta_merge(const logkv_beta_args* a, int32_t* status, void* stream) {
  if (!a) return fail(LOGKV_EINVAL, "Beta merge args are NULL");
  if (a->n_rows < 0 || a->n_rows % 2) return fail(LOGKV_EINVAL, "Beta merge needs an even row count, got %lld",
                                                  (long long)a->n_rows);
  if (a->dk < 1 || a->dv < 1 || a->dk > logkv::kMaxDim || a->dv > logkv::kMaxDim)
    return fail(LOGKV_EINVAL, "Beta merge widths must be in [1, %d], got %d/%d", logkv::kMaxDim, a->dk, a->dv);
  if (a->k_st < a->dk || a->v_st < a->dv) return fail(LOGKV_EINVAL, "Beta merge row strides below the widths");
  if (a->n_groups < 0 || a->n_groups > a->n_rows / 2 + 1)
    return fail(LOGKV_EINVAL, "Beta merge layout of %lld groups for %lld rows", (long long)a->n_groups,
                (long long)a->n_rows);
  if (a->n_groups == 0) return LOGKV_OK;
  if (!a->k || !a->v || !a->w || !a->layout || !a->cuts)
    return fail(LOGKV_EINVAL, "Beta merge rows, masses, layout or cuts are NULL");
  if (a->out_k && (!a->out_v || !a->out_w)) return fail(LOGKV_EINVAL, "Beta merge outputs K, V and w go together");
  if (a->apply && !a->out_k) return fail(LOGKV_EINVAL, "applying recorded cuts needs the outputs");
  const int rc = logkv::launch_beta_merge(*a, status, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "Beta merge");
  return LOGKV_OK;
}

int logkv_pack_slots(const logkv_slot_pack_args* a, void* stream) {
  if (!a) return fail(LOGKV_EINVAL, "slot pack args are NULL");
  if (a->n_batch < 1 || a->n_groups < 1 || a->slots < 0 || a->slots > a->out_cap)
    return fail(LOGKV_EINVAL, "slot pack shape: batch %d, groups %d, %d slots into %d rows", a->n_batch,
                a->n_groups, a->slots, a->out_cap);
  if (a->dk < 4 || a->dv < 4 || a->dk % 4 || a->dv % 4 || a->dim % 8 || a->dim <= a->dk || a->dim < a->dv ||
      a->dim > 264)
    return fail(LOGKV_EINVAL, "slot pack widths dk %d, dv %d, dim %d", a->dk, a->dv, a->dim);
  if (a->s_m < 0 || a->s_m > a->slots || a->s_valid < 0 || a->s_valid > a->slots)
    return fail(LOGKV_EINVAL, "slot pack prefix lengths out of range");
  if (a->slots && (!a->k || !a->v || !a->w || !a->out_k || !a->out_v || (a->s_m && !a->m) ||
                   (a->s_valid && !a->valid)))
    return fail(LOGKV_EINVAL, "slot pack buffer is NULL");
  if (reinterpret_cast<uintptr_t>(a->out_k) % 8 || reinterpret_cast<uintptr_t>(a->out_v) % 8)
    return fail(LOGKV_EINVAL, "packed rows must be 8-byte aligned");
  const int rc = logkv::launch_slot_pack(*a, static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "slot pack");
  return LOGKV_OK;
}

int64_t logkv_chunk_backward_workspace_bytes(const logkv_attention_args* a) {
  if (!a || a->n_groups < 1 || a->n_heads % a->n_groups) return -1;
  return logkv::chunk_backward_workspace_floats(*a) * 4;
}

int logkv_chunk_attention_backward(const logkv_attention_args* a, const int32_t* table, int64_t table_ints,
                                   const logkv_attention_grad_args* gr, void* ws, int64_t ws_bytes, void* stream) {
  if (!a || !gr || !table || table_ints < 1) return fail(LOGKV_EINVAL, "attention backward args or plan table are NULL");
  if (a->n_batch < 1 || a->n_groups < 1 || a->n_heads % a->n_groups || a->tq < 1)
    return fail(LOGKV_EINVAL, "attention backward shape: batch %d, heads %d, groups %d, tq %d", a->n_batch,
                a->n_heads, a->n_groups, a->tq);
  if (a->dk < 8 || a->dk % 8 || a->dk > 128 || a->dv % 32 || a->dv < 32 || a->dv > 128 || a->dim % 8 ||
      a->dim > 144 || a->dim <= a->dk || a->dim < a->dv)
    return fail(LOGKV_EINVAL, "attention backward takes dk a multiple of 8 up to 128, dv in {32, 64, 96, 128} and "
                "packed widths up to 144; got %d/%d/%d", a->dk, a->dv, a->dim);
  if (a->cap < 1 || a->tail < 0 || a->tail > a->cap || a->causal_tail < 0 || a->causal_tail > a->tail ||
      (a->causal_tail && a->causal_tail != a->tq))
    return fail(LOGKV_EINVAL, "attention backward rows: cap %d, tail %d, causal_tail %d", a->cap, a->tail,
                a->causal_tail);
  if (gr->grad_rows < 0 || gr->grad_rows > a->tail)
    return fail(LOGKV_EINVAL, "gradient rows %d outside [0, tail %d]", gr->grad_rows, a->tail);
  if (!a->q || !a->k || !a->v || !a->out || !gr->dout || !gr->dq || (gr->grad_rows && (!gr->dk || !gr->dv)))
    return fail(LOGKV_EINVAL, "attention backward buffer is NULL");
  if (reinterpret_cast<uintptr_t>(a->k) % 16 || reinterpret_cast<uintptr_t>(a->v) % 16)
    return fail(LOGKV_EINVAL, "packed K/V must be 16-byte aligned");
  if (!ws || ws_bytes < logkv::chunk_backward_workspace_floats(*a) * 4)
    return fail(LOGKV_EINVAL, "attention backward workspace too small");
  const int rc = logkv::launch_chunk_backward(*a, table + table_ints - 1, *gr, static_cast<float*>(ws),
                                              static_cast<hipStream_t>(stream));
  if (rc) return launch_failed(rc, "attention backward");
  return LOGKV_OK;
}

}  // extern "C"
