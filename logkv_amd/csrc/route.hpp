// Internal declarations shared by the route and ladder kernels.
#pragma once

#include "common.hpp"

namespace logkv {

using LadderArgs = logkv_ladder_view;
using RowsArgs = logkv_rows_view;
using RouteParams = logkv_route_params;

constexpr int kMaxOrderRows = 8192;   // rows per flush (position-order sort in LDS)
constexpr int kCenterTile = 32;       // rows per tile of the tiled center sum
constexpr int kOrderIndexBits = 13;
constexpr uint64_t kOrderIndexMask = (1ull << kOrderIndexBits) - 1;
constexpr int kMaxClusters = 32;      // K (alive bits are a 32-bit mask)
constexpr int kMaxDim = 256;          // dk, dv

// Valid rows of batch row b: counts[b] clamped to [0, tokens] (NULL counts = all rows).
__device__ __forceinline__ int valid_rows(const logkv_rows_view& r, int b) {
  if (!r.counts) return r.tokens;
  const int n = r.counts[b];
  return n < 0 ? 0 : (n > r.tokens ? r.tokens : n);
}

constexpr int kMaxLevels = 32;        // ladder levels L
constexpr int kMaxCandidates = 4096;  // Alpha span candidates per batch row (selection sorts them in LDS)
constexpr int kMaxLadders = 32768;    // batch * groups * K (a level's carry work table is staged in LDS)

// Per-ladder plan of one commit, written by the prepare launch and read by the
// level launches: counts before each level step and the rows staged into it.
struct LadderPlan {
  int32_t active;       // rows to append after the prepare step
  int32_t kind0;        // level-0 staged source: 0 flush rows (tok list), 1 S0 rows
  int32_t m_tok;        // entries of the tok list
  int32_t first;        // tok list offset of the first appended row
  int64_t order_base;   // order of staged flush row 0 (kind 0)
  int16_t cnt[kMaxLevels];
  int32_t m[kMaxLevels];
};

// Device scratch of one route/commit call, carved from the caller's workspace.
struct Workspace {
  int32_t* order;      // [n_batch, T]
  int8_t* assign;      // [lanes, T]
  float* s_win;        // [lanes, T]
  float* dist;         // [lanes, T]
  float* cap_dist;     // [lanes, T, K] orphan-to-candidate distances of a capped route (shares the
                       // ladder scratch, which only the commit launches after the route use)
  uint8_t* snap_alive; // [lanes, K] alive flags before the commit (written by its ladder blocks)
  uint8_t* ladder;     // per-ladder carry / staging rows
  int64_t ladder_stride;  // bytes per ladder
  int64_t s0_rows;        // delayed-archive staging rows per ladder
  int64_t m0_cap;         // most rows staged at level 0 (sizes the per-level carry buffers)
  int32_t sort_width;     // keys per block for the delayed-archive sort (0 without it)
  LadderPlan* plans;      // [ladders]
  uint16_t* tok;          // [ladders, T] each ladder's flush rows in position order
  int32_t* units;         // [L - 1, ladders + 1] prefix sums over ladders of each level's carry work units
  const int32_t* abort;   // optional: a nonzero value stops the commit before it writes anything
};

int64_t ladder_scratch_bytes(const LadderArgs& c, int64_t s0, int64_t m0);
int launch_route(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                 hipStream_t stream);
int launch_score(const logkv_span_args& a, float* out, hipStream_t stream);
int launch_partition(const logkv_partition_args& a, hipStream_t stream);
int64_t select_workspace_bytes(const logkv_alpha_select_args& a);
int launch_select(const logkv_alpha_select_args& a, void* ws, hipStream_t stream);
int launch_plan(const logkv_readout_view& c, int32_t* table, hipStream_t stream);
int launch_pack(const logkv_readout_view& c, const logkv_pack_args& p, const int32_t* table, hipStream_t stream);
int64_t attention_workspace_floats(const logkv_attention_args& a);
int launch_attention(const logkv_attention_args& a, const int32_t* width, float* part, hipStream_t stream);
int launch_chunk_attention(const logkv_attention_args& a, const int32_t* width, float* part, hipStream_t stream);
int64_t chunk_workspace_floats(const logkv_attention_args& a);
int launch_combine(const logkv_attention_args& a, const float* part, int n_split, hipStream_t stream);
int launch_commit(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                  hipStream_t stream);
int launch_order(const RowsArgs& r, int n_batch, int32_t* order, int32_t* clear, hipStream_t stream, int n_clear = 1);
int launch_record(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, const logkv_op_log_view& log,
                  hipStream_t stream);
int launch_beta_merge(const logkv_beta_args& a, int32_t* status, hipStream_t stream);
int launch_recent_append(const logkv_recent_args& a, int at, int n, hipStream_t stream);
int launch_recent_shift(const logkv_recent_args& a, int take, int count, hipStream_t stream);
int launch_slot_pack(const logkv_slot_pack_args& a, hipStream_t stream);
int64_t chunk_backward_workspace_floats(const logkv_attention_args& a);
int launch_chunk_backward(const logkv_attention_args& a, const int32_t* width, const logkv_attention_grad_args& g,
                          float* stats, hipStream_t stream);
int launch_replay(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, const logkv_op_log_view& log,
                  int64_t cursor, int32_t* status, hipStream_t stream);
int launch_record_wards(const LadderArgs& c, const int32_t* jobs, const int32_t* n_jobs, const logkv_op_log_view& log,
                        hipStream_t stream);
int launch_unified_replay(const LadderArgs& c, const RowsArgs& r, const Workspace& ws, const logkv_op_log_view& log,
                          const int64_t* cursors, int32_t* consumed, int32_t* jobs, int32_t* n_jobs, int32_t* status,
                          hipStream_t stream);

}  // namespace logkv
