// Internal declarations shared by the route and ladder kernels.
#pragma once

#include "common.hpp"

namespace logkv {

using LadderArgs = logkv_ladder_view;
using RowsArgs = logkv_rows_view;
using RouteParams = logkv_route_params;

constexpr int kMaxOrderRows = 8192;   // rows per flush (position-order sort in LDS)
constexpr int kOrderIndexBits = 13;
constexpr uint64_t kOrderIndexMask = (1ull << kOrderIndexBits) - 1;
constexpr int kAttachTile = 64;       // rows per attach block
constexpr int kMaxClusters = 32;      // K (alive bits are a 32-bit mask)
constexpr int kMaxDim = 256;          // dk, dv

// Valid rows of batch row b: counts[b] clamped to [0, tokens] (NULL counts = all rows).
__device__ __forceinline__ int valid_rows(const logkv_rows_view& r, int b) {
  if (!r.counts) return r.tokens;
  const int n = r.counts[b];
  return n < 0 ? 0 : (n > r.tokens ? r.tokens : n);
}

// Device scratch of one route/commit call, carved from the caller's workspace.
struct Workspace {
  int32_t* order;      // [n_batch, T]
  int8_t* assign;      // [lanes, T]
  float* s_win;        // [lanes, T]
  float* dist;         // [lanes, T]
  uint8_t* snap_alive; // [lanes, K] alive flags at the start of the flush
  uint8_t* ladder;     // per-ladder carry / staging rows
  int64_t ladder_stride;  // bytes per ladder
  int64_t s0_rows, carry_a_rows, carry_b_rows;
  int32_t sort_width;     // keys per block for the delayed-archive sort (0 without it)
};

int64_t ladder_scratch_rows(int64_t m0, int64_t slots, int64_t& s0, int64_t& ca, int64_t& cb, int64_t existing);
int64_t ladder_scratch_bytes(const LadderArgs& c, int64_t s0, int64_t ca, int64_t cb);
int64_t row_bytes(int dk, int dv);
int launch_route(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                 hipStream_t stream);
int launch_score(const logkv_span_args& a, float* out, hipStream_t stream);
int launch_partition(const logkv_partition_args& a, hipStream_t stream);
int launch_plan(const logkv_readout_view& c, int32_t* table, hipStream_t stream);
int launch_pack(const logkv_readout_view& c, const logkv_pack_args& p, const int32_t* table, hipStream_t stream);
int64_t attention_workspace_floats(const logkv_attention_args& a);
int launch_attention(const logkv_attention_args& a, const int32_t* width, float* part, hipStream_t stream);
int launch_commit(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                  hipStream_t stream);

}  // namespace logkv
