// Internal declarations of the unified (Ward / radius) route.
#pragma once

#include "route.hpp"

namespace logkv {

constexpr int kMaxNodes = 4608;   // rows of a flush + K (one lane's reducer state lives in LDS)

// Round bookkeeping of one lane's reducer stage (global memory, read by every
// phase launch of a round).
struct LaneCtl {
  int32_t count;    // live nodes
  int32_t ntrace;   // merges so far
  int32_t n_ok;     // merges of the current round
  int32_t nprop;    // mutual proposals of the current round
  int32_t active;   // 1: another round follows
  int32_t work;     // 1: the current round's Lance-Williams / rescan phases have work
  int32_t stuck;    // 1: clusters above the target and no pair left
  int32_t rounds;   // rounds run
  int32_t n_live;   // live rows after the current round's merges
  int32_t n_dirty;  // rows to rescan after the current round's merges
  int32_t lw_elems;    // sum over rounds of kept rows x live columns (Lance-Williams elements)
  int32_t scan_elems;  // sum over scans of rescanned rows x live columns (the first scan: n x n)
};

// Per lane and stage, what the stage's finish writes when ReduceArgs::stats is set:
// nodes, rounds, merges, Lance-Williams elements, rescanned elements, stuck.
constexpr int kStatsInts = 8;

// Arguments of one reducer stage over `lanes` lanes of M padded nodes.
struct ReduceArgs {
  float* dist;            // [lanes, M, M] squared distances (updated in place)
  float* mu;              // [lanes, M, D] centers (updated in place)
  const float* mass;      // [lanes, M] initial masses
  const int32_t* count;   // [lanes] nodes in use (the rest are padding)
  const float* limit;     // [lanes] radius limit, or NULL for none
  int32_t target;         // stop at this many clusters
  int32_t M, D;
  uint8_t* alive_out;     // [lanes, M] survivors
  int32_t* trace;         // [lanes, M, 2] merges (kept row, retired row) in round order
  int32_t* n_trace;       // [lanes]
  int32_t* stuck;         // [lanes] 1: clusters above the target and no pair left
  float* bound;           // [lanes, M] scratch: verified radius bounds of a round
  uint8_t* image;         // [lanes, image_stride] the reducer state (the LDS layout) between launches
  int64_t image_stride;
  LaneCtl* ctl;           // [lanes]
  int16_t* live;          // [lanes, 3, M] the round's live rows (ctl.n_live), rows to rescan
                          // (ctl.n_dirty) and kept rows (ctl.n_ok), each list ascending
  int32_t* stats;         // [lanes, stats_stride] the stage's counts (kStatsInts), or NULL
  int32_t stats_stride;
  int32_t passes;         // matching passes per round: > 1 adds frozen-center sweeps (no radius limit only)
  uint64_t* restricted;   // [lanes, M] the sweeps' restricted row minima (passes > 1)
};

// Full-recompute rounds of one reducer stage (a capacity-capped route): the
// stage's input and outputs as ReduceArgs names them, the cap, and the
// compacted node state, which alternates between two buffer sets round by
// round.
struct RoundArgs {
  float* mu;              // [lanes, M, D] the stage's nodes; the survivors' rows get their final centers
  const float* mass;      // [lanes, M]
  const int32_t* count;   // [lanes]
  const float* limit;     // [lanes] radius limit (the candidate stage), or NULL
  int32_t target, M, D, strict;   // strict: a lane with no pair above the target may take uncapped pairs,
                                  // and ends stuck (an error) if none is left either
  float cap;              // total-mass cap of a pair (> 0)
  float* cmu[2];          // [lanes, M, D] compacted centers
  float* cmass[2];        // [lanes, M]
  float* crad[2];         // [lanes, M] radius bounds (candidate stage)
  int32_t* croot[2];      // [lanes, M] the compacted rows' input ids
  int32_t* n_cur;         // [lanes] compacted nodes now
  int32_t* cbuf;          // [lanes] the buffer set holding the lane's nodes (its last round's output)
  int32_t* dcount;        // [lanes] n_cur of a lane with rounds to go, else 0 (the distance launch's count)
  uint64_t* keys;         // [lanes, M, 2] each row's least capped and uncapped packed cost
  float* dist;            // [lanes, M, M]
  uint8_t* alive_out;     // [lanes, M] survivors by input id
  int32_t* trace;         // [lanes, M, 2] merges in input ids, round by round, each round in cost order
  int32_t* n_trace;       // [lanes]
  int32_t* stuck;         // [lanes]
  int32_t* rounds;        // [lanes] rounds run
  int32_t* stats;         // [lanes, stats_stride] the stage's counts (kStatsInts), or NULL
  int32_t stats_stride;
};

// Device buffers of one unified plan (carved from the caller's workspace).
struct UnifiedBufs {
  int32_t M, D;
  const float* limit;     // [lanes]
  float* mu1;             // [lanes, M, D]
  float* mass1;           // [lanes, M]
  int32_t* count1;        // [lanes]
  float* mu2;
  float* mass2;
  int32_t* count2;
  float* dist;            // [lanes, M, M] (both stages)
  float* bound;           // [lanes, M]
  uint8_t* alive1;        // [lanes, M]
  uint8_t* alive2;
  int32_t* trace1;        // [lanes, M, 2]
  int32_t* trace2;
  int32_t* n_trace1;      // [lanes]
  int32_t* n_trace2;
  int32_t* stuck1;
  int32_t* stuck2;        // [lanes] read by the host: a stuck budget stage is an error
  int32_t* label1;        // [lanes, M]
  int32_t* label2;
  int32_t* n_roots1;
  int32_t* n_roots2;
  int32_t* n_old;         // [lanes]
  int32_t* old_ids;       // [lanes, kMaxClusters]
  int32_t* jobs;          // [lanes, kMaxClusters, 2] old-old merges (keep, retire) in order
  int32_t* n_jobs;        // [lanes]
  uint8_t* image;         // [lanes, image_stride] reducer state between the round launches
  int64_t image_stride;
  LaneCtl* ctl;           // [lanes]
  int16_t* live;          // [lanes, 3, M]
  int32_t* stats;         // [lanes, 2, kStatsInts] each stage's counts
  uint64_t* restricted;   // [lanes, M] the budget stage's restricted row minima (frozen-center sweeps)
  int32_t passes;         // matching passes per budget round (semantic_merge_passes)
  float cap;              // > 0: the capacity cap of a merged pair's mass (full-recompute rounds)
  float* cmu[2];          // full-recompute rounds' compacted node state (see RoundArgs)
  float* cmass[2];
  float* crad[2];
  int32_t* croot[2];
  int32_t* n_cur;
  int32_t* cbuf;
  int32_t* dcount;
  uint64_t* keys;         // [lanes, M, 2]
  int32_t* rounds;        // [lanes]
};

int launch_unified_plan(const LadderArgs& c, const RowsArgs& r, const UnifiedBufs& u, const Workspace& ws,
                        hipStream_t stream);
size_t unified_reduce_lds(int M);
int64_t unified_image_stride(int M);
// summary[0] = most old-old merges of a lane, summary[1] = 1 if a budget stage found no pair.
int launch_unified_summary(const LadderArgs& c, const UnifiedBufs& u, int32_t* summary, int tokens,
                           hipStream_t stream);
int launch_ward_step(const LadderArgs& c, const Workspace& ws, const int32_t* jobs, const int32_t* n_jobs, int step,
                     hipStream_t stream);
int launch_levels(const LadderArgs& c, const RowsArgs& r, const RouteParams& p, const Workspace& ws,
                  hipStream_t stream, struct SideStream* side = nullptr);

}  // namespace logkv
