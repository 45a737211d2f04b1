/* C ABI of the LogKV HIP library (liblogkv_hip.so, gfx950).
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * enqueues its kernels on the given HIP stream (NULL = the default stream),
 * never allocates and never synchronises the host. Scratch memory is passed in
 * by the caller; `*_workspace_bytes` reports how much. Return value: LOGKV_OK,
 * LOGKV_EINVAL for a shape / layout mismatch (the reference raises ValueError),
 * LOGKV_ERUNTIME for a HIP launch failure (RuntimeError); `logkv_last_error()`
 * gives the message of the calling thread's last failure.
 *
 * Storage follows the reference cache's buffers (litgpt/log_kv_cache.py:881-1121):
 * ladder fields are [lanes, K, L, B'] (+ feature axis), lanes = batch * groups;
 * several layer caches may share one allocation by folding layers into batch.
 * bf16 tensors are passed as uint16_t*, bool tensors as uint8_t*.
 */
#ifndef LOGKV_HIP_H
#define LOGKV_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { LOGKV_OK = 0, LOGKV_EINVAL = 1, LOGKV_ERUNTIME = 2 };

/* Persistent ladder and cluster state (all device pointers; level_k, level_v and
 * centroid 16-byte aligned). */
typedef struct logkv_ladder_view {
  uint16_t* level_k;      /* bf16 [lanes, K, L, B', dk] */
  uint16_t* level_v;      /* bf16 [lanes, K, L, B', dv] */
  float* level_w;         /* [lanes, K, L, B'] */
  int64_t* level_p_lo;
  int64_t* level_p_hi;
  int64_t* level_sum_wp;
  int64_t* level_order;
  uint8_t* pad_mask;
  int16_t* level_count;   /* [lanes, K, L] */
  float* centroid;        /* [lanes, K, dk] */
  float* n_eff;           /* [lanes, K] */
  int32_t* n_total;
  int64_t* p_hi_c;
  int32_t* level0_phase;
  uint8_t* alive;
  const float* s_h;       /* [lanes] */
  int32_t n_batch, n_groups, k_max, levels, slots, dk, dv;
} logkv_ladder_view;

/* The rows of one flush: k_raw / v [n_batch, G, T, d] bf16 with element strides
 * (last axis contiguous), positions [n_batch, T] int64, optional ragged counts. */
typedef struct logkv_rows_view {
  const uint16_t* k;
  int64_t k_sb, k_sg, k_st;
  const uint16_t* v;
  int64_t v_sb, v_sg, v_st;
  const int64_t* pos;
  int64_t pos_sb;
  const int32_t* counts;  /* [n_batch] device, rows at or past counts[b] are padding; NULL = T */
  int32_t tokens;
} logkv_rows_view;

typedef struct logkv_route_params {
  float eta;            /* temporal cost weight (seg_eta) */
  float g0;             /* temporal cost scale (seg_g0) */
  float lam;            /* radius multiplier (cluster_lambda_rel) */
  int32_t late_joins;   /* 1 with Alpha: re-sort clusters whose p_hi passes a new row */
  int32_t beta_merge;   /* 1: Beta 4->2 merges at non-top carry levels */
  int32_t center_tile;  /* 0 or 1: a center sums its new keys one row at a time in position order
                         * (semantic_centroid_backend="sequential"); 32: in position-ordered tiles of
                         * 32 rows, each tile summed by a halving tree, tiles added in order
                         * ("parallel", litgpt/log_kv_updates_triton.py:236-241, 274-275) */
  float hard_cap;       /* <= 0: no capacity cap. Else the cap (max_seq / K * semantic_capacity_hard_cap_mult
                         * as f32, litgpt/log_kv_cache.py:2347-2354): a frozen join needs n_total + 1 <= hard_cap,
                         * a cluster keeps at most hard_cap_rows - n_total of its direct rows (offset order)
                         * and orphans fill the nearest cluster with room (attach route only) */
  int32_t hard_cap_rows; /* int(cap), the truncated cap the rooms count against */
  int32_t merge_passes;  /* unified route: matching passes per budget-stage round (semantic_merge_passes); > 1 adds
                          * frozen-center sweeps (litgpt/log_kv_cache.py:561-588, :3314), 0 or 1 none. The attach
                          * route ignores it */
} logkv_route_params;

const char* logkv_last_error(void);

/* Bytes of scratch needed by logkv_attach_assign / logkv_route_commit. */
int64_t logkv_route_workspace_bytes(const logkv_ladder_view* cache, int32_t tokens, int32_t late_joins);

/* Final attach cluster of every valid row, in position order: assign[lane, t]
 * (int8, -1 past the row's count); order[b, t] (int32) lists row offsets by
 * position. Frozen joins + farthest-point seeds + orphan joins.
 * Replaces attach_assign (litgpt/log_kv_route_triton.py:894-917) and the seeding
 * planner _semantic_attach_plan_torch (litgpt/log_kv_cache.py:4636-4680). */
int logkv_attach_assign(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                        const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                        int8_t* assign, int32_t* order, void* stream);

/* One attach-routed flush committed into the ladders: decisions as above, new
 * clusters, ordinary and (with late_joins) delayed joins, Fenwick appends with
 * pair or Beta carries and the top-level fold, ordered centroid updates and the
 * cluster scalars. `assign` / `order` may be NULL.
 * Replaces the device work of _semantic_attach_commit / _alpha_commit_joins /
 * _semantic_apply_join_plan (litgpt/log_kv_cache.py:4682-4707, :3690-3788,
 * :4225-4361) and the kernels fill, merge_scatter, centroid_parallel
 * (litgpt/log_kv_updates_triton.py:79-87, :176-219, :268-282). */
int logkv_route_commit(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                       const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                       int8_t* assign, int32_t* order, void* stream);

/* The commit half of logkv_route_commit for decisions already in `assign` /
 * `order` (from logkv_attach_assign on the same rows and cache state, or NULL
 * for the copies left in the same workspace). Lets a caller time or overlap
 * the two halves; same replaced reference interfaces as logkv_route_commit. */
int logkv_commit_only(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                      const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                      const int8_t* assign, const int32_t* order, void* stream);

/* Unified (Ward / radius) route: bytes of scratch for logkv_unified_plan /
 * logkv_unified_commit (the route workspace sized for old-old merges, then
 * the reducer's per-lane distance matrices [T + K]^2 f32, centers and traces).
 * At most T + K <= 4608 per flush. */
int64_t logkv_unified_workspace_bytes(const logkv_ladder_view* cache, int32_t tokens, int32_t late_joins);

/* Byte offset, in that workspace, of the reducer's counts of the last
 * logkv_unified_plan: int32 [lanes, 2 stages, 8] = nodes, rounds, merges,
 * Lance-Williams elements (sum of kept rows x live columns over the rounds),
 * rescanned elements (sum of rescanned rows x live columns, the first scan
 * n x n), stuck flag, 0, 0; valid once the plan has run on the stream. -1 for
 * an invalid layout. No counterpart in the reference: the counts are the
 * roofline's byte model of the reducer (measurement only). */
int64_t logkv_unified_stats_offset(const logkv_ladder_view* cache, int32_t tokens, int32_t late_joins);

/* The decisions of one unified-routed flush, per lane (batch row, KV group):
 * the valid rows merge into candidates by mutual-nearest Ward rounds under
 * the radius limit limits[lane] (f32 [lanes] = sqrt(lambda * s_h)), then old
 * live clusters and candidates merge until at most K remain; every row's
 * final cluster and the lane's old-old merges stay in the workspace.
 * summary (device int32[2]) receives the most old-old merges of any lane and
 * 1 if a budget stage stopped above K with no pair left (an error).
 * Replaces _semantic_route_unified's planning (litgpt/log_kv_cache.py:
 * 3589-3660) with _semantic_unified_reduce_device / _incremental and
 * _UnifiedReduceTorch / UnifiedReduce (litgpt/log_kv_cache.py:3225-3376,
 * :448-637; litgpt/log_kv_route_triton.py:197-838) and the labels
 * (litgpt/log_kv_cache.py:3544-3568). With params->hard_cap > 0 the stages run
 * the full-recompute rounds of a capacity-capped route (_semantic_unified_reduce_rounds,
 * :3445-3519), and the call synchronizes `stream` every 8 rounds to read the lanes'
 * round flags (the reference polls every 4 rounds). */
int logkv_unified_plan(const logkv_ladder_view* cache, const logkv_rows_view* rows, const logkv_route_params* params,
                       const float* limits, void* workspace, int64_t workspace_bytes, int32_t* summary, void* stream);

/* Applies a plan left in the same workspace by logkv_unified_plan: merge_steps
 * (summary[0]) rounds of old-old merges, each the lane's next merge (both
 * ladders' entries re-appended into the lower cluster), then the commit of
 * the rows into their clusters (new clusters open the free ids in root
 * order). Replaces _semantic_ward_merge_batch (litgpt/log_kv_cache.py:
 * 2517-2580) and the commit tail of _semantic_route_unified (:3661-3688). */
int logkv_unified_commit(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                         const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                         int32_t merge_steps, void* stream);

/* Route op-log of a cache (litgpt/log_kv_cache.py:2006-2096): per lane (batch
 * row, KV group) int32 rows (op, cluster, arg, position) at rows[lane,
 * 0 .. lengths[lane]), op codes as the reference's (litgpt/log_kv_cache.py:
 * 90-94). lengths may pass capacity: rows past it are counted, not written
 * (the reference's "op_log overflow"; the caller reports it). */
typedef struct logkv_op_log_view {
  int32_t* rows;        /* [n_batch, G, capacity, 4] */
  int32_t* lengths;     /* [n_batch, G] */
  int64_t capacity;
} logkv_op_log_view;

enum {
  LOGKV_OP_NEW_CLUSTER = 0, LOGKV_OP_NEW_SEGMENT = 1, LOGKV_OP_JOIN = 2, LOGKV_OP_WARD_MERGE = 3,
  LOGKV_OP_PAD_INSERT = 4
};

/* Appends the op rows of the flush that logkv_route_commit / logkv_commit_only
 * just committed with the same workspace and rows: per lane, NEW_CLUSTER
 * (cluster, 0, earliest position) for every cluster it opened (ascending
 * cluster), then JOIN (cluster, 0, position) for the other rows of ordinary
 * joins (cluster ascending, rows in position order), then the same for
 * delayed-archive joins. Replaces the recording of _semantic_new_clusters,
 * _semantic_commit_joins_unsegmented and _alpha_commit_joins
 * (litgpt/log_kv_cache.py:2286-2297, :4153-4166, :3782-3788) with
 * _record_ops / _flush_recorded_ops (litgpt/log_kv_cache.py:2043-2096). */
int logkv_record_ops(const logkv_ladder_view* cache, const logkv_rows_view* rows, void* workspace,
                     int64_t workspace_bytes, const logkv_op_log_view* log, void* stream);

/* Replay status bits (logkv_replay_commit writes their OR to *status). */
enum {
  LOGKV_REPLAY_BAD_OP = 1,             /* not NEW_CLUSTER / JOIN of segment 0, or cluster out of range */
  LOGKV_REPLAY_UNKNOWN_POSITION = 2,   /* a row's position is not a row of this flush */
  LOGKV_REPLAY_DUPLICATE_POSITION = 4, /* two flush rows share a position */
  LOGKV_REPLAY_SHORT_LOG = 8,          /* fewer than the flush's rows logged past the cursor */
  LOGKV_REPLAY_UNCONSUMED = 16,        /* a flush row is named by no log row (another by two) */
  LOGKV_REPLAY_BAD_CLUSTER = 32,       /* NEW_CLUSTER of a live cluster, or JOIN of a dead one */
  LOGKV_REPLAY_BAD_ORDER = 64          /* a cluster's rows are not in increasing position order */
};

/* Re-applies the logged decisions of one flush without routing: per lane, the
 * rows [cursor, cursor + valid rows) of the log name each flush row's cluster
 * (by position), then the commit of logkv_route_commit runs on them. The
 * checks above are made on the device; on any failure *status (device int32)
 * gets the bits and no cache field is written. Replaces the replay branch of
 * _route_and_flush_batch with _semantic_build_replay_plan and
 * _semantic_commit_runs (litgpt/log_kv_cache.py:5067-5114, :4856-4926,
 * :4178-4223) for logs of attach-routed flushes. */
int logkv_replay_commit(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                        const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                        const logkv_op_log_view* log, int64_t cursor, int32_t* status, void* stream);

/* Op-log of a unified-routed flush, after logkv_unified_commit on the same
 * workspace: per lane the WARD_MERGE rows (keep, free, -1) of its old-old
 * merges in merge order, then the NEW_CLUSTER / JOIN rows logkv_record_ops
 * writes. Replaces the unified route's recording (litgpt/log_kv_cache.py:
 * 2597-2598, :3661-3688 with record=True). */
int logkv_unified_record_ops(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                             const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                             const logkv_op_log_view* log, void* stream);

/* Parses one logged unified flush for replay without routing: per lane from
 * cursors[lane] (device int64[lanes]), its leading WARD_MERGE rows become the
 * lane's old-old merges (each between two distinct clusters live at that
 * point), then one NEW_CLUSTER / JOIN row per valid flush row gives the
 * decisions, checked as logkv_replay_commit checks them against the clusters
 * live after the merges. consumed[lane] (device int32) receives the rows the
 * lane consumed; status (device int32[2]) receives the check bits and the most
 * merges of any lane. With status[0] == 0, logkv_unified_commit on the same
 * workspace with merge_steps = status[1] applies the flush. Replaces the
 * unified branch of _semantic_build_replay_plan and the replay loop
 * (litgpt/log_kv_cache.py:4856-4926, :5067-5114). */
int logkv_unified_replay_plan(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                              const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                              const logkv_op_log_view* log, const int64_t* cursors, int32_t* consumed,
                              int32_t* status, void* stream);

/* Copies a unified plan's decisions between the workspace and caller buffers
 * (into_workspace = 0: out of the workspace after logkv_unified_plan; 1: back
 * in before logkv_unified_commit): assign int8[lanes, T], order int32[n_batch,
 * T], jobs int32[lanes, 32, 2] (old-old merges), n_jobs int32[lanes]. The
 * update tape's record / replay of a unified flush (litgpt/log_kv_cache.py:
 * 4946-5031). */
int logkv_unified_decisions(const logkv_ladder_view* cache, const logkv_rows_view* rows,
                            const logkv_route_params* params, void* workspace, int64_t workspace_bytes,
                            int8_t* assign, int32_t* order, int32_t* jobs, int32_t* n_jobs, int32_t into_workspace,
                            void* stream);

/* The recent window's buffers and, for an append, the block's rows:
 * recent_k [n_batch, G, cap, dk], recent_k_raw [.., dkr], recent_v [.., dv]
 * (bf16, contiguous), recent_pos int64 [n_batch, cap], recent_ends uint8
 * [n_batch, cap] or NULL (no Alpha). Sources k / k_raw / v are bf16 with
 * element strides (batch, group, row; features contiguous), pos int64 with
 * strides (batch, row), ends uint8 [n_batch, n] rows of stride ends_sb.
 * Feature counts are multiples of 4; rows and strides 8-byte aligned. */
typedef struct logkv_recent_args {
  uint16_t* recent_k;
  uint16_t* recent_k_raw;
  uint16_t* recent_v;
  int64_t* recent_pos;
  uint8_t* recent_ends;
  int32_t n_batch, n_groups, cap, dk, dkr, dv;
  const uint16_t* k;
  int64_t k_sb, k_sg, k_st;
  const uint16_t* k_raw;
  int64_t kr_sb, kr_sg, kr_st;
  const uint16_t* v;
  int64_t v_sb, v_sg, v_st;
  const int64_t* pos;
  int64_t pos_sb, pos_st;
  const uint8_t* ends;
  int64_t ends_sb;
} logkv_recent_args;

/* Appends rows [0, n) of the sources to recent rows [at, at + n) of every
 * buffer in one launch. Replaces the recent-window writes of add_recent
 * (litgpt/log_kv_cache.py:5668-5718). */
int logkv_recent_append(const logkv_recent_args* args, int32_t at, int32_t n, void* stream);

/* After a flush of the first `take` of `count` recent rows: rows [take, count)
 * move to the front and rows [count - take, count) are cleared, every buffer
 * in one launch; needs count - take <= take. Replaces the shift and clear
 * after a flush (litgpt/log_kv_cache.py:5640-5659). */
int logkv_recent_shift(const logkv_recent_args* args, int32_t take, int32_t count, void* stream);

/* Candidate span table over the virtual rows [old exact pool (old_width rows) |
 * flush]: pool_* / flush_* are [n_batch, G, rows, d] bf16 with element strides;
 * span i covers tokens[span_offsets[i] .. span_offsets[i+1]) of batch row
 * span_rows[i]. With beta_novelty, centroids [n_batch, G, k_max, dk] f32 and
 * centroid_valid [n_batch, G, k_max] are the centers before the flush. */
typedef struct logkv_span_args {
  const uint16_t* pool_k;
  int64_t pk_sb, pk_sg, pk_st;
  const uint16_t* pool_v;
  int64_t pv_sb, pv_sg, pv_st;
  const uint16_t* flush_k;
  int64_t fk_sb, fk_sg, fk_st;
  const uint16_t* flush_v;
  int64_t fv_sb, fv_sg, fv_st;
  int32_t old_width;
  const int32_t* tokens;
  const int32_t* span_offsets;
  const int32_t* span_rows;
  int32_t n_spans;
  int32_t n_groups, dk, dv;
  const float* centroids;
  const uint8_t* centroid_valid;
  int32_t k_max;
  int32_t beta_novelty;
  const int32_t* n_spans_dev;  /* optional: only the first *n_spans_dev of the n_spans spans are scored */
} logkv_span_args;

/* Score of every candidate span (f32 [n_spans]): Alpha's normalised K/V
 * variance, or with beta_novelty the top-2 group mean of variance + novelty.
 * Replaces score_spans (litgpt/alpha_log_kv.py:125-174). */
int logkv_score_spans(const logkv_span_args* args, float* scores, void* stream);

/* Span selection of one Alpha flush on the device, with no host round trip:
 * the candidate whole spans of [exact pool | flush] (pool width = budget P),
 * their scores, and the bounded greedy choice. The current selection is
 * span_len / span_closed [n_batch, P] with span_count [n_batch]; the pool's
 * rows are those spans' tokens in order, at positions pool_pos [n_batch, P].
 * New rows: positions new_pos and boundary flags ends [n_batch, T]. `rows`
 * carries the K/V sources, groups, widths and centers for scoring (its
 * old_width must be P; its token tables are filled here). Outputs: keep
 * [n_batch, P] and archive [n_batch, P + T] source rows (indices into
 * [pool (P rows) | flush], -1 past the end), archive_count [n_batch], the new
 * selection's spans, alpha_count[0] = the largest kept count, and optionally
 * the candidates' scores. At most 4096 candidates per batch row. With
 * count_rows > 0 the batch rows are groups of count_rows consecutive rows
 * (caches stacked as batch rows, count_rows each) and alpha_count[i] is the
 * largest kept count of group i; 0 means one group of all rows.
 * Replaces the selection of _alpha_route_flush (litgpt/log_kv_cache.py:
 * 3904-3940): cut_spans, score_spans and choose_spans
 * (litgpt/alpha_log_kv.py:16-226). */
typedef struct logkv_alpha_select_args {
  const int32_t* span_len;
  const uint8_t* span_closed;
  const int32_t* span_count;
  const int64_t* pool_pos;
  const int64_t* new_pos;
  int64_t np_sb;
  const uint8_t* ends;
  int64_t ends_sb;
  int32_t tokens;
  int32_t n_batch, budget, max_span;
  logkv_span_args rows;
  int32_t* keep;
  int32_t* archive;
  int32_t* archive_count;
  int32_t* new_span_len;
  uint8_t* new_span_closed;
  int32_t* new_span_count;
  int32_t* alpha_count;
  float* scores;
  int32_t count_rows;
} logkv_alpha_select_args;

int64_t logkv_alpha_select_workspace_bytes(const logkv_alpha_select_args* args);
int logkv_alpha_select(const logkv_alpha_select_args* args, void* workspace, int64_t workspace_bytes, void* stream);

/* Exact-pool rewrite and archive gather over the same virtual rows: keep
 * [n_batch, P] and archive [n_batch, A] list source rows (-1 = zero row).
 * Outputs are contiguous: out_pool_k/v [n_batch, G, P, d], out_pool_pos /
 * out_pool_valid [n_batch, P], arch_k/v [n_batch, G, A, d], arch_pos
 * [n_batch, A]. The outputs must not alias the pool sources.
 * Replaces alpha_partition (litgpt/log_kv_updates_triton.py:285-328). */
typedef struct logkv_partition_args {
  const uint16_t* pool_k;
  int64_t pk_sb, pk_sg, pk_st;
  const uint16_t* pool_v;
  int64_t pv_sb, pv_sg, pv_st;
  const int64_t* pool_pos;
  int64_t pp_sb;
  const uint16_t* flush_k;
  int64_t fk_sb, fk_sg, fk_st;
  const uint16_t* flush_v;
  int64_t fv_sb, fv_sg, fv_st;
  const int64_t* flush_pos;
  int64_t fp_sb;
  int32_t old_width;
  const int32_t* keep;
  const int32_t* archive;
  int32_t P, A, n_batch, n_groups, dk, dv;
  uint16_t* out_pool_k;
  uint16_t* out_pool_v;
  int64_t* out_pool_pos;
  uint8_t* out_pool_valid;
  uint16_t* arch_k;
  uint16_t* arch_v;
  int64_t* arch_pos;
} logkv_partition_args;

int logkv_alpha_partition(const logkv_partition_args* args, void* stream);

/* Read-only view of one cache for the attention readout. Ladder fields as in
 * logkv_ladder_view; exact pool alpha_* [n_batch, G, alpha_cap, d] with
 * positions / valid flags [n_batch, alpha_cap] and alpha_count rows in use
 * (read from alpha_count_dev when that is not NULL, so a flush that chose the
 * exact pool on the device needs no host read); recent window (post-RoPE
 * keys) [n_batch, G, recent_cap, d]; RoPE tables cos / sin [positions, rope_n]
 * f32 or bf16 (table_bf16 = 1) with element strides. */
typedef struct logkv_readout_view {
  const uint16_t* level_k;
  const uint16_t* level_v;
  const float* level_w;
  const int64_t* level_sum_wp;
  const int16_t* level_count;
  int32_t n_batch, n_groups, k_max, levels, slots, dk, dv;
  const uint16_t* alpha_k;
  const uint16_t* alpha_v;
  const int64_t* alpha_pos;
  const uint8_t* alpha_valid;
  int32_t alpha_cap, alpha_count;
  const uint16_t* recent_k;
  const uint16_t* recent_v;
  int32_t recent_cap, recent_count;
  const void* cos;
  const void* sin;
  int64_t cos_s0, cos_s1, sin_s0, sin_s1;
  int32_t rope_n, table_bf16;
  int64_t rope_rows;  /* positions in the tables; anchors beyond clamp to the last row */
  const int32_t* alpha_count_dev;
} logkv_readout_view;

/* Ints of the plan table: per lane K*L + 1 pooled-row offsets (clusters in
 * order, levels top first), then the pooled width (largest lane count). */
int64_t logkv_plan_table_ints(const logkv_readout_view* cache);

/* Mid-anchor slot plan of the occupied entries, kept on the device.
 * Replaces _semantic_mid_attention_plan (litgpt/log_kv_cache.py:5979-6007). */
int logkv_mid_plan(const logkv_readout_view* cache, int32_t* table, void* stream);

/* Packed rows [pooled (width) | exact | recent | current] into out_k / out_v
 * [n_batch, G, out_cap, dim] bf16. With skip_pooled, only the rows from
 * recent window row recent_start on are written (a decode step re-packs only
 * its new rows). Current K/V [n_batch, G, cur_len, d] strided.
 * Replaces pack / pack_mid_kv (litgpt/log_kv_pack_triton.py:95-125,
 * litgpt/log_kv_pack.py:105-133). */
typedef struct logkv_pack_args {
  const uint16_t* cur_k;
  int64_t ck_sb, ck_sg, ck_st;
  const uint16_t* cur_v;
  int64_t cv_sb, cv_sg, cv_st;
  int32_t cur_len;
  uint16_t* out_k;
  uint16_t* out_v;
  int32_t out_cap, dim;
  int32_t skip_pooled, recent_start;
  /* Optional (NULL: not written): per packed row, float mass [n_batch, G, out_cap]
   * (a pooled slot's stored w, 0 for padding; 1 or 0 for an exact row by its
   * valid flag; 1 for recent and current rows) and uint8 validity. */
  float* out_w;
  uint8_t* out_valid;
} logkv_pack_args;

int logkv_pack(const logkv_readout_view* cache, const logkv_pack_args* args, const int32_t* table, void* stream);

/* Packed rows [n_batch, G, out_cap, dim] bf16 of unpacked attention slots: keys
 * k [n_batch, G, slots, dk] and values v (bf16, strided), masses w float
 * [n_batch, G, slots]; column dk of a key row is the mass bias lam * log(w), or
 * for the first s_m slots (anchor counts m int64 given) -log(max(m, 1)) +
 * lam * log(max(w, 1)); among the first s_valid slots, those whose uint8 valid
 * flag is 0 become zero rows with bias -10000. Bias rounded to bf16.
 * Replaces the slot encoding of log_kv_slot_attention's Flash path
 * (_slot_sdpa_inputs / _slot_mass_bias, litgpt/log_kv_cache.py:6418-6464,
 * anchor_mass_bias litgpt/log_kv_position.py:128-133). */
typedef struct logkv_slot_pack_args {
  const uint16_t* k;
  int64_t k_sb, k_sg, k_st;
  const uint16_t* v;
  int64_t v_sb, v_sg, v_st;
  const float* w;
  int64_t w_sb, w_sg;
  const int64_t* m;
  int64_t m_sb, m_sg;
  int32_t s_m;
  const uint8_t* valid;
  int64_t valid_sb, valid_sg;
  int32_t s_valid;
  float lam;
  int32_t n_batch, n_groups, slots, dk, dv, dim, out_cap;
  uint16_t* out_k;
  uint16_t* out_v;
} logkv_slot_pack_args;

int logkv_pack_slots(const logkv_slot_pack_args* args, void* stream);

/* Attention of queries q [n_batch, n_heads, tq, dk] (post-RoPE, bf16, strided)
 * over the packed rows k / v [n_batch, G, cap, dim]: pooled width (read from
 * the plan table) + `tail` rows (+ *alpha_count_dev when that is not NULL),
 * the last causal_tail rows causal; out
 * [n_batch, n_heads, tq, dv] bf16 strided. inv_scale_bf16 is 1/scale rounded
 * to bf16 (the packed query's bias coordinate).
 * Replaces the Flash SDPA call on the packed workspace
 * (litgpt/log_kv_cache.py:6751-6758) and log_kv_slot_attention's first-order
 * math (litgpt/log_kv_cache.py:6501-6630). */
typedef struct logkv_attention_args {
  const uint16_t* q;
  int64_t q_sb, q_sh, q_st;
  int32_t n_batch, n_heads, n_groups, tq, dk, dv, dim;
  const uint16_t* k;
  const uint16_t* v;
  int32_t cap;
  int32_t tail;
  int32_t causal_tail;
  float scale, inv_scale_bf16;
  uint16_t* out;
  int64_t o_sb, o_sh, o_st;
  const int32_t* alpha_count_dev;
} logkv_attention_args;

int64_t logkv_attention_workspace_bytes(const logkv_attention_args* args);
int logkv_decode_attention(const logkv_attention_args* args, const int32_t* table, int64_t table_ints,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* logkv_decode_attention without a workspace argument and without any
 * allocation: the split partials live in a device-resident scratch array of
 * the library (16 MiB per GPU, held until the process ends; its address is
 * looked up once per device on the first call there, with that device
 * current). No counterpart in the reference: it is for callers that cannot
 * allocate - code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc. Same arguments and result as logkv_decode_attention
 * (the same kernels); a call whose partials
 * (logkv_attention_workspace_bytes) exceed 16 MiB is rejected with
 * LOGKV_EINVAL. The stream must belong to the current device. Every call on
 * one GPU shares that GPU's scratch, so calls that overlap on one GPU (other
 * streams, other threads) race; serialize them. Each split writes its whole
 * partial before the combine reads it, so nothing needs clearing between
 * calls. */
int logkv_decode_attention_static(const logkv_attention_args* args, const int32_t* table, int64_t table_ints,
                                  void* stream);

/* The same attention for many query rows per KV group (a prefill or training
 * chunk), on the matrix cores (QK^T in bf16, PV in fp16 with P rounded to fp16,
 * fp32 accumulation): packed width <= 144, dv in {32, 64, 96, 128}. The
 * workspace (logkv_chunk_workspace_bytes, never 0) holds an exact fp16 copy of
 * each lane's V scaled by a power of two 2^-k (any k: the output is scaled
 * back by 2^k), made when the lane's nonzero magnitudes span at most 29
 * binades; a lane beyond that, or holding an infinity, NaN or subnormal, reads
 * its bf16 rows with P split into high and low bf16 parts instead. When the
 * key range is split over several blocks per query tile to fill the GPU, the
 * workspace also holds their partials, combined in split order.
 * Replaces the Flash SDPA call of _packed_flash_attention / _mid_chunk_attention
 * on a chunk (litgpt/log_kv_cache.py:6751-6758, :6802-6836). */
int64_t logkv_chunk_workspace_bytes(const logkv_attention_args* args);
int logkv_chunk_attention(const logkv_attention_args* args, const int32_t* table, int64_t table_ints,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* Gradient of that attention (matrix cores): given dout [n_batch, n_heads, tq, dv]
 * (bf16, strided) and the forward's output in args->out, writes dq
 * [n_batch, n_heads, tq, dk] (bf16, strided; the bias coordinate has no gradient)
 * and, for the last grad_rows packed rows of each lane (the in-flight chunk of a
 * training block, or every slot), dk [n_batch, G, grad_rows, dk] and dv
 * [n_batch, G, grad_rows, dv] (bf16, contiguous). grad_rows <= tail. dk a multiple
 * of 8 up to 128, dv in {32, 64, 96, 128}, packed width up to 144. The workspace
 * (logkv_chunk_backward_workspace_bytes) holds each query's log-sum-exp and
 * dout . out between the two launches.
 * Replaces the autograd backward of the Flash SDPA call on the packed workspace
 * (litgpt/log_kv_cache.py:6751-6758) that LogKVStreamTrainingAttention.backward
 * runs per block (litgpt/log_kv_cache.py:7032-7098). */
typedef struct logkv_attention_grad_args {
  const uint16_t* dout;
  int64_t do_sb, do_sh, do_st;
  uint16_t* dq;
  int64_t dq_sb, dq_sh, dq_st;
  uint16_t* dk;
  uint16_t* dv;
  int32_t grad_rows;
} logkv_attention_grad_args;

int64_t logkv_chunk_backward_workspace_bytes(const logkv_attention_args* args);
int logkv_chunk_attention_backward(const logkv_attention_args* args, const int32_t* table, int64_t table_ints,
                                   const logkv_attention_grad_args* grads, void* workspace,
                                   int64_t workspace_bytes, void* stream);

/* Beta 4->2 compaction of a block of n_rows entries (rows of each field
 * contiguous per row, K / V bf16 or float32 with row strides k_st / v_st in
 * elements): each layout row (start, width, out_start) of n_groups int64
 * triples is a group of width 4 or 2. apply = 0 chooses each full group's cut
 * in (2, 1, 3) of smallest normalised K + V distortion (ties keep the earlier)
 * and writes it to cuts (1 for a two-row tail); apply = 1 reads recorded cuts.
 * Outputs at out_start (+1 for the right side of a full group): float32
 * weighted means of K and V [n_rows / 2, d], mass, p_lo / p_hi over the side's
 * rows of positive mass (0 when the side has no mass), sum of sum_wp, smallest
 * order, AND of pad. With out_k NULL only the cuts are chosen. Metadata
 * pointers may be NULL (their outputs are skipped). A group whose layout or
 * recorded cut is out of range is skipped and sets bit 0 of *status (when not
 * NULL; the caller clears it).
 * Replaces beta_log_kv.select_cuts / apply_cuts / merge_blocks
 * (litgpt/beta_log_kv.py:29-105) and the fused _beta_merge kernel
 * (litgpt/log_kv_updates_triton.py:90-173). */
typedef struct logkv_beta_args {
  const void* k;
  int64_t k_st;
  int32_t k_f32;
  const void* v;
  int64_t v_st;
  int32_t v_f32;
  const float* w;
  const int64_t* p_lo;
  const int64_t* p_hi;
  const int64_t* sum_wp;
  const int64_t* order;
  const uint8_t* pad;
  int64_t n_rows;
  int32_t dk, dv;
  const int64_t* layout;
  int64_t n_groups;
  uint8_t* cuts;
  int32_t apply;
  float* out_k;
  float* out_v;
  float* out_w;
  int64_t* out_p_lo;
  int64_t* out_p_hi;
  int64_t* out_sum_wp;
  int64_t* out_order;
  uint8_t* out_pad;
} logkv_beta_args;

int logkv_beta_merge(const logkv_beta_args* args, int32_t* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOGKV_HIP_H */
