"""CPU restatement of one SemanticLogKV layer cache: recent window, flush, ladders, exact pool.

TEST INFRASTRUCTURE ONLY (the oracle): used by ``tests/``, the smoke check and
the CPU-baseline leg of the benchmark, never by the product package.

State uses the reference's buffer names and layouts
(litgpt/log_kv_cache.py:881-1121): ``level_*`` ``[Bt, G, K, L, B', ...]``,
``level_count`` ``[Bt, G, K, L]``, cluster scalars ``[Bt, G, K]``, recent window
``[Bt, G, 2*recent, D]``, exact pool ``[Bt, G, P, D]``. bf16 tensors are held as
float32 arrays of bf16 values.

One flush (litgpt/log_kv_cache.py:5609-5666, :5033-5128):
* Alpha on: snapshot ``[pool | flush]``, cut / score / choose whole spans,
  rewrite the exact pool, archive the rest (litgpt/log_kv_cache.py:3904-4003);
* attach route of the archived (or all flushed) rows (oracle.route);
* per (lane, cluster) job in position order: a dead cluster opens with its
  earliest row (litgpt/log_kv_cache.py:2268-2298); the other rows are joined -
  ordinary joins append ``w=1`` entries with ``order = phase + rank`` and
  update the center (litgpt/log_kv_cache.py:4116-4175, :4225-4361); with Alpha,
  a job whose earliest row precedes the cluster's ``p_hi`` re-sorts the whole
  cluster by ``p_lo`` and re-appends it (litgpt/log_kv_cache.py:3690-3788);
* the recent window shifts down by the flushed rows.
"""

from __future__ import annotations

import math

import numpy as np

from . import ladder as lad
from . import oplog, readout, route, spans, unified
from .numerics import bf16_round, f32

I64_MAX = np.iinfo(np.int64).max


def budget(batch, groups, max_seq, dk, dv, B, K, exact_tokens, element=2):
    """(B', L, baseline bytes, needed bytes) of the ladder (litgpt/log_kv_cache.py:857, :879-898)."""
    def levels(b):
        return max(2, math.ceil(math.log2(max_seq / max(K * b, 1) + 1.0)) + 2)

    L = levels(B)
    if not exact_tokens:
        return B, L, None, None
    pd = ((max(dk + 1, dv) + 7) // 8) * 8
    entry = (dk + dv + 2 * pd) * element + 41
    exact = exact_tokens * (groups * (dk + dv + 2 * pd) * element + 9)
    base = groups * K * L * (B * entry + 2)
    for cand in range(B - 1, 1, -1):
        lv = levels(cand)
        need = groups * K * lv * (cand * entry + 2) + exact
        if need <= base:
            return cand, lv, batch * base, batch * need
    raise ValueError("compressed ladder budget is too small for alpha_exact_tokens")


class OracleCache:
    def __init__(self, batch, groups, max_seq, dk, dv, *, B=128, recent_size=2048, K=12, lam=1.0, eta=1.0,
                 g0=2048.0, s_h=1.0, flush=2048, exact_tokens=0, span_max=64, beta_novelty=False,
                 beta_adaptive=False, cos=None, sin=None, table_bf16=False, unified=False, centroid_tile=1,
                 hard_cap_mult=0.0, merge_passes=1):
        self.batch, self.groups, self.max_seq, self.dk, self.dv = batch, groups, max_seq, dk, dv
        self.K, self.lam, self.eta, self.g0 = K, lam, eta, g0
        self.B, self.L, *_ = budget(batch, groups, max_seq, dk, dv, B, K, exact_tokens)
        self.recent_size, self.flush_n = recent_size, flush
        self.recent_capacity = 2 * recent_size
        self.P, self.span_max = exact_tokens, span_max
        self.beta_novelty, self.beta_adaptive = beta_novelty, beta_adaptive
        self.cos, self.sin, self.table_bf16 = cos, sin, table_bf16
        self.centroid_tile = centroid_tile       # 1: sequential centroid backend, 32: parallel
        # Capacity cap of the attach route (litgpt/log_kv_cache.py:2347-2354): max_seq / K rows
        # (at least 1) times the multiplier; none for a multiplier <= 0.
        self.hard_cap = max(float(max_seq) / max(K, 1), 1.0) * hard_cap_mult if hard_cap_mult > 0 else np.inf
        shp = (batch, groups, K, self.L, self.B)
        self.level_k = np.zeros(shp + (dk,), np.float32)
        self.level_v = np.zeros(shp + (dv,), np.float32)
        self.level_w = np.zeros(shp, np.float32)
        self.level_p_lo = np.full(shp, I64_MAX, np.int64)
        self.level_p_hi = np.full(shp, -1, np.int64)
        self.level_sum_wp = np.zeros(shp, np.int64)
        self.level_order = np.zeros(shp, np.int64)
        self.pad_mask = np.zeros(shp, bool)
        self.level_count = np.zeros((batch, groups, K, self.L), np.int64)
        self.centroid = np.zeros((batch, groups, K, dk), np.float32)
        self.n_eff = np.zeros((batch, groups, K), np.float32)
        self.n_total = np.zeros((batch, groups, K), np.int64)
        self.p_hi_c = np.full((batch, groups, K), -1, np.int64)
        self.level0_phase = np.zeros((batch, groups, K), np.int64)
        self.alive = np.zeros((batch, groups, K), bool)
        self.s_h = np.broadcast_to(f32(s_h), (batch, groups)).astype(np.float32).copy()
        cap = self.recent_capacity
        self.recent_k = np.zeros((batch, groups, cap, dk), np.float32)
        self.recent_k_raw = np.zeros((batch, groups, cap, dk), np.float32)
        self.recent_v = np.zeros((batch, groups, cap, dv), np.float32)
        self.recent_pos = np.zeros((batch, cap), np.int64)
        self.recent_ends = [[False] * cap for _ in range(batch)]
        self.recent_count = 0
        self.token_count = 0
        P = max(exact_tokens, 1)
        self.alpha_k_raw = np.zeros((batch, groups, P, dk), np.float32)
        self.alpha_v = np.zeros((batch, groups, P, dv), np.float32)
        self.alpha_pos = np.zeros((batch, P), np.int64)
        self.alpha_valid = np.zeros((batch, P), bool)
        self.alpha_count = 0
        self.alpha_spans = [[] for _ in range(batch)]
        self.alpha_positions = [[] for _ in range(batch)]
        self.beta_cuts = []
        self.late_joins = 0       # delayed-archive re-sorts performed (test coverage evidence)
        self.op_log = None        # per lane lists of (op, cluster, arg, position), see oracle.oplog
        self.unified = unified    # the unified Ward / radius route (oracle.unified) instead of attach
        self.merge_passes = int(merge_passes)   # frozen-center sweeps per budget round (unified route)
        self.ward_merges = 0      # old-old merges performed by the unified route (test coverage evidence)
        self.replay_cursor = None

    # ---- ladder access -------------------------------------------------
    def ladder(self, b, g, c) -> lad.Ladder:
        rows = {
            "k": self.level_k[b, g, c].reshape(-1, self.dk), "v": self.level_v[b, g, c].reshape(-1, self.dv),
            "w": self.level_w[b, g, c].reshape(-1), "p_lo": self.level_p_lo[b, g, c].reshape(-1),
            "p_hi": self.level_p_hi[b, g, c].reshape(-1), "sum_wp": self.level_sum_wp[b, g, c].reshape(-1),
            "order": self.level_order[b, g, c].reshape(-1), "pad": self.pad_mask[b, g, c].reshape(-1),
        }
        return lad.Ladder(rows, self.level_count[b, g, c], self.L, self.B)

    def _token_rows(self, k, v, pos, order0):
        n = len(pos)
        return {"k": f32(k), "v": f32(v), "w": np.ones(n, np.float32), "p_lo": pos.copy(), "p_hi": pos.copy(),
                "sum_wp": pos.copy(), "order": order0 + np.arange(n, dtype=np.int64), "pad": np.zeros(n, bool)}

    def _append(self, b, g, c, rows):
        cuts = self.ladder(b, g, c).append(rows, beta=self.beta_adaptive)
        self.beta_cuts.append(((b, g, c), cuts))

    # ---- commit ----------------------------------------------------------
    def new_cluster(self, b, g, c, key, value, pos):
        lad_ = self.ladder(b, g, c)
        lad_.clear()
        self.centroid[b, g, c] = f32(key)
        self.n_eff[b, g, c] = 1.0
        self._append(b, g, c, self._token_rows(key[None], value[None], np.asarray([pos], np.int64), 0))
        self.alive[b, g, c] = True
        self.n_total[b, g, c] = 1
        self.p_hi_c[b, g, c] = pos
        self.level0_phase[b, g, c] = 1

    def join(self, b, g, c, keys, values, pos):
        """Ordinary join of rows already in position order."""
        n = len(pos)
        phase = int(self.level0_phase[b, g, c])
        self._append(b, g, c, self._token_rows(keys, values, pos, phase))
        self.centroid[b, g, c], self.n_eff[b, g, c] = lad.centroid_update(
            self.centroid[b, g, c], self.n_eff[b, g, c], keys, tile=self.centroid_tile)
        self.level0_phase[b, g, c] = phase + n
        self.p_hi_c[b, g, c] = pos[-1]
        self.n_total[b, g, c] += n

    def join_late(self, b, g, c, keys, values, pos):
        """Delayed archive: re-sort the cluster's entries and the new rows by position."""
        self.late_joins += 1
        ladder = self.ladder(b, g, c)
        old = ladder.entries()
        new = self._token_rows(keys, values, pos, 0)
        combined = lad.concat([old, new])
        sort = np.argsort(combined["p_lo"], kind="stable")
        rows = lad.take(combined, sort)
        rows["order"] = np.arange(len(sort), dtype=np.int64)
        mu, ne = lad.centroid_update(self.centroid[b, g, c], self.n_eff[b, g, c], keys, tile=self.centroid_tile)
        high = max(int(self.p_hi_c[b, g, c]), int(pos.max()))
        total = int(self.n_total[b, g, c]) + len(pos)
        ladder.clear()
        self.centroid[b, g, c], self.n_eff[b, g, c] = mu, ne
        self.alive[b, g, c] = True
        self.n_total[b, g, c] = total
        self.p_hi_c[b, g, c] = high
        self.level0_phase[b, g, c] = len(sort)
        self._append(b, g, c, rows)

    def route_and_commit(self, ak, av, ap, counts):
        """Attach-route ``counts[b]`` rows of ``ak/av/ap`` and commit them; with
        ``op_log`` bound (``begin_op_log``) the flush's rows are appended to it.
        With ``unified`` the rows take the unified route instead."""
        if self.unified:
            return unified.route_unified(self, ak, av, ap, counts)
        assign, order = route.attach_assign(ak, ap, counts, self.centroid, self.alive, self.p_hi_c, self.s_h,
                                            self.eta, self.g0, self.lam, self.n_total, self.hard_cap)
        jobs = route.commit_jobs(assign, order, counts, self.alive)
        late = set()
        for (b, g, c), (new, rows) in sorted(jobs.items()):
            if new:
                t = rows[0]
                self.new_cluster(b, g, c, ak[b, g, t], av[b, g, t], int(ap[b, t]))
                rows = rows[1:]
            if not len(rows):
                continue
            pos = ap[b, rows].astype(np.int64)
            if self.P and pos.min() < self.p_hi_c[b, g, c]:
                late.add((b, g, c))
                self.join_late(b, g, c, ak[b, g, rows], av[b, g, rows], pos)
            else:
                self.join(b, g, c, ak[b, g, rows], av[b, g, rows], pos)
        if self.op_log is not None:
            for (b, g), rows in oplog.flush_rows(jobs, ap, late).items():
                self.op_log[b][g].extend(rows)
        return assign, order

    # ---- op-log ----------------------------------------------------------
    def begin_op_log(self):
        self.op_log = [[[] for _ in range(self.groups)] for _ in range(self.batch)]
        self.replay_cursor = None

    def replay_rows(self, k_raw, v, pos, host_log):
        """Re-apply one logged flush of ``T`` rows without routing
        (litgpt/log_kv_cache.py:5067-5114, :4178-4223): each run appends its rows
        in log order, each new cluster opens with its row."""
        k_raw, v = f32(k_raw), f32(v)
        pos = np.asarray(pos, np.int64)
        n_batch, n_groups, T, _ = k_raw.shape
        if self.replay_cursor is None:
            self.replay_cursor = [[0] * n_groups for _ in range(n_batch)]
        ends, rounds = oplog.replay_plan(host_log, self.replay_cursor, pos.tolist(), n_groups, T)
        self.replay_cursor = [list(row) for row in ends]
        for joins, specials in rounds:
            for b, g, c, _arg, _new_segment, offsets in joins:
                rows = np.asarray(offsets, np.int64)
                self.join(b, g, c, k_raw[b, g, rows], v[b, g, rows], pos[b, rows])
            for b, g, (kind, c, token, offset, _) in specials:
                if kind == "ward":
                    # A logged old-old merge of the unified route: cluster `token`
                    # (the row's arg) merges into c (litgpt/log_kv_cache.py:2597-2598).
                    unified.ward_merge(self, b, g, c, token)
                    continue
                if kind != "new":
                    raise NotImplementedError("segment pads are not part of this path")
                self.new_cluster(b, g, c, k_raw[b, g, offset], v[b, g, offset], int(token))

    # ---- flush -----------------------------------------------------------
    def flush_rows(self, k_raw, v, pos, ends=None):
        """One flush of ``T`` rows ``k_raw/v [Bt, G, T, D]``, ``pos [Bt, T]``."""
        k_raw, v = f32(k_raw), f32(v)
        pos = np.asarray(pos, np.int64)
        n_batch, _, T, _ = k_raw.shape
        if not self.P:
            return self.route_and_commit(k_raw, v, pos, np.full(n_batch, T, np.int64))
        old_width = self.alpha_count
        keys = np.concatenate((self.alpha_k_raw[:, :, :old_width], k_raw), axis=2)
        values = np.concatenate((self.alpha_v[:, :, :old_width], v), axis=2)
        pos_all = np.concatenate((self.alpha_pos[:, :old_width], pos), axis=1)
        cut = spans.cut_spans(self.alpha_spans, self.alpha_positions, pos.tolist(), ends, old_width, self.span_max)
        if cut is None:
            keep = archive = [[] for _ in range(n_batch)]
            sel_spans = [[] for _ in range(n_batch)]
            sel_pos = [[] for _ in range(n_batch)]
            self.last_scores = np.zeros(0, np.float32)
        else:
            scores = spans.score_spans(keys, values, cut, self.beta_novelty, self.centroid, self.alive)
            self.last_scores = scores
            keep, archive, sel_spans, sel_pos = spans.choose_spans(cut, scores, self.P)
        self.last_selection = (keep, archive)
        self.alpha_k_raw[...] = 0
        self.alpha_v[...] = 0
        self.alpha_pos[...] = 0
        self.alpha_valid[...] = False
        for b in range(n_batch):
            kb = np.asarray(keep[b], np.int64)
            self.alpha_k_raw[b, :, :len(kb)] = keys[b][:, kb]
            self.alpha_v[b, :, :len(kb)] = values[b][:, kb]
            self.alpha_pos[b, :len(kb)] = pos_all[b, kb]
            self.alpha_valid[b, :len(kb)] = True
        self.alpha_count = max(map(len, keep), default=0)
        self.alpha_spans, self.alpha_positions = sel_spans, sel_pos
        counts = np.asarray([len(a) for a in archive], np.int64)
        width = int(counts.max(initial=0))
        if not width:
            return None
        ak = np.zeros((n_batch, self.groups, width, self.dk), np.float32)
        av = np.zeros((n_batch, self.groups, width, self.dv), np.float32)
        ap = np.zeros((n_batch, width), np.int64)
        for b in range(n_batch):
            ab = np.asarray(archive[b], np.int64)
            ak[b, :, :len(ab)] = keys[b][:, ab]
            av[b, :, :len(ab)] = values[b][:, ab]
            ap[b, :len(ab)] = pos_all[b, ab]
        return self.route_and_commit(ak, av, ap, counts)

    def add_recent(self, k, v, k_raw, pos, ends=None):
        """Append a block to the recent window; flush in whole granules on overflow
        (litgpt/log_kv_cache.py:5668-5718)."""
        n = k.shape[2]
        if n > self.recent_size:
            raise ValueError("chunk size exceeds recent_size")
        if self.token_count + n > self.max_seq:
            raise RuntimeError("token overflow")
        self.token_count += n
        c = self.recent_count
        self.recent_k[:, :, c:c + n] = bf16_round(k)
        self.recent_k_raw[:, :, c:c + n] = bf16_round(k_raw)
        self.recent_v[:, :, c:c + n] = bf16_round(v)
        self.recent_pos[:, c:c + n] = np.asarray(pos, np.int64)
        if self.P:
            for b in range(self.batch):
                self.recent_ends[b][c:c + n] = list(ends[b])
        self.recent_count += n
        overflow = self.recent_count - self.recent_size
        if overflow > 0:
            F = self.flush_n
            pending = F * ((overflow + F - 1) // F)
            while pending > 0:
                take = min(F, pending)
                ends_now = [row[:take] for row in self.recent_ends] if self.P else None
                self.flush_rows(self.recent_k_raw[:, :, :take].copy(), self.recent_v[:, :, :take].copy(),
                                self.recent_pos[:, :take].copy(), ends_now)
                rem = self.recent_count - take
                for arr in (self.recent_k, self.recent_k_raw, self.recent_v):
                    arr[:, :, :rem] = arr[:, :, take:self.recent_count].copy()
                    arr[:, :, rem:self.recent_count] = 0
                self.recent_pos[:, :rem] = self.recent_pos[:, take:self.recent_count].copy()
                self.recent_pos[:, rem:self.recent_count] = 0
                if self.P:
                    for b in range(self.batch):
                        row = self.recent_ends[b]
                        row[:rem] = row[take:self.recent_count]
                        row[rem:self.recent_count] = [False] * (self.recent_count - rem)
                self.recent_count = rem
                pending -= take

    # ---- readout ---------------------------------------------------------
    def plan(self):
        return readout.mid_plan(self.level_count, self.level_w, self.level_sum_wp)

    def pack(self, k_cur=None, v_cur=None):
        return readout.pack(self, k_cur, v_cur, self.cos, self.sin, table_bf16=self.table_bf16)
