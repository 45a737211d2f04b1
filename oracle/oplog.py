"""CPU restatement of the route op-log: what a routed flush records, and how a
logged flush is parsed back into commits.

TEST INFRASTRUCTURE ONLY (the oracle): used by ``tests/`` and never by the
product package.

Row format (litgpt/log_kv_cache.py:90-94, :2006-2096): per lane (batch row,
KV group) tuples ``(op, cluster, arg, position)``; the attach route records
* ``NEW_CLUSTER (c, 0, earliest position)`` for each cluster a flush opens,
  lanes' new clusters in ascending id (litgpt/log_kv_cache.py:2286-2297,
  called first from :4702-4703);
* ``JOIN (c, 0, position)`` for the other rows of every ordinary join, jobs in
  ascending cluster, rows in position order (litgpt/log_kv_cache.py:4153-4166);
* with Alpha's delayed archival, the delayed clusters' ``JOIN`` rows after all
  ordinary ones (litgpt/log_kv_cache.py:3782-3788).

Replay parse (litgpt/log_kv_cache.py:4856-4926): from each lane's cursor,
consume one row per flushed token; consecutive ``JOIN`` rows of one cluster
and segment form one run; joins of distinct clusters share a round and a
structural op (a new cluster here) follows its round's joins.
"""

from __future__ import annotations

import numpy as np

NEW_CLUSTER, NEW_SEGMENT, JOIN, WARD_MERGE, PAD_INSERT = 0, 1, 2, 3, 4


def flush_rows(jobs, pos, late):
    """Rows one flush appends per lane.

    ``jobs``: ``{(b, g, c): (new, rows)}`` with flush offsets in position
    order (``oracle.route.commit_jobs``); ``pos``: ``[Bt, T]`` positions;
    ``late``: the set of ``(b, g, c)`` committed by delayed archival.
    Returns ``{(b, g): [(op, c, arg, position), ...]}``.
    """
    lanes = {}
    for (b, g, c), (new, rows) in sorted(jobs.items()):
        new_rows, ordinary, delayed = lanes.setdefault((b, g), ([], [], []))
        rows = list(rows)
        if new:
            new_rows.append((NEW_CLUSTER, c, 0, int(pos[b, rows[0]])))
            rows = rows[1:]
        target = delayed if (b, g, c) in late else ordinary
        target.extend((JOIN, c, 0, int(pos[b, t])) for t in rows)
    return {lane: a + o + d for lane, (a, o, d) in lanes.items()}


def replay_plan(host_log, cursors, positions_host, n_groups, n_tokens):
    """(end cursors, rounds) of one logged flush (litgpt/log_kv_cache.py:4856-4926).

    ``rounds`` is a list of ``(joins, specials)``: ``joins`` holds
    ``(b, g, cluster, arg, new_segment, offsets)`` runs of distinct clusters,
    ``specials`` holds ``(b, g, (kind, cluster, arg, offset, None))`` applied
    after them. Raises ``RuntimeError`` / ``ValueError`` as the reference does.
    """
    offset_by_token = []
    for b, row in enumerate(positions_host):
        offsets = {int(t): i for i, t in enumerate(row)}
        if len(offsets) != len(row):
            raise RuntimeError(f"semantic LogKV replay positions contain duplicate token ids for batch={b}")
        offset_by_token.append(offsets)
    lane_items, end_cursors = [], []
    try:
        for b in range(len(cursors)):
            ends = []
            for g in range(n_groups):
                consumed, rows, cursor, items = 0, host_log[b][g], cursors[b][g], []
                while consumed < n_tokens and cursor < len(rows):
                    op, cluster, arg, token = rows[cursor]
                    cursor += 1
                    if op == PAD_INSERT:
                        items.append(("pad", cluster, token, None, None))
                    elif op == WARD_MERGE:
                        items.append(("ward", cluster, arg, None, None))
                    elif op == NEW_CLUSTER:
                        items.append(("new", cluster, token, offset_by_token[b][int(token)], None))
                        consumed += 1
                    elif op in (JOIN, NEW_SEGMENT):
                        offsets = [offset_by_token[b][int(token)]]
                        while cursor < len(rows) and consumed + len(offsets) < n_tokens:
                            nop, nc, narg, token = rows[cursor]
                            if nop != JOIN or nc != cluster or narg != arg:
                                break
                            offsets.append(offset_by_token[b][int(token)])
                            cursor += 1
                        items.append(("join", cluster, arg, offsets, op == NEW_SEGMENT))
                        consumed += len(offsets)
                    else:
                        raise ValueError(f"unknown semantic LogKV op {op}")
                if consumed != n_tokens:
                    raise RuntimeError(
                        f"semantic LogKV replay consumed {consumed}/{n_tokens} tokens for batch={b}, group={g}")
                ends.append(cursor)
                lane_items.append((b, g, items))
            end_cursors.append(tuple(ends))
    except KeyError as exc:
        raise RuntimeError(f"semantic LogKV replay token {exc.args[0]} not in current flush positions") from exc
    ptr = [0] * len(lane_items)
    rounds = []
    while any(ptr[i] < len(items) for i, (_, _, items) in enumerate(lane_items)):
        joins, specials = [], []
        for i, (b, g, items) in enumerate(lane_items):
            used = set()
            while ptr[i] < len(items):
                kind, cluster, arg, offsets, new_segment = items[ptr[i]]
                if kind != "join" or cluster in used:
                    break
                used.add(cluster)
                joins.append((b, g, cluster, arg, new_segment, offsets))
                ptr[i] += 1
            if ptr[i] < len(items) and items[ptr[i]][0] != "join":
                specials.append((b, g, items[ptr[i]]))
                ptr[i] += 1
        rounds.append((joins, specials))
    return tuple(end_cursors), rounds


def as_lists(lanes, n_batch, n_groups):
    """``{(b, g): rows}`` -> the reference's host log layout ``[b][g] -> rows``."""
    return [[list(lanes.get((b, g), [])) for g in range(n_groups)] for b in range(n_batch)]


def to_array(host_log, capacity=None):
    """Host log -> (rows ``[Bt, G, cap, 4]`` int32, lengths ``[Bt, G]`` int32), zeros past each length."""
    n_batch, n_groups = len(host_log), len(host_log[0])
    lengths = np.array([[len(host_log[b][g]) for g in range(n_groups)] for b in range(n_batch)], np.int32)
    cap = int(capacity if capacity is not None else max(1, lengths.max(initial=0)))
    out = np.zeros((n_batch, n_groups, cap, 4), np.int32)
    for b in range(n_batch):
        for g in range(n_groups):
            rows = host_log[b][g]
            if rows:
                out[b, g, :len(rows)] = np.asarray(rows, np.int32)
    return out, lengths
