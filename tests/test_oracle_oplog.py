"""Pins of the oracle's op-log restatement (oracle/oplog.py) without the device.

* hand-derived logs of small flushes, read off the reference's record sites
  (litgpt/log_kv_cache.py:2286-2297, :4153-4166, :3782-3788): a lane's opened
  clusters come first in ascending cluster id (not in position order), then
  the joins by cluster with rows in position order, the opening row left
  out; delayed-archive joins follow every ordinary join of the lane;
* the replay schedule of the reference's parse (litgpt/log_kv_cache.py:
  4856-4926) on a known log: one structural op per round after that round's
  joins, consecutive joins of one cluster merged into one run;
* replaying a recorded stream into an empty cache reproduces every recorded
  state bit for bit (the reference's tests/test_log_kv_update_replay.py:75-94);
* the parse's errors: unknown token, duplicate positions, a short log, an
  unknown op code.
"""

import numpy as np
import pytest

from workloads import Mixture
from oracle import OracleCache, oplog

FIELDS = ("level_k", "level_v", "level_w", "level_p_lo", "level_p_hi", "level_sum_wp", "level_order", "pad_mask",
          "level_count", "centroid", "n_eff", "n_total", "p_hi_c", "level0_phase", "alive")


def e(*x):
    return np.asarray(x, np.float32)


def test_attach_log_known_answer():
    # Clusters 0 (center +10 e0) and 2 (-10 e0) live, 1 and 3 free, radius^2 4.
    # Rows at positions 10..15: 10 -> 0, 11 orphan, 12 -> 2, 13 -> 0, 14 orphan
    # (farther from every center than 11, so the first seed: slot 1), 11 the
    # second seed (slot 3), 15 joins the seed at 11 (slot 3).
    c = OracleCache(1, 1, 256, 4, 4, B=4, recent_size=8, K=4, s_h=4.0, flush=8)
    c.new_cluster(0, 0, 0, e(10, 0, 0, 0), e(1, 1, 1, 1), 2)
    c.new_cluster(0, 0, 2, e(-10, 0, 0, 0), e(1, 1, 1, 1), 3)
    c.begin_op_log()
    k = np.stack([e(10.5, 0, 0, 0), e(0, 0, 50, 0), e(-10.2, 0, 0, 0), e(10.1, 0, 0, 0), e(0, 0, 0, -60),
                  e(0, 0, 49, 0)])[None, None]
    c.flush_rows(k, np.ones_like(k), np.arange(10, 16)[None])
    assert c.op_log == [[[(0, 1, 0, 14), (0, 3, 0, 11), (2, 0, 0, 10), (2, 0, 0, 13), (2, 2, 0, 12),
                          (2, 3, 0, 15)]]]


def test_delayed_joins_follow_ordinary_known_answer():
    # Alpha archive rows 3 and 4 join cluster 0 (p_hi 40: delayed), 20 joins
    # cluster 1 (p_hi 5: ordinary); the ordinary row is logged first.
    c = OracleCache(1, 1, 256, 4, 4, B=4, recent_size=8, K=4, s_h=4.0, flush=8, exact_tokens=4, span_max=2)
    c.new_cluster(0, 0, 0, e(10, 0, 0, 0), e(1, 1, 1, 1), 40)
    c.new_cluster(0, 0, 1, e(-10, 0, 0, 0), e(1, 1, 1, 1), 5)
    c.begin_op_log()
    ak = np.stack([e(10.2, 0, 0, 0), e(-10.1, 0, 0, 0), e(9.9, 0, 0, 0)])[None, None]
    c.route_and_commit(ak, np.ones_like(ak), np.asarray([[3, 20, 4]]), np.asarray([3]))
    assert c.late_joins == 1
    assert c.op_log == [[[(2, 1, 0, 20), (2, 0, 0, 3), (2, 0, 0, 4)]]]


def test_replay_schedule_known_answer():
    log = [[[(0, 1, 0, 14), (0, 3, 0, 11), (2, 0, 0, 10), (2, 0, 0, 13), (2, 2, 0, 12), (2, 3, 0, 15)]]]
    ends, rounds = oplog.replay_plan(log, [[0]], [list(range(10, 16))], 1, 6)
    assert ends == ((6,),)
    assert rounds == [
        ([], [(0, 0, ("new", 1, 14, 4, None))]),
        ([], [(0, 0, ("new", 3, 11, 1, None))]),
        ([(0, 0, 0, 0, False, [0, 3]), (0, 0, 2, 0, False, [2]), (0, 0, 3, 0, False, [5])], []),
    ]
    # A run stops at the flush's token count even when the next row continues it.
    ends, rounds = oplog.replay_plan([[[(2, 0, 0, 1), (2, 0, 0, 2), (2, 0, 0, 3)]]], [[0]], [[1, 2]], 1, 2)
    assert ends == ((2,),) and rounds == [([(0, 0, 0, 0, False, [0, 1])], [])]


@pytest.mark.parametrize("batch,groups", [(1, 1), (2, 2)])
def test_replay_reproduces_recorded_states(batch, groups):
    dim, T = 8, 16
    kw = dict(B=4, recent_size=T, K=4, s_h=6.0, flush=T)
    rec = OracleCache(batch, groups, 1024, dim, dim, **kw)
    rec.begin_op_log()
    mix = Mixture(batch, groups, dim, clusters=5, seed=9)
    flushes, states = [], []
    for i in range(12):
        k, v = mix.rows(T).float().numpy(), mix.rows(T).float().numpy()
        pos = np.broadcast_to(np.arange(i * T, (i + 1) * T), (batch, T)).copy()
        rec.flush_rows(k, v, pos)
        flushes.append((k, v, pos))
        states.append({f: getattr(rec, f).copy() for f in FIELDS})
    assert rec.level_count.sum() > 0 and rec.alive.all()
    assert all(len(rec.op_log[b][g]) == 12 * T for b in range(batch) for g in range(groups))
    rep = OracleCache(batch, groups, 1024, dim, dim, **kw)
    for (k, v, pos), want in zip(flushes, states):
        rep.replay_rows(k, v, pos, rec.op_log)
        for f in FIELDS:
            assert np.array_equal(getattr(rep, f), want[f]), f
    assert rep.replay_cursor == [[12 * T] * groups for _ in range(batch)]


def test_replay_parse_errors():
    log = [[[(0, 1, 0, 14), (2, 1, 0, 15)]]]
    with pytest.raises(RuntimeError, match="not in current flush positions"):
        oplog.replay_plan(log, [[0]], [[14, 16]], 1, 2)
    with pytest.raises(RuntimeError, match="duplicate token ids"):
        oplog.replay_plan(log, [[0]], [[14, 14]], 1, 2)
    with pytest.raises(RuntimeError, match="consumed 2/3 tokens"):
        oplog.replay_plan(log, [[0]], [[14, 15, 16]], 1, 3)
    with pytest.raises(ValueError, match="unknown semantic LogKV op 7"):
        oplog.replay_plan([[[(7, 1, 0, 14)]]], [[0]], [[14]], 1, 1)


def test_replay_schedule_leading_ward_rows():
    """A unified flush's WARD_MERGE rows lead its lane and replay one a round,
    before any of the flush's opening or join rounds."""
    log = [[[(3, 2, 0, -1), (3, 1, 3, -1), (0, 0, 0, 11), (2, 1, 0, 10)]]]
    ends, rounds = oplog.replay_plan(log, [[0]], [[10, 11]], 1, 2)
    assert ends == ((4,),)
    assert rounds == [
        ([], [(0, 0, ("ward", 2, 0, None, None))]),
        ([], [(0, 0, ("ward", 1, 3, None, None))]),
        ([], [(0, 0, ("new", 0, 11, 1, None))]),
        ([(0, 0, 1, 0, False, [0])], []),
    ]


def test_unified_replay_reproduces_recorded_states():
    """A unified-routed stream's log (old-old Ward merges first in each lane)
    replays into every recorded state; lanes with Ward rows end at their own
    cursors."""
    from workloads import rope_tables

    batch, groups, dim, K, B, T, n, s_h = 2, 2, 16, 4, 8, 24, 8, 4.0
    cos, sin = rope_tables(T * (n + 2), dim)
    kw = dict(B=B, recent_size=T, K=K, s_h=s_h, flush=T, exact_tokens=0, span_max=4, beta_novelty=False,
              beta_adaptive=False, cos=cos.numpy(), sin=sin.numpy(), unified=True)
    rec = OracleCache(batch, groups, T * (n + 2), dim, dim, **kw)
    rec.begin_op_log()
    mix = Mixture(batch, groups, dim, clusters=K + 2, seed=17, drift_every=48)
    flushes, states = [], []
    for i in range(n):
        k, v = mix.rows(T).float().numpy(), mix.rows(T).float().numpy()
        pos = np.broadcast_to(np.arange(i * T, (i + 1) * T), (batch, T)).copy()
        rec.flush_rows(k, v, pos)
        flushes.append((k, v, pos))
        states.append({f: getattr(rec, f).copy() for f in FIELDS})
    assert rec.ward_merges > 0
    wards = [[sum(r[0] == oplog.WARD_MERGE for r in rec.op_log[b][g]) for g in range(groups)] for b in range(batch)]
    lengths = [[len(rec.op_log[b][g]) for g in range(groups)] for b in range(batch)]
    assert lengths == [[n * T + w for w in row] for row in wards]
    assert len({c for row in lengths for c in row}) > 1
    rep = OracleCache(batch, groups, T * (n + 2), dim, dim, **kw)
    for i, ((k, v, pos), want) in enumerate(zip(flushes, states)):
        rep.replay_rows(k, v, pos, rec.op_log)
        for f in FIELDS:
            assert np.array_equal(getattr(rep, f), want[f]), (i, f)
    assert rep.replay_cursor == lengths
