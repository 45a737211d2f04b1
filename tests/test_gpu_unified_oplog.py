"""Op-log and update tape of the unified route: the recorded rows (each lane's
WARD_MERGE rows, then its NEW_CLUSTER / JOIN rows) against the oracle's, a
replay from per-lane cursors into the recorded states, an oracle-written log
replayed on the device into the oracle's states, the replay checks (which
raise and write nothing), and the update tape (litgpt/log_kv_cache.py:
2597-2598, :3661-3688, :4856-4926, :4946-5114)."""

import numpy as np
import pytest
import torch

from harness import compare_state, to_np
from oracle import oplog as ora_oplog
from test_gpu_unified import _pair
from workloads import Mixture, rope_tables

pytestmark = pytest.mark.gpu

# batch, groups, dim, K, B, T, flushes, s_h (drifting centers force old-old merges)
CASE = (2, 2, 16, 4, 8, 24, 8, 4.0)


def _flushes(batch, groups, dim, K, T, n, seed=17, drift=48):
    mix = Mixture(batch, groups, dim, clusters=K + 2, seed=seed, drift_every=drift)
    out = []
    for i in range(n):
        k, v = mix.rows(T), mix.rows(T)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).expand(batch, -1).contiguous()
        out.append((k, v, pos))
    return out


def _state(cache):
    return {name: t.clone() for name, t in cache.named_buffers()}


def _same_state(cache, want):
    return [name for name, t in cache.named_buffers() if not torch.equal(t, want[name])]


def test_unified_recorded_rows_match_oracle():
    batch, groups, dim, K, B, T, n, s_h = CASE
    print("case unified record", flush=True)
    gpu, ora = _pair(batch, groups, dim, K, B, T, T * (n + 2), s_h)
    gpu.begin_op_log()
    ora.begin_op_log()
    dev = gpu.level_k.device
    for i, (k, v, pos) in enumerate(_flushes(batch, groups, dim, K, T, n)):
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), record_op_log=True)
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy())
        log, lengths = gpu.take_op_log()
        want, want_len = ora_oplog.to_array(ora.op_log, capacity=log.size(2))
        assert np.array_equal(to_np(lengths), want_len), f"flush {i}: lengths"
        assert np.array_equal(to_np(log), want), f"flush {i}: rows"
        assert gpu._last_op_log_host == ora.op_log
        bad = compare_state(gpu, ora)
        assert not bad, f"flush {i}: " + "; ".join(bad)
    assert ora.ward_merges > 0, "no old-old merge was logged"
    assert any(row[0] == ora_oplog.WARD_MERGE for lane in ora.op_log for rows in lane for row in rows)


def test_unified_replay_reproduces_recorded_states():
    batch, groups, dim, K, B, T, n, s_h = CASE
    print("case unified replay", flush=True)
    gpu, _ = _pair(batch, groups, dim, K, B, T, T * (n + 2), s_h)
    dev = gpu.level_k.device
    flushes = [(k.to(dev), v.to(dev), pos.to(dev)) for k, v, pos in _flushes(batch, groups, dim, K, T, n)]
    gpu.begin_op_log()
    states = []
    for k, v, pos in flushes:
        gpu.route_and_flush_batch(k, v, pos, record_op_log=True)
        states.append(_state(gpu))
    log, lengths = gpu.take_op_log()
    ends = to_np(lengths).astype(int).tolist()
    assert len({c for row in ends for c in row}) > 1, "the lanes' logs should differ in length (Ward rows)"
    for rep in range(2):
        gpu.reset_parameters()
        for i, ((k, v, pos), want) in enumerate(zip(flushes, states)):
            gpu.route_and_flush_batch(k, v, pos, replay_op_log=log, replay_op_log_len=lengths)
            torch.cuda.synchronize()
            bad = _same_state(gpu, want)
            assert not bad, f"pass {rep}, flush {i}: {bad}"
        assert gpu._op_replay_cursor_host == ends


def test_unified_replay_of_oracle_log_matches_oracle():
    """A unified log written by the oracle replays on the device into the oracle's states."""
    batch, groups, dim, K, B, T, n, s_h = CASE
    print("case unified oracle log", flush=True)
    gpu, ora = _pair(batch, groups, dim, K, B, T, T * (n + 2), s_h)
    ora.begin_op_log()
    flushes = _flushes(batch, groups, dim, K, T, n, seed=23)
    for k, v, pos in flushes:
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy())
    assert ora.ward_merges > 0
    rows, lengths = ora_oplog.to_array(ora.op_log)
    dev = gpu.level_k.device
    log, lens = torch.from_numpy(rows).to(dev), torch.from_numpy(lengths).to(dev)
    ora2 = _pair(batch, groups, dim, K, B, T, T * (n + 2), s_h)[1]
    for i, (k, v, pos) in enumerate(flushes):
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), replay_op_log=log, replay_op_log_len=lens)
        ora2.replay_rows(k.float().numpy(), v.float().numpy(), pos.numpy(), ora.op_log)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora2)
        assert not bad, f"flush {i}: " + "; ".join(bad)


def test_unified_replay_checks_raise_and_write_nothing():
    batch, groups, dim, K, B, T, n, s_h = CASE
    gpu, _ = _pair(batch, groups, dim, K, B, T, T * (n + 2), s_h)
    dev = gpu.level_k.device
    flushes = [(k.to(dev), v.to(dev), pos.to(dev)) for k, v, pos in _flushes(batch, groups, dim, K, T, n)]
    gpu.begin_op_log()
    for k, v, pos in flushes:
        gpu.route_and_flush_batch(k, v, pos, record_op_log=True)
    log, lengths = gpu.take_op_log()
    # The first flush whose lane (0, 0) rows open with a Ward merge (a flush
    # without one consumes exactly T rows of the lane).
    rows = gpu._last_op_log_host[0][0]
    at = None
    cursor = 0
    for flush in range(n):
        if cursor < len(rows) and rows[cursor][0] == ora_oplog.WARD_MERGE:
            at = cursor
            break
        cursor += T
    assert at is not None, "no Ward merge logged in lane (0, 0)"

    def expect(what, log_):
        gpu.reset_parameters()
        for k, v, pos in flushes[:flush]:
            gpu.route_and_flush_batch(k, v, pos, replay_op_log=log, replay_op_log_len=lengths)
        before = _state(gpu)
        cursors = [list(r) for r in gpu._op_replay_cursor_host]
        k, v, pos = flushes[flush]
        with pytest.raises(RuntimeError, match=what):
            gpu.route_and_flush_batch(k, v, pos, replay_op_log=log_, replay_op_log_len=lengths)
        assert not _same_state(gpu, before)
        assert gpu._op_replay_cursor_host == cursors

    bad = log.clone()
    bad[0, 0, at, 2] = bad[0, 0, at, 1]        # keep == free
    expect("Ward merges only lead", bad)
    bad = log.clone()
    bad[0, 0, at, 1] = K                       # a cluster out of range
    expect("Ward merges only lead", bad)


def test_unified_update_tape_replays_without_routing():
    from unittest.mock import patch

    from logkv_amd import LogStructuredKVCache
    from logkv_amd.log_kv_cache import _SemanticReplayUpdates

    batch, groups, dim, K, B, T, n, s_h = CASE
    print("case unified tape", flush=True)
    cos, sin = rope_tables(T * (n + 2), dim)
    cache = LogStructuredKVCache(
        (batch, groups, T * (n + 2), dim), (batch, groups, T * (n + 2), dim), B=B, recent_size=T, device="cuda",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=s_h,
        semantic_flush_granularity=T, semantic_anchor_mode="mid", allocate_second_order=False,
        semantic_unified_route=True, semantic_replay_updates=True, cos_cache=cos, sin_cache=sin, rope_n_elem=dim)
    dev = cache.level_k.device
    tape = _SemanticReplayUpdates()
    cache.begin_op_log()
    inputs, expected = [], []
    for k, v, pos in _flushes(batch, groups, dim, K, T, n):
        k, v, pos = k.to(dev), v.to(dev), pos.to(dev)
        host = pos.cpu().tolist()
        inputs.append((k, v, pos, host))
        with cache._semantic_update_context(tape):
            cache.route_and_flush_batch(k, v, pos, positions_host=host, record_op_log=True)
        expected.append(_state(cache))
    log, lengths = cache.take_op_log()
    assert any(row[0] == ora_oplog.WARD_MERGE for lane in cache._last_op_log_host for rows in lane for row in rows)
    for rep in range(2):
        cache.reset_parameters()
        with patch.object(cache, "_route_commit", side_effect=AssertionError("rerouted")):
            for i, ((k, v, pos, host), want) in enumerate(zip(inputs, expected)):
                with cache._semantic_update_context(tape, replay=True):
                    cache.route_and_flush_batch(k, v, pos, positions_host=host, replay_op_log=log,
                                                replay_op_log_len=lengths)
                torch.cuda.synchronize()
                bad = _same_state(cache, want)
                assert not bad, f"pass {rep}, flush {i}: {bad}"
