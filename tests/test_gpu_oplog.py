"""Device op-log: recorded rows against the oracle's, replay against the
recorded states (the reference's tests/test_log_kv_update_replay.py:75-94 and
tests/test_log_kv_replay_plan.py), and the replay checks, which must raise and
leave the cache untouched."""

import numpy as np
import pytest
import torch

from harness import compare_state, make_pair, to_np
from logkv_amd.log_kv_cache import _SemanticReplayPlans
from workloads import Mixture
from oracle import oplog as ora_oplog

pytestmark = pytest.mark.gpu


def _state(cache):
    return {name: t.clone() for name, t in cache.named_buffers()}


def _same_state(cache, want):
    return [name for name, t in cache.named_buffers() if not torch.equal(t, want[name])]


def _flushes(batch, groups, dim, K, T, n, seed=5, ends=False):
    mix = Mixture(batch, groups, dim, clusters=K, seed=seed)
    out = []
    for i in range(n):
        k, v = mix.rows(T), mix.rows(T)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).expand(batch, -1).contiguous()
        e = [[(p + 3 * b) % 7 == 0 for p in range(i * T, (i + 1) * T)] for b in range(batch)] if ends else None
        out.append((k, v, pos, e))
    return out


CASES = {
    # name: (batch, groups, dim, K, B, T, flushes, exact, span, beta)
    "attach": (2, 2, 64, 4, 8, 32, 8, 0, 16, False),
    "qwen_layer": (1, 8, 128, 12, 128, 2048, 3, 0, 16, False),
    "alpha_beta": (2, 2, 64, 4, 8, 32, 10, 16, 4, True),
}


@pytest.mark.parametrize("name", list(CASES))
def test_recorded_rows_match_oracle(name):
    batch, groups, dim, K, B, T, n, exact, span, beta = CASES[name]
    print(f"case {name}", flush=True)
    gpu, ora = make_pair(batch, groups, dim, K, B, recent=T, flush=T, max_seq=T * (n + 1), s_h=16.0, exact=exact,
                         span=span, beta_novelty=beta, beta_adaptive=beta)
    gpu.begin_op_log()
    ora.begin_op_log()
    dev = gpu.level_k.device
    for i, (k, v, pos, ends) in enumerate(_flushes(batch, groups, dim, K, T, n, ends=bool(exact))):
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), span_ends=ends, record_op_log=True)
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy(), ends)
        log, lengths = gpu.take_op_log()
        want, want_len = ora_oplog.to_array(ora.op_log, capacity=log.size(2))
        assert np.array_equal(to_np(lengths), want_len), f"flush {i}: lengths"
        assert np.array_equal(to_np(log), want), f"flush {i}: rows"
        assert gpu._last_op_log_host == ora.op_log
        bad = compare_state(gpu, ora)
        assert not bad, f"flush {i}: " + "; ".join(bad)
    if exact:
        assert ora.late_joins > 0, "no delayed-archive join was logged"


@pytest.mark.parametrize("name", ["attach", "qwen_layer"])
@pytest.mark.parametrize("host_plans", [False, True])
def test_replay_reproduces_recorded_states(name, host_plans):
    batch, groups, dim, K, B, T, n, _, _, _ = CASES[name]
    print(f"case {name} host_plans={host_plans}", flush=True)
    gpu, _ = make_pair(batch, groups, dim, K, B, recent=T, flush=T, max_seq=T * (n + 1), s_h=16.0)
    dev = gpu.level_k.device
    flushes = [(k.to(dev), v.to(dev), pos.to(dev)) for k, v, pos, _ in _flushes(batch, groups, dim, K, T, n)]
    gpu.begin_op_log()
    states = []
    for k, v, pos in flushes:
        gpu.route_and_flush_batch(k, v, pos, record_op_log=True)
        states.append(_state(gpu))
    log, lengths = gpu.take_op_log()
    plans = _SemanticReplayPlans(gpu._last_op_log_host) if host_plans else None
    for rep in range(2):
        gpu.reset_parameters()
        for i, ((k, v, pos), want) in enumerate(zip(flushes, states)):
            host = pos.cpu().tolist()
            gpu.route_and_flush_batch(k, v, pos, positions_host=host, replay_op_log=log, replay_op_log_len=lengths,
                                      replay_op_log_host=plans.host_log if plans else None, replay_plans=plans)
            torch.cuda.synchronize()
            bad = _same_state(gpu, want)
            assert not bad, f"pass {rep}, flush {i}: {bad}"
        assert gpu._op_replay_cursor_host == [[n * T] * groups for _ in range(batch)]
    if plans is not None:
        assert len(plans.plans) == n


def test_replay_of_oracle_log_matches_oracle():
    """A log written by the oracle replays on the device into the oracle's states."""
    batch, groups, dim, K, B, T, n, _, _, _ = CASES["attach"]
    gpu, ora = make_pair(batch, groups, dim, K, B, recent=T, flush=T, max_seq=T * (n + 1), s_h=16.0)
    ora.begin_op_log()
    flushes = _flushes(batch, groups, dim, K, T, n, seed=8)
    states = []
    for k, v, pos, _ in flushes:
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy())
        states.append({f: np.array(getattr(ora, f)) for f in ("level_k", "level_w", "centroid", "n_total")})
    rows, lengths = ora_oplog.to_array(ora.op_log)
    dev = gpu.level_k.device
    log, lens = torch.from_numpy(rows).to(dev), torch.from_numpy(lengths).to(dev)
    ora2 = make_pair(batch, groups, dim, K, B, recent=T, flush=T, max_seq=T * (n + 1), s_h=16.0)[1]
    for i, (k, v, pos, _) in enumerate(flushes):
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), replay_op_log=log, replay_op_log_len=lens)
        ora2.replay_rows(k.float().numpy(), v.float().numpy(), pos.numpy(), ora.op_log)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora2)
        assert not bad, f"flush {i}: " + "; ".join(bad)
        for f, want in states[i].items():
            assert np.array_equal(np.asarray(getattr(ora2, f)), want), f


def test_replay_checks_raise_and_write_nothing():
    batch, groups, dim, K, B, T, n, _, _, _ = CASES["attach"]
    gpu, _ = make_pair(batch, groups, dim, K, B, recent=T, flush=T, max_seq=T * (n + 1), s_h=16.0)
    dev = gpu.level_k.device
    flushes = [(k.to(dev), v.to(dev), pos.to(dev)) for k, v, pos, _ in _flushes(batch, groups, dim, K, T, 3)]
    gpu.begin_op_log()
    for k, v, pos in flushes:
        gpu.route_and_flush_batch(k, v, pos, record_op_log=True)
    log, lengths = gpu.take_op_log()
    k, v, pos = flushes[0]

    def expect(what, log_, lengths_, pos_=pos):
        gpu.reset_parameters()
        before = _state(gpu)
        with pytest.raises(RuntimeError, match=what):
            gpu.route_and_flush_batch(k, v, pos_, replay_op_log=log_, replay_op_log_len=lengths_)
        assert not _same_state(gpu, before)
        assert gpu._op_replay_cursor_host == [[0] * groups for _ in range(batch)]

    expect("not in the current flush positions", log, lengths, pos + 1000)
    dup = pos.clone()
    dup[:, 1] = dup[:, 0]
    expect("duplicate token ids", log, lengths, dup)
    expect("fewer rows", log, torch.full_like(lengths, T - 1))
    bad = log.clone()
    bad[0, 0, 0, 0] = 3          # a Ward merge row
    expect("not a NEW_CLUSTER / JOIN", bad, lengths)
    bad = log.clone()
    bad[0, 0, 0, 0] = 2          # the opening NEW_CLUSTER turned into a JOIN of a dead cluster
    expect("dead one", bad, lengths)
    bad = log.clone()
    bad[0, 0, 1, 3] = bad[0, 0, 2, 3]   # one token named twice, another not at all
    expect("exactly once", bad, lengths)
    # The unchanged log still replays after the failures.
    gpu.reset_parameters()
    gpu.route_and_flush_batch(k, v, pos, replay_op_log=log, replay_op_log_len=lengths)
    assert gpu._op_replay_cursor_host == [[T] * groups for _ in range(batch)]


def test_op_log_overflow_and_alpha_replay_refused():
    batch, groups, dim, K, B, T, n, exact, span, beta = CASES["alpha_beta"]
    gpu, _ = make_pair(batch, groups, dim, K, B, recent=T, flush=T, max_seq=T * 4, s_h=16.0, exact=exact,
                       span=span, beta_novelty=beta, beta_adaptive=beta)
    dev = gpu.level_k.device
    (k, v, pos, ends), = _flushes(batch, groups, dim, K, T, 1, ends=True)
    gpu.begin_op_log()
    gpu.op_log = torch.zeros(batch, groups, 5, 4, dtype=torch.int32, device=dev)
    gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), span_ends=ends, record_op_log=True)
    with pytest.raises(RuntimeError, match="op_log overflow"):
        gpu.take_op_log()
    with pytest.raises(RuntimeError, match="requires semantic_replay_updates"):
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), span_ends=ends, replay_op_log=gpu.op_log,
                                  replay_op_log_len=gpu.op_log_len)
