"""The capacity-capped attach planner on the device against the oracle
(litgpt/log_kv_cache.py:2347-2354, :2677-2680, :4497-4516, :4734-4822).

* the reference's known-answer flushes (tests/test_log_kv_cache.py:1996-2014,
  :3630-3655) through the device: the oracle's state bit for bit, and the
  reference's cluster counts (the initial clusters come from a first flush,
  whose farthest-point seeding numbers them the other way round);
* streams whose cap binds (mixtures drifting past it, with and without Alpha's
  ragged archives, a cap under one row), every flush bit-exact;
* the op-log of a capped stream equals the oracle's and replays into every
  recorded state.
"""

import numpy as np
import pytest
import torch

from harness import compare_state, feed, make_pair, to_np
from oracle import oplog as ora_oplog
from workloads import Mixture

pytestmark = pytest.mark.gpu


def _flush(gpu, ora, keys, positions):
    dev = gpu.level_k.device
    k = torch.from_numpy(keys).to(torch.bfloat16)
    pos = torch.as_tensor(positions, dtype=torch.int64)[None]
    gpu.route_and_flush_batch(k.to(dev), k.to(dev), pos.to(dev))
    ora.flush_rows(k.float().numpy(), k.float().numpy(), pos.numpy())
    bad = compare_state(gpu, ora)
    assert not bad, "; ".join(bad)


def test_full_winner_opens_a_new_cluster():
    # cap = 16 / 2 * 0.5 = 4; four rows at key 0 fill cluster 0 (n_total 4 after
    # a first flush that opens it and a second that joins three), then a fifth
    # row at key 0 cannot join and opens cluster 1.
    print("case full winner", flush=True)
    gpu, ora = make_pair(batch=1, groups=1, dim=8, K=2, B=3, recent=8, flush=8, max_seq=16, s_h=1.0,
                         hard_cap_mult=0.5)
    _flush(gpu, ora, np.zeros((1, 1, 1, 8), np.float32), [0])
    _flush(gpu, ora, np.zeros((1, 1, 3, 8), np.float32), [1, 2, 3])
    assert to_np(gpu.n_total)[0, 0].tolist() == [4, 0]
    _flush(gpu, ora, np.zeros((1, 1, 1, 8), np.float32), [4])
    assert to_np(gpu.n_total)[0, 0].tolist() == [4, 1] and bool(gpu.alive[0, 0, 1])


@pytest.mark.parametrize("case", ["orphans", "direct_and_orphans", "identical_seeds", "overflow"])
def test_reference_capacity_cases(case):
    print(f"case {case}", flush=True)
    gpu, ora = make_pair(batch=1, groups=1, dim=8, K=2, B=3, recent=8, flush=8, max_seq=16, s_h=1.0,
                         hard_cap_mult=0.5, lam=0.01)
    initial = 0 if case == "identical_seeds" else 2
    if initial:
        first = np.zeros((1, 1, 2, 8), np.float32)
        first[0, 0, 0, 0] = 100.0          # the farthest row seeds cluster 0
        _flush(gpu, ora, first, [0, 1])
    n = 8 if case == "overflow" else 6 if case == "identical_seeds" else 4
    keys = np.zeros((1, 1, n, 8), np.float32)
    keys[..., 0] = 10.0
    if case == "direct_and_orphans":
        keys[0, 0, 1, 0] = 0.0
    _flush(gpu, ora, keys, list(range(2, n + 2)))
    counts = to_np(gpu.n_total)[0, 0].astype(int).tolist()
    assert sum(counts) == initial + n
    assert float(gpu.level_w.float().sum()) == initial + n
    if case == "overflow":
        assert counts == [4, 6]
    elif case == "identical_seeds":
        assert counts == [4, 2]
    else:
        assert counts == [2, 4]


STREAMS = {
    # name: (batch, groups, dim, K, B, flush, max_seq, s_h, cap_mult, exact, tokens)
    "binding": (2, 2, 64, 6, 16, 32, 512, 64.0, 0.5, 0, 480),
    "tight": (1, 2, 32, 4, 8, 24, 384, 16.0, 0.25, 0, 360),
    "under_one_row": (1, 2, 32, 4, 8, 24, 256, 16.0, 0.005, 0, 240),
    "alpha_ragged": (2, 2, 64, 6, 16, 32, 512, 64.0, 0.5, 24, 480),
    "qwen_layer": (1, 2, 128, 12, 32, 256, 4096, 64.0, 1.0, 0, 4096),
}


@pytest.mark.parametrize("name", list(STREAMS))
def test_capped_stream_matches_oracle(name):
    batch, groups, dim, K, B, flush, max_seq, s_h, mult, exact, tokens = STREAMS[name]
    print(f"case {name}", flush=True)
    gpu, ora = make_pair(batch=batch, groups=groups, dim=dim, K=K, B=B, recent=flush, flush=flush, max_seq=max_seq,
                         s_h=s_h, exact=exact, span=8, beta_novelty=bool(exact), beta_adaptive=bool(exact),
                         hard_cap_mult=mult)
    assert gpu._params.hard_cap > 0
    mix = Mixture(batch, groups, dim, clusters=K + 3, seed=29, drift_every=4 * flush)
    cap_rows = int(gpu._semantic_hard_cap())
    for start in range(0, tokens, flush):
        feed(gpu, ora, mix, start, flush, with_ends=bool(exact))
        bad = compare_state(gpu, ora)
        assert not bad, f"flush at {start}: " + "; ".join(bad)
    # The cap binds: some cluster reached it.
    assert int(to_np(gpu.n_total).max()) >= max(cap_rows, 1)


def test_capped_op_log_matches_oracle_and_replays():
    batch, groups, dim, K, B, flush, max_seq, s_h, mult = 2, 2, 32, 4, 8, 24, 384, 16.0, 0.25
    print("case capped op-log", flush=True)
    gpu, ora = make_pair(batch=batch, groups=groups, dim=dim, K=K, B=B, recent=flush, flush=flush, max_seq=max_seq,
                         s_h=s_h, hard_cap_mult=mult)
    gpu.begin_op_log()
    ora.begin_op_log()
    mix = Mixture(batch, groups, dim, clusters=K + 3, seed=31, drift_every=4 * flush)
    dev = gpu.level_k.device
    flushes, states = [], []
    for i in range(12):
        k, v = mix.rows(flush), mix.rows(flush)
        pos = torch.arange(i * flush, (i + 1) * flush).unsqueeze(0).expand(batch, -1).contiguous()
        flushes.append((k.to(dev), v.to(dev), pos.to(dev)))
        gpu.route_and_flush_batch(*flushes[-1], record_op_log=True)
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy())
        states.append({name: t.clone() for name, t in gpu.named_buffers()})
    log, lengths = gpu.take_op_log()
    want, want_len = ora_oplog.to_array(ora.op_log, capacity=log.size(2))
    assert np.array_equal(to_np(lengths), want_len) and np.array_equal(to_np(log), want)
    gpu.reset_parameters()
    for i, ((k, v, pos), want_state) in enumerate(zip(flushes, states)):
        gpu.route_and_flush_batch(k, v, pos, replay_op_log=log, replay_op_log_len=lengths)
        torch.cuda.synchronize()
        bad = [name for name, t in gpu.named_buffers() if not torch.equal(t, want_state[name])]
        assert not bad, f"flush {i}: {bad}"
