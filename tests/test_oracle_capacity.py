"""Pins of the oracle's capacity-capped attach planner (oracle/route.py) without the device.

* the reference's own known answers (tests/test_log_kv_cache.py:1996-2014 and
  :3630-3655): a full winner pushes a token into a new cluster; orphans fill
  the nearest cluster up to its room first (direct rows counted), identical
  seeds open both free slots, and only when every cluster is full does a
  cluster exceed the cap;
* a hand-derived case: a cluster's direct rows are kept in flush-offset order,
  not position order;
* a cap too large to bind gives exactly the uncapped decisions, on random
  lanes with and without free slots;
* on random lanes with a binding cap: a cluster ends past the cap only when
  every candidate ends at or past it, the clusters opened are the lowest free
  slots, and every valid row gets a cluster.
"""

import numpy as np
import pytest

from oracle import OracleCache, oplog
from oracle import route


def _cache(**kw):
    args = dict(B=3, recent_size=8, K=2, lam=0.01, s_h=1.0, flush=8, hard_cap_mult=0.5)
    args.update(kw)
    max_seq = args.pop("max_seq", 16)
    return OracleCache(1, 1, max_seq, 8, 8, **args)


def test_full_winner_opens_a_new_cluster():
    # tests/test_log_kv_cache.py:1996-2014: cap = 8 / 2 * 1.0 = 4 and the winner holds 4.
    c = _cache(max_seq=8, lam=10.0, B=4, recent_size=2, flush=2, hard_cap_mult=1.0)
    assert c.hard_cap == 4.0
    c.alive[0, 0, 0] = True
    c.centroid[0, 0, 0] = 0.0
    c.n_eff[0, 0, 0] = 4.0
    c.n_total[0, 0, 0] = 4
    c.p_hi_c[0, 0, 0] = 3
    rng = np.random.default_rng(0)
    c.route_and_commit(np.zeros((1, 1, 1, 8), np.float32), rng.standard_normal((1, 1, 1, 8)).astype(np.float32),
                       np.asarray([[4]]), np.asarray([1]))
    assert int(c.n_total[0, 0, 0]) == 4
    assert bool(c.alive[0, 0, 1]) and int(c.n_total[0, 0, 1]) == 1


@pytest.mark.parametrize("case", ["orphans", "direct_and_orphans", "identical_seeds", "overflow"])
def test_orphans_reserve_capacity_before_commit(case):
    # tests/test_log_kv_cache.py:3630-3655: cap = 16 / 2 * 0.5 = 4.
    c = _cache()
    c.begin_op_log()
    initial = 0 if case == "identical_seeds" else 2
    for cl in range(initial):
        key = np.zeros(8, np.float32)
        key[0] = (0.0, 100.0)[cl]
        c.new_cluster(0, 0, cl, key, key, cl)
    n = 8 if case == "overflow" else 6 if case == "identical_seeds" else 4
    keys = np.zeros((1, 1, n, 8), np.float32)
    keys[..., 0] = 10.0
    if case == "direct_and_orphans":
        keys[0, 0, 1, 0] = 0.0
    c.route_and_commit(keys, keys, np.arange(2, n + 2)[None], np.asarray([n]))
    counts = c.n_total[0, 0].tolist()
    assert sum(counts) == initial + n
    assert c.level_w.sum() == initial + n
    if case == "overflow":
        assert min(counts) >= 4
        assert counts == [6, 4]        # 3 + 3 while room lasts, then both to the nearest
    else:
        assert counts == [4, 2]
    assert all(op != oplog.WARD_MERGE for op, *_ in c.op_log[0][0])


def test_direct_rows_keep_offset_order():
    """Hand-derived from litgpt/log_kv_cache.py:4497-4516: a cluster's direct rows
    are bucketed by flush offset (a stable sort of the decisions), so with room
    for one row the lower offset stays even when its position is later; the
    other becomes the orphan that opens the free slot."""
    x = np.zeros((2, 8), np.float32)           # rows in position order: position 5 (offset 1), 9 (offset 0)
    mu = np.zeros((2, 8), np.float32)
    alive = np.asarray([True, False])
    assign = route.lane_assign(x, np.asarray([5, 9]), mu, alive, np.asarray([3, -1]), 1.0, 1.0, 64.0, 10.0,
                               np.asarray([3, 0]), 4.0, np.asarray([1, 0]))
    assert assign.tolist() == [1, 0]
    # Uncapped, both join the live cluster.
    assert route.lane_assign(x, np.asarray([5, 9]), mu, alive, np.asarray([3, -1]), 1.0, 1.0, 64.0,
                             10.0).tolist() == [0, 0]


def _lane(rng, n, k, dim, n_alive, spread=3.0):
    x = (rng.standard_normal((n, dim)) * spread).astype(np.float32)
    mu = (rng.standard_normal((k, dim)) * spread).astype(np.float32)
    alive = np.zeros(k, bool)
    alive[rng.choice(k, n_alive, replace=False)] = True
    mu[~alive] = 0.0
    pos = np.sort(rng.choice(10 * n, n, replace=False)).astype(np.int64) + 100
    p_hi = rng.integers(0, 100, k).astype(np.int64)
    n_total = np.where(alive, rng.integers(1, 6, k), 0).astype(np.int64)
    offsets = rng.permutation(n)
    return x, pos, mu, alive, p_hi, n_total, offsets


@pytest.mark.parametrize("n_alive", [0, 2, 4, 6])
@pytest.mark.parametrize("seed", range(4))
def test_unbinding_cap_equals_uncapped(n_alive, seed):
    rng = np.random.default_rng(seed)
    x, pos, mu, alive, p_hi, n_total, offsets = _lane(rng, 40, 6, 16, n_alive)
    lam = 2.0 * 16 * 9 * rng.uniform(0.2, 2.0)
    want = route.lane_assign(x, pos, mu, alive, p_hi, 1.0, 1.0, 64.0, lam)
    got = route.lane_assign(x, pos, mu, alive, p_hi, 1.0, 1.0, 64.0, lam, n_total, 1e6, offsets)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n_alive", [0, 3, 6])
@pytest.mark.parametrize("cap", [1.0, 3.5, 8.0, 12.0])
@pytest.mark.parametrize("seed", range(3))
def test_binding_cap_invariants(n_alive, cap, seed):
    rng = np.random.default_rng(100 + seed)
    k = 6
    x, pos, mu, alive, p_hi, n_total, offsets = _lane(rng, 40, k, 16, n_alive)
    lam = 2.0 * 16 * 9 * 0.5
    assign = route.lane_assign(x, pos, mu, alive, p_hi, 1.0, 1.0, 64.0, lam, n_total, cap, offsets)
    assert assign.min() >= 0 and assign.max() < k
    # The clusters opened are the lowest free slots, at most one per orphan.
    free = np.flatnonzero(~alive).tolist()
    opened = sorted(set(free) & set(assign.tolist()))
    assert opened == free[:len(opened)]
    after = n_total + np.bincount(assign, minlength=k)
    over = [c for c in range(k) if after[c] > max(int(cap), n_total[c]) and (alive[c] or c in opened)]
    if over:
        # Someone exceeded the cap: then every candidate is at or past it.
        cands = [c for c in range(k) if alive[c] or c in opened]
        assert all(after[c] >= int(cap) for c in cands), (after.tolist(), cap)
