"""Pins of the oracle's unified route (oracle/unified.py) without the device.

* known answers of the reducer, worked by hand from the reference's rules
  (litgpt/log_kv_cache.py:437-637, docs/semantic-unified-routing.md:11-60):
  Ward cost n_a n_b / (n_a + n_b) d^2 and the Lance-Williams update (three
  points on a line merge at 0.5 then at 60.17 = 2/3 * 9.5^2); the radius bound
  max(r_a + beta d, r_b + alpha d) stops the second merge under a limit of 0.6;
  the symmetric ``row ^ col`` tie rule pairs (0,1) and (2,3) of four equally
  spaced points in one round (a lowest-index rule would not); the budget takes
  the cheapest pairs first;
* the incremental rounds equal a full recompute (centers and distances rebuilt
  from scratch every round) on separated data, as the reference states
  (litgpt/log_kv_cache.py:449-455);
* frozen-center sweeps (``merge_passes > 1``, the budget stage): a round's
  pairs equal an independent peeling of the cost matrix (per pass each row's
  minimum under the ``row ^ col`` tie rule, mutual pairs taken, their rows
  and columns struck; the reference's own test oracle,
  tests/test_log_kv_unified.py:503-526) on its integer data, and the
  incremental rounds equal full-recompute peeling rounds in float64 on
  distinct random costs (tests/test_log_kv_unified.py:690-706);
* the full-recompute rounds of a capacity-capped route (``reduce_rounds``)
  equal the incremental rounds without a cap on separated data (the
  reference's own check, tests/test_log_kv_unified.py:560-580), and with a
  cap give hand-worked answers: the nearest pair over the cap leaves the
  second-cheapest pair to merge, the budget stage overflows the cap when no
  capped pair is left, the candidate stage stops there instead;
* labels and the Ward entry order on hand-built cases;
* route invariants: at most K live clusters, every row accounted for once,
  n_total equal to the ladder mass, each candidate's rows within the radius
  limit of its center; an old-old merge frees a cluster id that a new
  candidate then opens.
"""

import math

import numpy as np
import pytest

from workloads import Mixture
from oracle import OracleCache
from oracle import unified as U

ONES = lambda n: np.ones(n, np.float32)  # noqa: E731


def line(*x):
    return np.asarray(x, np.float32)[:, None]


def test_reducer_known_answers():
    s, t, mu = U.reduce(line(0, 1, 10), ONES(3), 3, None, 1)
    assert s.tolist() == [0] and t == [(0, 1), (0, 2)]
    assert np.allclose(mu[0], [11 / 3])
    s, t, _ = U.reduce(line(0, 1, 10), ONES(3), 3, 0.6, 1)
    assert s.tolist() == [0, 2] and t == [(0, 1)]
    s, t, _ = U.reduce(line(0, 1, 2, 3), ONES(4), 4, None, 1)
    assert t == [(0, 1), (2, 3), (0, 2)]
    s, t, _ = U.reduce(line(0, 1, 10, 10.5), ONES(4), 4, None, 2)
    assert s.tolist() == [0, 2] and t == [(2, 3), (0, 1)]
    s, t, _ = U.reduce(line(0, 1, 10, 10.5), ONES(4), 4, None, 3)
    assert s.tolist() == [0, 1, 2] and t == [(2, 3)]


def test_lance_williams_distance_is_the_merged_center_distance():
    r = U.Reducer(U.pair_distances(line(0, 1, 10)), line(0, 1, 10), ONES(3), 3, None, 1)
    r.step()
    assert r.dist[0, 2] == r.dist[2, 0] == np.float32(90.25)
    assert r.mass.tolist() == [2, 0, 1] and r.alive.tolist() == [True, False, True]
    cost = (r.packed[0] >> np.uint64(32)).astype(np.uint32).view(np.float32)
    assert cost == np.float32(np.float32(90.25) * (np.float32(2) / np.float32(3)))


class _FullRecompute(U.Reducer):
    """Every round rebuilds distances from the current centers and rescans every row."""

    def step(self):
        live = np.flatnonzero(self.alive)
        d = U.pair_distances(self.mu)
        self.dist[np.ix_(live, live)] = d[np.ix_(live, live)]
        self.packed[live] = self._scan(live)
        return super().step()


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("limit", [None, 6.0])
def test_incremental_rounds_equal_full_recompute(seed, limit):
    rng = np.random.default_rng(seed)
    centers = rng.standard_normal((6, 16)).astype(np.float32) * 8
    x = (centers[rng.integers(0, 6, 40)] + rng.standard_normal((40, 16)) * 0.7).astype(np.float32)
    mass = np.ones(40, np.float32)
    runs = []
    for cls in (U.Reducer, _FullRecompute):
        r = cls(U.pair_distances(x), x, mass, 40, limit, 4 if limit is None else 1)
        for _ in range(200):
            if not r.step():
                break
        runs.append((np.flatnonzero(r.alive).tolist(), r.trace))
    assert runs[0] == runs[1]
    assert len(runs[0][1]) > 10


def _peel_pairs(cost, passes):
    """Frozen-center matching restated from the reference test's peeling oracle: per pass every row's
    least cost (ties to the least row ^ col), the mutual pairs taken and their rows and columns
    struck; the pairs sorted by (cost, lower row)."""
    n = cost.shape[0]
    remaining = cost.copy()
    chosen = []
    for _ in range(passes):
        best = np.full(n, -1)
        for i in range(n):
            m = remaining[i].min()
            if np.isfinite(m):
                cands = np.flatnonzero(remaining[i] == m)
                best[i] = min(cands, key=lambda j: i ^ j)
        pairs = [(i, int(best[i])) for i in range(n) if best[i] > i and best[best[i]] == i]
        chosen.extend(pairs)
        for i, j in pairs:
            remaining[[i, j], :] = np.inf
            remaining[:, [i, j]] = np.inf
    return sorted(chosen, key=lambda p: (cost[p], p[0]))


def _ward_costs(mu, mass):
    d2 = ((mu[:, None, :] - mu[None, :, :]) ** 2).sum(-1)
    cost = d2 * (mass[:, None] * mass[None, :] / np.maximum(mass[:, None] + mass[None, :], 1))
    cost[~((mass > 0)[:, None] & (mass > 0)[None, :])] = np.inf
    np.fill_diagonal(cost, np.inf)
    return cost


def test_frozen_center_sweeps_match_peeling():
    rng = np.random.default_rng(98)
    mu = rng.integers(-4, 5, (3, 65, 8)).astype(np.float32)
    mu[0] = 0                                   # every cost 0: the tie rule alone pairs the rows
    mass = np.ones((3, 65), np.float32)
    mass[1, 51:] = 0                            # massless rows take no pair
    mass[2] = 0
    extra = 0
    for lane in range(3):
        cost = _ward_costs(mu[lane].astype(np.float64), mass[lane].astype(np.float64))
        want = _peel_pairs(cost, 4)
        r = U.Reducer(U.pair_distances(mu[lane]), mu[lane], mass[lane], 65, None, 1, passes=4)
        r.step()
        assert r.trace == want, f"lane {lane}"
        one = U.Reducer(U.pair_distances(mu[lane]), mu[lane], mass[lane], 65, None, 1)
        one.step()
        assert one.trace == _peel_pairs(cost, 1), f"lane {lane}, one pass"
        extra += len(r.trace) - len(one.trace)
        assert len({x for pair in r.trace for x in pair}) == 2 * len(r.trace)
    assert extra > 0, "the sweeps added no pair"


def _peel_reduce(x, w, target, passes):
    """Full-recompute rounds in float64: each round the Ward costs of the live clusters' centers,
    the peeled pairs budgeted by cost (count - target), merged in that order."""
    mu, mass = x.astype(np.float64).copy(), w.astype(np.float64).copy()
    trace = []
    for _ in range(4 * len(w)):
        count = int((mass > 0).sum())
        pairs = _peel_pairs(_ward_costs(mu, mass), passes)[:max(count - target, 0)]
        if not pairs:
            break
        for a, b in pairs:
            total = mass[a] + mass[b]
            mu[a] = (mass[a] * mu[a] + mass[b] * mu[b]) / max(total, 1)
            mass[a], mass[b] = total, 0
            trace.append((a, b))
    return np.flatnonzero(mass > 0).tolist(), trace


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_frozen_sweep_rounds_equal_full_recompute(seed):
    rng = np.random.default_rng(223 + seed)
    for i, n in enumerate((70, 33, 5, 90)):
        w = rng.integers(1, 4, n).astype(np.float32)
        x = (rng.standard_normal((n, 8)) * (i + 1)).astype(np.float32)
        surv, trace, _ = U.reduce(x, w, n, None, 4, passes=4)
        want_surv, want_trace = _peel_reduce(x, w, 4, 4)
        assert surv.tolist() == want_surv and trace == want_trace, f"n={n}"
        assert len(surv) == min(n, 4)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("limit", [None, 6.0])
def test_full_recompute_rounds_equal_incremental_without_cap(seed, limit):
    rng = np.random.default_rng(seed)
    centers = rng.standard_normal((6, 16)).astype(np.float32) * 8
    x = (centers[rng.integers(0, 6, 40)] + rng.standard_normal((40, 16)) * 0.7).astype(np.float32)
    mass = rng.integers(1, 4, 40).astype(np.float32)
    target = 4 if limit is None else 1
    s1, t1, m1 = U.reduce(x, mass, 40, limit, target)
    s2, t2, m2 = U.reduce_rounds(x, mass, 40, limit, target)
    assert s1.tolist() == s2.tolist() and t1 == t2 and len(t1) > 10
    assert np.allclose(m1[s1], m2[s2], rtol=1e-5, atol=1e-5)


def test_full_recompute_rounds_with_a_cap():
    # Masses 2, 2, 1 at 0, 1, 5, cap 3.5: the nearest pair (0, 1) (cost 1 * 4/4 = 1) would
    # hold mass 4, so row 0's least capped cost is row 2 (25 * 2/3) and rows 1 and 2 pick
    # each other (16 * 2/3): (1, 2) merges, center (2 * 1 + 1 * 5) / 3.
    x, w = line(0, 1, 5), np.asarray([2, 2, 1], np.float32)
    s, t, mu = U.reduce_rounds(x, w, 3, None, 2, cap=3.5)
    assert s.tolist() == [0, 1] and t == [(1, 2)]
    assert mu[1, 0] == np.float32(np.float32(2 + 5) / np.float32(3))
    s, t, _ = U.reduce_rounds(x, w, 3, None, 2)
    assert t == [(0, 1)]
    # 0, 1, 10, 11 with mass 1 and cap 2.5: both close pairs merge (mass 2 each); the last
    # pair would hold 4. The budget stage (strict) takes it anyway, the candidate stage stops.
    x, w = line(0, 1, 10, 11), ONES(4)
    s, t, _ = U.reduce_rounds(x, w, 4, None, 1, cap=2.5, strict=True)
    assert s.tolist() == [0] and t == [(0, 1), (2, 3), (0, 2)]
    s, t, _ = U.reduce_rounds(x, w, 4, 100.0, 1, cap=2.5)
    assert s.tolist() == [0, 2] and t == [(0, 1), (2, 3)]


def test_labels_and_ward_entry_order():
    assert U.labels(5, [0, 4], [(0, 1), (2, 3), (0, 2)]).tolist() == [0, 0, 0, 0, 1]
    # keep entries: order 0..2 at p_lo 5, 7, 9; free: order 0..1 at p_lo 6, 8
    assert U.ward_entry_order([0, 1, 2, 0, 1], [5, 7, 9, 6, 8], [1, 1, 1, 1, 1], 3) == [0, 3, 1, 4, 2]
    # a massless keep entry takes the p_lo of the next massive entry (9)
    assert U.ward_entry_order([0, 1, 2, 0, 1], [5, 7, 9, 6, 8], [1, 0, 1, 1, 1], 3) == [0, 3, 4, 1, 2]
    # stored out of order: each side is sorted by order first
    assert U.ward_entry_order([2, 0, 1, 0], [9, 5, 7, 6], [1, 1, 1, 1], 3) == [1, 3, 2, 0]


def _stream(cache, batch, groups, dim, T, n, exact, seed=3):
    mix = Mixture(batch, groups, dim, clusters=6, seed=seed, drift_every=3 * T)
    total = 0
    for i in range(n):
        k, v = mix.rows(T).float().numpy(), mix.rows(T).float().numpy()
        pos = np.broadcast_to(np.arange(i * T, (i + 1) * T), (batch, T)).copy()
        ends = [[(p + 3 * b) % 5 == 0 for p in range(i * T, (i + 1) * T)] for b in range(batch)] if exact else None
        cache.flush_rows(k, v, pos, ends)
        total += T
        yield total


@pytest.mark.parametrize("exact", [0, 8])
def test_route_invariants(exact):
    batch, groups, dim, T, K = 2, 2, 16, 24, 4
    c = OracleCache(batch, groups, 4096, dim, dim, B=8, recent_size=T, K=K, s_h=4.0, flush=T, exact_tokens=exact,
                    span_max=4, unified=True)
    for total in _stream(c, batch, groups, dim, T, 8, exact):
        assert (c.alive.sum(-1) <= K).all()
        mass = c.level_w.sum((2, 3, 4)) + (c.alpha_valid.sum(-1)[:, None] if exact else 0)
        assert (mass == total).all()
        assert (c.level_w.sum((-1, -2)) == c.n_total).all()
        assert ((c.level_w.sum((-1, -2)) > 0) == c.alive).all()


def test_candidates_respect_the_radius():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 8))[rng.integers(0, 3, 60)] * 6 + rng.standard_normal((60, 8))).astype(np.float32)
    limit = np.float32(math.sqrt(4.0))
    surv, trace, mu = U.reduce(x, ONES(60), 60, limit, 1)
    lab = U.labels(60, surv, trace)
    assert len(trace) > 20
    for r, root in enumerate(surv):
        members = x[lab == r]
        far = np.sqrt(((members - mu[root]) ** 2).sum(-1)).max()
        assert far <= limit * (1 + 1e-5)


def test_old_old_merge_frees_a_cluster_for_a_new_candidate():
    dim = 8
    c = OracleCache(1, 1, 256, dim, dim, B=4, recent_size=4, K=2, s_h=1.0, flush=4, unified=True)
    e = np.eye(dim, dtype=np.float32)
    c.new_cluster(0, 0, 0, e[0] * 1, e[0], 10)
    c.join(0, 0, 0, np.stack([e[0] * 1.1]), np.stack([e[0]]), np.asarray([11]))
    c.new_cluster(0, 0, 1, e[0] * 2, e[1], 12)
    rows = np.stack([e[2] * 50, e[2] * 50.2, e[2] * 50.1, e[2] * 49.9])[None, None]
    out = c.flush_rows(rows, rows, np.arange(20, 24)[None])
    # the two old clusters (1.05 e0 and 2 e0) are the cheapest pair: 1 merges into 0
    assert c.n_total[0, 0].tolist() == [3, 4]
    assert c.p_hi_c[0, 0].tolist() == [12, 23]
    assert out[0, 0].tolist() == [1, 1, 1, 1]
    w = c.level_w[0, 0, 0].reshape(-1)
    assert sorted(c.level_p_lo[0, 0, 0].reshape(-1)[w > 0].tolist()) == [10, 11, 12]
