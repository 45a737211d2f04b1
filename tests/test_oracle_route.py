"""Pins of the oracle's attach routing (oracle/route.py) without the device.

* frozen joins against a float64 brute force of the reference's rule
  (litgpt/log_kv_cache.py:2649-2681): winner = argmin over live clusters of
  semantic distance + eta * gap / (gap + g0), direct when the winner's semantic
  distance is within lam * s_h; rows whose decision margin is below float32
  noise are skipped;
* orphan seeding (litgpt/log_kv_cache.py:4636-4680): the first seed is the
  orphan farthest from the live clusters, later seeds are farthest-point picks,
  free slots open in ascending id and each seed lands in its own slot; every
  orphan joins its nearest live-or-seed cluster (float64 brute force);
* invariants: every valid row gets one cluster in [0, K), padding rows -1, and
  the order is the stable position order.
"""

import numpy as np
import pytest

from oracle import route


def lanes(rng, n, K, D, alive_frac=1.0):
    centers = (rng.standard_normal((K, D)) * 4).astype(np.float32)
    label = rng.integers(0, K, n)
    x = centers[label] + rng.standard_normal((n, D)).astype(np.float32) * 0.5
    far = rng.random(n) < 0.1
    x[far] = rng.standard_normal((far.sum(), D)).astype(np.float32) * 12
    alive = rng.random(K) < alive_frac
    return x.astype(np.float32), centers, alive


def brute_force_frozen(x, pos, mu, alive, p_hi, s_h, eta, g0, lam):
    x64, mu64 = x.astype(np.float64), mu.astype(np.float64)
    sem = ((x64[:, None, :] - mu64[None]) ** 2).sum(-1)
    gap = np.maximum(pos[:, None] - p_hi[None, :], 0).astype(np.float64)
    cost = np.where(alive[None, :], sem + eta * gap / (gap + g0), np.inf)
    winner = cost.argmin(1)
    srt = np.sort(cost, axis=1)
    margin = srt[:, 1] - srt[:, 0] if cost.shape[1] > 1 else np.full(len(x), np.inf)
    s_win = sem[np.arange(len(x)), winner]
    return winner, s_win, margin, sem


@pytest.mark.parametrize("seed", range(4))
def test_frozen_joins_match_float64(seed):
    rng = np.random.default_rng(seed)
    n, K, D = 300, 12, 64
    x, mu, _ = lanes(rng, n, K, D)
    alive = np.ones(K, bool)
    alive[rng.integers(0, K)] = False
    pos = np.arange(1000, 1000 + n, dtype=np.int64)
    p_hi = rng.integers(0, 1200, K).astype(np.int64)
    s_h, eta, g0, lam = 64.0, 1.0, 2048.0, 1.0
    winner, s_win, direct, _ = route.lane_decisions(x, pos, mu, alive, p_hi, s_h, eta, g0, lam)
    w64, s64, margin, _ = brute_force_frozen(x, pos, mu, alive, p_hi, s_h, eta, g0, lam)
    clear = margin > 1e-3 * np.maximum(1.0, s64)
    assert clear.mean() > 0.9
    np.testing.assert_array_equal(winner[clear], w64[clear])
    far_from_radius = np.abs(s64 - lam * s_h) > 1e-3 * lam * s_h
    np.testing.assert_array_equal(direct[clear & far_from_radius], (s64 <= lam * s_h)[clear & far_from_radius])
    assert (~direct).sum() > 0 and direct.sum() > 0


def test_orphans_seed_free_slots_in_order():
    rng = np.random.default_rng(7)
    n, K, D = 200, 6, 32
    x, mu, _ = lanes(rng, n, K, D)
    alive = np.asarray([True, False, True, False, False, True])
    pos = np.arange(n, dtype=np.int64)
    p_hi = np.zeros(K, np.int64)
    s_h = 64.0
    assign = route.lane_assign(x, pos, mu, alive, p_hi, s_h, 1.0, 2048.0, 1.0)
    _, s64, _, sem = brute_force_frozen(x, pos, mu, alive, p_hi, s_h, 1.0, 2048.0, 1.0)
    orphan = ~(s64 <= s_h)
    free = [1, 3, 4]
    # first seed: the orphan farthest (winner's semantic distance) from the live clusters
    first = int(np.argmax(np.where(orphan, s64, -np.inf)))
    assert assign[first] == free[0]
    # farthest-point picks, float64
    x64 = x.astype(np.float64)
    picks = [first]
    dist = np.where(orphan, ((x64 - x64[first]) ** 2).sum(1), -np.inf)
    for _ in range(len(free) - 1):
        dist[picks[-1]] = -np.inf
        nxt = int(np.argmax(dist))
        picks.append(nxt)
        dist = np.minimum(dist, ((x64 - x64[nxt]) ** 2).sum(1))
    for slot, t in zip(free, picks):
        assert assign[t] == slot
    cand = mu.astype(np.float64).copy()
    for slot, t in zip(free, picks):
        cand[slot] = x64[t]
    d = ((x64[:, None, :] - cand[None]) ** 2).sum(-1)
    srt = np.sort(d, 1)
    clear = srt[:, 1] - srt[:, 0] > 1e-3 * srt[:, 0]
    rest = orphan & clear & ~np.isin(np.arange(n), picks)
    np.testing.assert_array_equal(assign[rest], d.argmin(1)[rest])
    assert set(assign.tolist()) <= set(range(K))


def test_attach_assign_invariants_and_order():
    rng = np.random.default_rng(3)
    Bt, G, T, K, D = 2, 3, 50, 5, 16
    x = rng.standard_normal((Bt, G, T, D)).astype(np.float32) * 4
    pos = np.stack([rng.permutation(T) + 100, rng.permutation(T)]).astype(np.int64)
    counts = np.asarray([T, 37])
    centroid = rng.standard_normal((Bt, G, K, D)).astype(np.float32) * 4
    alive = rng.random((Bt, G, K)) < 0.6
    p_hi = np.zeros((Bt, G, K), np.int64)
    s_h = np.full((Bt, G), 64.0, np.float32)
    out, order = route.attach_assign(x, pos, counts, centroid, alive, p_hi, s_h, 1.0, 2048.0, 1.0)
    for b in range(Bt):
        n = counts[b]
        assert np.array_equal(pos[b, order[b, :n]], np.sort(pos[b, :n]))
        assert (out[b, :, :n] >= 0).all() and (out[b, :, :n] < K).all()
        assert (out[b, :, n:] == -1).all()
