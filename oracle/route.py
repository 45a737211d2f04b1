"""Attach routing of one flush: frozen-center joins, farthest-point seeds, orphan joins.

TEST INFRASTRUCTURE ONLY (the oracle). Restates, per (batch row, KV group) lane:

* position order of the flushed rows, padding last
  (litgpt/log_kv_cache.py:4599-4606);
* frozen joins: ``semantic = max(|x|^2 + |mu|^2 - 2 x.mu, 0)``, temporal cost
  ``eta * gap / (gap + g0)`` with ``gap = max(pos - p_hi, 0)``, dead clusters at
  +inf, argmin with the lowest index on ties, ``direct = any alive and
  semantic(winner) <= lam * s_h`` (litgpt/log_kv_cache.py:2649-2681,
  litgpt/log_kv_route_triton.py:876-889);
* orphans with free cluster slots: first seed is the orphan farthest (by its
  winner's semantic distance) from the live clusters, later seeds are
  farthest-point picks over exact squared differences with earlier picks
  masked; seeds open the free slots in ascending id; every orphan joins the
  nearest live-or-seed cluster by exact squared differences and each seed is
  forced into its own slot (litgpt/log_kv_cache.py:4636-4680);
* orphans without free slots join the nearest live cluster by exact squared
  differences (litgpt/log_kv_route_triton.py:887-889);
* with a capacity cap (``cap`` finite, litgpt/log_kv_cache.py:2347-2354) the
  capped planner instead (:2677-2680, :4497-4516, :4734-4822): a frozen join
  needs ``float32(n_total[winner] + 1) <= float32(cap)``; each cluster keeps its
  first ``max(0, int(cap) - n_total)`` direct rows in offset order and the
  rest become orphans; seeds as above; every other orphan, in position order,
  takes the nearest candidate (ascending distance, then cluster id) whose
  room ``max(0, int(cap) - n_total - taken)`` is still positive, ``taken``
  being its kept direct rows or 1 for a seeded slot, each pick using one unit
  of room; with no room anywhere, the nearest candidate.

Deliberate restatement choices: feature sums use ``numerics.dsum`` (the
reference's GEMM/cdist orders are unspecified); the seeded orphan join compares
squared distances where the reference's ``torch.cdist`` compares their square
roots - the argmin differs only when two squared distances round to the same
square root, which the margin checks in the tests exclude.
"""

from __future__ import annotations

import numpy as np

from .numerics import argmax_first, argmin_first, dsum, f32

I64_MAX = np.iinfo(np.int64).max


def position_order(pos: np.ndarray, counts: np.ndarray) -> np.ndarray:
    """Stable position order per batch row; rows at or past ``counts[b]`` sort last."""
    n_batch, tokens = pos.shape
    valid = np.arange(tokens)[None, :] < np.asarray(counts)[:, None]
    keyed = np.where(valid, pos, I64_MAX)
    return np.argsort(keyed, axis=1, kind="stable")


def lane_decisions(x, pos, mu, alive, p_hi, s_h, eta, g0, lam):
    """Frozen-join quantities for one lane's rows (already in position order).

    Returns (winner, s_winner, direct, exact) where ``exact[t, c]`` is the
    squared difference distance used for orphan joins.
    """
    x = f32(x)
    mu = f32(mu)
    xx = dsum(x * x)                                   # [n]
    mm = dsum(mu * mu)                                 # [K]
    dot = dsum(x[:, None, :] * mu[None, :, :])         # [n, K]
    semantic = np.maximum((xx[:, None] + mm[None, :]) - f32(2.0) * dot, f32(0.0))
    gap = np.maximum(np.asarray(pos, dtype=np.int64)[:, None] - np.asarray(p_hi, dtype=np.int64)[None, :], 0)
    gap = gap.astype(np.float32)
    cost = semantic + f32(eta) * (gap / (gap + f32(g0)))
    cost = np.where(np.asarray(alive, dtype=bool)[None, :], cost, np.float32(np.inf))
    winner = argmin_first(cost, axis=1)
    s_winner = semantic[np.arange(len(winner)), winner]
    direct = bool(np.any(alive)) & (s_winner <= f32(lam) * f32(s_h))
    diff = x[:, None, :] - mu[None, :, :]
    exact = dsum(diff * diff)
    return winner, s_winner, direct, exact


def lane_assign(x, pos, mu, alive, p_hi, s_h, eta, g0, lam, n_total=None, cap=np.inf, offsets=None):
    """Final cluster of each row of one lane (rows in position order; ``offsets``
    are their flush offsets, which order a capped cluster's kept direct rows)."""
    alive = np.asarray(alive, dtype=bool)
    k = len(alive)
    winner, s_winner, direct, exact = lane_decisions(x, pos, mu, alive, p_hi, s_h, eta, g0, lam)
    capped = bool(np.isfinite(cap))
    if capped:
        n_total = np.asarray(n_total, dtype=np.int64)
        direct = direct & ((n_total[winner].astype(np.float32) + f32(1.0)) <= f32(cap))
        cap_rows = int(cap)
        kept = np.zeros(k, dtype=np.int64)
        for i in np.argsort(np.asarray(offsets), kind="stable"):
            if direct[i]:
                c = int(winner[i])
                if kept[c] < max(0, cap_rows - int(n_total[c])):
                    kept[c] += 1
                else:
                    direct[i] = False
    orphan = ~direct
    free = [c for c in range(k) if not alive[c]]
    n_use = min(len(free), int(orphan.sum()))
    if n_use == 0 and not capped:
        nearest = argmin_first(np.where(alive[None, :], exact, np.float32(np.inf)), axis=1)
        return np.where(direct, winner, nearest).astype(np.int64)
    if n_use == 0:
        picks = []
        return _capped_orphans(x, mu, alive, winner, direct, picks, free, n_total, cap_rows, kept)
    x = f32(x)

    def distance_to(t):
        diff = x - x[t][None, :]
        return dsum(diff * diff)

    nxt = int(argmax_first(np.where(orphan, s_winner, np.float32(-np.inf))))
    picks = [nxt]
    dist = np.where(orphan, distance_to(nxt), np.float32(-np.inf))
    for _ in range(n_use - 1):
        dist[nxt] = np.float32(-np.inf)
        nxt = int(argmax_first(dist))
        picks.append(nxt)
        dist = np.minimum(dist, distance_to(nxt))
    if capped:
        return _capped_orphans(x, mu, alive, winner, direct, picks, free, n_total, cap_rows, kept)
    d_or = _candidate_distances(x, mu, alive, picks, free)
    assign = np.where(direct, winner, argmin_first(d_or, axis=1)).astype(np.int64)
    for i, t in enumerate(picks):
        assign[t] = free[i]
    return assign


def _candidate_distances(x, mu, alive, picks, free):
    """Exact squared distances of every row to the live centers and the seed
    rows at their free slots (+inf for other slots)."""
    x = f32(x)
    mu_ext = f32(mu).copy()
    candidates = np.asarray(alive, dtype=bool).copy()
    for i, t in enumerate(picks):
        mu_ext[free[i]] = x[t]
        candidates[free[i]] = True
    diff = x[:, None, :] - mu_ext[None, :, :]
    return np.where(candidates[None, :], dsum(diff * diff), np.float32(np.inf))


def _capped_orphans(x, mu, alive, winner, direct, picks, free, n_total, cap_rows, kept):
    """Capped orphan placement (litgpt/log_kv_cache.py:4802-4822): rooms of the
    candidates, then each non-seed orphan in position order takes the nearest
    candidate with room left, else the nearest candidate."""
    d_or = _candidate_distances(x, mu, alive, picks, free)
    assign = np.where(direct, winner, -1).astype(np.int64)
    seeded = {free[i]: t for i, t in enumerate(picks)}
    for c, t in seeded.items():
        assign[t] = c
    room = {}
    for c in range(len(alive)):
        if alive[c] or c in seeded:
            room[c] = max(0, cap_rows - int(n_total[c]) - (1 if c in seeded else int(kept[c])))
    for i in np.flatnonzero(assign < 0):
        order = np.argsort(d_or[i], kind="stable").tolist()
        c = next((c for c in order if room.get(c, 0) > 0), order[0])
        room[c] = room.get(c, 0) - 1
        assign[i] = c
    return assign


def attach_assign(x, pos, counts, centroid, alive, p_hi, s_h, eta, g0, lam, n_total=None, cap=np.inf):
    """int8 cluster per row in position order ``[Bt, G, T]`` (-1 past ``counts``) and the order."""
    x = f32(x)
    n_batch, n_groups, tokens, _ = x.shape
    counts = np.asarray(counts, dtype=np.int64)
    order = position_order(np.asarray(pos, dtype=np.int64), counts)
    out = np.full((n_batch, n_groups, tokens), -1, dtype=np.int8)
    for b in range(n_batch):
        n = int(counts[b])
        if n == 0:
            continue
        rows = order[b, :n]
        for g in range(n_groups):
            out[b, g, :n] = lane_assign(
                x[b, g, rows], pos[b, rows], centroid[b, g], alive[b, g], p_hi[b, g], s_h[b, g], eta, g0, lam,
                None if n_total is None else n_total[b, g], cap, rows)
    return out, order


def commit_jobs(assign, order, counts, alive):
    """Group one flush's decisions by (lane, cluster) in position order.

    Returns ``{(b, g, c): (new, rows)}`` where ``rows`` are flush offsets in
    position order and ``new`` says the cluster was dead, so ``rows[0]`` opens
    it (litgpt/log_kv_cache.py:4682-4707).
    """
    n_batch, n_groups, _ = assign.shape
    jobs = {}
    for b in range(n_batch):
        n = int(counts[b])
        rows = order[b, :n]
        for g in range(n_groups):
            lane = assign[b, g, :n].astype(np.int64)
            for c in np.unique(lane):
                sel = rows[lane == c]
                jobs[(b, g, int(c))] = (not bool(alive[b, g, c]), sel)
    return jobs
