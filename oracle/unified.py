"""CPU restatement of the unified (Ward / radius) route.

TEST INFRASTRUCTURE ONLY (the oracle): used by ``tests/`` and never by the
product package.

Follows litgpt/log_kv_cache.py:3589-3688 (the route), :448-637 (the
incremental reducer ``_UnifiedReduceTorch``, restated per lane),
:3544-3568 (labels), :2517-2580 and :2395-2447 (Ward merge of old clusters
and its entry order), docs/semantic-unified-routing.md:11-96.

Two stages per lane (batch row, KV group):
1. candidates: the flushed rows start as singletons (mass 1, radius 0) and
   mutual-nearest Ward pairs merge while the radius bound
   ``max(r_a + beta d, r_b + alpha d) <= sqrt(lambda s_h)`` holds;
2. global budget: old live clusters (mass n_total) and the candidates compete
   until at most K remain, the ``count - K`` cheapest mutual pairs per round.
Old-old merges re-append both ladders into the lower cluster id; new roots
open the free cluster ids in ascending order; the rows are then committed as
attach-routed rows are.

Float order. Every element operation is one IEEE float32 operation in the
reference's order (``_unified_pair_cost``, ``_merge``). Where the reference
leaves an order to a library, one order is fixed here and on the device:
initial squared distances are canonical feature sums (``numerics.dsum``) of
squared differences, ``sum((x_i - x_j)^2)`` (the reference's small-matrix
``cdist`` form; it uses a centred Gram GEMM above 32 nodes), and the exact
radius check's squared distance likewise.
"""

from __future__ import annotations

import functools
import math

import numpy as np

from . import ladder as lad
from . import oplog
from .numerics import dsum, f32

INF = np.float32(np.inf)
INF_KEY = np.uint64(0x7F800000) << np.uint64(32)
LOW = np.uint64(0xFFFFFFFF)


def pack(cost, key):
    """(cost bits << 32) | key, +0.0 for a zero cost (litgpt/log_kv_cache.py:431-434)."""
    cost = np.where(cost == 0, np.float32(0), cost).astype(np.float32)
    return (cost.view(np.uint32).astype(np.uint64) << np.uint64(32)) | np.asarray(key).astype(np.uint64)


def pair_cost(d2, mi, mj, ri, rj, limit, valid):
    """Ward cost and validity (litgpt/log_kv_cache.py:437-445)."""
    one = np.float32(1)
    denom = np.maximum(mi + mj, one)
    valid = valid & (mi > 0) & (mj > 0)
    if limit is not None:
        distance = np.sqrt(d2)
        bound = np.maximum(ri + (mj / denom) * distance, rj + (mi / denom) * distance)
        valid = valid & (bound <= limit)
    cost = np.where(valid, d2 * (mi * mj / denom), INF).astype(np.float32)
    return cost, valid


def pair_distances(mu):
    """Squared distances ``[M, M]``: canonical sums of squared differences for
    i < j, mirrored, zero diagonal."""
    mu = f32(mu)
    m = mu.shape[0]
    out = np.zeros((m, m), np.float32)
    for i in range(m - 1):
        diff = mu[i][None, :] - mu[i + 1:]
        out[i, i + 1:] = dsum(diff * diff)
    iu = np.triu_indices(m, 1)
    out[iu[1], iu[0]] = out[iu]
    return out


def clamp0(x):
    return np.where(x < 0, np.float32(0), x).astype(np.float32)


class Reducer:
    """One lane's incremental rounds (litgpt/log_kv_cache.py:448-637). With
    ``passes > 1`` (the budget stage only) a round also runs frozen-center
    sweeps (:561-588): rows whose restricted partner was matched rescan the
    unmatched columns, unmatched mutual pairs join the round, and every pair
    of the round is budgeted by cost."""

    def __init__(self, dist, mu, mass, count, limit, target, passes=1):
        self.dist, self.mu, self.mass = f32(dist).copy(), f32(mu).copy(), f32(mass).copy()
        self.limit = None if limit is None else np.float32(limit)
        self.target = int(target)
        self.passes = max(1, int(passes))
        size = self.mass.shape[0]
        self.ids = np.arange(size)
        self.alive = self.ids < count
        self.radius = np.zeros(size, np.float32)
        self.count = int(count)
        self.stuck = False
        self.trace = []
        self.packed = np.full(size, INF_KEY, np.uint64)
        rows = np.flatnonzero(self.alive)
        if len(rows):
            self.packed[rows] = self._scan(rows)
        # Work counts (the device reports the same): rounds, kept rows x live columns of the
        # Lance-Williams updates, rescanned rows x live columns (the first scan: every row).
        self.rounds, self.lw_elems, self.scan_elems = 0, 0, len(rows) * len(rows)

    def _scan(self, rows, excluded=None):
        """Packed row minima (litgpt/log_kv_cache.py:473-488); ``excluded`` columns (matched
        this round) take no mass."""
        lim = self.limit is not None
        mass = self.mass if excluded is None else np.where(excluded, np.float32(0), self.mass).astype(np.float32)
        cost, _ = pair_cost(self.dist[rows], self.mass[rows][:, None], mass[None, :],
                            self.radius[rows][:, None] if lim else None, self.radius[None, :] if lim else None,
                            self.limit, self.ids[None, :] != rows[:, None])
        return pack(cost, rows[:, None] ^ self.ids[None, :]).min(1)

    def step(self):
        size = self.mass.shape[0]
        ids = self.ids
        best = np.clip(((self.packed & LOW).astype(np.int64)) ^ ids, 0, size - 1)
        cost = (self.packed >> np.uint64(32)).astype(np.uint32).view(np.float32)
        valid = self.alive & (ids < best) & (best[best] == ids) & (cost < INF)
        nprop = int(valid.sum())
        rejected = np.zeros(size, bool)
        bound = None
        if self.limit is not None:
            rows = np.flatnonzero(valid)
            other = best[rows]
            diff = self.mu[rows] - self.mu[other]
            exact2 = dsum(diff * diff)
            exact = np.sqrt(exact2)
            ma, mb = self.mass[rows], self.mass[other]
            denom = np.maximum(ma + mb, np.float32(1))
            verified = np.maximum(self.radius[rows] + (mb / denom) * exact,
                                  self.radius[other] + (ma / denom) * exact).astype(np.float32)
            bad = verified > self.limit
            self.dist[rows[bad], other[bad]] = exact2[bad]
            self.dist[other[bad], rows[bad]] = exact2[bad]
            rejected[rows[bad]] = True
            rejected[other[bad]] = True
            valid[rows[bad]] = False
            bound = np.zeros(size, np.float32)
            bound[rows] = verified
        pair = np.where(valid, cost, INF).astype(np.float32)
        mate = best
        if self.passes > 1:
            mate, pair, extra = self._sweeps(valid, best, pair)
            nprop += extra
        order = np.argsort(pair, kind="stable")[:size // 2]
        ok = pair[order] < INF
        ok &= np.cumsum(ok) <= self.count - self.target
        a = order[ok]
        b = mate[a]
        keep = np.zeros(size, bool)
        merged = np.zeros(size, bool)
        if len(a):
            self._merge(a, b, bound, keep, merged)
        dirty = self.alive & ~keep & (merged[best] | rejected)
        rows = np.flatnonzero(dirty)
        if len(rows):
            self.packed[rows] = self._scan(rows)
        live = int(self.alive.sum())
        self.rounds += 1
        self.lw_elems += len(a) * live
        self.scan_elems += len(rows) * live
        self.count -= int(ok.sum())
        remaining = self.count > self.target
        if remaining and nprop == 0:
            self.stuck = True
        return remaining and nprop > 0

    def _sweeps(self, valid, best, pair):
        """Frozen-center sweeps after the round's mutual pairs (litgpt/log_kv_cache.py:561-588):
        returns each row's mate, the pair costs (at a pair's lower row) and the pairs added."""
        size = self.mass.shape[0]
        ids = self.ids
        matched = np.zeros(size, bool)
        rows = np.flatnonzero(valid)
        matched[rows] = True
        matched[best[rows]] = True
        restricted = self.packed.copy()
        mate, extra = best.copy(), 0
        pair = pair.copy()
        for _ in range(self.passes - 1):
            partner = np.clip(((restricted & LOW).astype(np.int64)) ^ ids, 0, size - 1)
            rows = np.flatnonzero(self.alive & ~matched & matched[partner])
            if len(rows):
                restricted[rows] = self._scan(rows, excluded=matched)
                self.scan_elems += len(rows) * int(self.alive.sum())
            partner = np.clip(((restricted & LOW).astype(np.int64)) ^ ids, 0, size - 1)
            cost = (restricted >> np.uint64(32)).astype(np.uint32).view(np.float32)
            more = (self.alive & ~matched & (ids < partner) & (partner[partner] == ids) & (cost < INF)
                    & ~matched[partner])
            extra += int(more.sum())
            rows = np.flatnonzero(more)
            matched[rows] = True
            matched[partner[rows]] = True
            mate = np.where(more, partner, mate)
            pair = np.where(more, cost, pair).astype(np.float32)
        return mate, pair, extra

    def _merge(self, a, b, bound, keep, merged):
        size = self.mass.shape[0]
        ids = self.ids
        ma, mb = self.mass[a], self.mass[b]
        dab = self.dist[a, b]
        total = ma + mb
        alpha, beta = ma / total, mb / total
        shift = alpha * beta * dab
        keep[a] = True
        merged[a] = True
        merged[b] = True
        partner = np.zeros(size, np.int64)
        partner[a] = b
        pma, pmb, pdab = np.ones(size, np.float32), np.zeros(size, np.float32), np.zeros(size, np.float32)
        pma[a], pmb[a], pdab[a] = ma, mb, dab
        self.mass[a] = total
        self.mass[b] = 0
        self.alive[b] = False
        if bound is not None:
            self.radius[a] = bound[a]
        self.mu[a] = (ma[:, None] * self.mu[a] + mb[:, None] * self.mu[b]) / np.maximum(total, np.float32(1))[:, None]
        al, be, sh = alpha[:, None], beta[:, None], shift[:, None]
        x_aa, x_ba = self.dist[a], self.dist[b]
        new = al * x_aa + be * x_ba - sh
        q = partner
        x_ab, x_bb = self.dist[a[:, None], q[None, :]], self.dist[b[:, None], q[None, :]]
        qalpha, qbeta = pma / (pma + pmb), pmb / (pma + pmb)
        qshift = qalpha * qbeta * pdab
        own_first = qalpha * new + qbeta * (al * x_ab + be * x_bb - sh) - qshift
        other_first = al * (qalpha * x_aa + qbeta * x_ab - qshift) + be * (qalpha * x_ba + qbeta * x_bb - qshift) - sh
        both = np.where(a[:, None] < ids[None, :], own_first, other_first)
        new = clamp0(np.where(keep[None, :], both, new))
        new[np.arange(len(a)), a] = 0
        alive = self.alive
        cols = np.flatnonzero(alive & ~keep)
        for p in range(len(a)):
            self.dist[cols, a[p]] = new[p, cols]
        cols = np.flatnonzero(alive)
        for p in range(len(a)):
            self.dist[a[p], cols] = new[p, cols]
        lim = self.limit is not None
        cost, valid = pair_cost(new, total[:, None], self.mass[None, :],
                                self.radius[a][:, None] if lim else None, self.radius[None, :] if lim else None,
                                self.limit, alive[None, :] & (ids[None, :] != a[:, None]))
        packed = pack(cost, ids[None, :] ^ a[:, None])
        push = valid & ~keep[None, :]
        for p in range(len(a)):
            cols = np.flatnonzero(push[p])
            self.packed[cols] = np.minimum(self.packed[cols], packed[p, cols])
        self.packed[a] = packed.min(1)
        self.trace.extend(zip(a.tolist(), b.tolist()))


def reduce(mu, mass, count, limit, target, strict=False, counts=None, passes=1):
    """Rounds until no mutual pair is left or ``count <= target``
    (litgpt/log_kv_cache.py:3303-3376). Returns (survivors, trace, centers).
    ``counts``: a list that gets the stage's (nodes, rounds, merges,
    Lance-Williams elements, rescanned elements). ``passes``: frozen-center
    sweeps per round, used only without a radius limit (:3314)."""
    if count <= target:
        if counts is not None:
            counts.append((count, 0, 0, 0, 0))
        return np.arange(count), [], f32(mu).copy()
    r = Reducer(pair_distances(mu), mu, mass, count, limit, target, passes if limit is None else 1)
    size = r.mass.shape[0]
    for _ in range(2 * size + 7):
        if not r.step():
            break
    if strict and r.stuck:
        raise RuntimeError("unified route: no mutual pair below the cluster budget")
    if counts is not None:
        counts.append((count, r.rounds, len(r.trace), r.lw_elems, r.scan_elems))
    return np.flatnonzero(r.alive), r.trace, r.mu


def mutual_pairs(cost):
    """Disjoint mutual-minimum pairs of a cost matrix (litgpt/log_kv_cache.py:2988-3016): each row's
    least cost, ties to the least ``row ^ col``; a pair is named by its lower row, the pairs in
    (cost, row) order. Returns [(left, right, cost)]."""
    n = cost.shape[0]
    ids = np.arange(n)
    best_cost = cost.min(1) if n else np.zeros(0, np.float32)
    tie = ids[:, None] ^ ids[None, :]
    best = np.where(cost == best_cost[:, None], tie, 2 * n).argmin(1) if n else ids
    valid = (ids < best) & (best[best] == ids) & np.isfinite(best_cost)
    rows = np.flatnonzero(valid)
    order = rows[np.argsort(best_cost[rows], kind="stable")]
    return [(int(r), int(best[r]), best_cost[r]) for r in order]


def round_pairs(mu, mass, radius, limit, cap, overflow):
    """One full-recompute round's pairs over the current nodes (litgpt/log_kv_cache.py:3067-3117, the
    unfused form): Ward costs, with a limit the radius bound, with a finite cap no pair whose total
    mass exceeds it (``overflow``: a lane left with no capped pair takes the uncapped ones); mutual
    minima in (cost, row) order; with a limit each pair's bound re-checked from its exact distance
    and the pairs that fail dropped."""
    n = len(mass)
    d2 = pair_distances(mu)
    mi, mj = mass[:, None], mass[None, :]
    total = (mi + mj).astype(np.float32)
    denom = np.maximum(total, np.float32(1))
    cost = (d2 * (mi * mj / denom)).astype(np.float32)
    live = mass > 0
    cost = np.where(live[:, None] & live[None, :], cost, INF).astype(np.float32)
    np.fill_diagonal(cost, INF)
    if limit is not None:
        distance = np.sqrt(d2)
        bound = np.maximum(radius[:, None] + (mj / denom) * distance, radius[None, :] + (mi / denom) * distance)
        cost = np.where(bound > limit, INF, cost).astype(np.float32)
    capped = np.isfinite(cap)
    pairs = mutual_pairs(np.where(total > cap, INF, cost).astype(np.float32) if capped else cost)
    if overflow and capped and not pairs:
        pairs = mutual_pairs(cost)
    if limit is not None:
        kept = []
        for l, r, c in pairs:
            diff = mu[l] - mu[r]
            exact = np.sqrt(dsum((diff * diff)[None])[0])
            ml, mr = mass[l], mass[r]
            den = np.maximum(ml + mr, np.float32(1))
            bound = max(radius[l] + mr / den * exact, radius[r] + ml / den * exact)
            if not bound > limit:
                kept.append((l, r, c))
        pairs = kept
    return pairs


def reduce_rounds(mu, mass, count, limit, target, cap=INF, strict=False, counts=None, passes=1):
    """Full-recompute rounds (litgpt/log_kv_cache.py:3445-3519), the reducer of a capacity-capped
    unified route: each round prices the current nodes afresh (``round_pairs``), takes its first
    ``count - target`` pairs, merges each pair into its lower row (``_semantic_unified_merge_pack``,
    :3134-3156: the mass-weighted center, summed mass, with a limit the pair's radius bound from
    their exact distance) and compacts the survivors in order, until no pair is left or ``count <=
    target``. Returns ``reduce``'s (survivors, trace, centers) in input row ids; ``strict``: a round
    with no pair above the target raises. ``counts`` gets (nodes, rounds, merges, 0, 0)."""
    if passes > 1 and limit is None and not np.isfinite(cap):
        raise NotImplementedError("frozen-center sweeps of the full-recompute rounds are not restated")
    out = f32(mu).copy()
    if count <= target:
        if counts is not None:
            counts.append((count, 0, 0, 0, 0))
        return np.arange(count), [], out
    cur, m, rad = f32(mu[:count]).copy(), f32(mass[:count]).copy(), np.zeros(count, np.float32)
    roots = np.arange(count)
    trace, rounds = [], 0
    cap = np.float32(cap)
    while len(roots) > target:
        pairs = round_pairs(cur, m, rad, limit, cap, strict)[:len(roots) - target]
        rounds += 1
        if not pairs:
            if strict:
                raise RuntimeError("unified route: no mutual pair below the cluster budget")
            break
        trace.extend((int(roots[l]), int(roots[r])) for l, r, _ in pairs)
        partner = np.full(len(roots), -1)
        keep = np.ones(len(roots), bool)
        for l, r, _ in pairs:
            partner[l] = r
            keep[r] = False
        surv = np.flatnonzero(keep)
        new_mu, new_m, new_r = cur[surv].copy(), m[surv].copy(), np.zeros(len(surv), np.float32)
        for i, s_ in enumerate(surv):
            b = partner[s_]
            if limit is not None:
                new_r[i] = rad[s_]
            if b < 0:
                continue
            ma, mb = m[s_], m[b]
            comb = ma + mb
            scale = np.maximum(comb, np.float32(1))
            new_mu[i] = ((ma * cur[s_] + mb * cur[b]) / scale).astype(np.float32)
            new_m[i] = comb
            if limit is not None:
                diff = cur[s_] - cur[b]
                dist = np.sqrt(dsum((diff * diff)[None])[0])
                new_r[i] = max(rad[s_] + mb / scale * dist, rad[b] + ma / scale * dist)
        cur, m, rad, roots = new_mu, new_m, new_r, roots[surv]
    out[roots] = cur
    if counts is not None:
        counts.append((count, rounds, len(trace), 0, 0))
    return roots, trace, out


def labels(size, survivors, trace):
    """Leaf -> compact surviving row (litgpt/log_kv_cache.py:3544-3568)."""
    parent = np.arange(size)
    for a, b in trace:
        parent[b] = a
    while True:
        nxt = parent[parent]
        if np.array_equal(nxt, parent):
            break
        parent = nxt
    compact = np.full(size, -1, np.int64)
    compact[np.asarray(survivors, np.int64)] = np.arange(len(survivors))
    return compact[parent]


def ward_entry_order(order, p_lo, has_mass, split):
    """Two-way stable merge of the keep (``[:split]``) and free entries
    (litgpt/log_kv_cache.py:2425-2447)."""
    left = sorted(range(split), key=lambda i: order[i])
    right = sorted(range(split, len(order)), key=lambda i: order[i])
    effective = [0] * len(order)
    for seq in (left, right):
        nxt = None
        for i in reversed(seq):
            if has_mass[i]:
                nxt = p_lo[i]
            effective[i] = order[i] if nxt is None else nxt
    merged, i, j = [], 0, 0
    while i < len(left) and j < len(right):
        if effective[left[i]] <= effective[right[j]]:
            merged.append(left[i])
            i += 1
        else:
            merged.append(right[j])
            j += 1
    return merged + left[i:] + right[j:]


def ward_merge(cache, b, g, keep, free):
    """Merge old cluster ``free`` into ``keep`` (litgpt/log_kv_cache.py:2517-2580)."""
    cache.ward_merges += 1
    ents = [cache.ladder(b, g, c).entries() for c in (keep, free)]
    rows = lad.concat(ents)
    split = len(ents[0]["w"])
    idx = ward_entry_order(rows["order"].tolist(), rows["p_lo"].tolist(), (rows["w"] > 0).tolist(), split)
    rows = lad.take(rows, np.asarray(idx, np.int64))
    rows["order"] = np.arange(len(idx), dtype=np.int64)
    nk, nf = np.float32(cache.n_total[b, g, keep]), np.float32(cache.n_total[b, g, free])
    mu = (nk * cache.centroid[b, g, keep] + nf * cache.centroid[b, g, free]) / np.maximum(nk + nf, np.float32(1))
    ne = cache.n_eff[b, g, keep] + cache.n_eff[b, g, free]
    total = int(cache.n_total[b, g, keep]) + int(cache.n_total[b, g, free])
    high = max(int(cache.p_hi_c[b, g, keep]), int(cache.p_hi_c[b, g, free]))
    for c in (keep, free):
        cache.ladder(b, g, c).clear()
        cache.alive[b, g, c] = False
        cache.n_total[b, g, c] = 0
        cache.p_hi_c[b, g, c] = -1
        cache.level0_phase[b, g, c] = 0
    cache.centroid[b, g, keep] = mu.astype(np.float32)
    cache.n_eff[b, g, keep] = ne
    cache.n_eff[b, g, free] = 0
    cache.alive[b, g, keep] = True
    cache.n_total[b, g, keep] = total
    cache.p_hi_c[b, g, keep] = high
    cache.level0_phase[b, g, keep] = len(idx)
    if len(idx):
        cache._append(b, g, keep, rows)


def plan_lane(cache, keys, n, b, g, reduce_fn=reduce):
    """Both stages of one lane: (ward jobs [(keep, free)], target cluster root
    per row as (root index, n_old, old ids, survivors)). ``reduce_fn`` runs a
    reducer stage (``reduce``'s signature and results)."""
    limit = np.float32(math.sqrt(float(cache.lam) * float(cache.s_h[b, g])))
    mu = f32(keys[:n])
    cap = float(getattr(cache, "hard_cap", np.inf))
    if np.isfinite(cap):
        # A capacity cap runs the full-recompute rounds (litgpt/log_kv_cache.py:3283-3288).
        reduce_fn = functools.partial(reduce_rounds, cap=cap)
    surv1, trace1, mu1 = reduce_fn(mu, np.ones(n, np.float32), n, limit, 1)
    lab1 = labels(n, surv1, trace1)
    old = np.flatnonzero(cache.alive[b, g])
    weights = np.concatenate((cache.n_total[b, g, old].astype(np.float32),
                              np.bincount(lab1, minlength=len(surv1)).astype(np.float32)))
    centers = np.concatenate((cache.centroid[b, g, old].astype(np.float32), mu1[surv1]))
    m2 = len(weights)
    passes = getattr(cache, "merge_passes", 1)
    extra = {"passes": passes} if passes > 1 else {}
    surv2, trace2, _ = reduce_fn(centers, weights, m2, None, cache.K, strict=True, **extra)
    lab2 = labels(m2, surv2, trace2)
    jobs = [(int(old[a]), int(old[c])) for a, c in trace2 if c < len(old)]
    root = lab2[len(old) + lab1]
    return jobs, root, old, np.asarray(surv2)


def unified_jobs(cache, ak, ap, counts, reduce_fn=reduce):
    """The route half of a unified flush (litgpt/log_kv_cache.py:3589-3664): every lane planned,
    its old-old merges applied (and logged); returns the commit jobs ``{(b, g, c): (opened, rows
    in position order)}`` and per lane the cluster of every row (offset order), -1 past the
    count."""
    ak = f32(ak)
    n_batch, n_groups, width, _ = ak.shape
    out = np.full((n_batch, n_groups, width), -1, np.int64)
    plans = {}
    for b in range(n_batch):
        n = int(counts[b])
        if not n:
            continue
        for g in range(n_groups):
            plans[(b, g)] = plan_lane(cache, ak[b, g], n, b, g, reduce_fn)
    for (b, g), (jobs, _, _, _) in plans.items():
        for keep, free in jobs:
            ward_merge(cache, b, g, keep, free)
    # With an op-log bound, each lane's WARD_MERGE rows (keep, free, -1) come
    # first, in merge order (litgpt/log_kv_cache.py:2597-2598, called from the
    # merge steps at :3661-3664 before the new clusters and joins).
    if cache.op_log is not None:
        for (b, g), (jobs, _, _, _) in plans.items():
            cache.op_log[b][g].extend((oplog.WARD_MERGE, int(keep), int(free), -1) for keep, free in jobs)
    jobs_all = {}
    for (b, g), (_, root, old, surv2) in plans.items():
        n = int(counts[b])
        free_slots = iter(np.flatnonzero(~cache.alive[b, g]).tolist())
        rows = np.argsort(ap[b, :n], kind="stable")   # the lane's rows in position order
        by_root = root[rows]
        for r in range(len(surv2)):
            sel = rows[by_root == r]
            if not len(sel):
                continue
            opened = surv2[r] >= len(old)
            c = next(free_slots) if opened else int(old[surv2[r]])
            jobs_all[(b, g, c)] = (opened, sel)
            out[b, g, sel] = c
    return jobs_all, out


def route_unified(cache, ak, av, ap, counts):
    """Unified route + commit of ``counts[b]`` rows of ``ak/av/ap``
    (litgpt/log_kv_cache.py:3589-3688). Returns per lane the cluster of every
    row (offset order), -1 past the count."""
    ak, av = f32(ak), f32(av)
    jobs_all, out = unified_jobs(cache, ak, ap, counts)
    late = set()
    for (b, g, c), (new, rows) in sorted(jobs_all.items()):
        if new:
            t = rows[0]
            cache.new_cluster(b, g, c, ak[b, g, t], av[b, g, t], int(ap[b, t]))
            rows = rows[1:]
        if not len(rows):
            continue
        pos = ap[b, rows].astype(np.int64)
        if cache.P and pos.min() < cache.p_hi_c[b, g, c]:
            late.add((b, g, c))
            cache.join_late(b, g, c, ak[b, g, rows], av[b, g, rows], pos)
        else:
            cache.join(b, g, c, ak[b, g, rows], av[b, g, rows], pos)
    if cache.op_log is not None:
        for (b, g), rows in oplog.flush_rows(jobs_all, ap, late).items():
            cache.op_log[b][g].extend(rows)
    return out
