"""A batched Torch-CPU flush: the CPU baseline's implementation of one layer's flush.

TEST INFRASTRUCTURE ONLY: ``bench.py``'s ``cpu_baseline`` leg times it and tests/test_torch_cpu.py
checks it; the product package never imports it.

The oracle (``oracle.cache.OracleCache``) walks ladders and Beta groups one at a time, which is
what makes it a readable restatement and a slow baseline. The reference's CPU path instead schedules
every ladder of a flush together, level by level, and evaluates the Beta groups of a level as
tensor operations (litgpt/log_kv_cache.py:1756-1929, ``_semantic_append_entries_batched``;
litgpt/beta_log_kv.py:29-105, ``select_cuts`` / ``apply_cuts`` over all groups). ``TorchCpuCache``
restates that schedule on top of the oracle's state (same arrays, same driver, same Alpha
selection and attach decisions):

* one commit per flush: the opened, delayed-archive and joined ladders are staged first (the
  oracle's per-cluster rules, centers in position order), then appended together;
* each level once for all staged ladders: free slots filled, the overflowing pool's oldest rows
  paired (or Beta-compacted) in one batched call over every ladder's groups, survivors moved;
* Beta cut costs and merges as torch float32 tensor operations over all groups at once, in the
  oracle's canonical orders, so every state field stays bit-identical to the oracle's (checked by
  tests/test_torch_cpu.py); torch's intra-op threads parallelise the large operations.

The unified (Ward / radius) route's reducer (litgpt/log_kv_cache.py:448-637, ``_UnifiedReduceTorch``)
is restated on torch tensors as ``TorchReducer``, element operation for element operation the
oracle's ``oracle.unified.Reducer``, and its commit takes the same batched level-by-level append.
``slot_attention`` is the readout's attention over packed rows as the reference evaluates it on the
CPU (``torch.nn.functional.scaled_dot_product_attention`` over the Flash encoding of the slots,
litgpt/log_kv_cache.py:6751-6758), in float32.
"""

from __future__ import annotations

import numpy as np
import torch

from . import ladder as lad
from . import readout, route, unified
from .cache import OracleCache
from .numerics import WAVE, bf16_round, f32

I64_MAX = np.iinfo(np.int64).max
I64_MIN = np.iinfo(np.int64).min
_CUTS = (2, 1, 3)


def _dsum(t: torch.Tensor) -> torch.Tensor:
    """The oracle's canonical feature sum (``numerics.dsum``) of the last axis, batched."""
    d = t.shape[-1]
    chunks = max(1, -(-d // WAVE))
    if d != chunks * WAVE:
        t = torch.nn.functional.pad(t, (0, chunks * WAVE - d))
    s = t[..., :WAVE]
    for j in range(1, chunks):
        s = s + t[..., j * WAVE:(j + 1) * WAVE]
    width = WAVE
    while width > 1:
        width //= 2
        s = s[..., :width] + s[..., width:2 * width]
    return s[..., 0]


def _side_mean(x: torch.Tensor, wt: torch.Tensor):
    """sum_i x_i * w_i in row order / max(sum_i w_i, 1e-12); x ``[n, 4, d]``, wt ``[n, 4]``."""
    acc = x[:, 0] * wt[:, 0, None]
    for i in range(1, 4):
        acc = acc + x[:, i] * wt[:, i, None]
    mass = wt[:, 0]
    for i in range(1, 4):
        mass = mass + wt[:, i]
    return acc / torch.clamp(mass, min=1e-12)[:, None], mass


def beta_merge_batched(rows: dict, lengths):
    """``oracle.ladder.beta_merge`` over every group at once: returns (carries, cuts uint8)."""
    layout = lad.beta_layout(lengths)
    n_out = len(rows["w"]) // 2
    out = lad.empty_rows(n_out, rows["k"].shape[1], rows["v"].shape[1])
    if not len(layout):
        return out, np.zeros(0, np.uint8)
    start, width, dest = (torch.from_numpy(layout[:, j].copy()) for j in range(3))
    n = len(layout)
    idx = start[:, None] + torch.arange(4)[None, :]
    valid = torch.arange(4)[None, :] < width[:, None]
    gidx = torch.where(valid, idx, start[:, None])
    # Rows past a tail's width are zeros, as in the oracle's zero-filled groups.
    k4 = torch.where(valid[..., None], torch.from_numpy(f32(rows["k"]))[gidx], torch.zeros(()))
    v4 = torch.where(valid[..., None], torch.from_numpy(f32(rows["v"]))[gidx], torch.zeros(()))
    w4 = torch.where(valid, torch.from_numpy(f32(rows["w"]))[gidx], torch.zeros(()))

    # Cut costs (beta_select_cut): options (2, 1, 3), K then V, left then right side.
    total = torch.clamp(((w4[:, 0] + w4[:, 1]) + w4[:, 2]) + w4[:, 3], min=1e-12)
    costs = torch.zeros(n, 3)
    for x in (k4, v4):
        sq = _dsum(x * x)
        e = sq[:, 0] * w4[:, 0]
        for i in range(1, 4):
            e = e + sq[:, i] * w4[:, i]
        energy = torch.clamp(e / total, min=1e-12)
        for j, c in enumerate(_CUTS):
            for side in (0, 1):
                member = (torch.arange(4) < c) if side == 0 else (torch.arange(4) >= c)
                wt = torch.where(member[None, :], w4, torch.zeros(()))
                mean, _ = _side_mean(x, wt)
                d = x - mean[:, None, :]
                per = _dsum(d * d)
                loss = per[:, 0] * wt[:, 0]
                for i in range(1, 4):
                    loss = loss + per[:, i] * wt[:, i]
                costs[:, j] = costs[:, j] + loss / energy
    best = torch.zeros(n, dtype=torch.long)
    best = torch.where(costs[:, 1] < costs[:, 0], 1, best)
    best = torch.where(costs[:, 2] < costs.gather(1, best[:, None])[:, 0], 2, best)
    cut = torch.tensor(_CUTS)[best]
    cut = torch.where(width == 2, torch.ones_like(cut), cut)

    # Outputs (beta_apply): per group the left side (all valid rows for a tail) and the right side.
    ar = torch.arange(4)[None, :]
    left = valid & ((width[:, None] == 2) | (ar < cut[:, None]))
    right = valid & (width[:, None] == 4) & (ar >= cut[:, None])
    meta = {f: torch.from_numpy(np.asarray(rows[f]))[gidx] for f in ("p_lo", "p_hi", "sum_wp", "order")}
    pad = torch.from_numpy(np.asarray(rows["pad"]))[gidx]
    w_raw = torch.from_numpy(f32(rows["w"]))[gidx]
    for side, mask in ((0, left), (1, right)):
        has = mask.any(1) if side == 1 else torch.ones(n, dtype=torch.bool)
        wt = torch.where(mask, w4, torch.zeros(()))
        ko, mass = _side_mean(k4, wt)
        vo, _ = _side_mean(v4, wt)
        live = mask & (w_raw > 0)
        lo = torch.where(live, meta["p_lo"], torch.full((), I64_MAX)).min(1).values
        hi = torch.where(live, meta["p_hi"], torch.full((), I64_MIN)).max(1).values
        pos = mass > 0
        sel = torch.nonzero(has)[:, 0]
        d = (dest + side)[sel].numpy()
        out["k"][d] = ko[sel].numpy()
        out["v"][d] = vo[sel].numpy()
        out["w"][d] = mass[sel].numpy()
        out["p_lo"][d] = torch.where(pos, lo, torch.zeros((), dtype=torch.long))[sel].numpy()
        out["p_hi"][d] = torch.where(pos, hi, torch.zeros((), dtype=torch.long))[sel].numpy()
        out["sum_wp"][d] = torch.where(mask, meta["sum_wp"], torch.zeros((), dtype=torch.long)).sum(1)[sel].numpy()
        out["order"][d] = torch.where(mask, meta["order"], torch.full((), I64_MAX)).min(1).values[sel].numpy()
        out["pad"][d] = torch.where(mask, pad, torch.ones((), dtype=torch.bool)).all(1)[sel].numpy()
    return out, cut.to(torch.uint8).numpy()


def _bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even) as float32, as ``numerics.bf16_round``."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def _storage(rows: dict) -> dict:
    out = dict(rows)
    out["k"], out["v"] = _bf16(rows["k"]), _bf16(rows["v"])
    return out


def attach_assign_batched(x, pos, counts, centroid, alive, p_hi, s_h, eta, g0, lam):
    """``oracle.route.attach_assign`` with every KV group of a batch row evaluated at once in torch
    (the frozen-join distances, costs and winners, and the orphans' nearest live cluster); a lane
    whose orphans open free clusters takes the oracle's seeding path."""
    x = f32(x)
    n_batch, n_groups, tokens, _ = x.shape
    counts = np.asarray(counts, dtype=np.int64)
    order = route.position_order(np.asarray(pos, dtype=np.int64), counts)
    out = np.full((n_batch, n_groups, tokens), -1, dtype=np.int8)
    for b in range(n_batch):
        n = int(counts[b])
        if n == 0:
            continue
        rows = order[b, :n]
        xs = torch.from_numpy(np.ascontiguousarray(x[b][:, rows]))                 # [G, n, D]
        mu = torch.from_numpy(f32(centroid[b]))                                    # [G, K, D]
        live = torch.from_numpy(np.asarray(alive[b], dtype=bool))                  # [G, K]
        xx = _dsum(xs * xs)
        mm = _dsum(mu * mu)
        dot = _dsum(xs[:, :, None, :] * mu[:, None, :, :])
        semantic = torch.clamp((xx[:, :, None] + mm[:, None, :]) - 2.0 * dot, min=0.0)
        gap = torch.clamp(torch.from_numpy(np.asarray(pos[b, rows], np.int64))[None, :, None]
                          - torch.from_numpy(np.asarray(p_hi[b], np.int64))[:, None, :], min=0).float()
        cost = semantic + np.float32(eta) * (gap / (gap + np.float32(g0)))
        cost = torch.where(live[:, None, :], cost, torch.full((), float("inf")))
        winner = torch.argmin(cost, dim=2)
        s_winner = semantic.gather(2, winner[..., None])[..., 0]
        limit = torch.from_numpy(f32(np.float32(lam) * f32(s_h[b])))               # [G]
        direct = live.any(1)[:, None] & (s_winner <= limit[:, None])
        diff = xs[:, :, None, :] - mu[:, None, :, :]
        exact = _dsum(diff * diff)
        nearest = torch.argmin(torch.where(live[:, None, :], exact, torch.full((), float("inf"))), dim=2)
        assign = torch.where(direct, winner, nearest).numpy()
        for g in range(n_groups):
            orphans = int((~direct[g]).sum())
            free = int((~live[g]).sum())
            if orphans and free:
                assign[g] = route.lane_assign(x[b, g, rows], pos[b, rows], centroid[b, g], alive[b, g], p_hi[b, g],
                                              s_h[b, g], eta, g0, lam)
        out[b, :, :n] = assign
    return out, order


def _rope(x: torch.Tensor, anchors: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, table_bf16: bool):
    """``readout.rope`` in torch: rotate-half RoPE of bf16-valued ``x`` at ``anchors``, rounded to bf16."""
    n = cos.shape[1]
    half = n // 2
    c, s = cos[anchors], sin[anchors]
    xr = x[..., :n]
    rotated = torch.cat((-xr[..., half:], xr[..., :half]), dim=-1)
    if table_bf16:
        out = _bf16t(_bf16t(xr * c) + _bf16t(rotated * s))
    else:
        out = _bf16t(xr * c + rotated * s)
    return torch.cat((out, x[..., n:]), dim=-1)


def _bf16t(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


_INF = float("inf")
_I64_TOP = torch.iinfo(torch.int64).max


def _pack_key(cost: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
    """``oracle.unified.pack`` as int64: (cost bits << 32) | key, -0.0 stored as +0.0 (costs are
    >= 0 or +inf, so the bits fit in 31)."""
    cost = torch.where(cost == 0, torch.zeros((), dtype=torch.float32), cost)
    return (cost.view(torch.int32).to(torch.int64) << 32) | key.to(torch.int64)


def _pair_cost(d2, mi, mj, ri, rj, limit, valid):
    """``oracle.unified.pair_cost`` on tensors (litgpt/log_kv_cache.py:437-445)."""
    denom = torch.clamp(mi + mj, min=1.0)
    valid = valid & (mi > 0) & (mj > 0)
    if limit is not None:
        distance = torch.sqrt(d2)
        bound = torch.maximum(ri + (mj / denom) * distance, rj + (mi / denom) * distance)
        valid = valid & (bound <= limit)
    cost = torch.where(valid, d2 * (mi * mj / denom), torch.full((), _INF))
    return cost, valid


def pair_distances(mu: torch.Tensor, block: int = 32) -> torch.Tensor:
    """Squared distances ``[M, M]`` of rows of ``mu``, canonical feature sums of squared
    differences: the oracle's upper triangle and its mirror (x_i - x_j and x_j - x_i square to the
    same float), computed in row blocks."""
    m = mu.shape[0]
    out = torch.empty(m, m, dtype=torch.float32)
    for i0 in range(0, m, block):
        diff = mu[i0:i0 + block, None, :] - mu[None, :, :]
        out[i0:i0 + block] = _dsum(diff * diff)
    return out


def gram_distances(mu: torch.Tensor) -> torch.Tensor:
    """Squared distances as the reference forms them above 32 nodes (litgpt/log_kv_cache.py:3028-3047):
    rows centred on the first one, squared norms plus the Gram matrix (a GEMM), ``|a|^2 + |b|^2 - 2 a.b``
    clamped at zero. The CPU baseline times this form, the reference's own; its last-ulp values differ
    from the canonical direct differences (``pair_distances``), so it is not used for parity."""
    centred = mu - mu[:1]
    norm = (centred * centred).sum(-1)
    return torch.clamp(norm[:, None] + norm[None, :] - 2 * (centred @ centred.T), min=0.0)


class TorchReducer:
    """One lane's incremental reducer rounds on torch tensors: ``oracle.unified.Reducer`` with the
    same element operations in the same order (litgpt/log_kv_cache.py:448-637)."""

    def __init__(self, dist, mu, mass, count, limit, target):
        self.dist, self.mu, self.mass = dist, mu.clone(), mass.clone()
        self.limit = None if limit is None else float(np.float32(limit))
        self.target = int(target)
        size = self.mass.shape[0]
        self.ids = torch.arange(size)
        self.alive = self.ids < count
        self.radius = torch.zeros(size)
        self.count = int(count)
        self.stuck = False
        self.trace = []
        self.packed = torch.full((size,), int(unified.INF_KEY), dtype=torch.int64)
        rows = torch.nonzero(self.alive)[:, 0]
        if len(rows):
            self.packed[rows] = self._scan(rows)

    def _scan(self, rows):
        lim = self.limit is not None
        cost, _ = _pair_cost(self.dist[rows], self.mass[rows][:, None], self.mass[None, :],
                             self.radius[rows][:, None] if lim else None, self.radius[None, :] if lim else None,
                             self.limit, self.ids[None, :] != rows[:, None])
        return _pack_key(cost, rows[:, None] ^ self.ids[None, :]).min(1).values

    def step(self):
        size = self.mass.shape[0]
        ids = self.ids
        best = torch.clamp((self.packed & 0xFFFFFFFF) ^ ids, 0, size - 1)
        cost = (self.packed >> 32).to(torch.int32).view(torch.float32)
        valid = self.alive & (ids < best) & (best[best] == ids) & (cost < _INF)
        nprop = int(valid.sum())
        rejected = torch.zeros(size, dtype=torch.bool)
        bound = None
        if self.limit is not None:
            rows = torch.nonzero(valid)[:, 0]
            other = best[rows]
            diff = self.mu[rows] - self.mu[other]
            exact2 = _dsum(diff * diff)
            exact = torch.sqrt(exact2)
            ma, mb = self.mass[rows], self.mass[other]
            denom = torch.clamp(ma + mb, min=1.0)
            verified = torch.maximum(self.radius[rows] + (mb / denom) * exact,
                                     self.radius[other] + (ma / denom) * exact)
            bad = verified > self.limit
            self.dist[rows[bad], other[bad]] = exact2[bad]
            self.dist[other[bad], rows[bad]] = exact2[bad]
            rejected[rows[bad]] = True
            rejected[other[bad]] = True
            valid[rows[bad]] = False
            bound = torch.zeros(size)
            bound[rows] = verified
        pair = torch.where(valid, cost, torch.full((), _INF))
        order = torch.sort(pair, stable=True).indices[:size // 2]
        ok = pair[order] < _INF
        ok &= torch.cumsum(ok.to(torch.int64), 0) <= self.count - self.target
        a = order[ok]
        b = best[a]
        keep = torch.zeros(size, dtype=torch.bool)
        merged = torch.zeros(size, dtype=torch.bool)
        if len(a):
            self._merge(a, b, bound, keep, merged)
        dirty = self.alive & ~keep & (merged[best] | rejected)
        rows = torch.nonzero(dirty)[:, 0]
        if len(rows):
            self.packed[rows] = self._scan(rows)
        self.count -= int(ok.sum())
        remaining = self.count > self.target
        if remaining and nprop == 0:
            self.stuck = True
        return remaining and nprop > 0

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
        partner = torch.zeros(size, dtype=torch.int64)
        partner[a] = b
        pma, pmb, pdab = torch.ones(size), torch.zeros(size), torch.zeros(size)
        pma[a], pmb[a], pdab[a] = ma, mb, dab
        self.mass[a] = total
        self.mass[b] = 0
        self.alive[b] = False
        if bound is not None:
            self.radius[a] = bound[a]
        self.mu[a] = (ma[:, None] * self.mu[a] + mb[:, None] * self.mu[b]) / torch.clamp(total, min=1.0)[:, None]
        al, be, sh = alpha[:, None], beta[:, None], shift[:, None]
        x_aa, x_ba = self.dist[a], self.dist[b]
        new = al * x_aa + be * x_ba - sh
        x_ab, x_bb = self.dist[a[:, None], partner[None, :]], self.dist[b[:, None], partner[None, :]]
        qalpha, qbeta = pma / (pma + pmb), pmb / (pma + pmb)
        qshift = qalpha * qbeta * pdab
        own_first = qalpha * new + qbeta * (al * x_ab + be * x_bb - sh) - qshift
        other_first = al * (qalpha * x_aa + qbeta * x_ab - qshift) + be * (qalpha * x_ba + qbeta * x_bb - qshift) - sh
        both = torch.where(a[:, None] < ids[None, :], own_first, other_first)
        new = torch.where(keep[None, :], both, new)
        new = torch.where(new < 0, torch.zeros(()), new)
        new[torch.arange(len(a)), a] = 0
        alive = self.alive
        cols = torch.nonzero(alive & ~keep)[:, 0]
        self.dist[cols[:, None], a[None, :]] = new[:, cols].T
        cols = torch.nonzero(alive)[:, 0]
        self.dist[a[:, None], cols[None, :]] = new[:, cols]
        lim = self.limit is not None
        cost, valid = _pair_cost(new, total[:, None], self.mass[None, :],
                                 self.radius[a][:, None] if lim else None, self.radius[None, :] if lim else None,
                                 self.limit, alive[None, :] & (ids[None, :] != a[:, None]))
        packed = _pack_key(cost, ids[None, :] ^ a[:, None])
        push = valid & ~keep[None, :]
        colmin = torch.where(push, packed, torch.full((), _I64_TOP, dtype=torch.int64)).min(0).values
        self.packed = torch.minimum(self.packed, colmin)
        self.packed[a] = packed.min(1).values
        self.trace.extend(zip(a.tolist(), b.tolist()))


def reduce(mu, mass, count, limit, target, strict=False, gram=False, passes=1):
    """``oracle.unified.reduce`` with ``TorchReducer``: (survivors, trace, centers) as numpy. ``gram``:
    initial distances in the reference's Gram form above 32 nodes (``gram_distances``), else the
    canonical differences. Frozen-center sweeps (``passes > 1``) are not restated here."""
    if passes > 1 and limit is None:
        raise NotImplementedError("the Torch-CPU reducer restates one matching pass per round")
    if count <= target:
        return np.arange(count), [], f32(mu).copy()
    mu_t = torch.from_numpy(np.ascontiguousarray(f32(mu)))
    dist = gram_distances(mu_t) if gram and count > 32 else pair_distances(mu_t)
    r = TorchReducer(dist, mu_t, torch.from_numpy(np.ascontiguousarray(f32(mass))), count, limit, target)
    size = r.mass.shape[0]
    for _ in range(2 * size + 7):
        if not r.step():
            break
    if strict and r.stuck:
        raise RuntimeError("unified route: no mutual pair below the cluster budget")
    return torch.nonzero(r.alive)[:, 0].numpy(), r.trace, r.mu.numpy()


def slot_attention(q: torch.Tensor, ka: torch.Tensor, va: torch.Tensor, scale: float, dv: int) -> torch.Tensor:
    """Attention of queries ``[Bt, Hq, Tq, Dk]`` over packed rows ``[Bt, G, S, dim]`` (keys with their
    bias column at Dk, values in the first ``dv`` columns) as the reference's Flash encoding is
    evaluated (litgpt/log_kv_cache.py:6418-6464, :6751-6758): the query extended by ``1/scale`` in bf16
    at column Dk, so the bias adds to the scaled scores, then ``scaled_dot_product_attention`` per KV
    group over its query heads, in float32. No causal mask: one decode query per head."""
    n_batch, hq, tq, dk = q.shape
    n_groups, total, dim = ka.shape[1], ka.shape[2], ka.shape[3]
    rep = hq // n_groups
    qa = torch.zeros(n_batch, n_groups, rep * tq, dim)
    qa[..., :dk] = q.float().reshape(n_batch, n_groups, rep * tq, dk)
    qa[..., dk] = torch.tensor(1.0 / scale, dtype=torch.float32).to(torch.bfloat16).float()
    out = torch.nn.functional.scaled_dot_product_attention(qa, ka, va[..., :dv], scale=scale)
    return out.reshape(n_batch, hq, tq, dv)


class TorchCpuCache(OracleCache):
    """``OracleCache`` whose commit appends every ladder of a flush together, level by level, with
    the Beta groups of a level batched, whose unified route reduces on torch tensors, and whose pack
    is batched tensor code (see the module docstring). Op-log recording keeps the oracle's
    per-cluster path."""

    # The unified route's initial distances: False, the canonical differences (bit-identical to the
    # oracle); True, the reference's Gram form (the CPU baseline's timing).
    gram_distances = False

    def pack(self, k_cur=None, v_cur=None):
        """``readout.pack`` (the reference's Torch packer, litgpt/log_kv_pack.py:27-72) as batched
        torch gathers and RoPE; the log-mass column keeps numpy's float32 log."""
        dk, dv = self.dk, self.dv
        dim = readout.packed_dim(dk, dv)
        idx, anchors, valid = self.plan()
        pooled, exact, recent = idx.shape[-1], self.alpha_count, self.recent_count
        cur = 0 if k_cur is None else k_cur.shape[2]
        n_batch, n_groups = self.batch, self.groups
        ka = torch.zeros(n_batch, n_groups, pooled + exact + recent + cur, dim)
        va = torch.zeros_like(ka)
        cos, sin = torch.from_numpy(f32(self.cos)), torch.from_numpy(f32(self.sin))
        neg = float(bf16_round(np.float32(-10000.0)).reshape(-1)[0])
        if pooled:
            ti = torch.from_numpy(idx)
            kk = torch.from_numpy(self.level_k.reshape(n_batch, n_groups, -1, dk))
            vv = torch.from_numpy(self.level_v.reshape(n_batch, n_groups, -1, dv))
            kk = torch.gather(kk, 2, ti[..., None].expand(-1, -1, -1, dk))
            vv = torch.gather(vv, 2, ti[..., None].expand(-1, -1, -1, dv))
            ww = np.take_along_axis(self.level_w.reshape(n_batch, n_groups, -1), idx, axis=2)
            tv = torch.from_numpy(valid)
            keys = _rope(kk, torch.from_numpy(anchors), cos, sin, self.table_bf16)
            ka[:, :, :pooled, :dk] = torch.where(tv[..., None], keys, torch.zeros(()))
            va[:, :, :pooled, :dv] = torch.where(tv[..., None], vv, torch.zeros(()))
            bias = torch.from_numpy(bf16_round(np.log(np.maximum(ww, np.float32(1.0))).astype(np.float32)))
            ka[:, :, :pooled, dk] = torch.where(tv, bias, torch.full((), neg))
        if exact:
            ev = torch.from_numpy(np.ascontiguousarray(np.broadcast_to(self.alpha_valid[:, None, :exact],
                                                                       (n_batch, n_groups, exact))))
            ea = torch.from_numpy(np.ascontiguousarray(np.broadcast_to(self.alpha_pos[:, None, :exact],
                                                                       (n_batch, n_groups, exact))))
            keys = _rope(torch.from_numpy(f32(self.alpha_k_raw[:, :, :exact])), torch.where(ev, ea, 0), cos, sin,
                         self.table_bf16)
            ka[:, :, pooled:pooled + exact, :dk] = torch.where(ev[..., None], keys, torch.zeros(()))
            va[:, :, pooled:pooled + exact, :dv] = torch.where(ev[..., None],
                                                               torch.from_numpy(f32(self.alpha_v[:, :, :exact])),
                                                               torch.zeros(()))
            ka[:, :, pooled:pooled + exact, dk] = torch.where(ev, torch.zeros(()), torch.full((), neg))
        p = pooled + exact
        ka[:, :, p:p + recent, :dk] = torch.from_numpy(f32(self.recent_k[:, :, :recent]))
        va[:, :, p:p + recent, :dv] = torch.from_numpy(f32(self.recent_v[:, :, :recent]))
        if cur:
            ka[:, :, p + recent:, :dk] = torch.from_numpy(f32(k_cur))
            va[:, :, p + recent:, :dv] = torch.from_numpy(f32(v_cur))
        return ka.numpy(), va.numpy()

    def route_and_commit(self, ak, av, ap, counts):
        if self.op_log is not None:
            return super().route_and_commit(ak, av, ap, counts)
        if self.unified:
            fn = (lambda *a, **k: reduce(*a, gram=True, **k)) if self.gram_distances else reduce
            jobs, out = unified.unified_jobs(self, ak, ap, counts, reduce_fn=fn)
            self._commit(jobs, f32(ak), f32(av), ap)
            return out
        assign, order = attach_assign_batched(ak, ap, counts, self.centroid, self.alive, self.p_hi_c, self.s_h,
                                              self.eta, self.g0, self.lam)
        jobs = route.commit_jobs(assign, order, counts, self.alive)
        self._commit(jobs, ak, av, ap)
        return assign, order

    def _commit(self, jobs, ak, av, ap):
        """Stage every job's rows (opened clusters, delayed archives, joins: the oracle's per-cluster
        rules, centers in position order), then append all of them together level by level."""
        lanes, staged = [], []
        for (b, g, c), (new, rows) in sorted(jobs.items()):
            parts = []
            if new:
                t = rows[0]
                self.ladder(b, g, c).clear()
                self.centroid[b, g, c] = f32(ak[b, g, t])
                self.n_eff[b, g, c] = 1.0
                self.alive[b, g, c] = True
                self.n_total[b, g, c] = 1
                self.p_hi_c[b, g, c] = int(ap[b, t])
                self.level0_phase[b, g, c] = 1
                parts.append(self._token_rows(ak[b, g, t][None], av[b, g, t][None],
                                              np.asarray([ap[b, t]], np.int64), 0))
                rows = rows[1:]
            if len(rows):
                keys, values = ak[b, g, rows], av[b, g, rows]
                pos = ap[b, rows].astype(np.int64)
                if self.P and pos.min() < self.p_hi_c[b, g, c]:
                    self.late_joins += 1
                    ladder = self.ladder(b, g, c)
                    combined = lad.concat([ladder.entries(), self._token_rows(keys, values, pos, 0)])
                    sort = np.argsort(combined["p_lo"], kind="stable")
                    rows_sorted = lad.take(combined, sort)
                    rows_sorted["order"] = np.arange(len(sort), dtype=np.int64)
                    self.centroid[b, g, c], self.n_eff[b, g, c] = lad.centroid_update(
                        self.centroid[b, g, c], self.n_eff[b, g, c], keys, tile=self.centroid_tile)
                    self.p_hi_c[b, g, c] = max(int(self.p_hi_c[b, g, c]), int(pos.max()))
                    self.n_total[b, g, c] += len(pos)
                    self.level0_phase[b, g, c] = len(sort)
                    self.alive[b, g, c] = True
                    ladder.clear()
                    parts = [rows_sorted]
                else:
                    phase = int(self.level0_phase[b, g, c])
                    parts.append(self._token_rows(keys, values, pos, phase))
                    self.centroid[b, g, c], self.n_eff[b, g, c] = lad.centroid_update(
                        self.centroid[b, g, c], self.n_eff[b, g, c], keys, tile=self.centroid_tile)
                    self.level0_phase[b, g, c] = phase + len(pos)
                    self.p_hi_c[b, g, c] = pos[-1]
                    self.n_total[b, g, c] += len(pos)
            if parts:
                lanes.append((b, g, c))
                staged.append(parts[0] if len(parts) == 1 else lad.concat(parts))
        self._append_many(lanes, staged)

    def _append_many(self, lanes, staged):
        """``Ladder.append`` of ``staged[i]`` into ladder ``lanes[i]`` for every i, one level at a time
        for all of them (the pairs / Beta groups of a level in one batched call)."""
        B, L = self.B, self.L
        views = [self.ladder(*lane) for lane in lanes]
        active = [i for i in range(len(lanes)) if len(staged[i]["w"])]
        # Staged rows are rounded once here; carries are rounded when they are made, so every level
        # reads storage-rounded rows as the oracle's per-level rounding does.
        stage = {i: _storage(staged[i]) for i in active}
        for ell in range(L):
            if not active:
                return
            top = ell == L - 1
            pools, pair_ids, carry_lens = {}, [], []
            for i in active:
                ladder, st = views[i], stage[i]
                m = len(st["w"])
                filled = int(ladder.count[ell])
                take_n = min(B - filled, m)
                if take_n:
                    ladder._write(ell, filled, lad.take(st, slice(0, take_n)))
                filled += take_n
                mr = m - take_n
                if mr == 0:
                    ladder.count[ell] = filled
                    continue
                pool = lad.concat([lad.take(ladder.rows, ladder.level(ell)), lad.take(st, slice(take_n, m))])
                if top:
                    acc = lad.take(pool, slice(0, 1))
                    for t in range(1, mr + 1):
                        acc = lad.to_storage(lad.pair_merge(acc, lad.take(pool, slice(t, t + 1))))
                    ladder._write(ell, 0, acc)
                    ladder._write(ell, 1, lad.take(pool, slice(mr + 1, mr + B)))
                    ladder.count[ell] = B
                    continue
                n_pair = 2 * ((mr + 1) // 2)
                pools[i] = (pool, n_pair, mr)
                pair_ids.append(i)
                carry_lens.append(n_pair)
            if not pair_ids:
                return
            pairs = lad.concat([lad.take(pools[i][0], slice(0, pools[i][1])) for i in pair_ids])
            if self.beta_adaptive:
                carries, cuts = beta_merge_batched(pairs, carry_lens)
                carries = _storage(carries)
                groups = [(n + 3) // 4 for n in carry_lens]
                offs = np.concatenate(([0], np.cumsum(groups)))
                for j, i in enumerate(pair_ids):
                    self.beta_cuts.append((lanes[i], [(ell, cuts[offs[j]:offs[j + 1]])]))
            else:
                carries = _storage(lad.merge_pairs(pairs))
            off = 0
            next_active = []
            for i in pair_ids:
                pool, n_pair, mr = pools[i]
                ladder = views[i]
                lvl = ladder.level(ell)
                for f in lad.FIELDS:
                    ladder.rows[f][lvl] = 0
                ladder._write(ell, 0, lad.take(pool, slice(n_pair, B + mr)))
                ladder.count[ell] = B + mr - n_pair
                n_carry = n_pair // 2
                stage[i] = lad.take(carries, slice(off, off + n_carry))
                off += n_carry
                next_active.append(i)
            active = next_active
