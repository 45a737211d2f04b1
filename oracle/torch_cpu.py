"""A batched Torch-CPU flush: the CPU baseline's implementation of one layer's flush.

TEST INFRASTRUCTURE ONLY: ``bench.py``'s ``cpu_baseline`` leg times it and tests/test_torch_cpu.py
checks it; the product package never imports it.

The oracle (``oracle.cache.OracleCache``) walks ladders and Beta groups one at a time, which is
what makes it a readable checker and a slow baseline. The reference's CPU path instead schedules
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
"""

from __future__ import annotations

import numpy as np
import torch

from . import ladder as lad
from . import readout, route
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


class TorchCpuCache(OracleCache):
    """``OracleCache`` whose attach-route commit appends every ladder of a flush together, level by
    level, with the Beta groups of a level batched, and whose pack is batched tensor code (see the
    module docstring). Unified-route flushes and op-log recording keep the oracle's per-cluster path."""

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
        if self.unified or self.op_log is not None:
            return super().route_and_commit(ak, av, ap, counts)
        assign, order = attach_assign_batched(ak, ap, counts, self.centroid, self.alive, self.p_hi_c, self.s_h,
                                              self.eta, self.g0, self.lam)
        jobs = route.commit_jobs(assign, order, counts, self.alive)
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
        return assign, order

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
