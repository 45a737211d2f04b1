"""Per-cluster ladder: pair merges, Beta 4->2 merges, Fenwick append, top-level fold.

TEST INFRASTRUCTURE ONLY (the oracle). One ladder is the ``[L, B']`` block of
entries of one (batch row, KV group, cluster). An entry has eight fields
(litgpt/log_kv_updates_triton.py:12): key and value payload (bf16 storage,
float32 math), mass ``w`` (float32), ``p_lo``/``p_hi``/``sum_wp``/``order``
(int64) and ``pad`` (bool).

Rules restated:
* pair merge ``alpha = wa / max(wa + wb, 1e-8)``, payload ``alpha*a + (1-alpha)*b``,
  anchors over real (w > 0) members only, ``order = min``, ``pad = and``
  (litgpt/log_kv_cache.py:5217-5312, litgpt/log_kv_position.py:13-30,
  litgpt/log_kv_updates_triton.py:37-57);
* Beta: per four consecutive carry rows choose the cut in (2, 1, 3) with the
  lowest normalised K/V distortion (ties keep the earlier option), two-row
  tails use cut 1; outputs are ``sum w x / max(sum w, 1e-12)``
  (litgpt/beta_log_kv.py:7-105);
* Fenwick append: fill the free slots of a level, then the oldest
  ``2*ceil(m/2)`` rows of ``[stored | staged]`` pair into carries for the next
  level, survivors move to slots ``[0, n_surv)`` and the rest are cleared
  (litgpt/log_kv_cache.py:1815-1929);
* saturated top level: slot 0 becomes the left fold of ``S[0..m]`` (rounded to
  storage after every step) and slots ``1..B'-1`` take ``S[m+1..m+B'-1]``
  (litgpt/log_kv_cache.py:1670-1728);
* carries stay float32 until the next level reads them, which rounds them to
  the storage dtype (litgpt/log_kv_updates_triton.py:16-23).

Feature sums in the Beta costs use ``numerics.dsum``; sums over the four rows
run in row order. The cost accumulation order follows the Torch reference:
K left, K right, V left, V right (litgpt/beta_log_kv.py:29-46).
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_round, dsum, f32

FIELDS = ("k", "v", "w", "p_lo", "p_hi", "sum_wp", "order", "pad")
I64_MAX = np.iinfo(np.int64).max
I64_MIN = np.iinfo(np.int64).min


def empty_rows(n: int, dk: int, dv: int) -> dict:
    return {
        "k": np.zeros((n, dk), np.float32), "v": np.zeros((n, dv), np.float32),
        "w": np.zeros(n, np.float32), "p_lo": np.zeros(n, np.int64), "p_hi": np.zeros(n, np.int64),
        "sum_wp": np.zeros(n, np.int64), "order": np.zeros(n, np.int64), "pad": np.zeros(n, bool),
    }


def take(rows: dict, index) -> dict:
    return {f: rows[f][index] for f in FIELDS}


def concat(parts) -> dict:
    return {f: np.concatenate([p[f] for p in parts], axis=0) for f in FIELDS}


def to_storage(rows: dict) -> dict:
    """Round payload to bf16 storage (what every read of a staged carry does)."""
    out = dict(rows)
    out["k"] = bf16_round(rows["k"])
    out["v"] = bf16_round(rows["v"])
    return out


def pair_merge(a: dict, b: dict) -> dict:
    """Merge row i of ``a`` with row i of ``b`` (a older). Payload stays float32."""
    wa, wb = f32(a["w"]), f32(b["w"])
    alpha = wa / np.maximum(wa + wb, np.float32(1e-8))
    al = alpha[:, None]
    k = al * f32(a["k"]) + (np.float32(1.0) - al) * f32(b["k"])
    v = al * f32(a["v"]) + (np.float32(1.0) - al) * f32(b["v"])
    ra, rb = wa > 0, wb > 0
    both = ra & rb
    lo = np.where(both, np.minimum(a["p_lo"], b["p_lo"]), np.where(ra, a["p_lo"], b["p_lo"]))
    hi = np.where(both, np.maximum(a["p_hi"], b["p_hi"]), np.where(ra, a["p_hi"], b["p_hi"]))
    return {
        "k": k, "v": v, "w": wa + wb, "p_lo": lo.astype(np.int64), "p_hi": hi.astype(np.int64),
        "sum_wp": (a["sum_wp"] + b["sum_wp"]).astype(np.int64),
        "order": np.minimum(a["order"], b["order"]).astype(np.int64), "pad": a["pad"] & b["pad"],
    }


def merge_pairs(rows: dict) -> dict:
    """Pairs (0,1), (2,3), ... of an even-length block."""
    n = len(rows["w"]) // 2
    return pair_merge(take(rows, slice(0, 2 * n, 2)), take(rows, slice(1, 2 * n, 2)))


def beta_layout(lengths) -> np.ndarray:
    """Rows ``(start, width, out_start)`` of the 4-row groups of each even lane length."""
    out = []
    start = 0
    for n in lengths:
        n = int(n)
        if n < 0 or n % 2:
            raise ValueError("Beta compaction requires even nonnegative lane lengths")
        for off in range(0, n, 4):
            out.append((start + off, min(4, n - off), (start + off) // 2))
        start += n
    return np.asarray(out, dtype=np.int64).reshape(-1, 3)


def _side_mean(x, weights):
    """sum_i x_i * w_i (row order) / max(sum_i w_i, 1e-12) for four rows."""
    acc = x[0] * weights[0]
    for i in range(1, 4):
        acc = acc + x[i] * weights[i]
    mass = weights[0]
    for i in range(1, 4):
        mass = mass + weights[i]
    return acc / np.maximum(mass, np.float32(1e-12)), mass


def beta_select_cut(k4, v4, w4, width) -> int:
    """Cut of one group (rows already float32; ``w4`` zero past ``width``)."""
    if width == 2:
        return 1
    w = f32(w4)
    total = np.maximum(w[0] + w[1] + w[2] + w[3], np.float32(1e-12))
    costs = [np.float32(0.0)] * 3
    for x in (f32(k4), f32(v4)):
        sq = dsum(x * x)                                  # [4]
        e = sq[0] * w[0]
        for i in range(1, 4):
            e = e + sq[i] * w[i]
        energy = np.maximum(e / total, np.float32(1e-12))
        for j, cut in enumerate((2, 1, 3)):
            for side in (0, 1):
                mask = (np.arange(4) < cut) if side == 0 else (np.arange(4) >= cut)
                weights = np.where(mask, w, np.float32(0.0)).astype(np.float32)
                mean, _ = _side_mean(x, weights)
                d = x - mean[None, :]
                per = dsum(d * d)
                loss = per[0] * weights[0]
                for i in range(1, 4):
                    loss = loss + per[i] * weights[i]
                costs[j] = np.float32(costs[j] + loss / energy)
    best = 0
    for j in (1, 2):
        if costs[j] < costs[best]:
            best = j
    return (2, 1, 3)[best]


def beta_apply(rows4: dict, width: int, cut: int):
    """Two output rows (left, right) of one group; right is None for a 2-row tail."""
    w = np.zeros(4, np.float32)
    w[:width] = rows4["w"][:width]
    k = np.zeros((4, rows4["k"].shape[1]), np.float32)
    v = np.zeros((4, rows4["v"].shape[1]), np.float32)
    k[:width], v[:width] = rows4["k"][:width], rows4["v"][:width]
    valid = np.arange(4) < width
    outs = []
    for side in (0, 1):
        if side == 1 and width == 2:
            outs.append(None)
            continue
        if width == 2:
            mask = valid.copy()
        else:
            mask = valid & ((np.arange(4) < cut) if side == 0 else (np.arange(4) >= cut))
        weights = np.where(mask, w, np.float32(0.0)).astype(np.float32)
        ko, mass = _side_mean(k, weights)
        vo, _ = _side_mean(v, weights)
        idx = np.arange(width)
        m = mask[:width]
        live = m & (rows4["w"][:width] > 0)
        lo = rows4["p_lo"][idx][live].min() if live.any() else I64_MAX
        hi = rows4["p_hi"][idx][live].max() if live.any() else I64_MIN
        outs.append({
            "k": ko, "v": vo, "w": np.float32(mass),
            "p_lo": np.int64(lo if mass > 0 else 0), "p_hi": np.int64(hi if mass > 0 else 0),
            "sum_wp": np.int64(rows4["sum_wp"][idx][m].sum()),
            "order": np.int64(rows4["order"][idx][m].min() if m.any() else I64_MAX),
            "pad": bool(rows4["pad"][idx][m].all()),
        })
    return outs


def beta_merge(rows: dict, lengths, cuts=None):
    """Beta merge of concatenated even-length lanes; returns (carries, cuts uint8)."""
    layout = beta_layout(lengths)
    n_out = len(rows["w"]) // 2
    out = empty_rows(n_out, rows["k"].shape[1], rows["v"].shape[1])
    chosen = np.zeros(len(layout), np.uint8)
    for gi, (start, width, dest) in enumerate(layout):
        rows4 = take(rows, slice(start, start + width))
        if cuts is None:
            k4 = np.zeros((4, rows["k"].shape[1]), np.float32)
            v4 = np.zeros((4, rows["v"].shape[1]), np.float32)
            w4 = np.zeros(4, np.float32)
            k4[:width], v4[:width], w4[:width] = rows4["k"], rows4["v"], rows4["w"]
            cut = beta_select_cut(k4, v4, w4, width)
        else:
            cut = int(cuts[gi])
        chosen[gi] = cut
        for side, row in enumerate(beta_apply(rows4, width, cut)):
            if row is None:
                continue
            for f in FIELDS:
                out[f][dest + side] = row[f]
    return out, chosen


class Ladder:
    """View of one cluster's ladder: ``rows[f]`` are ``[L*B']`` views, ``count`` is ``[L]``."""

    def __init__(self, rows: dict, count: np.ndarray, levels: int, slots: int):
        self.L, self.B = levels, slots
        self.rows = rows
        self.count = count

    def clear(self):
        """Every field zeroed (p_lo and p_hi included) and counts reset
        (litgpt/log_kv_cache.py:2476-2492)."""
        for f in FIELDS:
            self.rows[f][...] = 0
        self.count[:] = 0

    def level(self, ell):
        return slice(ell * self.B, (ell + 1) * self.B)

    def _write(self, ell, slot0, rows):
        n = len(rows["w"])
        base = ell * self.B + slot0
        for f in FIELDS:
            self.rows[f][base:base + n] = rows[f]

    def append(self, staged: dict, beta: bool = False) -> list:
        """Fenwick-append ``staged`` rows (payload rounded to storage first).

        Returns the Beta cuts chosen per level (empty lists without Beta).
        """
        cuts_log = []
        stage = staged
        m = len(stage["w"])
        B = self.B
        for ell in range(self.L):
            if m == 0:
                break
            stage = to_storage(stage)
            top = ell == self.L - 1
            filled = int(self.count[ell])
            take_n = min(B - filled, m)
            if take_n:
                self._write(ell, filled, take(stage, slice(0, take_n)))
            filled += take_n
            rest = take(stage, slice(take_n, m))
            mr = m - take_n
            if mr == 0:
                self.count[ell] = filled
                break
            stored = take(self.rows, self.level(ell))
            pool = concat([stored, rest])
            if top:
                acc = take(pool, slice(0, 1))
                for t in range(1, mr + 1):
                    acc = to_storage(pair_merge(acc, take(pool, slice(t, t + 1))))
                self._write(ell, 0, acc)
                self._write(ell, 1, take(pool, slice(mr + 1, mr + B)))
                self.count[ell] = B
                break
            carry_n = (mr + 1) // 2
            n_pair = 2 * carry_n
            pairs = take(pool, slice(0, n_pair))
            if beta:
                carry, cuts = beta_merge(pairs, [n_pair])
                cuts_log.append((ell, cuts))
            else:
                carry = merge_pairs(pairs)
            n_surv = B + mr - n_pair
            survivors = take(pool, slice(n_pair, B + mr))
            lvl = self.level(ell)
            for f in FIELDS:
                self.rows[f][lvl] = 0
            self._write(ell, 0, survivors)
            self.count[ell] = n_surv
            stage = carry
            m = carry_n
        return cuts_log

    def entries(self) -> dict:
        """Occupied entries level by level, slots in order (the late-archive gather)."""
        idx = np.concatenate([np.arange(ell * self.B, ell * self.B + self.count[ell]) for ell in range(self.L)])
        return take(self.rows, idx.astype(np.int64))


def tiled_sum(keys, tile: int):
    """Row sum of ``keys`` in position-ordered tiles of ``tile`` rows: each tile (zeros past the
    last row) summed by a halving tree (row i with row i + tile/2, then + tile/4, ...), the tile
    sums added in order (the "parallel" centroid backend, litgpt/log_kv_updates_triton.py:236-241)."""
    keys = f32(keys)
    acc = None
    for t0 in range(0, len(keys), tile):
        x = np.zeros((tile, keys.shape[1]), np.float32)
        part = keys[t0:t0 + tile]
        x[:len(part)] = part
        h = tile // 2
        while h >= 1:
            x[:h] = x[:h] + x[h:2 * h]
            h //= 2
        acc = x[0].copy() if acc is None else np.float32(acc + x[0])
    return acc


def centroid_update(mu, n_eff, keys, forget: float = 1.0, tile: int = 1):
    """Ordered run update ``mu <- (pre*mu + sum k) / (pre + n)``, ``pre = n_eff*forget``
    (litgpt/log_kv_cache.py:4344-4359); keys summed one row at a time in row order, or with
    ``tile`` > 1 by ``tiled_sum``."""
    keys = f32(keys)
    n = np.float32(len(keys))
    acc = np.add.accumulate(keys, axis=0, dtype=np.float32)[-1] if tile == 1 else tiled_sum(keys, tile)
    pre = np.float32(n_eff) * np.float32(forget)
    denom = np.float32(pre + n)
    if pre > 0:
        mu = (pre * f32(mu) + acc) / denom
    else:
        mu = acc / n
    return mu.astype(np.float32), denom
