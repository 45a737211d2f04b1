"""Deferred, stacked flushes of a model's per-layer caches.

litgpt/model.py keeps one LogStructuredKVCache per layer and calls its
``add_recent`` once per layer and block (litgpt/model.py:1252-1340). A layer's
flush is a few dozen launches over 8 lanes, bound by launch latency rather than
by the GPU; every kernel is independent across batch rows, so the 28 layers'
flushes can run as one launch sequence over their stacked rows at the cost of
about one.

Caches built with the same configuration on one device form a flush group.
When a member first has a flush to run, the group moves every member's state
into the batch rows of one hidden owner cache (member ``l`` owns rows
``[l * Bt, (l + 1) * Bt)``) and each member's state buffers become views of its
rows. From then on a member's ``add_recent`` appends its rows and leaves the
flush pending, with its host counters advanced as if the flush had run; the
first read of a pending member's state (any reader of the cache, a state
buffer's attribute, the next ``add_recent``) runs every pending flush of the
group: one flush of the owner when every member is pending with the same
length and the same route parameters, otherwise each pending member's own
flush. Either way each member's rows end exactly as its own flush leaves them.

Flushes that record or replay an op-log or an update tape, and caches with a
side stream (``flush_stream``), are never deferred. ``set_flush_grouping``
turns grouping off for caches built afterwards.
"""

from __future__ import annotations

import contextlib
import weakref

import torch

# Member buffers that become views of the owner's rows (the whole flush and readout state).
STATE = (
    "recent_k", "recent_v", "recent_k_raw", "recent_pos", "recent_span_ends",
    "alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid", "alpha_span_len", "alpha_span_closed", "alpha_span_count",
    "level_k", "level_v", "level_w", "level_imp", "level_count", "pad_mask", "level_p_lo", "level_p_hi",
    "level_sum_wp", "level_order", "centroid", "n_eff", "n_total", "p_hi_c", "current_segment", "level0_phase",
    "alive", "s_h", "_unified_limits", "alpha_count_dev",
)
STATE_SET = frozenset(STATE)
# The exact pool's buffer set, which the owner swaps with its spare set at every Alpha flush.
ALPHA_SET = ("alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid", "alpha_span_len", "alpha_span_closed",
             "alpha_span_count")

_enabled = True
_open: dict = {}          # configuration key -> the group new caches join (not yet adopted)
_building_owner = False


def set_flush_grouping(enabled: bool) -> None:
    """Group caches built from now on (True, the default) or keep every cache's flushes immediate."""
    global _enabled
    _enabled = bool(enabled)


def flush_grouping() -> bool:
    return _enabled


def register(cache) -> None:
    """Called by every cache's constructor: join the open group of its configuration."""
    if not _enabled or _building_owner or cache.level_k.device.type != "cuda":
        return
    key = cache._group_key()
    group = _open.get(key)
    if group is None:
        group = _open[key] = FlushGroup(key)
    group.refs.append(weakref.ref(cache))
    cache._group = group


@contextlib.contextmanager
def _owner_construction():
    global _building_owner
    _building_owner = True
    try:
        yield
    finally:
        _building_owner = False


def _alpha_sets(cache):
    current = (cache.alpha_k_raw, cache.alpha_v, cache.alpha_pos, cache.alpha_valid, cache.alpha_span_len,
               cache.alpha_span_closed, cache.alpha_span_count)
    return current, cache._alpha_spare


class FlushGroup:
    """The members of one configuration and, once adopted, the owner cache whose rows they view."""

    def __init__(self, key):
        self.key = key
        self.refs = []          # weak references to the members, in registration order
        self.owner = None
        self.rows = 0           # batch rows per member
        self.broken = False     # a member left the stacked storage: no more stacked flushes
        self.stacked_runs = 0   # flushes run as one owner flush
        self.member_runs = 0    # flushes run by a member itself

    def members(self):
        return [m for m in (r() for r in self.refs) if m is not None]

    # ------------------------------------------------------------------
    def adopt(self) -> bool:
        """Move the live members' state into one owner cache (once); False when fewer than two live."""
        if self.broken:
            return False
        if self.owner is not None:
            return True
        members = self.members()
        if len(members) < 2:
            return False
        if _open.get(self.key) is self:
            del _open[self.key]          # later caches of this configuration start a new group
        for m in members:
            m._await_flush()
        first = members[0]
        bt = first.batch_size
        kw = dict(first._init_kwargs)
        k_shape, v_shape = list(kw["k_shape"]), list(kw["v_shape"])
        k_shape[0] = v_shape[0] = bt * len(members)
        kw.update(k_shape=tuple(k_shape), v_shape=tuple(v_shape), semantic_s_h=None)
        with _owner_construction():
            from .log_kv_cache import LogStructuredKVCache
            owner = LogStructuredKVCache(**kw)
        owner._group = None
        if owner.alpha_exact_tokens:
            owner.register_buffer("alpha_count_dev", torch.zeros(len(members), dtype=torch.int32,
                                                                 device=owner.level_k.device), persistent=False)
            owner._alpha_count_rows = bt
        lanes = bt * first.n_groups
        with torch.no_grad():
            for i, m in enumerate(members):
                for name in STATE:
                    src = m._buffers.get(name)
                    if src is not None:
                        self._slice(owner._buffers[name], name, i, bt, lanes).copy_(src)
                if owner.alpha_exact_tokens:
                    for dst, src in zip(owner._alpha_spare, m._alpha_spare):
                        dst[i * bt:(i + 1) * bt].copy_(src)
        self.owner, self.rows = owner, bt
        for i, m in enumerate(members):
            self._point(m, i)
        self.refs = [weakref.ref(m) for m in members]
        return True

    @staticmethod
    def _slice(t, name, i, bt, lanes):
        if name == "alpha_count_dev":
            return t[i:i + 1]
        if name == "_unified_limits":
            return t[i * lanes:(i + 1) * lanes]
        return t[i * bt:(i + 1) * bt]

    def _point(self, m, i, fresh=True):
        """Member ``i``'s state buffers as views of its owner rows (the owner's current exact-pool set).
        ``fresh``: the member's cached argument structs are dropped (they held its own buffers); after
        a flush they stay, since a member's exact-pool parity always names the same owner set."""
        owner, bt = self.owner, self.rows
        lanes = bt * m.n_groups
        for name in STATE:
            if name in m._buffers:
                m._buffers[name] = self._slice(owner._buffers[name], name, i, bt, lanes)
        if owner.alpha_exact_tokens:
            m._alpha_spare = tuple(t[i * bt:(i + 1) * bt] for t in owner._alpha_spare)
            m._alpha_parity = owner._alpha_parity
        m._group_index = i
        if fresh:
            m._views = {}
        m._mid_decode_state = None

    def _swap_alpha(self, m):
        """After a stacked Alpha flush only the exact-pool set changed (the owner swapped its two
        sets): member ``m`` takes its views of the owner's current set, built once per set."""
        owner, i, bt = self.owner, m._group_index, self.rows
        cur = owner._buffers["alpha_k_raw"]
        cache = m.__dict__.setdefault("_alpha_view_sets", {})
        hit = cache.get(owner._alpha_parity)
        if hit is None or hit[0] is not cur:
            views = {name: owner._buffers[name][i * bt:(i + 1) * bt] for name in ALPHA_SET if name in m._buffers}
            spare = tuple(t[i * bt:(i + 1) * bt] for t in owner._alpha_spare)
            hit = cache[owner._alpha_parity] = (cur, views, spare)
        m._buffers.update(hit[1])
        d = m.__dict__
        d["_alpha_spare"] = hit[2]
        d["_alpha_parity"] = owner._alpha_parity
        d["_mid_decode_state"] = None

    def _realign(self, m):
        """After a member's own Alpha flushes left its exact pool in the other buffer set, copy it back
        into the owner's current set, so the member's rows and the owner's current set agree again."""
        owner = self.owner
        if not owner.alpha_exact_tokens or m._alpha_parity == owner._alpha_parity:
            return
        i, bt = m._group_index, self.rows
        current, _ = _alpha_sets(m)
        owner_current, _ = _alpha_sets(owner)
        with torch.no_grad():
            for dst, src in zip(owner_current, current):
                dst[i * bt:(i + 1) * bt].copy_(src)
        self._point(m, i, fresh=False)

    def leave(self, m):
        """``m`` leaves the group (its buffers moved): pending flushes run first; an adopted group then
        runs every later flush per member."""
        self.run()
        if self.owner is not None:
            self.broken = True
        self.refs = [r for r in self.refs if r() is not None and r() is not m]
        m._group = None

    # ------------------------------------------------------------------
    def _stackable(self, members, pend):
        owner = self.owner
        if self.broken or owner is None or len(pend) != len(members) or len(self.refs) != len(members):
            return False
        first = pend[0]._pending
        params = tuple(getattr(owner._params, f) for f, _ in owner._params._fields_)
        for m in pend:
            if m._pending != first or m._alpha_parity != owner._alpha_parity or m._group is not self:
                return False
            if tuple(getattr(m._params, f) for f, _ in m._params._fields_) != params:
                return False
        return True

    def run(self) -> None:
        """Run every pending flush of the group (see the module docstring)."""
        members = self.members()
        pend = [m for m in members if m._pending is not None]
        if not pend:
            return
        stacked = self._stackable(members, pend)
        jobs = [(m, m._pending) for m in pend]
        for m in pend:
            m._pending = None
        if stacked:
            take, count = jobs[0][1]
            owner = self.owner
            owner.recent_count = count
            owner._semantic_flush_tokens(take)
            self.stacked_runs += 1
            if owner.alpha_exact_tokens:
                for m in members:
                    self._swap_alpha(m)
            return
        for m, (take, count) in jobs:
            m.recent_count = count
            m._semantic_flush_tokens(take)
            self.member_runs += 1
            if self.owner is not None and m._group is self:
                self._realign(m)
