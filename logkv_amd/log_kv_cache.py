"""LogStructuredKVCache for MI355X: the SemanticLogKV flush path on HIP kernels.

Drop-in for the reference class (litgpt/log_kv_cache.py:640) on the path the
current configurations use: semantic clusters (K > 1), attach routing, mid
anchors, first-order entries, optional Alpha exact spans and Beta. The
constructor keeps the reference signature (litgpt/log_kv_cache.py:681-720);
options outside that path raise NotImplementedError instead of silently
changing behaviour.

Design: the cache state lives on the device in the reference's buffer layout,
and a flush is a fixed sequence of kernels (position order, attach decisions,
seeds, per-ladder commit) with no host planning and no device-to-host
readback. The reference's host mirrors (``_semantic_counts`` ...) are
read-only properties that copy from the device when asked.
"""

from __future__ import annotations

import contextlib
import ctypes as C
import math
from typing import NamedTuple

import torch
import torch.nn as nn

from . import _lib
from . import flush_group as _flush_group
from ._lib import LadderView, RouteParams, RowsView, check, lib, ptr, require_device, stream_of

# Rows per tile of a center's new-key sum, by semantic_centroid_backend.
_CENTER_TILES = {"sequential": 1, "parallel": 32}


class CacheAttentionState(NamedTuple):
    """Unpacked attention slots of a cache (litgpt/log_kv_cache.py:151-161): keys, values and masses
    ``[B, G, S(, d)]``, validity and anchor counts of the pooled (+ exact) prefix, and the rank-1
    statistics (always None here: first-order entries only)."""
    slot_k: torch.Tensor
    slot_v: torch.Tensor
    slot_w: torch.Tensor
    slot_valid: torch.Tensor | None = None
    M_s: torch.Tensor | None = None
    slot_sigma_u: torch.Tensor | None = None
    slot_sigma2: torch.Tensor | None = None
    slot_gamma_a: torch.Tensor | None = None
    slot_gamma_b: torch.Tensor | None = None
    slot_gamma: torch.Tensor | None = None


def ladder_budget(batch_size, n_groups, max_seq_length, k_dim, v_dim, B, K, exact_tokens, element):
    """(B', L, budget bytes) of the Alpha-adjusted ladder (litgpt/log_kv_cache.py:857, :879-898)."""
    def levels(b):
        return max(2, math.ceil(math.log2(max_seq_length / max(K * b, 1) + 1.0)) + 2)

    L = levels(B)
    if not exact_tokens:
        return B, L, None
    packed = ((max(k_dim + 1, v_dim) + 7) // 8) * 8
    entry = (k_dim + v_dim + 2 * packed) * element + 41
    exact = exact_tokens * (n_groups * (k_dim + v_dim + 2 * packed) * element + 9)
    baseline = n_groups * K * L * (B * entry + 2)
    for cand in range(B - 1, 1, -1):
        lv = levels(cand)
        need = n_groups * K * lv * (cand * entry + 2) + exact
        if need <= baseline:
            return cand, lv, (batch_size * baseline, batch_size * need)
    raise ValueError("compressed ladder budget is too small for alpha_exact_tokens; increase B or reduce exact capacity")


class _SemanticReplayUpdates:
    """One training invocation's flush records, replayed without routing
    (litgpt/log_kv_cache.py:111-139).

    A record holds a flush's rows and its decisions as detached device
    tensors: the attach cluster of every row and the position order, and with
    Alpha the exact-pool selection (kept / archived rows, span state). A replay
    re-runs only the kernels that write the cache from those decisions, so the
    restored state is the recorded one bit for bit.
    """

    def __init__(self, flushes=None, tensors=None):
        self.flushes = {} if flushes is None else flushes
        self.tensors = [] if tensors is None else tensors

    def wait(self, device):
        if device.type == "cuda":
            stream = torch.cuda.current_stream(device)
            for record in self.flushes.values():
                if record[-1] is not None:
                    stream.wait_event(record[-1])

    def save(self, tensor, owned=False):
        """Keep ``tensor`` for replay (a copy unless the caller owns it outright); returns its index."""
        if tensor is None:
            return None
        self.tensors.append(tensor.detach() if owned else tensor.detach().clone())
        return len(self.tensors) - 1


class _SemanticReplayPlans:
    """Host-only replay state of one invocation (litgpt/log_kv_cache.py:97-108).

    Freezes the CPU op-log so later caller mutations cannot change it, and
    remembers the flush positions seen at each replay cursor, so a replay with
    different positions at the same cursor is rejected. The log itself is
    parsed on the device; this object holds no tensors and no cache reference.
    """

    def __init__(self, host_log):
        if host_log is None:
            raise RuntimeError("semantic replay plans require an existing CPU op-log")
        self.host_log = tuple(tuple(tuple(map(tuple, lane)) for lane in batch) for batch in host_log)
        self.plans = {}


class LogStructuredKVCache(nn.Module):
    """Semantic LogKV cache whose flush runs as HIP kernels on one MI355X.

    Buffers keep the reference names and shapes (litgpt/log_kv_cache.py:881-1121):
    ``level_{k,v}`` ``[Bt, G, K, L, B', D]`` bf16, ``level_w`` / ``level_imp`` f32,
    ``level_{p_lo,p_hi,sum_wp,order}`` i64, ``pad_mask`` bool, ``level_count`` i16
    ``[Bt, G, K, L]``, ``centroid`` f32 ``[Bt, G, K, D]``, ``n_eff`` f32,
    ``n_total`` i32, ``p_hi_c`` i64, ``level0_phase`` i32, ``alive`` bool
    ``[Bt, G, K]``, the recent window ``[Bt, G, 2*recent, D]`` and the exact pool.
    """

    def __init__(
        self,
        k_shape,
        v_shape,
        B: int = 512,
        recent_size: int = 0,
        device=None,
        dtype=None,
        importance_pooling: bool = False,
        importance_pooling_lambda: float = 1.0,
        importance_pooling_temperature: float = 1.0,
        semantic_clusters: bool = False,
        cluster_k_max: int = 1,
        cluster_lambda_rel: float = 1.0,
        seg_eta: float = 1.0,
        seg_g0: float = 2048.0,
        seg_gap_max: float | None = None,
        seg_block_level: int = 0,
        seg_forget: float = 0.5,
        semantic_s_h=None,
        semantic_flush_granularity: int = 2,
        semantic_cluster_chunk_size: int = 0,
        semantic_capacity_beta: float = 0.0,
        semantic_capacity_hard_cap_mult: float = 0.0,
        semantic_legacy_route: bool = False,
        semantic_unified_route: bool = False,
        semantic_merge_passes: int = 1,
        semantic_anchor_mode: str = "multi",
        semantic_pack_backend: str = "auto",
        semantic_centroid_backend: str = "sequential",
        semantic_replay_updates: bool = False,
        cos_cache: torch.Tensor | None = None,
        sin_cache: torch.Tensor | None = None,
        rope_n_elem: int | None = None,
        allocate_second_order: bool = True,
        alpha_exact_tokens: int = 0,
        alpha_span_max_tokens: int = 64,
        beta_novelty: bool = False,
        beta_adaptive_merge: bool = False,
    ) -> None:
        super().__init__()
        self._pending = None     # a deferred flush (its token count, the window's rows before it)
        self._group = None
        self._init_kwargs = dict(
            k_shape=tuple(k_shape), v_shape=tuple(v_shape), B=B, recent_size=recent_size, device=device, dtype=dtype,
            importance_pooling=importance_pooling, importance_pooling_lambda=importance_pooling_lambda,
            importance_pooling_temperature=importance_pooling_temperature, semantic_clusters=semantic_clusters,
            cluster_k_max=cluster_k_max, cluster_lambda_rel=cluster_lambda_rel, seg_eta=seg_eta, seg_g0=seg_g0,
            seg_gap_max=seg_gap_max, seg_block_level=seg_block_level, seg_forget=seg_forget,
            semantic_s_h=semantic_s_h, semantic_flush_granularity=semantic_flush_granularity,
            semantic_cluster_chunk_size=semantic_cluster_chunk_size, semantic_capacity_beta=semantic_capacity_beta,
            semantic_capacity_hard_cap_mult=semantic_capacity_hard_cap_mult,
            semantic_legacy_route=semantic_legacy_route, semantic_unified_route=semantic_unified_route,
            semantic_merge_passes=semantic_merge_passes, semantic_anchor_mode=semantic_anchor_mode,
            semantic_pack_backend=semantic_pack_backend, semantic_centroid_backend=semantic_centroid_backend,
            semantic_replay_updates=semantic_replay_updates, rope_n_elem=rope_n_elem,
            allocate_second_order=allocate_second_order, alpha_exact_tokens=alpha_exact_tokens,
            alpha_span_max_tokens=alpha_span_max_tokens, beta_novelty=beta_novelty,
            beta_adaptive_merge=beta_adaptive_merge)
        batch_size, n_groups, max_seq_length, k_dim = k_shape
        v_dim = v_shape[-1]
        device = torch.device(device) if device is not None else torch.device("cuda")
        dtype = dtype or torch.bfloat16
        self.batch_size, self.n_groups, self.max_seq_length = batch_size, n_groups, max_seq_length
        self.k_dim, self.v_dim = k_dim, v_dim
        self.B = B
        self.semantic_clusters = bool(semantic_clusters)
        self.alpha_exact_tokens = int(alpha_exact_tokens)
        self.alpha_span_max_tokens = int(alpha_span_max_tokens)
        self.beta_novelty = bool(beta_novelty)
        self.beta_adaptive_merge = bool(beta_adaptive_merge)
        self.allocate_second_order = bool(allocate_second_order)
        # Validation with the reference's messages (litgpt/log_kv_cache.py:739-898).
        if (self.beta_novelty or self.beta_adaptive_merge) and not self.alpha_exact_tokens:
            raise ValueError("BetaLogKV requires the Alpha exact-span cache (alpha_exact_tokens > 0)")
        if self.alpha_exact_tokens < 0:
            raise ValueError("alpha_exact_tokens must be >= 0")
        if self.alpha_exact_tokens:
            if not (semantic_clusters and semantic_anchor_mode == "mid" and not allocate_second_order
                    and cluster_k_max > 1):
                raise ValueError("AlphaLogKV requires semantic clusters, K > 1, mid anchors and no second-order allocation")
            if semantic_legacy_route or semantic_cluster_chunk_size:
                raise ValueError("AlphaLogKV archives through the attach or unified route; legacy/chunk-tree routing is not supported")
            if (seg_gap_max is not None and math.isfinite(seg_gap_max)) or seg_block_level:
                raise ValueError("AlphaLogKV requires disabled segment gaps/padding for delayed archival")
            if not 1 <= self.alpha_span_max_tokens <= self.alpha_exact_tokens:
                raise ValueError("alpha_span_max_tokens must be in [1, alpha_exact_tokens]")
        if semantic_anchor_mode not in ("mid", "multi"):
            raise ValueError("semantic_anchor_mode must be 'mid' or 'multi'")
        if semantic_pack_backend not in ("auto", "torch", "triton", "hip"):
            raise ValueError("semantic_pack_backend must be 'auto', 'torch', 'triton' or 'hip'")
        if semantic_centroid_backend not in ("sequential", "parallel"):
            raise ValueError("semantic_centroid_backend must be sequential or parallel")
        if semantic_merge_passes < 1:
            raise ValueError("semantic_merge_passes must be >= 1")
        recent = recent_size if recent_size > 0 else 2
        if recent < 2:
            raise ValueError(f"recent_size ({recent}) must be >= 2")
        if not 1 <= semantic_flush_granularity <= recent:
            raise ValueError(
                "semantic_flush_granularity must be in [1, recent_size], got "
                f"{semantic_flush_granularity} for recent_size={recent}")
        if not (math.isfinite(cluster_lambda_rel) and cluster_lambda_rel > 0.0):
            raise ValueError(f"cluster_lambda_rel must be finite and > 0, got {cluster_lambda_rel}")
        if not (math.isfinite(seg_g0) and seg_g0 > 0.0):
            raise ValueError(f"seg_g0 must be finite and > 0, got {seg_g0}")
        cap_mult = float(semantic_capacity_hard_cap_mult)
        if not (math.isfinite(cap_mult) and cap_mult >= 0.0):
            raise ValueError(f"semantic_capacity_hard_cap_mult must be finite >= 0, got {semantic_capacity_hard_cap_mult}")
        if cos_cache is None or sin_cache is None or rope_n_elem is None:
            raise ValueError("semantic LogKV requires cos_cache, sin_cache, and rope_n_elem")
        # The path this library implements; everything else is a different algorithm.
        unsupported = []
        if not semantic_clusters or cluster_k_max <= 1:
            unsupported.append("semantic_clusters with cluster_k_max > 1")
        if semantic_legacy_route or semantic_cluster_chunk_size:
            unsupported.append("attach routing (no legacy / chunk-tree route)")
        if semantic_capacity_beta:
            unsupported.append("no capacity penalty")
        if (seg_gap_max is not None and math.isfinite(seg_gap_max)) or seg_block_level:
            unsupported.append("no segment gaps or padding")
        if semantic_anchor_mode != "mid":
            unsupported.append("semantic_anchor_mode='mid'")
        if allocate_second_order:
            unsupported.append("allocate_second_order=False")
        if importance_pooling:
            unsupported.append("importance_pooling=False")
        if dtype not in _lib.ACTIVATION_DTYPES:
            unsupported.append("a bfloat16, float16 or float32 dtype")
        if cluster_k_max > 32:
            unsupported.append("cluster_k_max <= 32")
        if unsupported:
            raise NotImplementedError("logkv_amd implements the attach/mid/first-order flush path only; requires "
                                      + "; ".join(unsupported))
        if device.type != "cuda":
            raise ValueError(f"logkv_amd caches live on a ROCm device, got {device}")

        self.K_max = int(cluster_k_max)
        self.cluster_lambda_rel = float(cluster_lambda_rel)
        self.seg_eta, self.seg_g0 = float(seg_eta), float(seg_g0)
        self.seg_gap_max, self.seg_block_level, self.seg_forget = math.inf, 0, float(seg_forget)
        self.recent_size = recent
        self.semantic_flush_granularity = int(semantic_flush_granularity)
        self.semantic_anchor_mode = semantic_anchor_mode
        self.semantic_pack_backend = semantic_pack_backend
        self.semantic_centroid_backend = semantic_centroid_backend
        self.semantic_replay_updates = bool(semantic_replay_updates)
        self.semantic_unified_route = bool(semantic_unified_route)
        self._merge_passes = int(semantic_merge_passes)
        self.semantic_capacity_beta = 0.0
        self.semantic_capacity_hard_cap_mult = cap_mult
        self.semantic_legacy_route = False
        self.rope_n_elem = int(rope_n_elem)
        self.register_buffer("cos_cache", cos_cache.to(device=device), persistent=False)
        self.register_buffer("sin_cache", sin_cache.to(device=device), persistent=False)
        self.slot_k_dim = int(cos_cache.size(1)) + k_dim - self.rope_n_elem
        # The Alpha budget is priced at the constructor's dtype, as the reference prices it before any
        # later _convert_dtype; the entries themselves are stored as bfloat16 whatever the dtype.
        element = torch.empty((), dtype=dtype).element_size()
        self.activation_dtype = dtype
        dtype = torch.bfloat16
        B_eff, L, budget = ladder_budget(batch_size, n_groups, max_seq_length, k_dim, v_dim, B, self.K_max,
                                         self.alpha_exact_tokens, element)
        if budget is not None:
            self.alpha_baseline_B = B
            self.alpha_budget_bytes = budget
        if not 2 <= B_eff <= 32767:
            # Per-level slot counts are int16 (level_count and the device's ladder plans).
            raise ValueError(f"slots per level B'={B_eff} must be in [2, 32767]")
        self.B = self.B_prime = B_eff
        self.max_levels = self.L_alloc = L
        self.recent_capacity = 2 * recent
        self.token_count = 0
        self.recent_count = 0
        self._mid_decode_state = None
        self._second_order = False

        def buf(name, value):
            self.register_buffer(name, value, persistent=False)

        cap = self.recent_capacity
        buf("recent_k", torch.zeros(batch_size, n_groups, cap, self.slot_k_dim, device=device, dtype=dtype))
        buf("recent_v", torch.zeros(batch_size, n_groups, cap, v_dim, device=device, dtype=dtype))
        buf("recent_k_raw", torch.zeros(batch_size, n_groups, cap, k_dim, device=device, dtype=dtype))
        buf("recent_pos", torch.zeros(batch_size, cap, device=device, dtype=torch.int64))
        self._alpha_count_host = 0
        if self.alpha_exact_tokens:
            P = self.alpha_exact_tokens
            buf("alpha_k_raw", torch.zeros(batch_size, n_groups, P, k_dim, device=device, dtype=dtype))
            buf("alpha_v", torch.zeros(batch_size, n_groups, P, v_dim, device=device, dtype=dtype))
            buf("alpha_pos", torch.zeros(batch_size, P, device=device, dtype=torch.int64))
            buf("alpha_valid", torch.zeros(batch_size, P, device=device, dtype=torch.bool))
            # The exact pool's selection lives on the device: spans (length,
            # closed) of the kept rows and the kept count, so a flush chooses
            # spans with no host round trip.
            buf("alpha_span_len", torch.zeros(batch_size, P, device=device, dtype=torch.int32))
            buf("alpha_span_closed", torch.zeros(batch_size, P, device=device, dtype=torch.uint8))
            buf("alpha_span_count", torch.zeros(batch_size, device=device, dtype=torch.int32))
            buf("alpha_count_dev", torch.zeros(1, device=device, dtype=torch.int32))
            # The pool and its spans are rewritten into this second buffer set,
            # then the sets swap, so nothing reads a row it has overwritten.
            self._alpha_spare = (torch.zeros_like(self.alpha_k_raw), torch.zeros_like(self.alpha_v),
                                 torch.zeros_like(self.alpha_pos), torch.zeros_like(self.alpha_valid),
                                 torch.zeros_like(self.alpha_span_len), torch.zeros_like(self.alpha_span_closed),
                                 torch.zeros_like(self.alpha_span_count))
            # Natural span boundary flags of the recent rows, shifted with them.
            buf("recent_span_ends", torch.zeros(batch_size, cap, device=device, dtype=torch.uint8))
        shp = (batch_size, n_groups, self.K_max, L, B_eff)
        i64max = torch.iinfo(torch.int64).max
        buf("level_k", torch.zeros(*shp, k_dim, device=device, dtype=dtype))
        buf("level_v", torch.zeros(*shp, v_dim, device=device, dtype=dtype))
        buf("level_w", torch.zeros(shp, device=device, dtype=torch.float32))
        buf("level_imp", torch.zeros(shp, device=device, dtype=torch.float32))
        buf("level_count", torch.zeros(shp[:-1], device=device, dtype=torch.int16))
        buf("pad_mask", torch.zeros(shp, device=device, dtype=torch.bool))
        buf("level_p_lo", torch.full(shp, i64max, device=device, dtype=torch.int64))
        buf("level_p_hi", torch.full(shp, -1, device=device, dtype=torch.int64))
        buf("level_sum_wp", torch.zeros(shp, device=device, dtype=torch.int64))
        buf("level_order", torch.zeros(shp, device=device, dtype=torch.int64))
        lanes = (batch_size, n_groups, self.K_max)
        buf("centroid", torch.zeros(*lanes, k_dim, device=device, dtype=torch.float32))
        buf("n_eff", torch.zeros(lanes, device=device, dtype=torch.float32))
        buf("n_total", torch.zeros(lanes, device=device, dtype=torch.int32))
        buf("p_hi_c", torch.full(lanes, -1, device=device, dtype=torch.int64))
        buf("current_segment", torch.zeros(lanes, device=device, dtype=torch.int32))
        buf("level0_phase", torch.zeros(lanes, device=device, dtype=torch.int32))
        buf("alive", torch.zeros(lanes, device=device, dtype=torch.bool))
        if semantic_s_h is None:
            s_h = torch.ones(batch_size, n_groups, device=device, dtype=torch.float32)
        elif isinstance(semantic_s_h, torch.Tensor):
            s_h = semantic_s_h.to(device=device, dtype=torch.float32)
            if s_h.shape == (n_groups,):
                s_h = s_h.unsqueeze(0).expand(batch_size, -1).contiguous()
            elif s_h.shape != (batch_size, n_groups):
                raise ValueError(f"semantic_s_h must have shape ({n_groups},) or ({batch_size},{n_groups}), got {tuple(s_h.shape)}")
        else:
            s_h = torch.full((batch_size, n_groups), float(semantic_s_h), device=device, dtype=torch.float32)
        if not bool(torch.isfinite(s_h).all().item()) or not bool((s_h > 0).all().item()):
            raise ValueError("semantic_s_h must be finite and > 0")
        buf("s_h", s_h.contiguous())
        # Radius limits of the unified route's candidates, sqrt(lambda * s_h) per
        # lane (litgpt/log_kv_cache.py:3617-3620, :2728-2729), refreshed from the
        # live s_h before every unified flush.
        buf("_unified_limits", torch.zeros(batch_size * n_groups, dtype=torch.float32, device=device))
        self._workspace = None
        self._alpha_keep_alive = None
        # C-ABI argument structs and per-flush-length buffers, built once and
        # reused (raw pointers: cleared whenever buffers move).
        self._views = {}
        self._alpha_parity = 0   # flips with every swap of the exact pool's two buffer sets
        # The capacity cap (litgpt/log_kv_cache.py:2347-2354): the direct test
        # compares float32 counts with it, the rooms count against int(cap).
        cap = self._semantic_hard_cap()
        self._params = RouteParams(self.seg_eta, self.seg_g0, self.cluster_lambda_rel,
                                   1 if self.alpha_exact_tokens else 0, 1 if self.beta_adaptive_merge else 0,
                                   _CENTER_TILES[self._centroid_backend],
                                   cap if cap != math.inf else 0.0,   # stored as float32
                                   min(int(cap), 2**31 - 1) if cap != math.inf else 0,
                                   self._merge_passes)
        self.op_log: torch.Tensor | None = None
        self.op_log_len: torch.Tensor | None = None
        self._op_replay_cursor_host = None
        self._last_op_log_host = None
        # Update tape (semantic_replay_updates): the bound tape, whether it is
        # replayed, and the flushes recorded / replayed since the log began.
        self._active_updates = None
        self._replaying_updates = False
        self._update_actions = None
        self._tape_index = 0
        # Side-stream flushes: with `flush_stream` set (a torch.cuda.Stream of
        # the cache's device), add_recent queues its append and flush there,
        # after the caller's stream; every reader of the cache's device state
        # then waits on the last such flush (`_flush_done`).
        self.flush_stream = None
        self._flush_done = None
        # Rows per count of alpha_count_dev (0: one count for all rows; the owner of a flush group keeps
        # one count per member).
        self._alpha_count_rows = 0
        self._init_kwargs.update(cos_cache=self.cos_cache, sin_cache=self.sin_cache)
        _flush_group.register(self)

    def _group_key(self):
        """Caches whose flushes may run stacked share this key (same shapes, budget and route)."""
        kw = self._init_kwargs
        return (self.level_k.device, self.level_k.dtype, self.batch_size, self.n_groups, self.max_seq_length,
                self.k_dim, self.v_dim, self.B_prime, self.L_alloc, self.K_max, self.recent_size,
                self.semantic_flush_granularity, self.cluster_lambda_rel, self.seg_eta, self.seg_g0,
                self.semantic_capacity_hard_cap_mult, self.semantic_unified_route, self.semantic_merge_passes,
                self.alpha_exact_tokens, self.alpha_span_max_tokens, self.beta_novelty, self.beta_adaptive_merge,
                kw["semantic_centroid_backend"], self.semantic_replay_updates)

    def __getattr__(self, name):
        # A state buffer read while this cache's flush is deferred runs the flush first.
        if name in _flush_group.STATE_SET and self.__dict__.get("_pending") is not None:
            self._group.run()
        return super().__getattr__(name)

    def _await_flush(self, stream=None) -> None:
        """Make the device state current for ``stream`` (default: the current one): run a deferred
        flush of this cache (with the rest of its flush group), then order the stream after the last
        flush queued on ``flush_stream``."""
        if self._pending is not None:
            self._group.run()
        if self._flush_done is not None:
            (torch.cuda.current_stream(self.level_k.device) if stream is None else stream).wait_event(self._flush_done)

    def _semantic_capacity_target(self) -> float:
        """Rows per cluster if the sequence filled every cluster evenly (litgpt/log_kv_cache.py:2347-2348)."""
        return max(float(self.max_seq_length) / max(self.K_max, 1), 1.0)

    def _semantic_hard_cap(self) -> float:
        """The attach route's capacity cap, ``inf`` without one (litgpt/log_kv_cache.py:2350-2354)."""
        if self.semantic_capacity_hard_cap_mult <= 0.0:
            return math.inf
        return self._semantic_capacity_target() * self.semantic_capacity_hard_cap_mult

    # ------------------------------------------------------------------
    # C-ABI views
    # ------------------------------------------------------------------
    def _ladder_view(self) -> LadderView:
        view = self._views.get("ladder")
        if view is None:
            view = self._views["ladder"] = LadderView(
                ptr(self.level_k), ptr(self.level_v), ptr(self.level_w), ptr(self.level_p_lo), ptr(self.level_p_hi),
                ptr(self.level_sum_wp), ptr(self.level_order), ptr(self.pad_mask), ptr(self.level_count),
                ptr(self.centroid), ptr(self.n_eff), ptr(self.n_total), ptr(self.p_hi_c), ptr(self.level0_phase),
                ptr(self.alive), ptr(self.s_h),
                self.batch_size, self.n_groups, self.K_max, self.L_alloc, self.B_prime, self.k_dim, self.v_dim,
            )
        return view

    def _workspace_for(self, view: LadderView, tokens: int) -> torch.Tensor:
        need = self._views.get(("route_ws", tokens))
        if need is None:
            need = lib().logkv_route_workspace_bytes(C.byref(view), tokens, self._params.late_joins)
            if need < 0:
                raise ValueError("invalid cache layout for the HIP route")
            self._views[("route_ws", tokens)] = need
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(need, dtype=torch.uint8, device=self.level_k.device)
        return self._workspace

    @staticmethod
    def _rows_view(k_raw, v, positions, counts=None) -> RowsView:
        for name, t in (("k_raw", k_raw), ("v", v)):
            if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
                raise ValueError(f"{name} must be bf16 with a contiguous last axis")
        if positions.dtype != torch.int64 or positions.stride(-1) != 1:
            raise ValueError("positions must be int64 with a contiguous last axis")
        return RowsView(
            ptr(k_raw), k_raw.stride(0), k_raw.stride(1), k_raw.stride(2),
            ptr(v), v.stride(0), v.stride(1), v.stride(2),
            ptr(positions), positions.stride(0), ptr(counts), k_raw.size(2),
        )

    # ------------------------------------------------------------------
    # Flush
    # ------------------------------------------------------------------
    @torch.no_grad()
    def route_and_flush_batch(self, k_raw, v, positions, *, positions_host=None, record_op_log=False,
                              replay_op_log=None, replay_op_log_len=None, replay_op_log_host=None,
                              replay_plans=None, span_ends=None, counts=None, assign_out=None, order_out=None):
        """Route one flush of rows ``[Bt, G, T, D]`` and commit them (litgpt/log_kv_cache.py:4946-5128).

        ``record_op_log`` appends the flush's decisions to the op-log
        (``begin_op_log``); ``replay_op_log`` / ``replay_op_log_len`` re-apply
        a logged flush without routing (litgpt/log_kv_cache.py:5049-5114).
        """
        k_raw, v = _lib.as_storage(k_raw), _lib.as_storage(v)
        self._await_flush()
        if self._active_updates is not None:
            return self._tape_flush(self._active_updates, k_raw, v, positions, positions_host, span_ends, counts,
                                    record_op_log, replay_op_log is not None or replay_op_log_host is not None)
        if replay_plans is not None and replay_op_log is None:
            raise RuntimeError("semantic replay plans require the matching op-log; rerouting is not allowed")
        if record_op_log and self.op_log is None:
            self.begin_op_log()
        if positions.dim() == 1:
            positions = positions.unsqueeze(0).expand(k_raw.size(0), -1)
        for t, what in ((k_raw, "k_raw"), (v, "v"), (positions, "positions")):
            require_device(t, what)
        if k_raw.shape[:2] != (self.batch_size, self.n_groups) or v.shape[:3] != k_raw.shape[:3]:
            raise ValueError("flush rows must be [batch, groups, T, dim] matching the cache")
        if positions_host is None and replay_plans is not None:
            raise RuntimeError("semantic replay plans require CPU positions; device readback is not allowed")
        self._mid_decode_state = None
        if self.alpha_exact_tokens:
            if replay_op_log is not None:
                raise RuntimeError("AlphaLogKV replay requires semantic_replay_updates; reranking is not allowed")
            return self._alpha_route_flush(k_raw, v, positions, positions_host, span_ends, record=record_op_log)
        if replay_op_log is not None:
            return self._replay_flush(k_raw, v, positions, positions_host, counts, replay_op_log, replay_op_log_len,
                                      replay_op_log_host, replay_plans)
        self._route_commit(k_raw, v, positions, counts, assign_out, order_out, record=record_op_log)

    def _route_commit(self, k_raw, v, positions, counts=None, assign_out=None, order_out=None, record=False):
        """Route and commit one flush; with ``assign_out`` / ``order_out`` the
        decisions are also written there (for the update tape), and the unified
        route returns its old-old merges as well (``_unified_route_commit``)."""
        if self.semantic_unified_route:
            return self._unified_route_commit(k_raw, v, positions, counts, record=record, assign_out=assign_out,
                                              order_out=order_out)
        view = self._ladder_view()
        rows = self._rows_view(k_raw, v, positions, counts)
        ws = self._workspace_for(view, rows.tokens)
        stream = stream_of(k_raw.device)
        rc = lib().logkv_route_commit(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                      ptr(assign_out), ptr(order_out), stream)
        check(rc, "logkv_route_commit")
        if record:
            log = self._op_log_view()
            check(lib().logkv_record_ops(C.byref(view), C.byref(rows), ptr(ws), ws.numel(), C.byref(log), stream),
                  "logkv_record_ops")

    def _unified_workspace(self, k_raw, v, positions, counts):
        view = self._ladder_view()
        rows = self._rows_view(k_raw, v, positions, counts)
        key = ("unified_ws", rows.tokens)
        need = self._views.get(key)
        if need is None:
            need = lib().logkv_unified_workspace_bytes(C.byref(view), rows.tokens, self._params.late_joins)
            if need < 0:
                raise ValueError("invalid cache layout for the unified route")
            self._views[key] = need
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(need, dtype=torch.uint8, device=self.level_k.device)
        return view, rows, self._workspace

    def _unified_route_commit(self, k_raw, v, positions, counts=None, record=False, assign_out=None, order_out=None):
        """Unified route of one flush (litgpt/log_kv_cache.py:3589-3688): the plan
        on the device, one read of its two-word summary (the old-old merge
        rounds to launch and the budget stage's failure flag), then the merges
        and the commit. ``record`` appends the flush's op-log rows (its
        WARD_MERGE rows, then NEW_CLUSTER / JOIN). With ``assign_out`` /
        ``order_out`` the decisions are copied there and the old-old merges are
        returned as ``{"jobs", "n_jobs", "steps"}`` (an update-tape record)."""
        view, rows, ws = self._unified_workspace(k_raw, v, positions, counts)
        summary = self._views.get("unified_summary")
        if summary is None:
            summary = self._views["unified_summary"] = torch.zeros(2, dtype=torch.int32, device=self.level_k.device)
        stream = stream_of(k_raw.device)
        # sqrt(lambda * s_h) in double, rounded once to float32, as the reference's host
        # math.sqrt(lambda * s_h) (litgpt/log_kv_cache.py:3620-3621), from the s_h the attach
        # route also reads, so both routes follow a caller's update of s_h.
        self._unified_limits.copy_(self.s_h.reshape(-1).double().mul(self.cluster_lambda_rel).sqrt())
        check(lib().logkv_unified_plan(C.byref(view), C.byref(rows), C.byref(self._params), ptr(self._unified_limits),
                                       ptr(ws), ws.numel(), ptr(summary), stream), "logkv_unified_plan")
        steps, stuck = summary.tolist()
        if stuck:
            raise RuntimeError("unified route: a budget stage found no mutual pair above the cluster budget")
        merges = None
        if assign_out is not None:
            lanes = self.batch_size * self.n_groups
            jobs = torch.empty(lanes, 32, 2, dtype=torch.int32, device=k_raw.device)
            n_jobs = torch.empty(lanes, dtype=torch.int32, device=k_raw.device)
            check(lib().logkv_unified_decisions(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws),
                                                ws.numel(), ptr(assign_out), ptr(order_out), ptr(jobs), ptr(n_jobs), 0,
                                                stream), "logkv_unified_decisions")
            merges = {"jobs": jobs, "n_jobs": n_jobs, "steps": torch.tensor([int(steps)], dtype=torch.int32)}
        check(lib().logkv_unified_commit(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                         int(steps), stream), "logkv_unified_commit")
        if record:
            check(lib().logkv_unified_record_ops(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws),
                                                 ws.numel(), C.byref(self._op_log_view()), stream),
                  "logkv_unified_record_ops")
        return merges

    def unified_reduce_stats(self, tokens: int) -> torch.Tensor:
        """The reducer's counts of the last unified flush of ``tokens`` rows, int32 ``[Bt * G, 2, 8]`` on
        the host (one synchronisation): per lane and stage (radius candidates, cluster budget) its
        nodes, rounds, merges, Lance-Williams elements (kept rows x live columns, summed over the
        rounds), rescanned elements (rescanned rows x live columns, the first scan n x n) and stuck
        flag. Measurement only."""
        self._await_flush()
        view = self._ladder_view()
        at = lib().logkv_unified_stats_offset(C.byref(view), int(tokens), self._params.late_joins)
        lanes = self.batch_size * self.n_groups
        if at < 0 or self._workspace is None or self._workspace.numel() < at + lanes * 64:
            raise ValueError("no unified flush of this length has run on this cache")
        return self._workspace[at:at + lanes * 64].view(torch.int32).reshape(lanes, 2, 8).cpu()

    def _unified_commit_only(self, k_raw, v, positions, counts, assign, order, merges):
        """A recorded unified flush applied from its decisions and old-old merges."""
        view, rows, ws = self._unified_workspace(k_raw, v, positions, counts)
        stream = stream_of(k_raw.device)
        check(lib().logkv_unified_decisions(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                            ptr(assign), ptr(order), ptr(merges["jobs"]), ptr(merges["n_jobs"]), 1,
                                            stream), "logkv_unified_decisions")
        check(lib().logkv_unified_commit(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                         int(merges["steps"][0]), stream), "logkv_unified_commit")

    def _commit_only(self, k_raw, v, positions, counts, assign, order, merges=None):
        if self.semantic_unified_route:
            return self._unified_commit_only(k_raw, v, positions, counts, assign, order, merges)
        view = self._ladder_view()
        rows = self._rows_view(k_raw, v, positions, counts)
        ws = self._workspace_for(view, rows.tokens)
        check(lib().logkv_commit_only(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                      ptr(assign), ptr(order), stream_of(k_raw.device)), "logkv_commit_only")

    def _alpha_route_flush(self, k_raw, v, positions, positions_host, span_ends, record=False, tape=None):
        from .alpha_log_kv import alpha_flush
        return alpha_flush(self, k_raw, v, positions, positions_host, span_ends, record=record, tape=tape)

    # ------------------------------------------------------------------
    # Update tape (litgpt/log_kv_cache.py:4932-5031)
    # ------------------------------------------------------------------
    @contextlib.contextmanager
    def _semantic_update_context(self, updates, *, replay=False):
        previous = self._active_updates, self._replaying_updates
        self._active_updates, self._replaying_updates = updates, replay
        try:
            yield
        finally:
            self._active_updates, self._replaying_updates = previous

    def _tape_signature(self, k_raw, v, span_ends):
        ends = None
        if span_ends is not None and not isinstance(span_ends, torch.Tensor):
            ends = tuple(tuple(bool(x) for x in row) for row in span_ends)
        return (tuple(k_raw.shape), tuple(v.shape), k_raw.dtype, v.dtype, k_raw.device, self.K_max, self.B,
                self.L_alloc, self.recent_size, self.semantic_flush_granularity, self.alpha_exact_tokens,
                self.alpha_span_max_tokens, self.beta_novelty, self.beta_adaptive_merge, ends)

    def _tape_flush(self, updates, k_raw, v, positions, positions_host, span_ends, counts, record_op_log, replay):
        """Record a flush on the bound tape, or replay it from there
        (litgpt/log_kv_cache.py:4946-5031): keyed by the flush's CPU positions,
        replayed in recording order with the same shapes and configuration."""
        if positions.dim() == 1:
            positions = positions.unsqueeze(0).expand(k_raw.size(0), -1)
        host = positions_host
        if host is None:
            raise RuntimeError("update replay requires CPU flush positions; no device readback is allowed")
        if len(host) != k_raw.size(0) or any(len(row) != k_raw.size(2) for row in host):
            raise RuntimeError("update replay CPU positions do not match the flush shape")
        key = tuple(tuple(int(x) for x in row) for row in host)
        signature = self._tape_signature(k_raw, v, span_ends)
        dev = k_raw.device
        if self._replaying_updates:
            if not replay or key not in updates.flushes:
                raise RuntimeError("missing semantic update record; rerouting is not allowed")
            expected, index, saved, ready = updates.flushes[key]
            if index != self._tape_index:
                raise RuntimeError("semantic update replay flushes are out of order")
            if signature != expected:
                raise RuntimeError("semantic update record does not match this flush/configuration")
            stream = torch.cuda.current_stream(dev)
            if ready is not None:
                stream.wait_event(ready)   # device-side wait only
            tensors = {name: None if i is None else updates.tensors[i] for name, i in saved.items()}
            for t in tensors.values():
                if t is not None and t.is_cuda:   # a unified record's merge-round count stays on the host
                    t.record_stream(stream)
            self._mid_decode_state = None
            if self.alpha_exact_tokens:
                from .alpha_log_kv import alpha_replay
                alpha_replay(self, tensors)
            else:
                self._commit_only(tensors["k"], tensors["v"], tensors["pos"], tensors["counts"], tensors["assign"],
                                  tensors["order"], tensors)
            self._tape_index += 1
            return
        if replay or key in updates.flushes:
            raise RuntimeError("duplicate or incorrectly bound semantic update recording")
        if record_op_log and self.op_log is None:
            self.begin_op_log()
        if not record_op_log:
            raise RuntimeError("semantic update recording requires record_op_log=True")
        for t, what in ((k_raw, "k_raw"), (v, "v"), (positions, "positions")):
            require_device(t, what)
        if k_raw.shape[:2] != (self.batch_size, self.n_groups) or v.shape[:3] != k_raw.shape[:3]:
            raise ValueError("flush rows must be [batch, groups, T, dim] matching the cache")
        self._mid_decode_state = None
        if self.alpha_exact_tokens:
            saved = self._alpha_route_flush(k_raw, v, positions, positions_host, span_ends, record=True, tape=updates)
        else:
            T = k_raw.size(2)
            assign = torch.empty(self.batch_size * self.n_groups, T, dtype=torch.int8, device=dev)
            order = torch.empty(self.batch_size, T, dtype=torch.int32, device=dev)
            merges = self._route_commit(k_raw, v, positions, counts, assign, order, record=True)
            saved = {"k": updates.save(k_raw), "v": updates.save(v), "pos": updates.save(positions),
                     "counts": updates.save(counts), "assign": updates.save(assign, owned=True),
                     "order": updates.save(order, owned=True)}
            for name, t in (merges or {}).items():
                saved[name] = updates.save(t, owned=True)
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(dev))
        updates.flushes[key] = (signature, self._tape_index, saved, ready)
        self._tape_index += 1

    # ------------------------------------------------------------------
    # Op-log record / replay (litgpt/log_kv_cache.py:2006-2096, :4856-4926)
    # ------------------------------------------------------------------
    def begin_op_log(self) -> None:
        """Bind a fresh per-(batch, group) route log (litgpt/log_kv_cache.py:2006-2028).

        ``op_log`` ``[Bt, G, 3 * max_seq_length, 4]`` int32 rows (op, cluster,
        arg, position) and ``op_log_len`` ``[Bt, G]``, written on the device by
        every flush routed with ``record_op_log=True``.
        """
        self._await_flush()
        cap = max(1, self.max_seq_length * 3)
        dev = self.level_count.device
        self.op_log = torch.zeros(self.batch_size, self.n_groups, cap, 4, device=dev, dtype=torch.int32)
        self.op_log_len = torch.zeros(self.batch_size, self.n_groups, device=dev, dtype=torch.int32)
        self._op_replay_cursor_host = None
        self._tape_index = 0

    def _op_log_view(self, log=None, lengths=None) -> _lib.OpLogView:
        log = self.op_log if log is None else log
        lengths = self.op_log_len if lengths is None else lengths
        return _lib.OpLogView(ptr(log), ptr(lengths), log.size(2))

    def take_op_log(self):
        """(log ``[Bt, G, max_len, 4]``, lengths ``[Bt, G]``) copies (litgpt/log_kv_cache.py:2029-2038).

        Reads the lengths back (one synchronisation) and keeps the rows as host
        tuples in ``_last_op_log_host``. Raises ``RuntimeError`` when a lane
        logged more rows than the capacity (the rows past it were not written).
        """
        if getattr(self, "op_log", None) is None or getattr(self, "op_log_len", None) is None:
            return None, None
        self._await_flush()
        lengths = self.op_log_len.cpu()
        if int(lengths.max()) > self.op_log.size(2):
            raise RuntimeError("semantic LogKV op_log overflow")
        max_len = int(lengths.max())
        rows = self.op_log[:, :, :max_len].cpu().tolist()
        lens = lengths.tolist()
        self._last_op_log_host = [[[tuple(r) for r in rows[b][g][:lens[b][g]]] for g in range(self.n_groups)]
                                  for b in range(self.batch_size)]
        return self.op_log[:, :, :max_len].clone(), self.op_log_len.clone()

    def _replay_flush(self, k_raw, v, positions, positions_host, counts, log, lengths, log_host, plans):
        """Re-apply one logged flush (litgpt/log_kv_cache.py:5067-5114) on the device.

        Every lane of an attach-routed log consumes one row per flushed token,
        so the lanes share one cursor. The checks run on the device; their
        status is read back (one synchronisation) and a failed check raises
        ``RuntimeError`` with the cache left as it was.
        """
        if lengths is None:
            raise ValueError("replay_op_log_len is required with replay_op_log")
        if plans is not None and log_host is not plans.host_log:
            raise RuntimeError("semantic replay plan does not match the CPU op-log")
        if self.semantic_unified_route:
            return self._unified_replay_flush(k_raw, v, positions, positions_host, counts, log, lengths, plans)
        B, G, T = k_raw.shape[:3]
        if (log.dim() != 4 or tuple(log.shape[:2]) != (B, G) or log.size(3) != 4 or log.dtype != torch.int32
                or tuple(lengths.shape) != (B, G) or lengths.dtype != torch.int32):
            raise RuntimeError("semantic replay log does not match the current batch/groups")
        require_device(log, "replay_op_log")
        require_device(lengths, "replay_op_log_len")
        log, lengths = log.contiguous(), lengths.contiguous()
        if getattr(self, "_op_replay_cursor_host", None) is None:
            self._op_replay_cursor_host = [[0] * G for _ in range(B)]
        cursors = self._op_replay_cursor_host
        cursor = cursors[0][0]
        if any(c != cursor for row in cursors for c in row):
            raise RuntimeError("semantic LogKV replay cursors differ across lanes")
        if plans is not None:
            current = tuple(tuple(int(x) for x in row) for row in positions_host[:B])
            key = tuple(tuple(row[:G]) for row in cursors[:B])
            seen = plans.plans.setdefault(key, current)
            if seen != current:
                raise RuntimeError("semantic replay plan does not match the current flush positions")
        view = self._ladder_view()
        rows = self._rows_view(k_raw, v, positions, counts)
        ws = self._workspace_for(view, rows.tokens)
        status = self._views.get("replay_status")
        if status is None:
            status = self._views["replay_status"] = torch.zeros(1, dtype=torch.int32, device=self.level_k.device)
        lv = self._op_log_view(log, lengths)
        check(lib().logkv_replay_commit(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                        C.byref(lv), cursor, ptr(status), stream_of(k_raw.device)),
              "logkv_replay_commit")
        bits = int(status.item())
        if bits:
            why = "; ".join(msg for bit, msg in _lib.REPLAY_ERRORS.items() if bits & bit)
            raise RuntimeError(f"semantic LogKV replay of rows {cursor}.. failed (nothing was written): {why}")
        taken = [T] * B if counts is None else [max(0, min(T, int(c))) for c in counts.tolist()]
        for b in range(B):
            cursors[b][:G] = [cursors[b][g] + taken[b] for g in range(G)]

    def _unified_replay_flush(self, k_raw, v, positions, positions_host, counts, log, lengths, plans):
        """Re-apply one logged unified flush (litgpt/log_kv_cache.py:5067-5114):
        per lane from its own cursor, the leading WARD_MERGE rows are the old-old
        merges and one NEW_CLUSTER / JOIN row per flushed token the decisions.
        The parse and its checks run on the device; the check bits, the merge
        rounds and the rows each lane consumed are read back (one
        synchronisation), and a failed check raises ``RuntimeError`` before
        anything is written to the cache."""
        if lengths is None:
            raise ValueError("replay_op_log_len is required with replay_op_log")
        B, G, T = k_raw.shape[:3]
        if (log.dim() != 4 or tuple(log.shape[:2]) != (B, G) or log.size(3) != 4 or log.dtype != torch.int32
                or tuple(lengths.shape) != (B, G) or lengths.dtype != torch.int32):
            raise RuntimeError("semantic replay log does not match the current batch/groups")
        require_device(log, "replay_op_log")
        require_device(lengths, "replay_op_log_len")
        log, lengths = log.contiguous(), lengths.contiguous()
        if getattr(self, "_op_replay_cursor_host", None) is None:
            self._op_replay_cursor_host = [[0] * G for _ in range(B)]
        cursors = self._op_replay_cursor_host
        if plans is not None:
            current = tuple(tuple(int(x) for x in row) for row in positions_host[:B])
            key = tuple(tuple(row[:G]) for row in cursors[:B])
            seen = plans.plans.setdefault(key, current)
            if seen != current:
                raise RuntimeError("semantic replay plan does not match the current flush positions")
        if T == 0:
            return
        view, rows, ws = self._unified_workspace(k_raw, v, positions, counts)
        dev = k_raw.device
        lanes = B * G
        out = self._views.get(("unified_replay", lanes))
        if out is None:
            out = self._views[("unified_replay", lanes)] = torch.zeros(2 + lanes, dtype=torch.int32, device=dev)
        cur = torch.tensor([c for row in cursors[:B] for c in row[:G]], dtype=torch.int64).to(dev)
        stream = stream_of(dev)
        check(lib().logkv_unified_replay_plan(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                              C.byref(self._op_log_view(log, lengths)), ptr(cur), ptr(out[2:]),
                                              ptr(out), stream), "logkv_unified_replay_plan")
        host = out.tolist()
        bits, steps = host[0], host[1]
        if bits:
            why = "; ".join(msg for bit, msg in _lib.REPLAY_ERRORS.items() if bits & bit)
            raise RuntimeError(f"semantic LogKV replay of a unified flush failed (nothing was written): {why}")
        check(lib().logkv_unified_commit(C.byref(view), C.byref(rows), C.byref(self._params), ptr(ws), ws.numel(),
                                         int(steps), stream), "logkv_unified_commit")
        for b in range(B):
            cursors[b][:G] = [cursors[b][g] + host[2 + b * G + g] for g in range(G)]

    def _semantic_flush_tokens(self, flush_len: int, span_ends=None, **route) -> None:
        pending = int(flush_len)
        while pending > 0:
            take = min(self.semantic_flush_granularity, pending)
            if take > self.recent_count:
                raise RuntimeError(f"semantic LogKV cannot flush {take} tokens from recent_count={self.recent_count}")
            # CPU positions are read only where a caller needs them (update tape, replay plans).
            needs_host = self._active_updates is not None or route.get("replay_plans") is not None
            self.route_and_flush_batch(
                self.recent_k_raw[:, :, :take], self.recent_v[:, :, :take], self.recent_pos[:, :take],
                positions_host=self.recent_pos[:, :take].tolist() if needs_host else None,
                span_ends=self.recent_span_ends[:, :take] if self.alpha_exact_tokens else None,
                **route,
            )
            remaining = self.recent_count - take
            if remaining <= take:
                # One launch moves the remaining rows to the front and clears the rest.
                args = self._recent_args()
                check(lib().logkv_recent_shift(C.byref(args), take, self.recent_count,
                                               stream_of(self.recent_k.device)), "logkv_recent_shift")
                self.recent_count = remaining
                pending -= take
                continue
            if remaining > 0:
                stage = (lambda x: x) if remaining <= take else torch.Tensor.clone
                for name in ("recent_k", "recent_k_raw", "recent_v"):
                    t = getattr(self, name)
                    t[:, :, :remaining].copy_(stage(t[:, :, take:self.recent_count]))
                self.recent_pos[:, :remaining].copy_(stage(self.recent_pos[:, take:self.recent_count]))
                if self.alpha_exact_tokens:
                    self.recent_span_ends[:, :remaining].copy_(stage(self.recent_span_ends[:, take:self.recent_count]))
            # The vacated rows are cleared (litgpt/log_kv_cache.py:5652-5659).
            for name in ("recent_k", "recent_k_raw", "recent_v"):
                getattr(self, name)[:, :, remaining:self.recent_count].zero_()
            self.recent_pos[:, remaining:self.recent_count].zero_()
            if self.alpha_exact_tokens:
                self.recent_span_ends[:, remaining:self.recent_count].zero_()
            self.recent_count = remaining
            pending -= take

    def _recent_args(self):
        """The recent window's buffers as the C-ABI struct (built once; the sources are set per append)."""
        args = self._views.get("recent")
        if args is None:
            args = self._views["recent"] = _lib.RecentArgs()
            args.recent_k, args.recent_k_raw, args.recent_v = ptr(self.recent_k), ptr(self.recent_k_raw), ptr(self.recent_v)
            args.recent_pos = ptr(self.recent_pos)
            args.recent_ends = ptr(self.recent_span_ends) if self.alpha_exact_tokens else None
            args.n_batch, args.n_groups, args.cap = self.batch_size, self.n_groups, self.recent_capacity
            args.dk, args.dkr, args.dv = self.recent_k.size(-1), self.recent_k_raw.size(-1), self.recent_v.size(-1)
        return args

    def _recent_append(self, k, k_raw, v, positions, ends, n) -> bool:
        """Append rows with one launch (litgpt/log_kv_cache.py:5668-5718); False when a source's layout
        (dtype, feature stride, 8-byte rows) leaves it to tensor copies."""
        srcs = (k, k_raw, v)
        if n == 0 or any(t.dtype != torch.bfloat16 or t.stride(-1) != 1 or t.data_ptr() % 8
                         or any(st % 4 for st in t.stride()[:3]) or t.device != self.recent_k.device for t in srcs):
            return False
        if positions.dtype != torch.int64 or (ends is not None and (ends.dtype != torch.uint8 or ends.stride(-1) != 1)):
            return False
        if tuple(k.shape) != (self.batch_size, self.n_groups, n, self.recent_k.size(-1)) or \
                tuple(v.shape) != (self.batch_size, self.n_groups, n, self.recent_v.size(-1)):
            return False
        args = self._recent_args()
        args.k, (args.k_sb, args.k_sg, args.k_st) = ptr(k), k.stride()[:3]
        args.k_raw, (args.kr_sb, args.kr_sg, args.kr_st) = ptr(k_raw), k_raw.stride()[:3]
        args.v, (args.v_sb, args.v_sg, args.v_st) = ptr(v), v.stride()[:3]
        args.pos, (args.pos_sb, args.pos_st) = ptr(positions), positions.stride()
        args.ends, args.ends_sb = (ptr(ends), ends.stride(0)) if ends is not None else (None, 0)
        check(lib().logkv_recent_append(C.byref(args), self.recent_count, n, stream_of(self.recent_k.device)),
              "logkv_recent_append")
        return True

    def _input_positions(self, n, input_pos):
        """Positions of an appended block as a device tensor ``[Bt, n]`` (no host read)."""
        dev = self.recent_k.device
        if input_pos is None:
            return torch.arange(self.token_count, self.token_count + n, device=dev).unsqueeze(0).expand(
                self.batch_size, -1)
        if input_pos.dim() == 1:
            return input_pos.to(dev, torch.int64).unsqueeze(0).expand(self.batch_size, -1)
        if input_pos.dim() == 2:
            return input_pos.to(dev, torch.int64)
        raise ValueError(f"input_pos must be 1-D or 2-D, got shape {tuple(input_pos.shape)}")

    def _span_ends_block(self, span_ends, n):
        """Boundary flags of an appended block as uint8 ``[Bt, n]`` on the device: a tensor (bool or
        integer, any device) or per-row host lists, as the reference takes them."""
        dev = self.recent_k.device
        if isinstance(span_ends, torch.Tensor):
            if tuple(span_ends.shape) != (self.batch_size, n):
                raise ValueError("AlphaLogKV span boundaries must match the input batch and token count")
            return span_ends.to(dev, torch.uint8)
        if span_ends is None or len(span_ends) != self.batch_size or any(len(row) != n for row in span_ends):
            raise ValueError("AlphaLogKV span boundaries must match the input batch and token count")
        host = torch.tensor([[bool(x) for x in row] for row in span_ends], dtype=torch.uint8)
        return host.pin_memory().to(dev, non_blocking=True)

    @torch.no_grad()
    def add_recent(self, k, v, *, k_raw=None, input_pos=None, record_op_log=False, replay_op_log=None,
                   replay_op_log_len=None, replay_op_log_host=None, replay_plans=None, span_ends=None):
        """Append a block to the recent window; flush whole granules on overflow
        (litgpt/log_kv_cache.py:5668-5718, :5847). With ``flush_stream`` set the
        append and the flush are queued on that stream after the caller's, and
        the cache's readers wait for them; the host state advances at once."""
        k, v, k_raw = _lib.as_storage(k), _lib.as_storage(v), _lib.as_storage(k_raw)
        side = self.flush_stream
        if side is not None and side != torch.cuda.current_stream(self.level_k.device):
            side.wait_stream(torch.cuda.current_stream(self.level_k.device))
            for t in (k, v, k_raw, input_pos, span_ends):
                if isinstance(t, torch.Tensor) and t.is_cuda:
                    t.record_stream(side)
            with torch.cuda.stream(side):
                self._add_recent(k, v, k_raw=k_raw, input_pos=input_pos, record_op_log=record_op_log,
                                 replay_op_log=replay_op_log, replay_op_log_len=replay_op_log_len,
                                 replay_op_log_host=replay_op_log_host, replay_plans=replay_plans,
                                 span_ends=span_ends)
            done = self._flush_done if self._flush_done is not None else torch.cuda.Event()
            done.record(side)
            self._flush_done = done
            return
        self._add_recent(k, v, k_raw=k_raw, input_pos=input_pos, record_op_log=record_op_log,
                         replay_op_log=replay_op_log, replay_op_log_len=replay_op_log_len,
                         replay_op_log_host=replay_op_log_host, replay_plans=replay_plans, span_ends=span_ends)

    def _add_recent(self, k, v, *, k_raw=None, input_pos=None, record_op_log=False, replay_op_log=None,
                    replay_op_log_len=None, replay_op_log_host=None, replay_plans=None, span_ends=None):
        self._await_flush()
        if k_raw is None:
            raise ValueError("semantic LogKV add_recent requires pre-RoPE k_raw")
        n = k.size(2)
        if n > self.recent_size:
            raise ValueError(f"chunk size {n} exceeds recent_size {self.recent_size}")
        if k_raw.shape[:3] != k.shape[:3] or k_raw.size(-1) != self.k_dim:
            raise ValueError(f"k_raw shape {tuple(k_raw.shape)} does not match semantic cache shape")
        positions = self._input_positions(n, input_pos)
        ends = self._span_ends_block(span_ends, n) if self.alpha_exact_tokens else None
        if self.token_count + n > self.max_seq_length:
            raise RuntimeError(
                f"LogStructuredKVCache: token overflow! token_count={self.token_count}, n={n}, "
                f"max_seq_length={self.max_seq_length}.")
        self.token_count += n
        if self.recent_count + n > self.recent_capacity:
            raise RuntimeError(f"semantic LogKV recent buffer overflow: recent_count={self.recent_count}, n={n}, "
                               f"capacity={self.recent_capacity}")
        if not self._recent_append(k, k_raw, v, positions, ends, n):
            dst = slice(self.recent_count, self.recent_count + n)
            self.recent_k[:, :, dst] = k
            self.recent_k_raw[:, :, dst] = k_raw
            self.recent_v[:, :, dst] = v
            self.recent_pos[:, dst] = positions
            if ends is not None:
                self.recent_span_ends[:, dst] = ends
        self.recent_count += n
        overflow = self.recent_count - self.recent_size
        if overflow > 0:
            F = self.semantic_flush_granularity
            take = F * ((overflow + F - 1) // F)
            plain = not record_op_log and replay_op_log is None and replay_op_log_host is None and replay_plans is None
            if (plain and self._active_updates is None and self.flush_stream is None and self._group is not None
                    and self._group.adopt()):
                # Deferred: the group runs it, stacked with the other layers' flushes, at the first read.
                self._pending = (take, self.recent_count)
                self.recent_count -= take
                self._mid_decode_state = None
                return
            self._semantic_flush_tokens(take, record_op_log=record_op_log,
                                        replay_op_log=replay_op_log, replay_op_log_len=replay_op_log_len,
                                        replay_op_log_host=replay_op_log_host, replay_plans=replay_plans)

    def reset_parameters(self) -> None:
        """Empty cache (litgpt/log_kv_cache.py:6270)."""
        self._await_flush()
        i64max = torch.iinfo(torch.int64).max
        for name in ("recent_k", "recent_v", "recent_k_raw", "recent_pos", "level_k", "level_v", "level_w",
                     "level_imp", "level_count", "pad_mask", "level_sum_wp", "level_order", "centroid", "n_eff",
                     "n_total", "current_segment", "level0_phase", "alive"):
            getattr(self, name).zero_()
        self.level_p_lo.fill_(i64max)
        self.level_p_hi.fill_(-1)
        self.p_hi_c.fill_(-1)
        self.token_count = self.recent_count = 0
        self.alpha_count = 0
        self._mid_decode_state = None
        self.op_log = self.op_log_len = None
        self._op_replay_cursor_host = None
        self._tape_index = 0
        if self.alpha_exact_tokens:
            for name in ("alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid", "alpha_span_len", "alpha_span_closed",
                         "alpha_span_count", "alpha_count_dev"):
                getattr(self, name).zero_()
            for t in self._alpha_spare:
                t.zero_()
            self.recent_span_ends.zero_()

    def _apply(self, fn, recurse=True):
        # Moving or casting buffers invalidates raw pointers held in workspaces
        # (litgpt/log_kv_cache.py:6226-6232).
        self._await_flush()
        before = {name: t.data_ptr() for name, t in self._buffers.items() if t is not None}
        self._mid_decode_state = None
        self._workspace = None
        self._views = {}
        self._alpha_keep_alive = None
        # A cast of the module (``.float()``, ``.to(dtype)``) keeps every buffer's dtype - the kernels'
        # storage contract - and moves devices only; a floating cast (fn maps float32 and bf16 to one
        # dtype) sets the activation dtype instead, as ``_convert_dtype`` does.
        probes = [fn(torch.empty(0, dtype=dt, device=self.level_k.device)) for dt in (torch.float32, torch.bfloat16)]
        cast = probes[0].dtype if probes[0].dtype == probes[1].dtype else None

        def keep_dtype(t):
            target = fn(t.new_empty(0))
            return t if target.device == t.device else t.to(target.device)

        out = super()._apply(keep_dtype, recurse)
        if self.alpha_exact_tokens:
            self._alpha_spare = tuple(keep_dtype(t) for t in self._alpha_spare)
        if cast in _lib.ACTIVATION_DTYPES:
            self.activation_dtype = cast
        moved = any(t is not None and t.data_ptr() != before.get(name) for name, t in self._buffers.items())
        if moved and self._group is not None:
            self._group.leave(self)      # its buffers no longer view the group's stacked rows
        return out

    # ------------------------------------------------------------------
    # Readout plan
    # ------------------------------------------------------------------
    def _semantic_mid_attention_plan(self):
        """Plan of the occupied slots, built on the device (litgpt/log_kv_cache.py:5979-6007)."""
        from .log_kv_pack import semantic_mid_attention_plan
        return semantic_mid_attention_plan(self)

    def _semantic_attention_plan(self):
        """Mid-anchor plan (litgpt/log_kv_cache.py:5955-5958); the only anchor mode built."""
        return self._semantic_mid_attention_plan()

    def get_attention_state(self, with_stats: bool = False, *, plan=None) -> CacheAttentionState:
        """Unpacked slots for ``log_kv_slot_attention`` (litgpt/log_kv_cache.py:6116-6120): pooled slots in
        plan order, the exact pool, the recent window. Entries are first order, so ``with_stats`` yields
        no statistics (as the reference does without second-order storage)."""
        from .log_kv_pack import attention_state
        return attention_state(self, self._semantic_attention_plan() if plan is None else plan)

    def _semantic_attention_state(self, with_stats: bool = False, plan=None) -> CacheAttentionState:
        return self.get_attention_state(with_stats, plan=plan)

    def _convert_dtype(self, dtype: torch.dtype) -> None:
        """Reconcile the cache with the activation dtype (litgpt/log_kv_cache.py:6236-6268); a no-op
        once it matches. The reference converts its buffers to ``dtype``; here the entries stay
        bfloat16 (the kernels' storage type) and ``dtype`` becomes the activation dtype: float16 /
        float32 rows are rounded to bf16 where they enter (``add_recent``, ``route_and_flush_batch``,
        the attention entry points) and readouts come back in ``dtype``. As in the reference, the
        decode prefix kept for reuse is dropped when the dtype changes."""
        _lib.check_activation_dtype(dtype)
        if self.activation_dtype == dtype:
            return
        self._mid_decode_state = None
        self.activation_dtype = dtype

    # ------------------------------------------------------------------
    # Host mirrors of the reference, read from the device on demand
    # ------------------------------------------------------------------
    @property
    def semantic_merge_passes(self) -> int:
        """Matching passes per budget round of the unified route (litgpt/log_kv_cache.py:3314): more than
        one adds frozen-center sweeps (:561-588). Read by every later unified flush."""
        return self._merge_passes

    @semantic_merge_passes.setter
    def semantic_merge_passes(self, value: int) -> None:
        value = int(value)
        if value < 1:
            raise ValueError("semantic_merge_passes must be >= 1")
        self._merge_passes = value
        if "_params" in self.__dict__:
            self._params.merge_passes = value

    @property
    def semantic_centroid_backend(self) -> str:
        """Order of a center's new-key sum: "sequential" (one row at a time in position order) or
        "parallel" (position-ordered tiles of 32 rows, each summed by a halving tree, tiles added in
        order; litgpt/log_kv_updates_triton.py:236-241). Read by every later flush."""
        return self._centroid_backend

    @semantic_centroid_backend.setter
    def semantic_centroid_backend(self, value: str) -> None:
        if value not in _CENTER_TILES:
            raise ValueError("semantic_centroid_backend must be sequential or parallel")
        self._centroid_backend = value
        if "_params" in self.__dict__:
            self._params.center_tile = _CENTER_TILES[value]

    @property
    def alpha_count(self) -> int:
        """Rows of the exact pool in use (largest kept count); read from the device."""
        if not self.alpha_exact_tokens:
            return self._alpha_count_host
        self._await_flush()
        return int(self.alpha_count_dev.item())

    @alpha_count.setter
    def alpha_count(self, value: int) -> None:
        if self.alpha_exact_tokens:
            self._await_flush()
            self.alpha_count_dev.fill_(int(value))
        else:
            self._alpha_count_host = int(value)

    @property
    def _alpha_spans(self):
        """Per batch row, (length, closed) of the exact pool's spans (litgpt/log_kv_cache.py)."""
        self._await_flush()
        n = self.alpha_span_count.tolist()
        lens, closed = self.alpha_span_len.tolist(), self.alpha_span_closed.tolist()
        return [[(lens[b][i], bool(closed[b][i])) for i in range(n[b])] for b in range(self.batch_size)]

    @property
    def _alpha_positions(self):
        """Per batch row, positions of the exact pool's kept rows in span order."""
        rows = [sum(length for length, _ in spans) for spans in self._alpha_spans]
        pos = self.alpha_pos.tolist()
        return [pos[b][:rows[b]] for b in range(self.batch_size)]

    @property
    def _semantic_counts(self):
        self._await_flush()
        return self.level_count.long().cpu().tolist()

    @property
    def _semantic_alive(self):
        self._await_flush()
        return self.alive.cpu().tolist()

    @property
    def _semantic_p_hi_c(self):
        self._await_flush()
        return self.p_hi_c.cpu().tolist()

    @property
    def _semantic_n_total(self):
        self._await_flush()
        return self.n_total.long().cpu().tolist()

    @property
    def _semantic_level0_phase(self):
        self._await_flush()
        return self.level0_phase.long().cpu().tolist()

    @property
    def second_order(self) -> bool:
        return False

    @second_order.setter
    def second_order(self, value: bool) -> None:
        if value:
            raise RuntimeError("Second-order storage is disabled; rebuild the cache with allocate_second_order=True")


def append_exact_tokens(state, k_new, v_new):
    """Exact entries appended after a state's slots (litgpt/log_kv_cache.py:6391-6425)."""
    from .log_kv_pack import append_exact_tokens as _append
    return _append(state, k_new, v_new)


def log_kv_slot_attention(*args, **kwargs):
    """Slot attention over unpacked slots (litgpt/log_kv_cache.py:6501-6721); see log_kv_pack."""
    from .log_kv_pack import log_kv_slot_attention as _attend
    return _attend(*args, **kwargs)


def log_kv_chunk_attention(*args, **kwargs):
    """One streaming attention step over [cache | chunk] (litgpt/log_kv_cache.py:6802-6836); see log_kv_pack."""
    from .log_kv_pack import log_kv_chunk_attention as _chunk
    return _chunk(*args, **kwargs)


class LogKVStreamTrainingAttention(torch.autograd.Function):
    """Streaming training attention with memory independent of T * S (litgpt/log_kv_cache.py:6867-7098).

    Forward streams the sequence in ``train_block`` blocks with no recorded graph: each block's queries
    attend to the cache state at the block's start plus the block causally, then the block is committed
    while the route decisions are recorded (the op-log, and with ``semantic_replay_updates`` the update
    tape: rows, attach decisions, Alpha selections). Backward resets the cache and replays the same
    flushes from the records - no re-routing, no re-selection - recomputing each block's attention with
    a gradient (the matrix-core backward kernels) on exactly the state forward attended over. Gradients
    reach q, k and v through each token's own block only (the cache commits detached copies).
    """

    @staticmethod
    def forward(ctx, q, k, v, cache, scale, train_block, second_order_scale, k_raw=None, span_ends=None):
        commit_k_raw = k if k_raw is None else k_raw
        ctx.input_count = len(ctx.needs_input_grad)
        ctx.span_ends = None if span_ends is None else tuple(tuple(bool(x) for x in row) for row in span_ends)
        if cache.alpha_exact_tokens and (not cache.semantic_replay_updates or second_order_scale != 0.0):
            raise ValueError("AlphaLogKV training requires semantic_replay_updates and second_order_scale=0")
        T = q.size(2)
        train_block = int(train_block)
        if train_block < 2:
            raise ValueError(f"logKV train_block must be >= 2, got {train_block}")
        if train_block > cache.recent_size:
            raise ValueError(f"logKV train_block ({train_block}) must be <= recent_size ({cache.recent_size})")
        updates = _SemanticReplayUpdates() if cache.semantic_replay_updates else None
        outputs, plans = [], []
        with torch.no_grad():
            if updates is not None:
                updates.wait(q.device)
            cache.reset_parameters()
            cache.begin_op_log()
            for start in range(0, T, train_block):
                end = min(start + train_block, T)
                plan = cache._semantic_attention_plan()
                plans.append(plan)
                outputs.append(log_kv_chunk_attention(cache, q[:, :, start:end], k[:, :, start:end],
                                                      v[:, :, start:end], scale, second_order_scale,
                                                      attention_plan=plan))
                with cache._semantic_update_context(updates):
                    cache.add_recent(k[:, :, start:end], v[:, :, start:end], k_raw=commit_k_raw[:, :, start:end],
                                     record_op_log=True, span_ends=None if ctx.span_ends is None else
                                     [row[start:end] for row in ctx.span_ends])
        op_log, op_log_len = cache.take_op_log()
        ctx.replay_plans = _SemanticReplayPlans(cache._last_op_log_host)
        ctx.op_log, ctx.op_log_len, ctx.op_log_host = op_log, op_log_len, ctx.replay_plans.host_log
        ctx.updates, ctx.plans, ctx.cache = updates, plans, cache
        ctx.scale, ctx.train_block, ctx.second_order_scale = scale, train_block, second_order_scale
        ctx.config = (cache.semantic_anchor_mode, cache.semantic_centroid_backend, cache.semantic_replay_updates,
                      cache.semantic_unified_route, cache.semantic_merge_passes, cache.alpha_exact_tokens,
                      cache.alpha_span_max_tokens, cache.beta_novelty, cache.beta_adaptive_merge)
        ctx.save_for_backward(q, k, v, commit_k_raw)
        return torch.cat(outputs, dim=2)

    @staticmethod
    def backward(ctx, grad_y):
        q, k, v, k_raw = ctx.saved_tensors
        cache, updates = ctx.cache, ctx.updates
        if ctx.config != (cache.semantic_anchor_mode, cache.semantic_centroid_backend, cache.semantic_replay_updates,
                          cache.semantic_unified_route, cache.semantic_merge_passes, cache.alpha_exact_tokens,
                          cache.alpha_span_max_tokens, cache.beta_novelty, cache.beta_adaptive_merge):
            raise RuntimeError("semantic cache configuration changed between forward and backward")
        T = q.size(2)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        with torch.no_grad():
            if updates is not None:
                updates.wait(q.device)
            cache.reset_parameters()
        for i, start in enumerate(range(0, T, ctx.train_block)):
            end = min(start + ctx.train_block, T)
            q_b = q[:, :, start:end].detach().requires_grad_(True)
            k_b = k[:, :, start:end].detach().requires_grad_(True)
            v_b = v[:, :, start:end].detach().requires_grad_(True)
            with torch.enable_grad():
                y_b = log_kv_chunk_attention(cache, q_b, k_b, v_b, ctx.scale, ctx.second_order_scale,
                                             attention_plan=ctx.plans[i])
            g_q, g_k, g_v = torch.autograd.grad(y_b, (q_b, k_b, v_b), grad_y[:, :, start:end])
            dq[:, :, start:end] = g_q
            dk[:, :, start:end] = g_k
            dv[:, :, start:end] = g_v
            with torch.no_grad(), cache._semantic_update_context(updates, replay=True):
                cache.add_recent(k[:, :, start:end], v[:, :, start:end], k_raw=k_raw[:, :, start:end],
                                 replay_op_log=ctx.op_log, replay_op_log_len=ctx.op_log_len,
                                 replay_op_log_host=ctx.op_log_host, replay_plans=ctx.replay_plans,
                                 span_ends=None if ctx.span_ends is None else
                                 [row[start:end] for row in ctx.span_ends])
        return (dq, dk, dv) + (None,) * (ctx.input_count - 3)
