"""Attention readout of a LogKV cache on the device: slot plan, packed K/V, decode attention.

Mirrors the reference's first-order mid-anchor readout:

* ``semantic_mid_attention_plan`` -> ``LogStructuredKVCache._semantic_mid_attention_plan``
  (litgpt/log_kv_cache.py:5979-6007), here a device table of per-lane pooled-row
  offsets plus the pooled width, so building it never waits for the host;
* ``pack_mid_kv`` -> litgpt/log_kv_pack.py:105-133 (same arguments, checks and
  return value);
* ``log_kv_chunk_attention`` -> litgpt/log_kv_cache.py:6802-6836 for
  ``second_order_scale == 0`` with mid anchors (the path that reaches
  ``_mid_chunk_attention``, litgpt/log_kv_cache.py:6772-6799), including the
  decode-prefix reuse of ``reuse_prefix=True``.

Packed rows are ``[pooled (plan width) | exact pool | recent | current]`` of
width ``dim = 8*ceil(max(Dk + 1, Dv) / 8)``; the key's column ``Dk`` carries
``log(max(w, 1))`` for pooled slots, 0 for exact / recent / current rows and
-10000 for empty rows, and the query carries ``1/scale`` there, so the logit of
a slot is ``scale * q.k + log w`` (litgpt/log_kv_cache.py:6428-6464).
"""

from __future__ import annotations

import ctypes as C
import math

import torch

from ._lib import (AttentionArgs, AttentionGradArgs, PackArgs, ReadoutView, SlotPackArgs, as_storage, check, lib, ptr,
                   require_device, stream_of)

_BACKENDS = ("auto", "triton", "hip")


def packed_dim(k_dim: int, v_dim: int) -> int:
    return ((max(k_dim + 1, v_dim) + 7) // 8) * 8


class MidAttentionPlan:
    """Device plan of the occupied slots: ``table`` int32 ``[lanes * (K*L + 1) + 1]``.

    Per lane, ``K*L`` offsets of the (cluster, level top-down) blocks in the
    pooled rows and the lane's slot count; the last entry is the pooled width
    (the largest lane count). ``width`` reads that entry back once.
    """

    __slots__ = ("table", "lanes", "blocks", "_width")

    def __init__(self, table: torch.Tensor, lanes: int, blocks: int):
        self.table, self.lanes, self.blocks = table, lanes, blocks
        self._width = None

    @property
    def width(self) -> int:
        if self._width is None:
            self._width = int(self.table[-1].item())
        return self._width

    def lane_counts(self) -> torch.Tensor:
        return self.table[:-1].view(self.lanes, self.blocks + 1)[:, -1]


def readout_view(cache) -> ReadoutView:
    """The cache's readout struct: built once per exact-pool buffer set and
    reused (only the recent row count changes between calls)."""
    cache._await_flush()
    key = ("readout", cache._alpha_parity)
    view = cache._views.get(key)
    if view is None:
        view = cache._views[key] = _build_readout_view(cache)
    view.recent_count = cache.recent_count
    return view


def _build_readout_view(cache) -> ReadoutView:
    table_bf16 = cache.cos_cache.dtype == torch.bfloat16
    if cache.cos_cache.dtype not in (torch.float32, torch.bfloat16) or cache.sin_cache.dtype != cache.cos_cache.dtype:
        raise ValueError("RoPE tables must both be float32 or both bfloat16")
    if cache.cos_cache.size(1) != cache.rope_n_elem or cache.slot_k_dim != cache.k_dim:
        raise NotImplementedError("packed readout requires RoPE tables of width rope_n_elem")
    view = ReadoutView(
        ptr(cache.level_k), ptr(cache.level_v), ptr(cache.level_w), ptr(cache.level_sum_wp), ptr(cache.level_count),
        cache.batch_size, cache.n_groups, cache.K_max, cache.L_alloc, cache.B_prime, cache.k_dim, cache.v_dim)
    if cache.alpha_exact_tokens:
        view.alpha_k, view.alpha_v = ptr(cache.alpha_k_raw), ptr(cache.alpha_v)
        view.alpha_pos, view.alpha_valid = ptr(cache.alpha_pos), ptr(cache.alpha_valid)
        view.alpha_cap, view.alpha_count = cache.alpha_exact_tokens, 0
        view.alpha_count_dev = ptr(cache.alpha_count_dev)     # rows in use, read on the device
    view.recent_k, view.recent_v = ptr(cache.recent_k), ptr(cache.recent_v)
    view.recent_cap, view.recent_count = cache.recent_capacity, cache.recent_count
    view.cos, view.sin = ptr(cache.cos_cache), ptr(cache.sin_cache)
    view.cos_s0, view.cos_s1 = cache.cos_cache.stride()
    view.sin_s0, view.sin_s1 = cache.sin_cache.stride()
    view.rope_n, view.table_bf16 = cache.rope_n_elem, 1 if table_bf16 else 0
    view.rope_rows = min(cache.cos_cache.size(0), cache.sin_cache.size(0))
    return view


def semantic_mid_attention_plan(cache, view: ReadoutView | None = None) -> MidAttentionPlan:
    """Plan of the occupied slots (litgpt/log_kv_cache.py:5979-6007), built on the device."""
    view = readout_view(cache) if view is None else view
    n = int(lib().logkv_plan_table_ints(C.byref(view)))
    table = torch.empty(n, dtype=torch.int32, device=cache.level_k.device)
    check(lib().logkv_mid_plan(C.byref(view), ptr(table), stream_of(table.device)), "logkv_mid_plan")
    return MidAttentionPlan(table, cache.batch_size * cache.n_groups, cache.K_max * cache.L_alloc)


def _check_backend(backend):
    if backend == "torch":
        raise NotImplementedError("logkv_amd has no PyTorch packer; the HIP pack kernel is the only path")
    if backend not in _BACKENDS:
        raise ValueError("packing backend must be 'auto', 'torch' or 'triton'")


def _check_kv(cache, k, v):
    if (k.ndim != 4 or v.ndim != 4 or k.shape[:3] != v.shape[:3]
            or k.shape[:2] != (cache.batch_size, cache.n_groups)
            or k.size(-1) != cache.k_dim or v.size(-1) != cache.v_dim
            or k.device != cache.level_k.device or v.device != k.device
            or k.dtype != cache.level_k.dtype or v.dtype != k.dtype):
        raise ValueError("K/V shape, device and dtype must match the cache")


def _launch_pack(cache, view, plan, k, v, dim, ka, va, skip_pooled, recent_start, out_w=None, out_valid=None):
    """Pack into ``ka / va``; with ``skip_pooled`` only the rows from recent window row
    ``recent_start`` on (the exact pool's row count is read on the device). ``out_w`` /
    ``out_valid`` (float / uint8 ``[Bt, G, cap]``) also receive each row's mass and validity."""
    args = PackArgs(ptr(k), *k.stride()[:3], ptr(v), *v.stride()[:3], k.size(2), ptr(ka), ptr(va), ka.size(2), dim,
                    1 if skip_pooled else 0, recent_start, ptr(out_w), ptr(out_valid))
    if k.stride(3) != 1 or v.stride(3) != 1:
        raise ValueError("current K/V rows must be contiguous in the feature dimension")
    check(lib().logkv_pack(C.byref(view), C.byref(args), ptr(plan.table), stream_of(k.device)), "logkv_pack")


def pack_mid_kv(cache, plan, k, v, dim, *, backend=None, buffers=None, skip_pooled=False, recent_start=0):
    """Return final padded K/V ``[Bt, G, length, dim]``; K's extra coordinate stores log mass / masking.

    Same contract as litgpt/log_kv_pack.py:105-133; ``length`` is the plan's
    pooled width plus the exact, recent and current rows (reading the width
    back once per plan).
    """
    if (k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16) and buffers is None:
        # float16 / float32 rows: packed at the cache's bf16 precision, returned in k's dtype.
        ka, va = pack_mid_kv(cache, plan, as_storage(k), as_storage(v), dim, backend=backend,
                             skip_pooled=skip_pooled, recent_start=recent_start)
        return ka.to(k.dtype), va.to(v.dtype)
    backend = cache.semantic_pack_backend if backend is None else backend
    _check_backend(backend)
    if cache.semantic_anchor_mode != "mid":
        raise ValueError("mid packer requires semantic_anchor_mode='mid'")
    _check_kv(cache, k, v)
    if not isinstance(plan, MidAttentionPlan) or plan.lanes != cache.batch_size * cache.n_groups \
            or plan.table.device != k.device:
        raise ValueError("mid attention plan must match K/V lanes and device")
    if dim <= k.size(-1) or dim < v.size(-1):
        raise ValueError("packed dimension must hold K, its bias coordinate, and V")
    if ((skip_pooled and buffers is None) or (recent_start and not skip_pooled)
            or not 0 <= recent_start <= cache.recent_count):
        raise ValueError("prefix reuse requires a workspace and a valid recent offset")
    if buffers is not None and (k.requires_grad or v.requires_grad):
        raise ValueError("reusable decode buffers cannot hold differentiable K/V")
    if torch.is_grad_enabled() and (k.requires_grad or v.requires_grad):
        return _PackMidKV.apply(k, v, cache, plan, dim)
    length = plan.width + cache.alpha_count + cache.recent_count + k.size(2)
    if buffers is not None:
        if len(buffers) != 2 or any(buf.ndim != 4 or buf.shape[:2] != k.shape[:2] or buf.size(2) < length
                                    or buf.size(3) != dim or not buf.is_contiguous() or buf.dtype != k.dtype
                                    or buf.device != k.device for buf in buffers):
            raise ValueError("decode workspace does not match the packed layout")
        ka, va = buffers
    else:
        ka = k.new_empty((*k.shape[:2], length, dim))
        va = v.new_empty((*v.shape[:2], length, dim))
    view = readout_view(cache)
    _launch_pack(cache, view, plan, k, v, dim, ka, va, skip_pooled, recent_start)
    return ka[:, :, :length], va[:, :, :length]


class _PackMidKV(torch.autograd.Function):
    """pack_mid_kv with a gradient for the current rows (litgpt/log_kv_pack.py:75-97): the packed
    prefix is detached state, each current row is copied once, so the backward is the slice of the
    current rows' key and value features."""

    @staticmethod
    def forward(ctx, k, v, cache, plan, dim):
        ctx.start = plan.width + cache.alpha_count + cache.recent_count
        ctx.k_dim, ctx.v_dim = k.size(-1), v.size(-1)
        with torch.no_grad():
            return pack_mid_kv(cache, plan, k.detach(), v.detach(), dim)

    @staticmethod
    def backward(ctx, gka, gva):
        gk = gka[:, :, ctx.start:, :ctx.k_dim].contiguous() if ctx.needs_input_grad[0] and gka is not None else None
        gv = gva[:, :, ctx.start:, :ctx.v_dim].contiguous() if ctx.needs_input_grad[1] and gva is not None else None
        return gk, gv, None, None, None


def _inv_scale_bf16(scale: float) -> float:
    return torch.tensor(1.0 / scale, dtype=torch.float32).to(torch.bfloat16).item()


def packed_attention(q, ka, va, plan, tail, scale, causal_tail, v_dim, n_groups, workspace=None,
                     alpha_count_dev=None):
    """Attention of ``q [Bt, Hq, Tq, Dk]`` over packed rows ``[plan width + exact + tail]`` of ``ka / va``.

    The pooled width (and, given ``alpha_count_dev``, the exact pool's row
    count) is read on the device, so ``ka / va`` may be longer than the packed
    rows (a reusable decode workspace)."""
    bt, hq, tq, dk = q.shape
    if q.dtype != torch.bfloat16 or q.stride(3) != 1:
        raise ValueError("queries must be bfloat16 with contiguous features")
    if not ka.is_contiguous() or not va.is_contiguous() or ka.shape != va.shape:
        raise ValueError("packed K/V must be contiguous and of one shape")
    out = q.new_empty(bt, hq, tq, v_dim)
    args = AttentionArgs(ptr(q), *q.stride()[:3], bt, hq, n_groups, tq, dk, v_dim, ka.size(3), ptr(ka), ptr(va),
                         ka.size(2), tail, causal_tail, float(scale), _inv_scale_bf16(scale), ptr(out),
                         *out.stride()[:3], ptr(alpha_count_dev))
    if (hq // n_groups) * tq > 16:
        # Many query rows per KV group: the matrix-core chunk kernel.
        need = int(lib().logkv_chunk_workspace_bytes(C.byref(args)))
        if need < 0:
            raise ValueError("bad attention shape")
        if need and (workspace is None or workspace.numel() < need):
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        check(lib().logkv_chunk_attention(C.byref(args), ptr(plan.table), plan.table.numel(),
                                          ptr(workspace) if need else None, need, stream_of(q.device)),
              "logkv_chunk_attention")
        return out, workspace
    need = int(lib().logkv_attention_workspace_bytes(C.byref(args)))
    if need < 0:
        raise ValueError("bad attention shape")
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    check(lib().logkv_decode_attention(C.byref(args), ptr(plan.table), plan.table.numel(), ptr(workspace),
                                       workspace.numel(), stream_of(q.device)), "logkv_decode_attention")
    return out, workspace


def packed_attention_backward(q, ka, va, out, dout, plan, tail, scale, causal_tail, v_dim, n_groups, grad_rows,
                              alpha_count_dev=None):
    """Gradients of ``packed_attention``: dq ``[Bt, Hq, Tq, Dk]`` and, for the last ``grad_rows`` packed
    rows of every lane, dk / dv ``[Bt, G, grad_rows, D]`` (the matrix-core backward kernels)."""
    bt, hq, tq, dk = q.shape
    if dout.dtype != torch.bfloat16:
        dout = dout.to(torch.bfloat16)
    if dout.stride(-1) != 1:
        dout = dout.contiguous()
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    gk = q.new_empty(bt, n_groups, grad_rows, dk)
    gv = q.new_empty(bt, n_groups, grad_rows, v_dim)
    args = AttentionArgs(ptr(q), *q.stride()[:3], bt, hq, n_groups, tq, dk, v_dim, ka.size(3), ptr(ka), ptr(va),
                         ka.size(2), tail, causal_tail, float(scale), _inv_scale_bf16(scale), ptr(out),
                         *out.stride()[:3], ptr(alpha_count_dev))
    grads = AttentionGradArgs(ptr(dout), *dout.stride()[:3], ptr(dq), *dq.stride()[:3], ptr(gk), ptr(gv), grad_rows)
    need = int(lib().logkv_chunk_backward_workspace_bytes(C.byref(args)))
    if need < 0:
        raise ValueError("bad attention shape")
    ws = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    check(lib().logkv_chunk_attention_backward(C.byref(args), ptr(plan.table), plan.table.numel(), C.byref(grads),
                                               ptr(ws), ws.numel(), stream_of(q.device)),
          "logkv_chunk_attention_backward")
    return dq, gk, gv


class _PackedAttention(torch.autograd.Function):
    """Attention over packed rows whose gradient reaches the queries and the last ``grad_rows`` rows
    (the in-flight chunk, or every slot of a slot attention): forward by the decode / matrix-core
    kernels, backward by the matrix-core backward kernels. ``k_rows`` / ``v_rows`` are the tensors the
    gradient rows were packed from (their features only; masked rows get zero gradient through
    ``row_mask``)."""

    @staticmethod
    def forward(ctx, q, k_rows, v_rows, ka, va, plan, tail, scale, causal_tail, v_dim, n_groups, alpha_count_dev,
                row_mask):
        out, _ = packed_attention(q.detach(), ka, va, plan, tail, scale, causal_tail, v_dim, n_groups, None,
                                  alpha_count_dev)
        ctx.save_for_backward(q.detach(), ka, va, out)
        # The exact pool's row count as it was for these packed rows: the cache's counter moves on
        # with later flushes, and a graph may be differentiated after them.
        exact = None if alpha_count_dev is None else alpha_count_dev.clone()
        ctx.meta = (plan, tail, scale, causal_tail, v_dim, n_groups, exact, k_rows.size(2), row_mask)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, ka, va, out = ctx.saved_tensors
        plan, tail, scale, causal_tail, v_dim, n_groups, exact, rows, row_mask = ctx.meta
        dq, gk, gv = packed_attention_backward(q, ka, va, out, dout, plan, tail, scale, causal_tail, v_dim, n_groups,
                                               rows, exact)
        if row_mask is not None:
            gk = gk * row_mask[..., None]
            gv = gv * row_mask[..., None]
        return (dq if ctx.needs_input_grad[0] else None, gk if ctx.needs_input_grad[1] else None,
                gv if ctx.needs_input_grad[2] else None) + (None,) * 10


def _decode_capacity(cache, t: int) -> int:
    return cache.K_max * cache.L_alloc * cache.B_prime + cache.alpha_exact_tokens + cache.recent_capacity + max(2, t)


def log_kv_chunk_attention(cache, q_b, k_b, v_b, scale, second_order_scale=1.0, attention_plan=None, *,
                           causal_tail=None, reuse_prefix=False):
    """One streaming attention step over ``[cache state | current chunk (causal)]``, without committing the chunk.

    Restates litgpt/log_kv_cache.py:6802-6836 for the first-order mid-anchor
    path (``second_order_scale == 0``); the packed workspace and the softmax
    run in the HIP library. With ``reuse_prefix`` (inference, at most two query
    rows) the packed prefix is kept on the cache and later steps re-pack only
    their new rows, as in litgpt/log_kv_cache.py:6772-6799.
    """
    if q_b.dtype != torch.bfloat16 or k_b.dtype != torch.bfloat16 or v_b.dtype != torch.bfloat16:
        # float16 / float32 activations: the rows are rounded to the cache's bf16 storage and the output
        # is returned in the queries' dtype (both casts differentiable).
        out = log_kv_chunk_attention(cache, as_storage(q_b), as_storage(k_b), as_storage(v_b), scale,
                                     second_order_scale, attention_plan, causal_tail=causal_tail,
                                     reuse_prefix=reuse_prefix)
        return out.to(q_b.dtype)
    causal_tail = q_b.size(2) if causal_tail is None else causal_tail
    if causal_tail and causal_tail != q_b.size(2):
        raise ValueError("causal_tail must equal query length or be zero")
    if second_order_scale != 0.0 or not cache.semantic_clusters or cache.semantic_anchor_mode != "mid":
        raise NotImplementedError("logkv_amd reads out the first-order mid-anchor path (second_order_scale=0)")
    _check_backend(cache.semantic_pack_backend)
    _check_kv(cache, k_b, v_b)
    if not 1e-3 <= scale <= 1.0:
        raise NotImplementedError("attention scale must lie in [1e-3, 1]")
    if q_b.ndim != 4 or q_b.size(0) != cache.batch_size or q_b.size(1) % cache.n_groups \
            or q_b.size(-1) != cache.k_dim or q_b.device != k_b.device:
        raise ValueError("queries must be [B, n_heads, t, k_dim] on the cache's device with n_heads % n_groups == 0")
    dim = packed_dim(k_b.size(-1), v_b.size(-1))
    view = readout_view(cache)
    if torch.is_grad_enabled() and (q_b.requires_grad or k_b.requires_grad or v_b.requires_grad):
        # Training: the prefix is detached state; the gradient reaches the queries and the chunk.
        plan = semantic_mid_attention_plan(cache, view) if attention_plan is None else attention_plan
        cap = _decode_capacity(cache, k_b.size(2))
        ka = k_b.new_empty(*k_b.shape[:2], cap, dim)
        va = v_b.new_empty(*v_b.shape[:2], cap, dim)
        _launch_pack(cache, view, plan, k_b.detach(), v_b.detach(), dim, ka, va, False, 0)
        exact = cache.alpha_count_dev if cache.alpha_exact_tokens else None
        return _PackedAttention.apply(q_b, k_b, v_b, ka, va, plan, cache.recent_count + k_b.size(2), scale,
                                      causal_tail, v_b.size(-1), cache.n_groups, exact, None)
    reuse = (reuse_prefix and not torch.is_grad_enabled() and q_b.size(2) <= 2
             and not k_b.requires_grad and not v_b.requires_grad)
    key = (k_b.device, k_b.dtype, dim, id(cache.cos_cache), id(cache.sin_cache))
    buffers, skip_pooled, recent_start = None, False, 0
    if reuse:
        saved = cache._mid_decode_state
        if saved is not None and saved[0] == key:
            _, plan, buffers, recent_start, workspace = saved
            skip_pooled = True
        else:
            plan = semantic_mid_attention_plan(cache, view) if attention_plan is None else attention_plan
            workspace = None
        if buffers is None:
            cap = _decode_capacity(cache, k_b.size(2))
            buffers = (k_b.new_empty(*k_b.shape[:2], cap, dim), v_b.new_empty(*v_b.shape[:2], cap, dim))
    else:
        plan = semantic_mid_attention_plan(cache, view) if attention_plan is None else attention_plan
        workspace = None
        cap = _decode_capacity(cache, k_b.size(2))
        buffers = (k_b.new_empty(*k_b.shape[:2], cap, dim), v_b.new_empty(*v_b.shape[:2], cap, dim))
    ka, va = buffers
    _launch_pack(cache, view, plan, k_b, v_b, dim, ka, va, skip_pooled, recent_start)
    exact = cache.alpha_count_dev if cache.alpha_exact_tokens else None
    tail = cache.recent_count + k_b.size(2)
    out, workspace = packed_attention(q_b, ka, va, plan, tail, scale, causal_tail, v_b.size(-1), cache.n_groups,
                                      workspace, exact)
    if reuse:
        cache._mid_decode_state = (key, plan, buffers, cache.recent_count, workspace)
    return out


def attention_state(cache, plan):
    """The cache's attention state as unpacked slots (litgpt/log_kv_cache.py:6009-6114, first order):
    ``slot_k`` the pooled keys RoPE'd at their mid anchors, the exact pool's keys RoPE'd at their
    positions and the recent window's keys, ``slot_v`` the values, ``slot_w`` the pooled masses (1 for
    exact valid and recent rows), ``slot_valid`` over [pooled | exact] and ``M_s`` ones. Built by one
    pack launch that also writes every row's mass and validity; rows that are masked (pooled padding,
    invalid exact rows) are zero."""
    from .log_kv_cache import CacheAttentionState

    B, G, dk, dv = cache.batch_size, cache.n_groups, cache.k_dim, cache.v_dim
    dev = cache.level_k.device
    width, exact, recent = plan.width, cache.alpha_count, cache.recent_count
    rows = width + exact + recent
    dim = packed_dim(dk, dv)
    ka = torch.empty(B, G, max(rows, 1), dim, dtype=cache.level_k.dtype, device=dev)
    va = torch.empty_like(ka)
    w = torch.empty(B, G, max(rows, 1), dtype=torch.float32, device=dev)
    valid = torch.empty(B, G, max(rows, 1), dtype=torch.uint8, device=dev)
    empty = torch.empty(B, G, 0, dk, dtype=cache.level_k.dtype, device=dev)
    if rows:
        _launch_pack(cache, readout_view(cache), plan, empty, empty, dim, ka, va, False, 0, w, valid)
    slot_valid = valid[:, :, :width + exact].bool()
    act = cache.activation_dtype
    return CacheAttentionState(ka[:, :, :rows, :dk].to(act), va[:, :, :rows, :dv].to(act), w[:, :, :rows],
                               slot_valid=slot_valid,
                               M_s=torch.ones(B, G, width + exact, dtype=torch.int64, device=dev))


def append_exact_tokens(state, k_new, v_new):
    """The state with exact entries (mass 1) appended after its slots (litgpt/log_kv_cache.py:6391-6425):
    the in-flight chunk attends before it is committed. ``slot_valid`` / ``M_s`` cover the prefix only and
    pass through; appended entries get zero rank-1 statistics when the state carries them."""
    stats = (state.slot_sigma_u, state.slot_sigma2, state.slot_gamma_a, state.slot_gamma_b, state.slot_gamma)
    have = [x is not None for x in stats]
    if any(have) and not all(have):
        raise ValueError("append_exact_tokens() requires either all rank-1 stats or none")
    n = k_new.size(2)
    mass = state.slot_w.new_ones(state.slot_w.size(0), state.slot_w.size(1), n)
    grown = state._replace(slot_k=torch.cat([state.slot_k, k_new], dim=2), slot_v=torch.cat([state.slot_v, v_new], dim=2),
                           slot_w=torch.cat([state.slot_w, mass], dim=-1))
    if not all(have):
        return grown
    zero_row = mass.new_zeros(mass.shape)
    return grown._replace(
        slot_sigma_u=torch.cat([state.slot_sigma_u, torch.zeros_like(k_new)], dim=2),
        slot_sigma2=torch.cat([state.slot_sigma2, zero_row], dim=-1),
        slot_gamma_a=torch.cat([state.slot_gamma_a, torch.zeros_like(k_new)], dim=2),
        slot_gamma_b=torch.cat([state.slot_gamma_b, torch.zeros_like(v_new)], dim=2),
        slot_gamma=torch.cat([state.slot_gamma, zero_row], dim=-1))


def _slot_rows_visible(slot_valid, slots, tq, causal_tail):
    """Whether every query row keeps at least one visible valid slot (host check)."""
    s_valid = slot_valid.size(-1)
    if s_valid < slots - causal_tail or (causal_tail and s_valid < slots):
        return True   # an always-valid slot past the prefix is visible to every query
    dev = slot_valid.device
    cols = torch.arange(slots, device=dev)
    rows = torch.arange(tq, device=dev)
    visible = torch.ones(tq, slots, dtype=torch.bool, device=dev)
    if causal_tail:
        visible = (cols[None, :] < slots - causal_tail) | (cols[None, :] - (slots - causal_tail) <= rows[:, None])
    valid = torch.ones(*slot_valid.shape[:2], slots, dtype=torch.bool, device=dev)
    valid[..., :s_valid] = slot_valid
    return bool((valid[:, :, None, :] & visible).any(-1).all())


def log_kv_slot_attention(q, slot_k, slot_v, slot_w, scale, mask=None, lam=1.0, causal_tail=0, slot_M=None,
                          slot_valid=None, check_valid=True, slot_sigma_u=None, slot_sigma2=None, slot_gamma_a=None,
                          slot_gamma_b=None, slot_gamma=None, second_order_scale=1.0):
    """First-order slot attention ``softmax(scale * q.k_s + lam * log w_s - log M_s) . v_s`` over unpacked
    slots (litgpt/log_kv_cache.py:6501-6721), evaluated as the reference's Flash path does: each slot's
    bias rides in an extra key coordinate (rounded to bf16) against ``1/scale`` in the query, invalid
    slots carry -10000. The slots are packed on the device (``logkv_pack_slots``) and read by the
    decode / matrix-core attention kernels. ``q [B, nh, T_q, dk]``, slots ``[B, G, S, .]``; the last
    ``causal_tail`` slots are the in-flight chunk, causal against the queries."""
    B, nh, tq, dk = q.shape
    S = slot_k.size(2)
    if S == 0:
        return torch.zeros(B, nh, tq, slot_v.size(-1), device=q.device, dtype=q.dtype)
    stats = (slot_sigma_u, slot_sigma2, slot_gamma_a, slot_gamma_b, slot_gamma)
    if slot_sigma_u is not None and any(x is None for x in stats):
        raise ValueError("log_kv_slot_attention() requires either all rank-1 stats or none")
    if causal_tail:
        if mask is not None:
            raise ValueError("causal_tail and mask are mutually exclusive")
        if causal_tail != tq:
            raise ValueError(f"causal_tail ({causal_tail}) must equal T_q ({tq}): the tail entries are the "
                             "appended in-flight chunk, aligned one-to-one with the queries")
    if slot_sigma_u is not None and second_order_scale != 0.0:
        raise NotImplementedError("logkv_amd reads out first-order slots only (no rank-1 statistics)")
    if mask is not None:
        raise NotImplementedError("logkv_amd masks through causal_tail and slot_valid, not a (T_q, S) mask")
    if q.dtype != torch.bfloat16 or slot_k.dtype != torch.bfloat16 or slot_v.dtype != torch.bfloat16:
        # float16 / float32 activations: queries and slots rounded to bf16, the output in q's dtype.
        return log_kv_slot_attention(as_storage(q), as_storage(slot_k), as_storage(slot_v), slot_w, scale, mask,
                                     lam, causal_tail, slot_M, slot_valid, check_valid, slot_sigma_u, slot_sigma2,
                                     slot_gamma_a, slot_gamma_b, slot_gamma, second_order_scale).to(q.dtype)
    if not math.isfinite(scale) or not 1e-3 <= scale <= 1.0:
        raise NotImplementedError("attention scale must lie in [1e-3, 1]")
    G = slot_k.size(1)
    if nh % G or slot_k.shape[:3] != (B, G, S) or slot_v.shape[:3] != (B, G, S) or slot_w.shape != (B, G, S) \
            or slot_k.size(-1) != dk:
        raise ValueError("slots must be [B, G, S, d] with G dividing the query heads and masses [B, G, S]")
    for t, what in ((q, "q"), (slot_k, "slot_k"), (slot_v, "slot_v"), (slot_w, "slot_w")):
        require_device(t, what)
    if slot_valid is not None and check_valid and not _slot_rows_visible(slot_valid, S, tq, causal_tail):
        raise ValueError("log_kv_slot_attention(): a query row has no valid slot")
    dv = slot_v.size(-1)
    dim = packed_dim(dk, dv)
    ka = q.new_empty(B, G, S, dim)
    va = q.new_empty(B, G, S, dim)
    w = slot_w.float()
    if slot_k.stride(-1) != 1 or slot_v.stride(-1) != 1:
        raise ValueError("slot keys and values need contiguous features")
    m = None if slot_M is None else slot_M.to(torch.int64)
    valid = None if slot_valid is None else slot_valid.to(torch.uint8)
    slot_k_d, slot_v_d = slot_k.detach(), slot_v.detach()
    args = SlotPackArgs(ptr(slot_k_d), *slot_k.stride()[:3], ptr(slot_v_d), *slot_v.stride()[:3], ptr(w), *w.stride()[:2],
                        ptr(m), *(m.stride()[:2] if m is not None else (0, 0)), 0 if m is None else m.size(-1),
                        ptr(valid), *(valid.stride()[:2] if valid is not None else (0, 0)),
                        0 if valid is None else valid.size(-1), float(lam), B, G, S, dk, dv, dim, S, ptr(ka), ptr(va))
    check(lib().logkv_pack_slots(C.byref(args), stream_of(q.device)), "logkv_pack_slots")
    plan = MidAttentionPlan(torch.zeros(1, dtype=torch.int32, device=q.device), 0, 0)
    if torch.is_grad_enabled() and (q.requires_grad or slot_k.requires_grad or slot_v.requires_grad):
        mask = None
        if valid is not None:
            mask = torch.ones(B, G, S, dtype=q.dtype, device=q.device)
            mask[..., :valid.size(-1)] = valid.to(q.dtype)
        return _PackedAttention.apply(q, slot_k, slot_v, ka, va, plan, S, scale, causal_tail, dv, G, None, mask)
    return packed_attention(q, ka, va, plan, S, scale, causal_tail, dv, G)[0]
