"""Attention readout: mid-anchor slot plan, packed K/V workspace, mass-biased attention.

TEST INFRASTRUCTURE ONLY (the oracle).

* plan: per lane, occupied slots cluster-major, top level first, slots in
  order; ``anchor = (2*sum_wp + w) // (2*w)`` with ``w`` as an integer >= 1,
  ``valid = occupied and w > 0`` (litgpt/log_kv_cache.py:5979-6007);
* pack: ``[pooled | exact pool | recent | current]`` rows of width
  ``dim = 8*ceil(max(Dk+1, Dv)/8)``; pooled and exact keys are RoPE'd at their
  anchor (rotate-half, products rounded to the table dtype when that is bf16);
  column ``Dk`` carries ``log(max(w, 1))`` for valid pooled slots, 0 for exact
  valid / recent / current rows and -10000 for invalid ones; invalid rows are
  zero otherwise (litgpt/log_kv_pack.py:27-72, litgpt/log_kv_pack_triton.py:12-92,
  litgpt/log_kv_position.py:74-101);
* attention: ``softmax(scale * [q, 1/scale] . [k, bias])`` over the packed rows,
  the last ``causal_tail`` rows causal against the queries, GQA by
  ``head // (Hq / G)`` (litgpt/log_kv_cache.py:6428-6464, :6751-6758). The oracle
  evaluates it in float64 from the bf16 operands.
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_round, f32


def packed_dim(dk: int, dv: int) -> int:
    return ((max(dk + 1, dv) + 7) // 8) * 8


def mid_plan(level_count, level_w, level_sum_wp):
    """(indices [Bt,G,S], anchors, valid) with indices flat over (cluster, level, slot)."""
    n_batch, n_groups, K, L = level_count.shape
    B = level_w.shape[-1]
    lanes = []
    for b in range(n_batch):
        for g in range(n_groups):
            idx = []
            for c in range(K):
                for ell in range(L - 1, -1, -1):
                    base = (c * L + ell) * B
                    idx.extend(range(base, base + int(level_count[b, g, c, ell])))
            lanes.append(idx)
    width = max((len(x) for x in lanes), default=0)
    indices = np.full((n_batch, n_groups, width), -1, dtype=np.int64)
    for lane, idx in enumerate(lanes):
        indices[lane // n_groups, lane % n_groups, :len(idx)] = idx
    occupied = indices >= 0
    safe = np.maximum(indices, 0)
    w = np.take_along_axis(level_w.reshape(n_batch, n_groups, -1), safe, axis=2)
    s = np.take_along_axis(level_sum_wp.reshape(n_batch, n_groups, -1), safe, axis=2)
    valid = occupied & (w > 0)
    ww = np.maximum(w.astype(np.int64), 1)
    anchors = np.floor_divide(2 * s + ww, 2 * ww)
    anchors = np.where(valid, anchors, 0)
    return safe, anchors, valid


def rope(x, anchors, cos, sin, table_bf16=False):
    """Rotate-half RoPE of bf16-valued ``x [..., D]`` at integer ``anchors [...]`` -> bf16 values.

    ``table_bf16``: the cos/sin tables are bf16, so each product rounds to bf16
    before the sum (litgpt/log_kv_pack_triton.py:61-65)."""
    x = f32(x)
    n = cos.shape[1]
    half = n // 2
    c = f32(cos)[anchors]
    s = f32(sin)[anchors]
    xr = x[..., :n]
    rotated = np.concatenate((-xr[..., half:], xr[..., :half]), axis=-1)
    if table_bf16:
        a = bf16_round(xr * c)
        b = bf16_round(rotated * s)
        out = bf16_round(a + b)
    else:
        out = bf16_round(xr * c + rotated * s)
    return np.concatenate((out, x[..., n:]), axis=-1)


def pack(state, k_cur, v_cur, cos, sin, plan=None, table_bf16=False):
    """Packed K/V ``[Bt, G, S_tot, dim]`` as bf16-valued float32 arrays."""
    dk, dv = state.level_k.shape[-1], state.level_v.shape[-1]
    dim = packed_dim(dk, dv)
    n_batch, n_groups = state.level_k.shape[:2]
    if plan is None:
        plan = mid_plan(state.level_count, state.level_w, state.level_sum_wp)
    idx, anchors, valid = plan
    pooled = idx.shape[-1]
    exact = state.alpha_count
    recent = state.recent_count
    cur = 0 if k_cur is None else k_cur.shape[2]
    total = pooled + exact + recent + cur
    ka = np.zeros((n_batch, n_groups, total, dim), np.float32)
    va = np.zeros_like(ka)
    flat_k = state.level_k.reshape(n_batch, n_groups, -1, dk)
    flat_v = state.level_v.reshape(n_batch, n_groups, -1, dv)
    flat_w = state.level_w.reshape(n_batch, n_groups, -1)
    if pooled:
        kk = np.take_along_axis(flat_k, idx[..., None], axis=2)
        vv = np.take_along_axis(flat_v, idx[..., None], axis=2)
        ww = np.take_along_axis(flat_w, idx, axis=2)
        keys = rope(kk, anchors, cos, sin, table_bf16)
        ka[:, :, :pooled, :dk] = np.where(valid[..., None], keys, 0)
        va[:, :, :pooled, :dv] = np.where(valid[..., None], vv, 0)
        bias = bf16_round(np.log(np.maximum(ww, np.float32(1.0))).astype(np.float32))
        ka[:, :, :pooled, dk] = np.where(valid, bias, bf16_round(np.float32(-10000.0)))
    if exact:
        ev = np.broadcast_to(state.alpha_valid[:, None, :exact], (n_batch, n_groups, exact))
        ea = np.broadcast_to(state.alpha_pos[:, None, :exact], (n_batch, n_groups, exact))
        keys = rope(state.alpha_k_raw[:, :, :exact], np.where(ev, ea, 0), cos, sin, table_bf16)
        ka[:, :, pooled:pooled + exact, :dk] = np.where(ev[..., None], keys, 0)
        va[:, :, pooled:pooled + exact, :dv] = np.where(ev[..., None], state.alpha_v[:, :, :exact], 0)
        ka[:, :, pooled:pooled + exact, dk] = np.where(ev, 0.0, bf16_round(np.float32(-10000.0)))
    p = pooled + exact
    ka[:, :, p:p + recent, :dk] = state.recent_k[:, :, :recent]
    va[:, :, p:p + recent, :dv] = state.recent_v[:, :, :recent]
    if cur:
        ka[:, :, p + recent:, :dk] = f32(k_cur)
        va[:, :, p + recent:, :dv] = f32(v_cur)
    return ka, va


def attention(q, ka, va, scale, causal_tail, dv):
    """float64 attention of bf16-valued queries ``[Bt, Hq, Tq, Dk]`` over the packed rows."""
    q = f32(q)
    n_batch, hq, tq, dk = q.shape
    n_groups, total, dim = ka.shape[1], ka.shape[2], ka.shape[3]
    qa = np.zeros((n_batch, hq, tq, dim), np.float64)
    qa[..., :dk] = q
    qa[..., dk] = float(np.asarray(bf16_round(np.float32(1.0 / scale))).reshape(-1)[0])
    rep = hq // n_groups
    kk = np.repeat(ka.astype(np.float64), rep, axis=1)
    vv = np.repeat(va.astype(np.float64), rep, axis=1)
    scores = scale * np.einsum("bhqd,bhsd->bhqs", qa, kk)
    if causal_tail:
        start = total - causal_tail
        for i in range(tq):
            scores[:, :, i, start + i + 1:] = -np.inf
    scores -= scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqs,bhsd->bhqd", p, vv)[..., :dv]


def slot_pack(slot_k, slot_v, slot_w, lam=1.0, slot_M=None, slot_valid=None):
    """Packed rows of unpacked slots, the Flash encoding of log_kv_slot_attention
    (litgpt/log_kv_cache.py:6418-6464, anchor_mass_bias litgpt/log_kv_position.py:128-133):
    keys and values copied, column Dk = ``lam * log(w)`` (0 when ``lam == 0``), or for the first
    ``slot_M`` columns ``-log(max(M, 1)) + lam * log(max(w, 1))``, in float32 and rounded to
    bf16; among the first ``slot_valid`` columns, invalid slots are zero rows with bias -10000."""
    slot_k, slot_v, w = f32(slot_k), f32(slot_v), f32(slot_w)
    n_batch, n_groups, S, dk = slot_k.shape
    dv = slot_v.shape[-1]
    dim = packed_dim(dk, dv)
    ka = np.zeros((n_batch, n_groups, S, dim), np.float32)
    va = np.zeros_like(ka)
    with np.errstate(divide="ignore"):
        bias = (np.float32(lam) * np.log(w)).astype(np.float32) if lam != 0.0 else np.zeros_like(w)
        if slot_M is not None:
            s_m = slot_M.shape[-1]
            m = -np.log(np.maximum(np.asarray(slot_M, np.float32), np.float32(1.0))).astype(np.float32)
            if lam != 0.0:
                m = (m + np.float32(lam) * np.log(np.maximum(w[..., :s_m], np.float32(1.0)))).astype(np.float32)
            bias[..., :s_m] = m
    valid = np.ones((n_batch, n_groups, S), bool)
    if slot_valid is not None:
        valid[..., :slot_valid.shape[-1]] = np.asarray(slot_valid, bool)
    ka[..., :dk] = np.where(valid[..., None], slot_k, 0)
    va[..., :dv] = np.where(valid[..., None], slot_v, 0)
    ka[..., dk] = np.where(valid, bf16_round(bias), bf16_round(np.float32(-10000.0)))
    return ka, va


def attention_grad(q, ka, va, scale, causal_tail, dv, dout, grad_rows):
    """float64 gradients of ``attention``: (dq ``[Bt, Hq, Tq, Dk]``, dk and dv of the last
    ``grad_rows`` packed rows ``[Bt, G, grad_rows, D]``), the textbook softmax backward
    (litgpt/log_kv_cache.py:6867-7098 takes them per block through autograd): with
    ``p = softmax(scale * qa . ka)``, ``D = dout . o`` and ``ds = p * (dout . va - D)``,
    ``dq = scale * ds . ka[:Dk]``, ``dk = scale * ds^T . q`` and ``dv = p^T . dout``, summed over
    the query heads of a KV group; the bias coordinate carries no gradient."""
    q = f32(q).astype(np.float64)
    dout = f32(dout).astype(np.float64)
    n_batch, hq, tq, dk = q.shape
    n_groups, total, dim = ka.shape[1], ka.shape[2], ka.shape[3]
    rep = hq // n_groups
    qa = np.zeros((n_batch, hq, tq, dim), np.float64)
    qa[..., :dk] = q
    qa[..., dk] = float(np.asarray(bf16_round(np.float32(1.0 / scale))).reshape(-1)[0])
    kk = np.repeat(ka.astype(np.float64), rep, axis=1)
    vv = np.repeat(va.astype(np.float64), rep, axis=1)
    scores = scale * np.einsum("bhqd,bhsd->bhqs", qa, kk)
    if causal_tail:
        start = total - causal_tail
        for i in range(tq):
            scores[:, :, i, start + i + 1:] = -np.inf
    scores -= scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    o = np.einsum("bhqs,bhsd->bhqd", p, vv[..., :dv])
    dp = np.einsum("bhqd,bhsd->bhqs", dout, vv[..., :dv])
    ds = p * (dp - (dout * o).sum(-1, keepdims=True))
    dq = scale * np.einsum("bhqs,bhsd->bhqd", ds, kk[..., :dk])
    dk_all = scale * np.einsum("bhqs,bhqd->bhsd", ds, q)
    dv_all = np.einsum("bhqs,bhqd->bhsd", p, dout)
    dk_g = dk_all.reshape(n_batch, n_groups, rep, total, dk).sum(2)
    dv_g = dv_all.reshape(n_batch, n_groups, rep, total, dv).sum(2)
    return dq, dk_g[:, :, total - grad_rows:], dv_g[:, :, total - grad_rows:]
