"""Alpha exact spans: whole-span candidates, device scoring, bounded greedy choice.

Call surface of the reference module (litgpt/alpha_log_kv.py): ``SpanSelection``,
``SpanCut``, ``cut_spans``, ``score_spans``, ``choose_spans``, ``select_spans``
- host span cutting and greedy choice over host position / boundary lists, as
in the reference, with scoring in the HIP library (``logkv_score_spans``).
Indices there refer to ``[old exact pool (old_width rows) | current flush]``.

A cache's flush (``alpha_flush``) runs the same selection on the device
instead (``logkv_alpha_select``: candidates, scores and greedy against the
selection state the cache keeps on the device), then the exact-pool / archive
split (``logkv_alpha_partition``); there indices address ``[pool (P rows) |
flush]``.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib


@dataclass
class SpanSelection:
    keep: list[list[int]]
    archive: list[list[int]]
    spans: list[list[tuple[int, bool]]]
    positions: list[list[int]]


@dataclass
class SpanCut:
    """Candidate whole spans of one flush; host data only.

    ``candidates[b]`` = (list of (token ranges, old, closed), positions of the
    row's ``[pool | flush]`` rows); ``token_rows[b]`` flat token indices in span
    order; ``length_rows[b]`` span lengths.
    """
    candidates: list
    token_rows: list
    length_rows: list


def _cut_row(spans, old_pos, new_pos, flags, old_width, max_span):
    """One row's candidates ``[(ranges, old, closed)]`` and its ``[pool | flush]`` positions.

    Closed old spans are candidates as they are. The row's last unfinished old span (the tail) and
    the flush tokens are then walked as one sequence, in combined coordinates: ``c < t`` is the
    tail's ``c``-th token (pool row ``t0 + c``), ``c >= t`` the flush's token ``c - t`` (row
    ``old_width + c - t``). A run of that sequence closes at a boundary token or when its hard
    segment reaches a multiple of ``max_span`` tokens, and a position jump closes the open run
    before the jumping token; the run open at the end stays unfinished. The tail's own tokens never
    close a run (the previous flush left it open), they only count toward the first segment, and a
    tail of ``max_span`` tokens or more disables the cap until that segment ends. A run is reported
    as one row range per side of the tail / flush border it covers.
    """
    row, tail, offset = [], None, 0
    for length, closed in spans:
        if closed:
            row.append(([(offset, offset + length)], True, True))
        else:
            tail = (offset, length)
        offset += length
    positions = np.zeros(old_width + len(new_pos), dtype=np.int64)
    positions[:len(old_pos)] = old_pos
    positions[old_width:] = new_pos
    t0, t = tail if tail is not None else (0, 0)

    def ranges(a, z):
        out = [(t0 + a, t0 + min(z, t))] if a < t else []
        if z > t:
            out.append((old_width + max(a, t) - t, old_width + z - t))
        return out

    start, depth, capped = 0, t, t < max_span
    prev = int(positions[t0 + t - 1]) if t else None
    for i, p in enumerate(int(x) for x in new_pos):
        c = t + i
        if prev is not None and p != prev + 1:
            if start < c:
                row.append((ranges(start, c), False, True))
            start, depth, capped = c, 0, True
        prev = p
        depth += 1
        if flags[i] or (capped and depth % max_span == 0):
            row.append((ranges(start, c + 1), False, True))
            start = c + 1
            if flags[i]:
                depth, capped = 0, True
    if start < t + len(new_pos):
        row.append((ranges(start, t + len(new_pos)), False, False))
    return row, positions


def cut_spans(old_spans, old_positions, new_positions, ends, old_width, max_span):
    """Whole candidate spans per row (host only); None when no row has one
    (litgpt/alpha_log_kv.py:84-122).

    Row indices address ``[old exact pool (old_width rows) | current flush]``. A row's candidates
    are its closed old spans (old), then the runs of its unfinished old span followed by the flush
    (``_cut_row``): a position jump right after that span closes it alone, otherwise the flush's
    first run continues it. Each candidate is ``(ranges, old, closed)``.
    """
    candidates, token_rows, length_rows = [], [], []
    for spans, old_pos, new_pos, flags in zip(old_spans, old_positions, new_positions, ends):
        row, positions = _cut_row(spans, old_pos, new_pos, flags, old_width, max_span)
        candidates.append((row, positions))
        token_rows.append(np.asarray([i for rs, _, _ in row for a, z in rs for i in range(a, z)], dtype=np.int64))
        length_rows.append([sum(z - a for a, z in rs) for rs, _, _ in row])
    if not any(length_rows):
        return None
    return SpanCut(candidates, token_rows, length_rows)


def _span_tables(cut: SpanCut, device):
    """Device tables of the candidates: tokens int32, span offsets int32, span row int32."""
    tokens = np.concatenate(cut.token_rows).astype(np.int32)
    lengths = np.concatenate([np.asarray(x, dtype=np.int64) for x in cut.length_rows])
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    rows = np.repeat(np.arange(len(cut.length_rows)), [len(x) for x in cut.length_rows]).astype(np.int32)
    packed = np.concatenate((tokens, offsets, rows)).astype(np.int32)
    dev = torch.from_numpy(packed).pin_memory().to(device, non_blocking=True) if device.type == "cuda" else \
        torch.from_numpy(packed).to(device)
    n_tok, n_span = len(tokens), len(lengths)
    return dev, dev[:n_tok], dev[n_tok:n_tok + n_span + 1], dev[n_tok + n_span + 1:], n_span


def score_spans_split(pool_k, pool_v, flush_k, flush_v, old_width, cut: SpanCut, *, beta_novelty=False,
                      centroids=None, centroid_valid=None):
    """Scores of the candidates over ``[pool[:, :, :old_width] | flush]`` without materialising the cat."""
    if beta_novelty and (centroids is None or centroid_valid is None):
        raise ValueError("Beta span scoring requires centroids and centroid_valid from before the flush")
    dev = flush_k.device
    _lib.require_device(flush_k, "span scoring keys")
    keep, tokens, offsets, rows, n_span = _span_tables(cut, dev)
    out = torch.empty(n_span, dtype=torch.float32, device=dev)
    if pool_k is None:
        pool_k, pool_v = flush_k, flush_v
    args = _lib.SpanArgs(
        _lib.ptr(pool_k), pool_k.stride(0), pool_k.stride(1), pool_k.stride(2),
        _lib.ptr(pool_v), pool_v.stride(0), pool_v.stride(1), pool_v.stride(2),
        _lib.ptr(flush_k), flush_k.stride(0), flush_k.stride(1), flush_k.stride(2),
        _lib.ptr(flush_v), flush_v.stride(0), flush_v.stride(1), flush_v.stride(2),
        int(old_width), _lib.ptr(tokens), _lib.ptr(offsets), _lib.ptr(rows), n_span,
        flush_k.size(1), flush_k.size(-1), flush_v.size(-1),
        _lib.ptr(centroids) if beta_novelty else None, _lib.ptr(centroid_valid) if beta_novelty else None,
        centroids.size(2) if beta_novelty else 0, 1 if beta_novelty else 0)
    rc = _lib.lib().logkv_score_spans(C.byref(args), _lib.ptr(out), _lib.stream_of(dev))
    _lib.check(rc, "logkv_score_spans")
    out._logkv_keepalive = (keep, pool_k, pool_v, flush_k, flush_v, centroids, centroid_valid)
    return out


def score_spans(k, v, cut, *, beta_novelty=False, centroids=None, centroid_valid=None):
    """Device tensor of span scores in candidate order (litgpt/alpha_log_kv.py:125-174)."""
    for t in (k, v):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError("span scoring needs bf16 K/V with a contiguous last axis")
    if beta_novelty:
        centroids = centroids.float().contiguous()
        centroid_valid = centroid_valid.contiguous()
    return score_spans_split(None, None, k, v, 0, cut, beta_novelty=beta_novelty, centroids=centroids,
                             centroid_valid=centroid_valid)


def choose_spans(cut: SpanCut, host_scores, budget) -> SpanSelection:
    """Bounded whole-span greedy from host scores in candidate order (litgpt/alpha_log_kv.py:177-226).

    Per row, a candidate's density is its score, times 1.1 for an old span. Unfinished spans are
    kept unconditionally and old closed spans start kept; while over budget, kept closed spans are
    evicted cheapest first (lowest density, later candidate on ties). The remaining candidates are
    then offered densest first (earlier on ties): one fits in the free room, or displaces the
    cheapest kept closed spans only if its density * length strictly exceeds their summed
    density * length. A span kept this way may itself be displaced later.
    """
    keep, archive, out_spans, out_pos = [], [], [], []
    base = 0
    for (row, positions), tokens, sizes in zip(cut.candidates, cut.token_rows, cut.length_rows):
        n = len(row)
        dens = [float(host_scores[base + i]) * (1.1 if row[i][1] else 1.0) for i in range(n)]
        base += n
        cost_key = lambda i: (dens[i], -i)  # noqa: E731  cheapest victim first
        kept = [row[i][1] or not row[i][2] for i in range(n)]
        room = budget - sum(sizes[i] for i in range(n) if kept[i])
        # Kept closed spans in eviction order; kept in order as candidates join it.
        victims = sorted((i for i in range(n) if kept[i] and row[i][2]), key=cost_key)
        while room < 0 and victims:
            j = victims.pop(0)
            kept[j] = False
            room += sizes[j]
        for i in sorted((i for i in range(n) if not kept[i]), key=lambda i: (-dens[i], i)):
            need, free, lost, taken = sizes[i], room, 0.0, 0
            while free < need and taken < len(victims):
                j = victims[taken]
                free += sizes[j]
                lost += dens[j] * sizes[j]
                taken += 1
            if free < need or (taken and not dens[i] * need > lost):
                continue
            for j in victims[:taken]:
                kept[j] = False
            del victims[:taken]
            kept[i] = True
            room = free - need
            at = 0
            while at < len(victims) and cost_key(victims[at]) < cost_key(i):
                at += 1
            victims.insert(at, i)
        mask = np.repeat(np.asarray(kept, dtype=bool), sizes) if n else np.zeros(0, dtype=bool)
        keep.append(tokens[mask].tolist())
        archive.append(tokens[~mask].tolist())
        out_spans.append([(sizes[i], row[i][2]) for i in range(n) if kept[i]])
        out_pos.append(positions[tokens[mask]].tolist())
    return SpanSelection(keep, archive, out_spans, out_pos)


def select_spans(k, v, old_spans, old_positions, new_positions, ends, old_width, budget, max_span, *,
                 beta_novelty=False, centroids=None, centroid_valid=None):
    """Cut, score on the device (one score readback) and choose (litgpt/alpha_log_kv.py:69-81)."""
    cut = cut_spans(old_spans, old_positions, new_positions, ends, old_width, max_span)
    if cut is None:
        rows = len(ends)
        return SpanSelection([[] for _ in range(rows)], [[] for _ in range(rows)],
                             [[] for _ in range(rows)], [[] for _ in range(rows)])
    scores = score_spans(k, v, cut, beta_novelty=beta_novelty, centroids=centroids, centroid_valid=centroid_valid)
    return choose_spans(cut, scores.cpu().tolist(), budget)


def _table(rows, width, device):
    t = np.full((len(rows), max(width, 1)), -1, dtype=np.int32)
    for b, r in enumerate(rows):
        t[b, :len(r)] = r
    return torch.from_numpy(t).pin_memory().to(device, non_blocking=True)


def _pinned_upload(array: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(array).pin_memory().to(device, non_blocking=True)


def _span_ends_device(span_ends, n_batch: int, T: int, device) -> torch.Tensor:
    """Boundary flags as uint8 ``[n_batch, T]`` on the device: a device tensor
    (bool or uint8) is used in place, host lists are uploaded."""
    if isinstance(span_ends, torch.Tensor):
        if span_ends.device != device or span_ends.shape != (n_batch, T) or span_ends.stride(-1) != 1:
            raise ValueError("span_ends must be [batch, T] on the cache's device with contiguous rows")
        if span_ends.dtype == torch.bool:
            return span_ends.view(torch.uint8)
        if span_ends.dtype != torch.uint8:
            raise ValueError("span_ends must be bool or uint8")
        return span_ends
    rows = np.zeros((n_batch, T), dtype=np.uint8)
    for b, row in enumerate(span_ends):
        rows[b, :len(row)] = np.frombuffer(bytes(bytearray(bool(x) for x in row)), dtype=np.uint8)
    return _pinned_upload(rows, device)


class _AlphaCall:
    """Argument structs and output buffers of the Alpha flush of one cache, one
    flush length ``T`` and one of the pool's two buffer sets (``parity``): built
    once, then only the flush rows' pointers and strides change per call."""

    def __init__(self, cache, T: int, parity_sets, bufs):
        (pk, pv, ppos, _, slen, sclosed, scount), (nk, nv, npos, nvalid, nlen, nclosed, ncount) = parity_sets
        n_batch, G, P = cache.batch_size, cache.n_groups, cache.alpha_exact_tokens
        self.bufs = bufs
        keep, archive, archive_count, ak, av, ap = bufs["keep"], bufs["archive"], bufs["count"], bufs["k"], \
            bufs["v"], bufs["pos"]
        self.rows = _lib.SpanArgs(
            pk.data_ptr(), pk.stride(0), pk.stride(1), pk.stride(2), pv.data_ptr(), pv.stride(0), pv.stride(1),
            pv.stride(2), None, 0, 0, 0, None, 0, 0, 0, P, None, None, None, 0, G, cache.k_dim, cache.v_dim,
            cache.centroid.data_ptr() if cache.beta_novelty else None,
            cache.alive.data_ptr() if cache.beta_novelty else None, cache.K_max, 1 if cache.beta_novelty else 0,
            None)
        self.select = _lib.AlphaSelectArgs(
            slen.data_ptr(), sclosed.data_ptr(), scount.data_ptr(), ppos.data_ptr(), None, 0, None, 0, T,
            n_batch, P, cache.alpha_span_max_tokens, self.rows, keep.data_ptr(), archive.data_ptr(),
            archive_count.data_ptr(), nlen.data_ptr(), nclosed.data_ptr(), ncount.data_ptr(),
            cache.alpha_count_dev.data_ptr(), None, cache._alpha_count_rows)
        self.sized = False   # the selection workspace is sized on the first call (it checks the row pointers)
        self.part = _lib.PartitionArgs(
            pk.data_ptr(), pk.stride(0), pk.stride(1), pk.stride(2),
            pv.data_ptr(), pv.stride(0), pv.stride(1), pv.stride(2),
            ppos.data_ptr(), ppos.stride(0), None, 0, 0, 0, None, 0, 0, 0, None, 0,
            P, keep.data_ptr(), archive.data_ptr(), P, P + T, n_batch, G, cache.k_dim, cache.v_dim,
            nk.data_ptr(), nv.data_ptr(), npos.data_ptr(), nvalid.data_ptr(),
            ak.data_ptr(), av.data_ptr(), ap.data_ptr())

    def set_rows(self, k_raw, v, positions, ends):
        r, sel, part = self.select.rows, self.select, self.part
        ks, vs = k_raw.stride(), v.stride()
        r.flush_k, r.fk_sb, r.fk_sg, r.fk_st = k_raw.data_ptr(), ks[0], ks[1], ks[2]
        r.flush_v, r.fv_sb, r.fv_sg, r.fv_st = v.data_ptr(), vs[0], vs[1], vs[2]
        sel.new_pos, sel.np_sb = positions.data_ptr(), positions.stride(0)
        sel.ends, sel.ends_sb = ends.data_ptr(), ends.stride(0)
        part.flush_k, part.fk_sb, part.fk_sg, part.fk_st = r.flush_k, ks[0], ks[1], ks[2]
        part.flush_v, part.fv_sb, part.fv_sg, part.fv_st = r.flush_v, vs[0], vs[1], vs[2]
        part.flush_pos, part.fp_sb = sel.new_pos, sel.np_sb


def _alpha_call(cache, T: int, dtype) -> _AlphaCall:
    key = ("alpha", T, cache._alpha_parity)
    call = cache._views.get(key)
    if call is None:
        bufs = cache._views.get(("alpha_bufs", T))
        if bufs is None:
            n_batch, G, P = cache.batch_size, cache.n_groups, cache.alpha_exact_tokens
            A, dev = P + T, cache.alpha_k_raw.device
            bufs = cache._views[("alpha_bufs", T)] = {
                "keep": torch.empty(n_batch, P, dtype=torch.int32, device=dev),
                "archive": torch.empty(n_batch, A, dtype=torch.int32, device=dev),
                "count": torch.empty(n_batch, dtype=torch.int32, device=dev),
                "k": torch.empty(n_batch, G, A, cache.k_dim, dtype=dtype, device=dev),
                "v": torch.empty(n_batch, G, A, cache.v_dim, dtype=dtype, device=dev),
                "pos": torch.empty(n_batch, A, dtype=torch.int64, device=dev),
            }
        current = (cache.alpha_k_raw, cache.alpha_v, cache.alpha_pos, cache.alpha_valid, cache.alpha_span_len,
                   cache.alpha_span_closed, cache.alpha_span_count)
        call = cache._views[key] = _AlphaCall(cache, T, (current, cache._alpha_spare), bufs)
    return call


@torch.no_grad()
def alpha_flush(cache, k_raw, v, positions, positions_host, span_ends, record=False, tape=None):
    """One Alpha flush of ``cache`` (litgpt/log_kv_cache.py:3904-4003), all on the device.

    The span selection (candidates of ``[exact pool | flush]``, scores, bounded
    greedy) runs in ``logkv_alpha_select`` against the selection state the
    cache keeps on the device, so the flush never waits for the host; the
    exact pool is rewritten into the cache's second buffer set (then swapped)
    and the archived rows are attach-routed with delayed joins. Only the
    boundary flags travel from the host, and not even they when given as a
    device tensor. Row indices address ``[pool (P rows) | flush]``;
    ``positions_host`` is not needed. The argument structs and the kept /
    archived row buffers are built once per flush length and reused. With
    ``record`` the archived rows' route decisions are appended to the op-log
    (litgpt/log_kv_cache.py:3782-3788). With an update ``tape`` the flush's
    rows, selection and decisions are saved there and their indices returned.
    """
    if span_ends is None:
        raise ValueError("AlphaLogKV requires natural span boundaries")
    dev = k_raw.device
    T = k_raw.size(2)
    ends = _span_ends_device(span_ends, cache.batch_size, T, dev)
    if positions.dtype != torch.int64 or positions.stride(-1) != 1:
        positions = positions.to(torch.int64).contiguous()
    call = _alpha_call(cache, T, k_raw.dtype)
    call.set_rows(k_raw, v, positions, ends)
    bufs, stream = call.bufs, _lib.stream_of(dev)
    if not call.sized:
        need = int(_lib.lib().logkv_alpha_select_workspace_bytes(C.byref(call.select)))
        if need < 0:
            _lib.check(_lib.LOGKV_EINVAL, "logkv_alpha_select")
        if bufs.get("ws") is None or bufs["ws"].numel() < need:
            bufs["ws"] = torch.empty(need, dtype=torch.uint8, device=dev)
        call.sized = True
    ws = bufs["ws"]
    _lib.check(_lib.lib().logkv_alpha_select(C.byref(call.select), ws.data_ptr(), ws.numel(), stream),
               "logkv_alpha_select")
    _lib.check(_lib.lib().logkv_alpha_partition(C.byref(call.part), stream), "logkv_alpha_partition")
    _swap_pool(cache)
    # Inputs that may be temporaries stay referenced until the next flush on this stream.
    cache._alpha_keep_alive = (ends, positions)
    assign = order = None
    if tape is not None:
        A = bufs["k"].size(2)
        assign = torch.empty(cache.batch_size * cache.n_groups, A, dtype=torch.int8, device=dev)
        order = torch.empty(cache.batch_size, A, dtype=torch.int32, device=dev)
    merges = cache._route_commit(bufs["k"], bufs["v"], bufs["pos"], bufs["count"], assign, order, record=record)
    if tape is None:
        return None
    saved = {"k": tape.save(k_raw), "v": tape.save(v), "pos": tape.save(positions), "ends": tape.save(ends),
             "keep": tape.save(bufs["keep"]), "archive": tape.save(bufs["archive"]), "count": tape.save(bufs["count"]),
             "span_len": tape.save(cache.alpha_span_len), "span_closed": tape.save(cache.alpha_span_closed),
             "span_count": tape.save(cache.alpha_span_count), "alpha_count": tape.save(cache.alpha_count_dev),
             "assign": tape.save(assign, owned=True), "order": tape.save(order, owned=True)}
    # The unified route's old-old merges (its decisions are assign / order as the attach route's).
    for name, t in (merges or {}).items():
        saved[name] = tape.save(t, owned=True)
    return saved


def _swap_pool(cache):
    """The rewritten exact pool (second buffer set) becomes the current one."""
    spare = cache._alpha_spare
    cache._alpha_spare = (cache.alpha_k_raw, cache.alpha_v, cache.alpha_pos, cache.alpha_valid,
                          cache.alpha_span_len, cache.alpha_span_closed, cache.alpha_span_count)
    (cache.alpha_k_raw, cache.alpha_v, cache.alpha_pos, cache.alpha_valid, cache.alpha_span_len,
     cache.alpha_span_closed, cache.alpha_span_count) = spare
    cache._alpha_parity ^= 1


@torch.no_grad()
def alpha_replay(cache, saved):
    """Re-apply a recorded Alpha flush without selecting: the exact-pool rewrite
    and archive gather with the recorded keep / archive tables, the recorded
    span state, then the commit of the archived rows with their recorded attach
    decisions (the replay half of litgpt/log_kv_cache.py:4946-5011)."""
    k_raw, v, positions, ends = saved["k"], saved["v"], saved["pos"], saved["ends"]
    call = _alpha_call(cache, k_raw.size(2), k_raw.dtype)
    call.set_rows(k_raw, v, positions, ends)
    bufs = call.bufs
    for name in ("keep", "archive", "count"):
        bufs[name].copy_(saved[name])
    _lib.check(_lib.lib().logkv_alpha_partition(C.byref(call.part), _lib.stream_of(k_raw.device)),
               "logkv_alpha_partition")
    _swap_pool(cache)
    cache.alpha_span_len.copy_(saved["span_len"])
    cache.alpha_span_closed.copy_(saved["span_closed"])
    cache.alpha_span_count.copy_(saved["span_count"])
    cache.alpha_count_dev.copy_(saved["alpha_count"])
    cache._alpha_keep_alive = (ends, positions)
    cache._commit_only(bufs["k"], bufs["v"], bufs["pos"], bufs["count"], saved["assign"], saved["order"], saved)
