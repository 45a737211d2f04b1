"""Logical KV entries retained at request completion, relative to an uncompressed cache
(litgpt/kv_compression.py:1-82).

An entry is one stored K/V pair of one batch item, layer and KV group. The counts take
the recent window (and a pending tail held by the attention module), the Alpha exact
pool's valid rows (unfinished spans included) and the live ladder entries (slots of
positive mass); they leave out padding, preallocated capacity and packing workspaces,
so they are not a memory figure.

The log-structured counts are reductions over device buffers (one host read per
layer); a dense cache (anything without ``token_count``) is counted from
``processed_tokens``, or from its populated positions for a sliding window, as the
reference does.
"""

from __future__ import annotations

from typing import NamedTuple

_TOTAL_FIELDS = (
    "processed_tokens",
    "layer_group_count",
    "recent_slots",
    "exact_slots",
    "hierarchical_slots",
    "retained_slots",
    "dense_slots",
)


def _with_ratios(counts: dict) -> dict:
    """The totals plus the per-lane mean and the retention / saving / compression ratios
    (None where a denominator is zero; litgpt/kv_compression.py:20-29)."""
    retained, dense = counts["retained_slots"], counts["dense_slots"]
    lanes = counts["layer_group_count"]
    return {
        **counts,
        "retained_slots_per_layer_group": retained / lanes if lanes else None,
        "kv_retention_ratio": retained / dense if dense else None,
        "kv_saving_ratio": 1 - retained / dense if dense else None,
        "kv_compression_factor": dense / retained if dense and retained else None,
    }


class _LayerCount(NamedTuple):
    tokens: int        # the layer's token count (what a dense cache would hold per lane)
    lanes: int         # batch items x KV groups
    recent: int
    exact: int
    hierarchical: int


def _count_layer(attn, processed_tokens: int) -> _LayerCount:
    """One attention layer's retained entries. A log-structured cache (it tracks ``token_count``)
    counts its recent window plus a pending tail the attention module holds, the valid exact-pool
    rows of every KV group and the ladder slots of positive mass (device reductions, one host read);
    a dense cache holds ``processed_tokens`` per lane, or its populated positions when it is a
    sliding window."""
    cache = attn.kv_cache
    if cache is None:
        raise ValueError("every attention layer needs an initialized KV cache to measure compression")
    if hasattr(cache, "token_count"):
        await_flush = getattr(cache, "_await_flush", None)
        if await_flush is not None:
            await_flush()   # a flush queued on the cache's side stream is counted too
        tail = getattr(attn, "_log_kv_pending", None)
        tail_len = 0 if tail is None else tail[0].size(2)
        lanes = cache.batch_size * cache.n_groups
        exact = int(cache.alpha_valid.sum().item()) * cache.n_groups if cache.alpha_exact_tokens else 0
        live = int((cache.level_w > 0).sum().item())
        return _LayerCount(cache.token_count + tail_len, lanes, (cache.recent_count + tail_len) * lanes, exact, live)
    batch, groups = cache.k.shape[:2]
    lanes = batch * groups
    if getattr(cache, "is_sliding_window", False):
        held = int((cache.positions >= 0).sum().item()) * groups
    else:
        held = processed_tokens * lanes
    return _LayerCount(processed_tokens, lanes, held, 0, 0)


def cache_compression_snapshot(model, processed_tokens: int) -> dict:
    """Retained entries of every layer and batch / group lane of ``model``
    (``model.transformer.h[i].attn.kv_cache``), counted before the request's caches are reset
    (litgpt/kv_compression.py:32-76).

    A log-structured layer's own token count (with its attention module's pending tail) is
    authoritative; ``processed_tokens`` counts dense layers, which do not track it.
    ``layer_group_count`` includes the batch dimension. Raises ValueError for a layer without a
    cache, for layers whose token counts disagree and for a model without attention layers.
    """
    layers = [_count_layer(block.attn, processed_tokens) for block in model.transformer.h]
    if not layers:
        raise ValueError("the model has no attention layers to measure KV compression on")
    if len({layer.tokens for layer in layers}) != 1:
        raise ValueError("the layers' KV caches disagree on their token counts")
    tokens = layers[0].tokens
    counts = {
        "processed_tokens": tokens,
        "layer_group_count": sum(layer.lanes for layer in layers),
        "recent_slots": sum(layer.recent for layer in layers),
        "exact_slots": sum(layer.exact for layer in layers),
        "hierarchical_slots": sum(layer.hierarchical for layer in layers),
        "dense_slots": sum(tokens * layer.lanes for layer in layers),
    }
    counts["retained_slots"] = counts["recent_slots"] + counts["exact_slots"] + counts["hierarchical_slots"]
    return _with_ratios({field: counts[field] for field in _TOTAL_FIELDS})


def summarize_compression(records: list[dict]) -> dict:
    """Aggregate request snapshots by their summed entries, not by averaging their ratios
    (litgpt/kv_compression.py:79-82)."""
    counts = {field: sum(record[field] for record in records) for field in _TOTAL_FIELDS}
    return {"request_count": len(records), **_with_ratios(counts)}
