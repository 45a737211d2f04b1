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


def _log_cache_counts(cache, pending_len: int) -> tuple[int, int, int, int]:
    """(lanes, recent, exact, hierarchical) entries of one log-structured layer cache."""
    lanes = cache.batch_size * cache.n_groups
    recent = (cache.recent_count + pending_len) * lanes
    exact = 0
    if cache.alpha_exact_tokens:
        # Valid exact-pool rows per batch item, each stored once per KV group.
        exact = int(cache.alpha_valid.sum().item()) * cache.n_groups
    hierarchical = int((cache.level_w > 0).sum().item())
    return lanes, recent, exact, hierarchical


def cache_compression_snapshot(model, processed_tokens: int) -> dict:
    """Count every layer and batch / group lane of ``model`` (``model.transformer.h[i].attn.kv_cache``)
    before its request cache is reset (litgpt/kv_compression.py:32-76).

    A log-structured cache's own token count plus the pending tail its attention module
    holds (``attn._log_kv_pending``, keys first) is authoritative; ``processed_tokens`` is
    the count for dense caches, which do not track it (tokens actually forwarded, without
    an unforwarded final output). ``layer_group_count`` includes the batch dimension.
    Raises ValueError when a layer has no cache, when the layers' token counts differ or
    when the model has no attention layers.
    """
    counts = dict.fromkeys(_TOTAL_FIELDS, 0)
    token_count = None
    for block in model.transformer.h:
        cache = block.attn.kv_cache
        if cache is None:
            raise ValueError("Cannot measure KV compression without an initialized cache in every layer")
        log_structured = hasattr(cache, "token_count")
        pending = getattr(block.attn, "_log_kv_pending", None) if log_structured else None
        pending_len = 0 if pending is None else pending[0].size(2)
        current = cache.token_count + pending_len if log_structured else processed_tokens
        if token_count is not None and current != token_count:
            raise ValueError("KV cache token counts differ between layers")
        token_count = current
        if log_structured:
            lanes, recent, exact, hierarchical = _log_cache_counts(cache, pending_len)
        else:
            batch_size, n_groups = cache.k.shape[:2]
            lanes = batch_size * n_groups
            if getattr(cache, "is_sliding_window", False):
                recent = int((cache.positions >= 0).sum().item()) * n_groups
            else:
                recent = current * lanes
            exact = hierarchical = 0
        counts["layer_group_count"] += lanes
        counts["recent_slots"] += recent
        counts["exact_slots"] += exact
        counts["hierarchical_slots"] += hierarchical
        counts["dense_slots"] += current * lanes
    if token_count is None:
        raise ValueError("Cannot measure KV compression for a model without attention layers")
    counts["processed_tokens"] = token_count
    counts["retained_slots"] = counts["recent_slots"] + counts["exact_slots"] + counts["hierarchical_slots"]
    return _with_ratios(counts)


def summarize_compression(records: list[dict]) -> dict:
    """Aggregate request snapshots by their summed entries, not by averaging their ratios
    (litgpt/kv_compression.py:79-82)."""
    counts = {field: sum(record[field] for record in records) for field in _TOTAL_FIELDS}
    return {"request_count": len(records), **_with_ratios(counts)}
