"""Retained-entry accounting (litgpt/kv_compression.py:1-82) on the host: dense and
sliding-window caches, the log-structured count rule on a stand-in cache (its device
buffers are plain tensors here), summaries weighted by entries, and the error cases.
The reference's own tests (tests/test_kv_compression.py) are the model for these."""

from types import SimpleNamespace

import pytest
import torch

from logkv_amd.kv_compression import cache_compression_snapshot, summarize_compression


def model_with(*caches, pending=None):
    layers = [SimpleNamespace(attn=SimpleNamespace(kv_cache=c, _log_kv_pending=pending)) for c in caches]
    return SimpleNamespace(transformer=SimpleNamespace(h=layers))


def dense(batch=2, groups=3, sliding=None):
    k = torch.zeros(batch, groups, 128, 8)
    if sliding is None:
        return SimpleNamespace(k=k, is_sliding_window=False)
    return SimpleNamespace(k=k, is_sliding_window=True, positions=torch.tensor(sliding))


def log_like(tokens, recent, level_w, alpha_valid=None, groups=3):
    """The attributes the count rule reads from a LogStructuredKVCache."""
    batch = level_w.size(0)
    return SimpleNamespace(token_count=tokens, batch_size=batch, n_groups=groups, recent_count=recent,
                           alpha_exact_tokens=0 if alpha_valid is None else alpha_valid.size(1),
                           alpha_valid=alpha_valid, level_w=level_w)


def test_dense_cache_ignores_preallocated_capacity():
    snap = cache_compression_snapshot(model_with(dense(), dense()), 5)
    assert snap["layer_group_count"] == 12
    assert snap["recent_slots"] == snap["retained_slots"] == snap["dense_slots"] == 60
    assert snap["retained_slots_per_layer_group"] == 5
    assert snap["kv_retention_ratio"] == snap["kv_compression_factor"] == 1
    assert snap["kv_saving_ratio"] == 0


def test_sliding_window_counts_only_populated_positions():
    cache = dense(sliding=[6, 7, 8, -1])
    snap = cache_compression_snapshot(model_with(cache), 9)
    assert snap["recent_slots"] == 3 * 3
    assert snap["kv_retention_ratio"] == 9 / (9 * 6)


def test_log_cache_counts_recent_exact_and_live_entries():
    w = torch.zeros(2, 3, 4, 5, 6)
    w[0, 0, 1, 2, :3] = 1.0
    w[1, 2, 0, 0, :5] = 7.0
    valid = torch.tensor([[1, 1, 0, 1], [0, 1, 0, 0]], dtype=torch.bool)
    cache = log_like(tokens=40, recent=7, level_w=w, alpha_valid=valid)
    snap = cache_compression_snapshot(model_with(cache), processed_tokens=999)
    assert snap["processed_tokens"] == 40
    assert snap["recent_slots"] == 7 * 6
    assert snap["exact_slots"] == 4 * 3
    assert snap["hierarchical_slots"] == 8
    assert snap["retained_slots"] == 42 + 12 + 8
    assert snap["dense_slots"] == 40 * 6
    assert snap["kv_compression_factor"] == snap["dense_slots"] / snap["retained_slots"]


def test_pending_tail_counts_as_recent_and_as_tokens():
    cache = log_like(tokens=10, recent=2, level_w=torch.zeros(1, 3, 1, 1, 1))
    pending = (torch.zeros(1, 3, 1, 8), torch.zeros(1, 3, 1, 8))
    snap = cache_compression_snapshot(model_with(cache, pending=pending), 0)
    assert snap["processed_tokens"] == 11
    assert snap["recent_slots"] == 3 * 3
    assert snap["dense_slots"] == 11 * 3


def test_summary_weights_entries_instead_of_request_ratios():
    short = cache_compression_snapshot(model_with(log_like(4, 4, torch.zeros(2, 3, 1, 1, 1))), 0)
    w = torch.zeros(2, 3, 2, 3, 4)
    w[..., :2] = 1.0
    long = cache_compression_snapshot(model_with(log_like(64, 4, w)), 0)
    result = summarize_compression([short, long])
    expected = (short["retained_slots"] + long["retained_slots"]) / (short["dense_slots"] + long["dense_slots"])
    assert result["request_count"] == 2
    assert result["processed_tokens"] == 68
    assert result["kv_retention_ratio"] == expected
    assert result["kv_retention_ratio"] != (short["kv_retention_ratio"] + long["kv_retention_ratio"]) / 2
    assert result["kv_saving_ratio"] == 1 - expected
    assert result["kv_compression_factor"] == 1 / expected


def test_empty_cache_and_empty_summary_have_no_ratio():
    empty = cache_compression_snapshot(model_with(log_like(0, 0, torch.zeros(2, 3, 1, 1, 1))), 0)
    for result in (empty, summarize_compression([])):
        assert result["retained_slots"] == result["dense_slots"] == 0
        assert result["kv_retention_ratio"] is None
        assert result["kv_saving_ratio"] is None
        assert result["kv_compression_factor"] is None
    assert summarize_compression([])["request_count"] == 0


def test_inconsistent_layer_token_counts_are_rejected():
    caches = [log_like(4, 4, torch.zeros(1, 3, 1, 1, 1)), log_like(8, 0, torch.zeros(1, 3, 1, 1, 1))]
    with pytest.raises(ValueError, match="disagree on their token counts"):
        cache_compression_snapshot(model_with(*caches), 4)


def test_missing_cache_and_no_layers_are_rejected():
    with pytest.raises(ValueError, match="initialized KV cache"):
        cache_compression_snapshot(model_with(None), 4)
    with pytest.raises(ValueError, match="no attention layers"):
        cache_compression_snapshot(model_with(), 4)
