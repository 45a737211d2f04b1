"""The drop-in surface, checked on the CPU: every name litgpt/model.py imports from the cache module
(model.py:20-24), every cache method and attribute it touches on this path (model.py:1043-1361:
add_recent, reset_parameters, _convert_dtype, get_attention_state, second_order, token_count,
recent_size, semantic_clusters) and the Alpha / Beta module functions exist with the reference's
parameter names, in order (signatures from litgpt/log_kv_cache.py:681-720, :5847, :6116, :6236,
:6391, :6501, :6802, :6914; litgpt/alpha_log_kv.py; litgpt/beta_log_kv.py)."""

from __future__ import annotations

import inspect

import pytest
import torch


def params(fn):
    return [p for p in inspect.signature(fn).parameters if p not in ("self", "ctx")]


def test_model_imports_resolve():
    from logkv_amd.log_kv_cache import (CacheAttentionState, LogKVStreamTrainingAttention,  # noqa: F401
                                        LogStructuredKVCache, append_exact_tokens, log_kv_chunk_attention,
                                        log_kv_slot_attention)


def test_cache_constructor_takes_every_reference_argument():
    from logkv_amd import LogStructuredKVCache

    reference = ["k_shape", "v_shape", "B", "recent_size", "device", "dtype", "importance_pooling",
                 "importance_pooling_lambda", "importance_pooling_temperature", "semantic_clusters", "cluster_k_max",
                 "cluster_lambda_rel", "seg_eta", "seg_g0", "seg_gap_max", "seg_block_level", "seg_forget",
                 "semantic_s_h", "semantic_flush_granularity", "semantic_cluster_chunk_size",
                 "semantic_capacity_beta", "semantic_capacity_hard_cap_mult", "semantic_legacy_route",
                 "semantic_unified_route", "semantic_merge_passes", "semantic_anchor_mode", "semantic_pack_backend",
                 "semantic_centroid_backend", "semantic_replay_updates", "cos_cache", "sin_cache", "rope_n_elem",
                 "allocate_second_order", "alpha_exact_tokens", "alpha_span_max_tokens", "beta_novelty",
                 "beta_adaptive_merge"]
    assert set(reference) <= set(params(LogStructuredKVCache.__init__))
    assert params(LogStructuredKVCache.__init__)[:4] == reference[:4]


def test_cache_methods_used_by_the_model():
    from logkv_amd import LogStructuredKVCache as C

    assert params(C.add_recent) == ["k", "v", "k_raw", "input_pos", "record_op_log", "replay_op_log",
                                    "replay_op_log_len", "replay_op_log_host", "replay_plans", "span_ends"]
    assert params(C.reset_parameters) == []
    assert params(C._convert_dtype) == ["dtype"]
    assert params(C.get_attention_state) == ["with_stats", "plan"]
    assert params(C.route_and_flush_batch)[:3] == ["k_raw", "v", "positions"]
    for name in ("positions_host", "record_op_log", "replay_op_log", "replay_op_log_len", "replay_op_log_host",
                 "replay_plans", "span_ends"):
        assert name in params(C.route_and_flush_batch)
    for name in ("begin_op_log", "take_op_log", "_semantic_update_context", "_semantic_attention_plan",
                 "_semantic_mid_attention_plan", "_semantic_attention_state"):
        assert callable(getattr(C, name))
    prop = inspect.getattr_static(C, "second_order")
    assert isinstance(prop, property) and prop.fset is not None   # the model assigns it (model.py:1189)


def test_attention_functions():
    from logkv_amd.log_kv_cache import (LogKVStreamTrainingAttention, append_exact_tokens, log_kv_chunk_attention,
                                        log_kv_slot_attention)
    from logkv_amd.log_kv_pack import log_kv_chunk_attention as chunk
    from logkv_amd.log_kv_pack import log_kv_slot_attention as slot

    assert params(chunk) == ["cache", "q_b", "k_b", "v_b", "scale", "second_order_scale", "attention_plan",
                             "causal_tail", "reuse_prefix"]
    assert params(slot) == ["q", "slot_k", "slot_v", "slot_w", "scale", "mask", "lam", "causal_tail", "slot_M",
                            "slot_valid", "check_valid", "slot_sigma_u", "slot_sigma2", "slot_gamma_a",
                            "slot_gamma_b", "slot_gamma", "second_order_scale"]
    assert params(append_exact_tokens) == ["state", "k_new", "v_new"]
    assert params(LogKVStreamTrainingAttention.forward) == ["q", "k", "v", "cache", "scale", "train_block",
                                                            "second_order_scale", "k_raw", "span_ends"]
    assert callable(log_kv_chunk_attention) and callable(log_kv_slot_attention)
    assert hasattr(LogKVStreamTrainingAttention, "apply")


def test_cache_attention_state_fields():
    from logkv_amd import CacheAttentionState

    assert CacheAttentionState._fields == ("slot_k", "slot_v", "slot_w", "slot_valid", "M_s", "slot_sigma_u",
                                           "slot_sigma2", "slot_gamma_a", "slot_gamma_b", "slot_gamma")


def test_alpha_and_beta_modules():
    from logkv_amd import alpha_log_kv as a
    from logkv_amd import beta_log_kv as b

    assert params(a.cut_spans) == ["old_spans", "old_positions", "new_positions", "ends", "old_width", "max_span"]
    assert params(a.choose_spans) == ["cut", "host_scores", "budget"]
    assert params(a.select_spans)[:9] == ["k", "v", "old_spans", "old_positions", "new_positions", "ends",
                                          "old_width", "budget", "max_span"]
    assert params(a.score_spans)[:3] == ["k", "v", "cut"]
    assert [f for f in a.SpanSelection.__dataclass_fields__] == ["keep", "archive", "spans", "positions"]
    assert params(b.make_layout) == ["lengths", "device"]
    assert params(b.select_cuts) == ["block", "layout"]
    assert params(b.apply_cuts) == ["block", "layout", "cuts"]
    assert params(b.merge_blocks) == ["block", "lengths", "cuts"]


@pytest.mark.parametrize("name", ["cache_compression_snapshot", "summarize_compression"])
def test_compression_accounting(name):
    import logkv_amd

    assert callable(getattr(logkv_amd, name))


def test_activation_rows_round_to_bf16_storage():
    """float16 / float32 activations enter the cache rounded to bf16 (nearest even, differentiably);
    other dtypes are refused as the options this library does not implement."""
    from logkv_amd._lib import as_storage, check_activation_dtype

    x = torch.tensor([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -3.0e38, 65504.0], dtype=torch.float32)
    y = as_storage(x)
    assert y.dtype == torch.bfloat16
    # ties to even: 1+2^-8 -> 1, 1+3*2^-8 -> 1+2^-6; 65504 -> 65536 (bf16 spacing 256 there)
    assert [y[i].item() for i in (0, 1, 3)] == [1.0, 1.0 + 2.0 ** -6, 65536.0]
    assert torch.isfinite(y[2]) and y[2].item() < -2.99e38
    h = as_storage(torch.tensor([2050.0], dtype=torch.float16, requires_grad=True))
    assert h.dtype == torch.bfloat16 and h.requires_grad and h.item() == 2048.0
    b = torch.ones(2, dtype=torch.bfloat16)
    assert as_storage(b) is b and as_storage(None) is None
    with pytest.raises(NotImplementedError):
        check_activation_dtype(torch.float64)
    with pytest.raises(NotImplementedError):
        as_storage(torch.zeros(1, dtype=torch.float64))
