"""Update tape (semantic_replay_updates): flushes recorded under a tape replay
into an empty cache without routing or span selection and restore every
buffer bit for bit (the reference's tests/test_log_kv_update_replay.py:41-72
and tests/test_alpha_log_kv.py:282-311 for the exact pool)."""

from unittest.mock import patch

import pytest
import torch

from logkv_amd import LogStructuredKVCache, alpha_log_kv
from logkv_amd.log_kv_cache import _SemanticReplayUpdates
from workloads import Mixture, rope_tables

pytestmark = pytest.mark.gpu


def _cache(exact=0, beta=False, dim=8, groups=2, batch=2, max_seq=256, K=8, recent=16):
    # Three slots per level as the reference's test; eight with an exact pool
    # (its budget is carved from the ladders).
    B = 8 if exact else 3
    cos, sin = rope_tables(max_seq, dim)
    return LogStructuredKVCache(
        (batch, groups, max_seq, dim), (batch, groups, max_seq, dim), B=B, recent_size=recent, device="cuda",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=4.0,
        semantic_flush_granularity=recent, semantic_anchor_mode="mid", allocate_second_order=False,
        semantic_centroid_backend="parallel", semantic_replay_updates=True, cos_cache=cos, sin_cache=sin,
        rope_n_elem=dim, alpha_exact_tokens=exact, alpha_span_max_tokens=4, beta_novelty=beta,
        beta_adaptive_merge=beta)


def _state(cache):
    return {name: t.clone() for name, t in cache.named_buffers()}


def _diff(cache, want):
    return [name for name, t in cache.named_buffers() if not torch.equal(t, want[name])]


@pytest.mark.parametrize("exact,beta", [(0, False), (8, False), (8, True)])
def test_tape_replay_restores_all_state_without_routing(exact, beta):
    print(f"case exact={exact} beta={beta}", flush=True)
    torch.manual_seed(11)
    cache = _cache(exact, beta)
    tape = _SemanticReplayUpdates()
    cache.begin_op_log()
    dev = cache.level_k.device
    mix = Mixture(2, 2, 8, clusters=6, seed=4)
    inputs, expected = [], []
    for start in range(0, 128, 16):
        # Rows with a stride of two rows (a noncontiguous payload view).
        k = torch.cat([mix.rows(16), mix.rows(16)], 2).to(dev)[:, :, ::2]
        v = mix.rows(16).to(dev)
        p = torch.arange(start, start + 16, device=dev).expand(2, -1)
        host = [list(range(start, start + 16))] * 2
        ends = [[(q + 3 * b) % 5 == 0 for q in range(start, start + 16)] for b in range(2)] if exact else None
        inputs.append((k, v, p, host, ends))
        with cache._semantic_update_context(tape):
            cache.route_and_flush_batch(k, v, p, positions_host=host, record_op_log=True, span_ends=ends)
        expected.append((_state(cache), cache._semantic_counts))
    log, lengths = cache.take_op_log()
    assert tape.tensors and all(not t.requires_grad for t in tape.tensors)
    assert int(cache.level_count.sum()) > 0
    if exact:
        assert int(cache.alpha_valid.sum()) > 0
    for rep in range(2):
        cache.reset_parameters()
        with patch.object(cache, "_route_commit", side_effect=AssertionError("rerouted")), \
                patch.object(alpha_log_kv, "alpha_flush", side_effect=AssertionError("reselected")):
            for i, ((k, v, p, host, ends), (buffers, counts)) in enumerate(zip(inputs, expected)):
                with cache._semantic_update_context(tape, replay=True):
                    cache.route_and_flush_batch(k, v, p, positions_host=host, replay_op_log=log,
                                                replay_op_log_len=lengths, span_ends=ends)
                torch.cuda.synchronize()
                bad = _diff(cache, buffers)
                assert not bad, f"pass {rep}, flush {i}: {bad}"
                assert cache._semantic_counts == counts
    assert cache._active_updates is None
    k, v, p, host, ends = inputs[0]
    with cache._semantic_update_context(tape, replay=True), pytest.raises(RuntimeError, match="missing"):
        cache.route_and_flush_batch(k, v, p, positions_host=[[999] * 16] * 2, replay_op_log=log, span_ends=ends)
    cache.reset_parameters()
    k, v, p, host, ends = inputs[1]
    with cache._semantic_update_context(tape, replay=True), pytest.raises(RuntimeError, match="out of order"):
        cache.route_and_flush_batch(k, v, p, positions_host=host, replay_op_log=log, span_ends=ends)


def test_tape_recording_rules():
    cache = _cache()
    tape = _SemanticReplayUpdates()
    dev = cache.level_k.device
    k = torch.randn(2, 2, 16, 8, device=dev).to(torch.bfloat16)
    p = torch.arange(16, device=dev).expand(2, -1)
    host = [list(range(16))] * 2
    with cache._semantic_update_context(tape):
        with pytest.raises(RuntimeError, match="requires record_op_log=True"):
            cache.route_and_flush_batch(k, k, p, positions_host=host)
        with pytest.raises(RuntimeError, match="CPU flush positions"):
            cache.route_and_flush_batch(k, k, p, record_op_log=True)
        cache.route_and_flush_batch(k, k, p, positions_host=host, record_op_log=True)
        with pytest.raises(RuntimeError, match="duplicate"):
            cache.route_and_flush_batch(k, k, p, positions_host=host, record_op_log=True)
    cache.reset_parameters()
    narrow = k[..., :4].contiguous()
    with cache._semantic_update_context(tape, replay=True), pytest.raises(RuntimeError, match="does not match"):
        cache.route_and_flush_batch(narrow, narrow, p, positions_host=host, replay_op_log=p)
