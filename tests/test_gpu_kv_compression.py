"""Retained-entry accounting on the device cache (litgpt/kv_compression.py:32-76): after
every add_recent of an Alpha stream the snapshot's counts equal those of an oracle cache fed
the same stream (its exact-pool validity, live ladder slots and recent rows, computed on the
CPU), unfinished spans count, and the KV groups' ladders are counted separately (the
reference's test_alpha_counts_unfinished_spans_and_each_group workload: batch 2, 2 groups x 8,
B=8, recent 8, K=4, P=8, span cap 4)."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from logkv_amd import LogStructuredKVCache
from logkv_amd.kv_compression import cache_compression_snapshot

pytestmark = pytest.mark.gpu


def model_with(*caches):
    layers = [SimpleNamespace(attn=SimpleNamespace(kv_cache=c)) for c in caches]
    return SimpleNamespace(transformer=SimpleNamespace(h=layers))


def test_alpha_counts_unfinished_spans_and_each_group():
    shape = (2, 2, 128, 8)
    cache = LogStructuredKVCache(
        shape, shape, B=8, recent_size=8, device="cuda", dtype=torch.bfloat16, semantic_clusters=True,
        cluster_k_max=4, semantic_anchor_mode="mid", allocate_second_order=False, semantic_flush_granularity=8,
        cos_cache=torch.ones(128, 8), sin_cache=torch.zeros(128, 8), rope_n_elem=8, alpha_exact_tokens=8,
        alpha_span_max_tokens=4)
    from oracle import OracleCache

    ora = OracleCache(2, 2, 128, 8, 8, B=8, recent_size=8, K=4, flush=8, exact_tokens=8, span_max=4,
                      cos=np.ones((128, 8), np.float32), sin=np.zeros((128, 8), np.float32))
    g = torch.Generator().manual_seed(17)
    k, v = (torch.randn(2, 2, 96, 8, generator=g).to(torch.bfloat16).cuda() for _ in range(2))
    ends = [[i % 3 == 2 for i in range(96)], [i % 4 == 3 for i in range(96)]]
    saw_unfinished = saw_unequal_groups = False
    for start in range(0, 96, 8):
        pos = torch.arange(start, start + 8, device="cuda").unsqueeze(0).expand(2, -1).contiguous()
        block_ends = [row[start:start + 8] for row in ends]
        cache.add_recent(k[:, :, start:start + 8], v[:, :, start:start + 8], k_raw=k[:, :, start:start + 8],
                         input_pos=pos, span_ends=block_ends)
        kb, vb = (x[:, :, start:start + 8].float().cpu().numpy() for x in (k, v))
        ora.add_recent(kb, vb, kb, pos.cpu().numpy(), block_ends)
        snap = cache_compression_snapshot(model_with(cache), start + 8)
        exact = int(ora.alpha_valid.sum()) * 2
        hierarchical = int((ora.level_w > 0).sum())
        assert snap["processed_tokens"] == ora.token_count == start + 8
        assert snap["exact_slots"] == exact
        assert snap["hierarchical_slots"] == hierarchical
        assert snap["recent_slots"] == ora.recent_count * 4
        assert snap["retained_slots"] == ora.recent_count * 4 + exact + hierarchical
        assert snap["dense_slots"] == (start + 8) * 4
        counts = cache.alpha_span_count.tolist()
        closed = cache.alpha_span_closed.cpu()
        saw_unfinished |= any(not bool(closed[b, i]) for b in range(2) for i in range(counts[b]))
        saw_unequal_groups |= hierarchical != int((ora.level_w[0, 0] > 0).sum()) * 4
    assert saw_unfinished
    assert saw_unequal_groups
    assert snap["kv_retention_ratio"] < 1


def test_two_layers_and_retention_falls_with_length():
    """Two layer caches of a Qwen3-shaped stream (8 groups x 128, K=12, B=32, Alpha 32 / 16):
    the counts add over layers, and the retained share shrinks as the stream grows."""
    from workloads import Mixture, rope_tables

    cos, sin = rope_tables(8192, 128)
    caches = [LogStructuredKVCache(
        (1, 8, 8192, 128), (1, 8, 8192, 128), B=32, recent_size=512, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=12, semantic_flush_granularity=512, semantic_anchor_mode="mid",
        allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=128, alpha_exact_tokens=32,
        alpha_span_max_tokens=16, beta_novelty=True, beta_adaptive_merge=True) for _ in range(2)]
    mix = Mixture(1, 8, 128, clusters=12, seed=3)
    ratios = []
    for blk in range(12):
        k, v = mix.rows(512).cuda(), mix.rows(512).cuda()
        pos = torch.arange(blk * 512, (blk + 1) * 512, device="cuda").unsqueeze(0).contiguous()
        for c in caches:
            c.add_recent(k, v, k_raw=k, input_pos=pos, span_ends=mix.span_ends(blk * 512, 512))
        snap = cache_compression_snapshot(model_with(*caches), (blk + 1) * 512)
        per_layer = [cache_compression_snapshot(model_with(c), (blk + 1) * 512) for c in caches]
        for f in ("recent_slots", "exact_slots", "hierarchical_slots", "dense_slots"):
            assert snap[f] == sum(p[f] for p in per_layer)
        assert snap["layer_group_count"] == 16
        ratios.append(snap["kv_retention_ratio"])
    assert ratios[-1] < ratios[3] < 1
