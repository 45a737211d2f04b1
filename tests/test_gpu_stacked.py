"""Layer-stacked flush: one cache whose batch rows are the layers of a model at
batch 1, flushed with one call per step, against one cache per layer flushed
separately. Every flush-path kernel is independent across batch rows, so each
row of the stacked state must equal its layer's own state bit for bit (the
exact pool's row count is the largest over rows, as in any batched cache)."""

import numpy as np
import pytest
import torch

from harness import STATE_FIELDS, to_np
from workloads import Mixture, rope_tables

pytestmark = pytest.mark.gpu

FIELDS = STATE_FIELDS + ("alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid", "alpha_span_len",
                         "alpha_span_closed", "alpha_span_count")


def _cache(batch, groups, dim, K, B, flush, max_seq, exact, span, beta):
    from logkv_amd import LogStructuredKVCache

    cos, sin = rope_tables(max_seq, dim)
    return LogStructuredKVCache(
        (batch, groups, max_seq, dim), (batch, groups, max_seq, dim), B=B, recent_size=flush, device="cuda",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=8.0,
        semantic_flush_granularity=flush, semantic_anchor_mode="mid", allocate_second_order=False,
        cos_cache=cos, sin_cache=sin, rope_n_elem=dim, alpha_exact_tokens=exact, alpha_span_max_tokens=span,
        beta_novelty=beta, beta_adaptive_merge=beta)


@pytest.mark.parametrize("beta", [False, True])
def test_stacked_layers_match_separate_caches(beta):
    layers, groups, dim, K, B, flush, max_seq, exact, span = 3, 2, 64, 4, 16, 96, 2048, 32, 8
    stacked = _cache(layers, groups, dim, K, B, flush, max_seq, exact, span, beta)
    single = [_cache(1, groups, dim, K, B, flush, max_seq, exact, span, beta) for _ in range(layers)]
    mixes = [Mixture(1, groups, dim, clusters=K, seed=11 + r) for r in range(layers)]
    dev = stacked.level_k.device
    for step in range(8):
        ks, vs = [m.rows(flush) for m in mixes], [m.rows(flush) for m in mixes]
        pos = torch.arange(step * flush, (step + 1) * flush, device=dev)
        # Boundaries differ per layer row so that the rows' selections differ.
        ends = torch.tensor([[(p + 5 * r) % 7 == 0 for p in range(step * flush, (step + 1) * flush)]
                             for r in range(layers)], dtype=torch.uint8, device=dev)
        stacked.route_and_flush_batch(torch.cat(ks).to(dev), torch.cat(vs).to(dev),
                                      pos.unsqueeze(0).expand(layers, -1).contiguous(), span_ends=ends)
        for r, cache in enumerate(single):
            cache.route_and_flush_batch(ks[r].to(dev), vs[r].to(dev), pos.unsqueeze(0).contiguous(),
                                        span_ends=ends[r:r + 1].contiguous())
        torch.cuda.synchronize()
        for f in FIELDS:
            got = to_np(getattr(stacked, f))
            for r, cache in enumerate(single):
                want = to_np(getattr(cache, f))[0]
                assert np.array_equal(got[r], want, equal_nan=True), f"step {step}, layer {r}: {f}"
        assert stacked.alpha_count == max(c.alpha_count for c in single)
