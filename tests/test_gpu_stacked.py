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


def _cache(batch, groups, dim, K, B, flush, max_seq, exact, span, beta, s_h):
    from logkv_amd import LogStructuredKVCache

    cos, sin = rope_tables(max_seq, dim)
    return LogStructuredKVCache(
        (batch, groups, max_seq, dim), (batch, groups, max_seq, dim), B=B, recent_size=flush, device="cuda",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=s_h,
        semantic_flush_granularity=flush, semantic_anchor_mode="mid", allocate_second_order=False,
        cos_cache=cos, sin_cache=sin, rope_n_elem=dim, alpha_exact_tokens=exact, alpha_span_max_tokens=span,
        beta_novelty=beta, beta_adaptive_merge=beta)


SHAPES = {
    # name: (layers, groups, dim, K, B, flush, max_seq, exact, span, s_h, steps, checked steps)
    "small": (3, 2, 64, 4, 16, 96, 2048, 32, 8, 8.0, 8, range(8)),
    # the benchmarked stack: 28 Qwen3-1.7B layers (8 KV groups x 128), B'=125, L=7, Alpha 256 / 64
    "qwen_28_layers": (28, 8, 128, 12, 128, 2048, 32768, 256, 64, 64.0, 5, (1, 4)),
    # 32 x 4 x 8 = 1024 ladders (the stacked call takes the library's side stream, the single-layer
    # calls do not) with short ladders: B'=63, L = 3 (levels 0 and 1 finish on the side stream one
    # after the other) and B'=31, L = 4 (level 0, then levels 1 and 2 as one launch); rows from two
    # mixture centers, so a few clusters carry into the upper levels
    "wide_3_levels": (32, 4, 64, 8, 64, 64, 256, 16, 8, 8.0, 4, range(4)),
    "wide_4_levels": (32, 4, 64, 8, 32, 64, 512, 16, 8, 8.0, 8, (3, 5, 7)),
}
MIX_CENTERS = {"wide_3_levels": 2, "wide_4_levels": 2}   # default: K


@pytest.mark.parametrize("shape,beta", [("small", False), ("small", True), ("qwen_28_layers", True),
                                        ("wide_3_levels", False), ("wide_3_levels", True),
                                        ("wide_4_levels", True)])
def test_stacked_layers_match_separate_caches(shape, beta):
    layers, groups, dim, K, B, flush, max_seq, exact, span, s_h, steps, checked = SHAPES[shape]
    print(f"case {shape} beta={beta}", flush=True)
    stacked = _cache(layers, groups, dim, K, B, flush, max_seq, exact, span, beta, s_h)
    single = [_cache(1, groups, dim, K, B, flush, max_seq, exact, span, beta, s_h) for _ in range(layers)]
    mixes = [Mixture(1, groups, dim, clusters=MIX_CENTERS.get(shape, K), seed=11 + r) for r in range(layers)]
    dev = stacked.level_k.device
    for step in range(steps):
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
        if step not in checked:
            continue
        for f in FIELDS:
            got = getattr(stacked, f)
            for r, cache in enumerate(single):
                want = getattr(cache, f)[0]
                assert torch.equal(got[r], want) or (got[r].is_floating_point() and torch.equal(
                    torch.nan_to_num(got[r], nan=7.0), torch.nan_to_num(want, nan=7.0))), \
                    f"step {step}, layer {r}: {f}"
        assert stacked.alpha_count == max(c.alpha_count for c in single)
    if shape in MIX_CENTERS:   # the short ladders did carry: some clusters hold entries above level 0
        assert bool((stacked.level_count[..., 1:] > 0).any())
