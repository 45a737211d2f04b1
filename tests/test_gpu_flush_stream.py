"""Side-stream flushes: a cache whose ``flush_stream`` is set queues add_recent's
append and flush on that stream while the caller's stream goes on (the
attention of later layers), and every reader of the cache waits for them. The
attention outputs and the cache state must equal a cache driven on one stream,
bit for bit, over a prefill of several blocks with Alpha and Beta."""

import pytest
import torch

from harness import make_pair
from logkv_amd import log_kv_chunk_attention
from workloads import Mixture

pytestmark = pytest.mark.gpu


def _drive(caches, blocks, T, side=None):
    """Per block: every layer's chunk attention, then its add_recent (as a model's layers call them)."""
    dev = caches[0].level_k.device
    if side is not None:
        for cache in caches:
            cache.flush_stream = side
    mix = Mixture(1, caches[0].n_groups, caches[0].k_dim, clusters=6, seed=61)
    g = torch.Generator(device=dev).manual_seed(5)
    outs = []
    for blk in range(blocks):
        k, v = mix.rows(T).to(dev), mix.rows(T).to(dev)
        q = torch.randn(1, 4, T, caches[0].k_dim, generator=g, device=dev).to(torch.bfloat16)
        pos = torch.arange(blk * T, (blk + 1) * T, device=dev).unsqueeze(0)
        ends = torch.tensor([[(p + 7) % 16 == 0 for p in range(blk * T, (blk + 1) * T)]], dtype=torch.uint8, device=dev)
        for cache in caches:
            outs.append(log_kv_chunk_attention(cache, q, k, v, caches[0].k_dim ** -0.5, second_order_scale=0.0))
            cache.add_recent(k, v, k_raw=k, input_pos=pos, span_ends=ends)
    for cache in caches:
        cache._await_flush()
    torch.cuda.synchronize()
    return outs


def test_side_stream_flushes_match_one_stream():
    layers, T, blocks = 3, 64, 8
    print("case side-stream flushes", flush=True)
    one = [make_pair(batch=1, groups=2, dim=64, K=6, B=8, recent=T, flush=T, max_seq=T * (blocks + 2), s_h=16.0,
                     exact=32, span=8, beta_novelty=True, beta_adaptive=True)[0] for _ in range(layers)]
    two = [make_pair(batch=1, groups=2, dim=64, K=6, B=8, recent=T, flush=T, max_seq=T * (blocks + 2), s_h=16.0,
                     exact=32, span=8, beta_novelty=True, beta_adaptive=True)[0] for _ in range(layers)]
    want = _drive(one, blocks, T)
    got = _drive(two, blocks, T, side=torch.cuda.Stream(two[0].level_k.device))
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"attention output {i}"
    for layer, (a, b) in enumerate(zip(two, one)):
        bad = [name for (name, x), (_, y) in zip(a.named_buffers(), b.named_buffers()) if not torch.equal(x, y)]
        assert not bad, f"layer {layer}: {bad}"
        assert a.recent_count == b.recent_count and a.token_count == b.token_count


def test_side_stream_readers_wait_for_the_flush():
    """Readers that return host values (the compression snapshot, ``alpha_count``, the host
    mirrors, the exact pool's spans) read right after a side-stream ``add_recent`` see the
    flushed state: they equal the same reads of a one-stream cache after every block."""
    from types import SimpleNamespace

    from logkv_amd.kv_compression import cache_compression_snapshot

    T, blocks = 64, 6
    print("case side-stream readers", flush=True)
    kw = dict(batch=1, groups=2, dim=64, K=6, B=8, recent=T, flush=T, max_seq=T * (blocks + 2), s_h=16.0,
              exact=32, span=8, beta_novelty=True, beta_adaptive=True)
    one, two = make_pair(**kw)[0], make_pair(**kw)[0]
    dev = one.level_k.device
    side = torch.cuda.Stream(dev)
    two.flush_stream = side
    mix = Mixture(1, one.n_groups, one.k_dim, clusters=6, seed=67)

    def reads(cache):
        model = SimpleNamespace(transformer=SimpleNamespace(h=[SimpleNamespace(attn=SimpleNamespace(kv_cache=cache))]))
        return (cache_compression_snapshot(model, cache.token_count), cache.alpha_count, cache._alpha_spans,
                cache._alpha_positions, cache._semantic_counts, cache._semantic_alive, cache._semantic_n_total,
                cache._semantic_p_hi_c, cache._semantic_level0_phase)

    for blk in range(blocks):
        k, v = mix.rows(T).to(dev), mix.rows(T).to(dev)
        pos = torch.arange(blk * T, (blk + 1) * T, device=dev).unsqueeze(0)
        ends = torch.tensor([[(p + 7) % 16 == 0 for p in range(blk * T, (blk + 1) * T)]], dtype=torch.uint8,
                            device=dev)
        one.add_recent(k, v, k_raw=k, input_pos=pos, span_ends=ends)
        two.add_recent(k, v, k_raw=k, input_pos=pos, span_ends=ends)
        assert reads(two) == reads(one), f"block {blk}"
