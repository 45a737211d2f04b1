"""Deferred, stacked flushes of per-layer caches (logkv_amd/flush_group.py): caches of one configuration
driven as litgpt's model drives its layers (per block and layer: the chunk attention, then add_recent)
leave every state field and every attention output bit-identical to the same caches built with grouping
off, and every state field equal to an oracle cache per layer; the group runs the layers' flushes as
one stacked flush when all are pending, and each member's own flush (realigning its exact pool) when a
read forces one early."""

import pytest
import torch

from harness import STATE_FIELDS, compare_state, make_pair
from logkv_amd import flush_group, log_kv_chunk_attention
from workloads import Mixture

pytestmark = pytest.mark.gpu

ALPHA_FIELDS = ("alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid")


def _layers(n, grouped, **kw):
    flush_group.set_flush_grouping(grouped)
    try:
        pairs = [make_pair(**kw) for _ in range(n)]
    finally:
        flush_group.set_flush_grouping(True)
    return [p[0] for p in pairs], [p[1] for p in pairs]


def _run(layers, blocks, T, kw, early_read=None, step=None):
    """Per block and layer: attention of the grouped and ungrouped caches (compared), then add_recent
    on both and the layer's oracle. ``early_read``: (block, layer) after whose add_recent that layer's
    host mirror is read (a forced early flush). Returns the grouped caches."""
    grouped, oras = _layers(layers, True, **kw)
    plain, _ = _layers(layers, False, **kw)
    assert grouped[0]._group is not None and plain[0]._group is None
    dim, G, batch = kw["dim"], kw["groups"], kw["batch"]
    dev = grouped[0].level_k.device
    mixes = [Mixture(batch, G, dim, clusters=6, seed=40 + li) for li in range(layers)]
    gq = torch.Generator().manual_seed(9)
    step = step or T
    for blk in range(blocks * T // step):
        start = blk * step
        pos = torch.arange(start, start + step).unsqueeze(0).expand(batch, -1).contiguous()
        for li in range(layers):
            k, v = mixes[li].rows(step), mixes[li].rows(step)
            q = torch.randn(batch, 2 * G, step, dim, generator=gq).to(torch.bfloat16)
            ends = mixes[li].span_ends(start, step, 8) if kw.get("exact") else None
            outs = [log_kv_chunk_attention(c, q.to(dev), k.to(dev), v.to(dev), dim ** -0.5, second_order_scale=0.0)
                    for c in (grouped[li], plain[li])]
            assert torch.equal(outs[0], outs[1]), f"step {blk} layer {li}: attention output"
            for c in (grouped[li], plain[li]):
                c.add_recent(k.to(dev), v.to(dev), k_raw=k.to(dev), input_pos=pos.to(dev), span_ends=ends)
            oras[li].add_recent(k.float().numpy(), v.float().numpy(), k.float().numpy(), pos.numpy(), ends)
            if early_read == (blk, li):
                assert grouped[li]._semantic_counts == plain[li]._semantic_counts
    torch.cuda.synchronize()
    fields = STATE_FIELDS + (ALPHA_FIELDS if kw.get("exact") else ())
    for li in range(layers):
        bad = compare_state(grouped[li], oras[li], fields)   # its attribute reads run a pending flush
        assert not bad, f"layer {li}: " + "; ".join(bad)
        diff = [n for (n, a), (_, b) in zip(grouped[li].named_buffers(), plain[li].named_buffers())
                if not torch.equal(a, b)]
        assert not diff, f"layer {li}: {diff}"
        assert grouped[li].recent_count == plain[li].recent_count
        assert grouped[li].alpha_count == plain[li].alpha_count
    return grouped


BASE = dict(batch=2, groups=2, dim=64, K=4, B=8, recent=64, flush=64, max_seq=64 * 12, s_h=16.0)


@pytest.mark.parametrize("alpha", [False, True])
def test_grouped_layers_match_separate_caches_and_oracle(alpha):
    print(f"case grouped layers alpha={alpha}", flush=True)
    kw = dict(BASE, exact=32, span=8, beta_novelty=True, beta_adaptive=True) if alpha else dict(BASE)
    grouped = _run(3, 9, 64, kw)
    group = grouped[0]._group
    assert group.owner is not None and group.stacked_runs >= 7 and group.member_runs == 0


def test_early_read_runs_member_flushes_then_stacks_again():
    """A host read of layer 1 right after its add_recent flushes layers 0 and 1 by themselves (their
    exact pools realigned into the stacked storage); later blocks stack again."""
    print("case early read", flush=True)
    kw = dict(BASE, exact=32, span=8, beta_novelty=True, beta_adaptive=True)
    grouped = _run(3, 9, 64, kw, early_read=(4, 1))
    group = grouped[0]._group
    assert group.member_runs == 3 and group.stacked_runs >= 5


def test_decode_pairs_defer_and_stack():
    """Two-row appends (decode commits): every 16th append of a layer overflows its 32-row window."""
    print("case decode pairs", flush=True)
    kw = dict(BASE, recent=32, flush=32, max_seq=32 * 14, exact=16, span=4, beta_novelty=True,
              beta_adaptive=True)
    grouped = _run(2, 10, 32, kw, step=2)
    assert grouped[0]._group.stacked_runs >= 8


def test_unified_route_groups():
    from logkv_amd import LogStructuredKVCache
    from workloads import rope_tables

    print("case unified grouped", flush=True)
    cos, sin = rope_tables(2048, 32)

    def cache():
        return LogStructuredKVCache(
            (1, 2, 2048, 32), (1, 2, 2048, 32), B=8, recent_size=48, device="cuda", dtype=torch.bfloat16,
            semantic_clusters=True, cluster_k_max=4, semantic_s_h=4.0, semantic_flush_granularity=48,
            semantic_anchor_mode="mid", allocate_second_order=False, semantic_unified_route=True, cos_cache=cos,
            sin_cache=sin, rope_n_elem=32)

    grouped = [cache() for _ in range(3)]
    flush_group.set_flush_grouping(False)
    try:
        plain = [cache() for _ in range(3)]
    finally:
        flush_group.set_flush_grouping(True)
    mix = Mixture(1, 2, 32, clusters=6, seed=3, drift_every=3 * 48)
    for i in range(8):
        pos = torch.arange(i * 48, (i + 1) * 48, device="cuda").unsqueeze(0)
        for li in range(3):
            k, v = mix.rows(48).cuda(), mix.rows(48).cuda()
            for c in (grouped[li], plain[li]):
                c.add_recent(k, v, k_raw=k, input_pos=pos)
    for a, b in zip(grouped, plain):
        a._await_flush()     # named_buffers() reads the buffers directly, past the deferred-flush check
        diff = [n for (n, x), (_, y) in zip(a.named_buffers(), b.named_buffers()) if not torch.equal(x, y)]
        assert not diff, diff
    assert grouped[0]._group.stacked_runs >= 6


def test_same_device_move_keeps_the_group():
    print("case module moves", flush=True)
    grouped, _ = _layers(2, True, **BASE)
    for c in grouped:
        c.to(c.level_k.device)
    mix = Mixture(2, 2, 64, clusters=6, seed=1)
    for blk in range(3):
        pos = torch.arange(blk * 64, (blk + 1) * 64, device="cuda").unsqueeze(0).expand(2, -1).contiguous()
        for c in grouped:
            k = mix.rows(64).cuda()
            c.add_recent(k, k, k_raw=k, input_pos=pos)
    assert grouped[0]._group is not None and not grouped[0]._group.broken
    assert grouped[0]._pending is not None and grouped[0]._group.stacked_runs == 1
    grouped[0]._semantic_counts
    assert grouped[0]._group.stacked_runs == 2
