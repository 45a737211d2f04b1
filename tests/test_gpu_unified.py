"""Device unified (Ward / radius) route against the oracle, bit for bit: the
cluster state after every flush (ladders, centers, n_eff, n_total, p_hi,
phase, alive), with drifting mixtures that force old-old merges, with Alpha's
ragged archives and delayed joins, and with Beta carries."""

import numpy as np
import pytest
import torch

from harness import compare_state
from workloads import Mixture, rope_tables

pytestmark = pytest.mark.gpu


def _pair(batch, groups, dim, K, B, T, max_seq, s_h, exact=0, span=4, beta=False, passes=1, cap=0.0):
    from logkv_amd import LogStructuredKVCache
    from oracle import OracleCache

    cos, sin = rope_tables(max_seq, dim)
    gpu = LogStructuredKVCache(
        (batch, groups, max_seq, dim), (batch, groups, max_seq, dim), B=B, recent_size=T, device="cuda",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=s_h,
        semantic_flush_granularity=T, semantic_anchor_mode="mid", allocate_second_order=False,
        semantic_unified_route=True, semantic_merge_passes=passes, cos_cache=cos, sin_cache=sin, rope_n_elem=dim,
        alpha_exact_tokens=exact, alpha_span_max_tokens=span, beta_novelty=beta, beta_adaptive_merge=beta,
        semantic_capacity_hard_cap_mult=cap)
    ora = OracleCache(batch, groups, max_seq, dim, dim, B=B, recent_size=T, K=K, s_h=s_h, flush=T,
                      exact_tokens=exact, span_max=span, beta_novelty=beta, beta_adaptive=beta,
                      cos=cos.numpy(), sin=sin.numpy(), unified=True, merge_passes=passes, hard_cap_mult=cap)
    return gpu, ora


CASES = {
    # name: (batch, groups, dim, K, B, T, flushes, s_h, exact, beta, drift)
    "small": (2, 2, 16, 4, 8, 24, 8, 4.0, 0, False, 48),
    "wide": (1, 2, 128, 12, 16, 256, 5, 64.0, 0, False, 512),
    "alpha_beta": (2, 2, 16, 4, 8, 24, 10, 4.0, 8, True, 48),
}


@pytest.mark.parametrize("passes", [1, 4])
@pytest.mark.parametrize("name", list(CASES))
def test_unified_route_matches_oracle(name, passes):
    """``passes`` 4: the budget stage's frozen-center sweeps (semantic_merge_passes, the reference's
    evaluation setting for the mid anchor)."""
    batch, groups, dim, K, B, T, n, s_h, exact, beta, drift = CASES[name]
    print(f"case {name}, merge passes {passes}", flush=True)
    gpu, ora = _pair(batch, groups, dim, K, B, T, T * (n + 2), s_h, exact=exact, beta=beta, passes=passes)
    mix = Mixture(batch, groups, dim, clusters=K + 2, seed=17, drift_every=drift)
    dev = gpu.level_k.device
    for i in range(n):
        k, v = mix.rows(T), mix.rows(T)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).expand(batch, -1).contiguous()
        ends = [[(p + 3 * b) % 5 == 0 for p in range(i * T, (i + 1) * T)] for b in range(batch)] if exact else None
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), span_ends=ends)
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy(), ends)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"flush {i}: " + "; ".join(bad)
        assert (ora.alive.sum(-1) <= K).all()
    assert ora.ward_merges > 0, "no old-old merge was exercised"


@pytest.mark.parametrize("name", ["small", "alpha_beta", "wide"])
def test_capped_unified_route_matches_oracle(name):
    """A capacity cap (semantic_capacity_hard_cap_mult) runs the full-recompute rounds: each round
    prices the compacted nodes afresh, no pair above the cap merges, and the budget stage takes
    uncapped pairs when no capped one is left; the cluster state after every flush equals the
    oracle's bit for bit."""
    batch, groups, dim, K, B, T, n, s_h, exact, beta, drift = CASES[name]
    print(f"case capped {name}", flush=True)
    max_seq = T * (n + 2)
    # A cap of a few flushes' worth of rows per cluster: binding within the run.
    mult = 0.5 if name != "wide" else 0.75
    gpu, ora = _pair(batch, groups, dim, K, B, T, max_seq, s_h, exact=exact, beta=beta, cap=mult)
    mix = Mixture(batch, groups, dim, clusters=K + 2, seed=23, drift_every=drift)
    dev = gpu.level_k.device
    for i in range(n):
        k, v = mix.rows(T), mix.rows(T)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).expand(batch, -1).contiguous()
        ends = [[(p + 3 * b) % 5 == 0 for p in range(i * T, (i + 1) * T)] for b in range(batch)] if exact else None
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev), span_ends=ends)
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy(), ends)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"flush {i}: " + "; ".join(bad)
        assert (ora.alive.sum(-1) <= K).all()


def test_old_old_merge_frees_a_cluster():
    dim = 8
    gpu, ora = _pair(1, 1, dim, 2, 4, 4, 256, 1.0)
    e = np.eye(dim, dtype=np.float32)
    dev = gpu.level_k.device
    # Two old clusters (1 e0 and 5 e0: farther apart than the radius allows),
    # then a far candidate: the old pair is the cheapest merge, so cluster 1
    # merges into 0 and the candidate opens 1.
    first = np.stack([e[0] * 1, e[0] * 1.1, e[0] * 5, e[0] * 5.1])[None, None]
    second = np.stack([e[2] * 50, e[2] * 50.2, e[2] * 50.1, e[2] * 49.9])[None, None]
    for i, rows in enumerate((first, second)):
        t = torch.from_numpy(rows).to(torch.bfloat16)
        pos = torch.arange(10 * i, 10 * i + 4).unsqueeze(0)
        gpu.route_and_flush_batch(t.to(dev), t.to(dev), pos.to(dev))
        ora.flush_rows(t.float().numpy(), t.float().numpy(), pos.numpy())
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"flush {i}: " + "; ".join(bad)
        if i == 0:
            assert ora.n_total[0, 0].tolist() == [2, 2]
    assert ora.ward_merges == 1
    assert ora.alive[0, 0].tolist() == [True, True]
    assert ora.n_total[0, 0].tolist() == [4, 4]


@pytest.mark.parametrize("passes", [1, 4])
@pytest.mark.parametrize("scale", [1.0, 2.0])
def test_lattice_ties_and_radius_edge(scale, passes):
    """Rows on a binary lattice: duplicates (zero distances), many exactly
    equal costs, and with s_h = 1 (radius limit 1) singleton pairs at squared
    distance 4 whose radius bound equals the limit exactly, so the rescan
    screen's border and tie cases decide real rows."""
    print(f"case lattice scale {scale}, merge passes {passes}", flush=True)
    dim, T, K = 16, 64, 4
    gpu, ora = _pair(2, 2, dim, K, 8, T, T * 6, 1.0, passes=passes)
    g = torch.Generator().manual_seed(int(scale * 10))
    dev = gpu.level_k.device
    for i in range(4):
        bits = torch.randint(0, 2, (2, 2, T, 5), generator=g).float() * scale
        rows = torch.zeros(2, 2, T, dim)
        rows[..., :5] = bits
        rows = rows.to(torch.bfloat16)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).expand(2, -1).contiguous()
        gpu.route_and_flush_batch(rows.to(dev), rows.to(dev), pos.to(dev))
        ora.flush_rows(rows.float().numpy(), rows.float().numpy(), pos.numpy())
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"flush {i}: " + "; ".join(bad)


@pytest.mark.parametrize("passes", [1, 4])
def test_reducer_counts_match_oracle(passes):
    """The device reducer's work counts of each flush (``unified_reduce_stats``: per lane and stage the
    nodes, rounds, merges, Lance-Williams and rescanned elements - the byte model of the unified
    roofline; with sweeps, their restricted rescans too) equal the oracle reducer's on the same
    inputs."""
    from oracle import unified as U

    batch, groups, dim, K, B, T, n, s_h = 1, 2, 128, 12, 16, 256, 4, 64.0
    print(f"case reducer counts, merge passes {passes}", flush=True)
    gpu, ora = _pair(batch, groups, dim, K, B, T, T * (n + 2), s_h, passes=passes)
    mix = Mixture(batch, groups, dim, clusters=K + 2, seed=19, drift_every=512)
    dev = gpu.level_k.device
    for i in range(n):
        k, v = mix.rows(T), mix.rows(T)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).expand(batch, -1).contiguous()
        want = []
        for b in range(batch):
            for g in range(groups):
                stages = []
                U.plan_lane(ora, k[b, g].float().numpy(), T, b, g,
                            reduce_fn=lambda *a, **kw: U.reduce(*a, counts=stages, **kw))
                want.append(stages)
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev))
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy())
        got = gpu.unified_reduce_stats(T)
        for lane, stages in enumerate(want):
            for st, counts in enumerate(stages):
                assert tuple(got[lane, st, :5].tolist()) == counts, f"flush {i} lane {lane} stage {st}"
        assert want[0][0][2] > 0
