"""The batched Torch-CPU flush (oracle/torch_cpu.py, the CPU baseline) against the oracle: its
batched Beta merge equals the per-group one on every field, and whole streams (attach routing
with seeding; Alpha + Beta with delayed archives) leave every state field bit-identical."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import OracleCache
from oracle import ladder as lad
from oracle.numerics import bf16_round
from oracle.torch_cpu import TorchCpuCache, beta_merge_batched
from workloads import Mixture, rope_tables

FIELDS = ("level_k", "level_v", "level_w", "level_p_lo", "level_p_hi", "level_sum_wp", "level_order", "pad_mask",
          "level_count", "centroid", "n_eff", "n_total", "p_hi_c", "level0_phase", "alive", "alpha_k_raw",
          "alpha_v", "alpha_pos", "alpha_valid")


def random_rows(rng, n, dk, dv):
    rows = lad.empty_rows(n, dk, dv)
    rows["k"] = bf16_round(rng.standard_normal((n, dk)).astype(np.float32) * 3)
    rows["v"] = bf16_round(rng.standard_normal((n, dv)).astype(np.float32))
    rows["w"] = rng.integers(0, 9, n).astype(np.float32)
    rows["p_lo"] = rng.integers(0, 1000, n)
    rows["p_hi"] = rows["p_lo"] + rng.integers(0, 50, n)
    rows["sum_wp"] = rng.integers(0, 10000, n)
    rows["order"] = rng.integers(0, 500, n)
    rows["pad"] = rng.random(n) < 0.2
    return rows


@pytest.mark.parametrize("dk,dv", [(128, 128), (64, 96), (200, 40)])
def test_batched_beta_merge_equals_the_oracle(dk, dv):
    rng = np.random.default_rng(dk + dv)
    lengths = [8, 2, 6, 0, 12, 4, 10]
    rows = random_rows(rng, sum(lengths), dk, dv)
    rows["k"][:8] = rows["k"][0]            # near ties: identical rows
    rows["v"][:8] = rows["v"][0]
    rows["w"][12:14] = 0                    # empty masses
    want, want_cuts = lad.beta_merge(rows, lengths)
    got, got_cuts = beta_merge_batched(rows, lengths)
    np.testing.assert_array_equal(got_cuts, want_cuts)
    for f in lad.FIELDS:
        np.testing.assert_array_equal(got[f], want[f], err_msg=f)


def _pair(batch, groups, dim, K, B, recent, max_seq, s_h, exact, span, beta):
    cos, sin = rope_tables(max_seq, dim)
    args = (batch, groups, max_seq, dim, dim)
    kw = dict(B=B, recent_size=recent, K=K, s_h=s_h, flush=recent, exact_tokens=exact, span_max=span,
              beta_novelty=beta, beta_adaptive=beta, cos=cos.numpy(), sin=sin.numpy())
    return OracleCache(*args, **kw), TorchCpuCache(*args, **kw)


@pytest.mark.parametrize("case", ["attach_seeding", "alpha_beta"])
def test_stream_equals_the_oracle(case):
    torch.manual_seed(0)
    if case == "attach_seeding":
        ora, fast = _pair(1, 2, 64, 4, 8, 64, 2048, 4.0, 0, 4, False)
        mix = Mixture(1, 2, 64, clusters=6, seed=3, outlier=0.2)
    else:
        ora, fast = _pair(2, 2, 64, 4, 8, 64, 2048, 16.0, 32, 8, True)
        mix = Mixture(2, 2, 64, clusters=4, seed=5)
    for blk in range(10):
        k_raw, v, k = (mix.rows(64).float().numpy() for _ in range(3))
        pos = np.arange(blk * 64, (blk + 1) * 64)[None].repeat(ora.batch, 0)
        ends = mix.span_ends(blk * 64, 64, 5) if ora.P else None
        for c in (ora, fast):
            c.add_recent(k, v, k_raw, pos, ends)
        for f in FIELDS:
            np.testing.assert_array_equal(getattr(fast, f), getattr(ora, f), err_msg=f"block {blk}: {f}")
        assert fast.alpha_spans == ora.alpha_spans
    assert int(ora.level_count[..., 1:].sum()) > 0
    if case == "alpha_beta":
        assert ora.late_joins > 0 and fast.late_joins == ora.late_joins


@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16])
def test_batched_pack_equals_the_oracle(table_dtype):
    cos, sin = rope_tables(2048, 64, dtype=table_dtype)
    kw = dict(B=8, recent_size=64, K=4, s_h=16.0, flush=64, exact_tokens=32, span_max=8, beta_novelty=True,
              beta_adaptive=True, cos=cos.float().numpy(), sin=sin.float().numpy(),
              table_bf16=table_dtype is torch.bfloat16)
    ora, fast = OracleCache(2, 2, 2048, 64, 64, **kw), TorchCpuCache(2, 2, 2048, 64, 64, **kw)
    mix = Mixture(2, 2, 64, clusters=4, seed=9)
    for blk in range(8):
        k_raw, v, k = (mix.rows(64).float().numpy() for _ in range(3))
        pos = np.arange(blk * 64, (blk + 1) * 64)[None].repeat(2, 0)
        for c in (ora, fast):
            c.add_recent(k, v, k_raw, pos, mix.span_ends(blk * 64, 64, 5))
    cur_k, cur_v = (mix.rows(3).float().numpy() for _ in range(2))
    for a, b in zip(fast.pack(cur_k, cur_v), ora.pack(cur_k, cur_v)):
        np.testing.assert_array_equal(a, b)
    assert ora.alpha_count > 0 and int((ora.level_w > 0).sum()) > 0


def _lattice(rng, n, dim):
    """Rows on a coarse binary lattice: many exactly tied squared distances and Ward costs."""
    return (rng.integers(-2, 3, (n, dim)) * 0.5).astype(np.float32)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("limit", [None, 3.0, 6.0])
@pytest.mark.parametrize("lattice", [False, True])
def test_torch_reducer_equals_the_oracle(seed, limit, lattice):
    """The Torch reducer's rounds (survivors, merge trace, centers, radii, distances, row minima)
    equal the numpy oracle's after every round, on mixtures and on lattice rows with exact ties."""
    from oracle import unified as U
    from oracle.torch_cpu import TorchReducer, pair_distances

    rng = np.random.default_rng(seed)
    if lattice:
        x = _lattice(rng, 60, 8)
    else:
        centers = rng.standard_normal((6, 16)).astype(np.float32) * 8
        x = (centers[rng.integers(0, 6, 60)] + rng.standard_normal((60, 16)) * 0.7).astype(np.float32)
    mass = (rng.integers(1, 4, 60)).astype(np.float32) if limit is None else np.ones(60, np.float32)
    target = 4 if limit is None else 1
    ora = U.Reducer(U.pair_distances(x), x, mass, 60, limit, target)
    xt = torch.from_numpy(x)
    dist = pair_distances(xt)
    np.testing.assert_array_equal(dist.numpy(), U.pair_distances(x))
    fast = TorchReducer(dist, xt, torch.from_numpy(mass), 60, limit, target)
    np.testing.assert_array_equal(fast.packed.numpy().astype(np.uint64), ora.packed)
    for rnd in range(200):
        go_o, go_f = ora.step(), fast.step()
        assert go_o == go_f and fast.trace == ora.trace, rnd
        np.testing.assert_array_equal(fast.alive.numpy(), ora.alive, err_msg=f"round {rnd}")
        np.testing.assert_array_equal(fast.mu.numpy(), ora.mu, err_msg=f"round {rnd}")
        np.testing.assert_array_equal(fast.radius.numpy(), ora.radius, err_msg=f"round {rnd}")
        np.testing.assert_array_equal(fast.dist.numpy(), ora.dist, err_msg=f"round {rnd}")
        np.testing.assert_array_equal(fast.packed.numpy().astype(np.uint64), ora.packed, err_msg=f"round {rnd}")
        if not go_o:
            break
    assert len(ora.trace) > 10 and fast.stuck == ora.stuck


@pytest.mark.parametrize("exact", [0, 16])
def test_unified_stream_equals_the_oracle(exact):
    """Unified-route streams (drifting mixtures that force old-old Ward merges; with Alpha, ragged
    archives and delayed joins) through the Torch reducer and the batched commit leave every state
    field bit-identical to the oracle's."""
    cos, sin = rope_tables(2048, 32)
    kw = dict(B=4, recent_size=48, K=4, s_h=4.0, flush=48, exact_tokens=exact, span_max=4,
              beta_novelty=bool(exact), beta_adaptive=bool(exact), cos=cos.numpy(), sin=sin.numpy(), unified=True)
    ora, fast = OracleCache(2, 2, 2048, 32, 32, **kw), TorchCpuCache(2, 2, 2048, 32, 32, **kw)
    mix = Mixture(2, 2, 32, clusters=6, seed=3, drift_every=3 * 48)
    for i in range(8):
        k, v = mix.rows(48).float().numpy(), mix.rows(48).float().numpy()
        pos = np.broadcast_to(np.arange(i * 48, (i + 1) * 48), (2, 48)).copy()
        ends = [[(p + 3 * b) % 5 == 0 for p in range(i * 48, (i + 1) * 48)] for b in range(2)] if exact else None
        for c in (ora, fast):
            c.flush_rows(k, v, pos, ends)
        for f in FIELDS:
            np.testing.assert_array_equal(getattr(fast, f), getattr(ora, f), err_msg=f"flush {i}: {f}")
    assert ora.ward_merges > 0 and fast.ward_merges == ora.ward_merges
    assert int(ora.level_count[..., 1:].sum()) > 0


def test_slot_attention_matches_float64():
    """The CPU slot attention over packed rows equals the oracle's float64 attention within the
    readout's tolerance (2e-3 relative to max(1, |ref|))."""
    from oracle import readout as ro
    from oracle.torch_cpu import slot_attention

    rng = np.random.default_rng(4)
    n_batch, hq, groups, dk, rows = 2, 8, 4, 64, 300
    dim = ro.packed_dim(dk, dk)
    ka = bf16_round(rng.standard_normal((n_batch, groups, rows, dim)).astype(np.float32))
    ka[..., dk] = bf16_round(np.log(rng.uniform(1, 64, (n_batch, groups, rows))).astype(np.float32))
    ka[..., dk + 1:] = 0
    va = bf16_round(rng.standard_normal((n_batch, groups, rows, dim)).astype(np.float32) * 3)
    q = bf16_round(rng.standard_normal((n_batch, hq, 1, dk)).astype(np.float32))
    want = ro.attention(q, ka, va, dk ** -0.5, 0, dk)
    got = slot_attention(torch.from_numpy(q), torch.from_numpy(ka), torch.from_numpy(va), dk ** -0.5, dk).numpy()
    assert (np.abs(got - want) / np.maximum(1.0, np.abs(want))).max() <= 2e-3


def test_gram_distances_close_to_canonical():
    """The reference's Gram form (the CPU baseline's timing) agrees with the canonical differences up
    to rounding: relative to the rows' squared norms, within a few float32 ulps."""
    from oracle.torch_cpu import gram_distances, pair_distances

    g = torch.Generator().manual_seed(2)
    x = (torch.randn(200, 128, generator=g) * 4 + torch.randn(1, 128, generator=g) * 10).float()
    exact, gram = pair_distances(x), gram_distances(x)
    scale = (x - x[:1]).square().sum(-1).max()
    assert float((gram - exact).abs().max() / scale) < 1e-5
    assert float(gram.diagonal().abs().max() / scale) < 1e-5
