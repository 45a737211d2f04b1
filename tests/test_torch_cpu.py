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
