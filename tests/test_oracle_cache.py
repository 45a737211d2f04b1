"""Pins of the oracle's layer cache (oracle/cache.py) without the device.

* delayed archive known answer (tests/test_alpha_log_kv.py:198-208 of the
  reference): a cluster opened at position 40 that receives rows at 3 and 4
  keeps p_hi 40, holds mass 3 and sum(w*p) 47, n_total 3;
* Alpha budget closed form (litgpt/log_kv_cache.py:879-898): B=128, K=12,
  P=256 at 32K tokens gives B'=125, L=7; 128K gives L=9; without Alpha B=128;
  the product's ladder_budget agrees;
* streaming invariants of the reference's ragged-archive test
  (tests/test_alpha_log_kv.py:212-246 of the reference): every token is
  accounted for exactly once across ladders, exact pool and recent window;
  n_total and alive agree with the ladders; p_hi bounds every entry; the
  exact pool's positions are unique, disjoint from the recent window and its
  spans respect the budget and the cap; sum(w*k) is conserved within bf16
  rounding.
"""

import numpy as np
import pytest

from logkv_amd.log_kv_cache import ladder_budget
from workloads import Mixture
from oracle import OracleCache, budget


def test_delayed_archive_known_answer():
    rng = np.random.default_rng(0)
    c = OracleCache(2, 2, 128, 8, 8, B=8, recent_size=8, K=4, s_h=1.0, flush=8, exact_tokens=8, span_max=4)
    k = rng.standard_normal((8, 8)).astype(np.float32)
    c.new_cluster(0, 0, 0, k[0], k[0], 40)
    c.join_late(0, 0, 0, k[:2], k[:2], np.asarray([3, 4], np.int64))
    assert c.p_hi_c[0, 0, 0] == 40
    assert c.level_w[0, 0, 0].sum() == 3
    assert c.level_sum_wp[0, 0, 0].sum() == 47
    assert c.n_total[0, 0, 0] == 3
    # entries re-sorted by position: the two late rows come first
    lo = c.level_p_lo[0, 0, 0].reshape(-1)[c.level_w[0, 0, 0].reshape(-1) > 0]
    assert sorted(lo.tolist()) == [3, 4, 40]


@pytest.mark.parametrize("args,want", [
    ((1, 8, 32768, 128, 128, 128, 12, 256), (125, 7)),
    ((1, 8, 131072, 128, 128, 128, 12, 256), (125, 9)),
    ((1, 8, 32768, 128, 128, 128, 12, 0), (128, 7)),
])
def test_budget_closed_form(args, want):
    B, L, base, _ = budget(*args)
    assert (B, L) == want
    if args[-1] and args[2] == 32768:
        # ladder bytes at B=128, L=7: K*G*L*(B*C_entry + 2) with C_entry = 1097 B at D = 128
        assert base == 94_360_896
    got = ladder_budget(*args, 2)
    assert (got[0], got[1]) == want


@pytest.mark.parametrize("beta", [False, True])
def test_streaming_invariants(beta):
    batch, groups, dim = 2, 2, 16
    c = OracleCache(batch, groups, 1024, dim, dim, B=6, recent_size=16, K=4, s_h=16.0, flush=8, exact_tokens=12,
                    span_max=4, beta_novelty=beta, beta_adaptive=beta)
    mix = Mixture(batch, groups, dim, clusters=4, seed=3)
    ks, vs = [], []
    for start in range(0, 160, 8):
        k, v = mix.rows(8).float().numpy(), mix.rows(8).float().numpy()
        pos = np.broadcast_to(np.arange(start, start + 8), (batch, 8))
        ends = [[(p + 7 * b) % 5 == 0 for p in range(start, start + 8)] for b in range(batch)]
        c.add_recent(k, v, k, pos, ends)
        ks.append(k)
        vs.append(v)
        stop = start + 8
        mass = c.level_w.sum((2, 3, 4)) + c.alpha_valid.sum(-1)[:, None] + c.recent_count
        assert (mass == stop).all()
        assert (c.level_w.sum((-1, -2)) == c.n_total).all()
        live = c.level_w.sum((-1, -2)) > 0
        assert (live == c.alive).all()
        hi = np.where(c.level_w > 0, c.level_p_hi, -1).max((-1, -2))
        assert (np.where(live, hi, 0) <= np.where(live, c.p_hi_c, 0)).all()
        for b in range(batch):
            assert sum(n for n, _ in c.alpha_spans[b]) <= 12
            assert all(n <= 4 for n, _ in c.alpha_spans[b])
            p = c.alpha_pos[b, c.alpha_valid[b]].tolist()
            assert p == c.alpha_positions[b] and len(set(p)) == len(p)
            assert not set(p) & set(c.recent_pos[b, :c.recent_count].tolist())
    src = np.concatenate(ks, axis=2).astype(np.float64)
    total = (c.level_k.astype(np.float64) * c.level_w[..., None]).sum((2, 3, 4))
    total += (c.alpha_k_raw.astype(np.float64) * c.alpha_valid[:, None, :, None]).sum(2)
    total += c.recent_k_raw[:, :, :c.recent_count].astype(np.float64).sum(2)
    np.testing.assert_allclose(total, src.sum(2), atol=0.12 * np.abs(src).sum(2).max() / 100 + 0.12, rtol=0.01)
