"""Alpha / Beta on the device against the oracle: span scores and whole flushes, bit for bit."""

import numpy as np
import pytest
import torch

from harness import STATE_FIELDS, compare_state, feed, make_pair, to_np
from logkv_amd import alpha_log_kv as prod
from logkv_amd.workloads import Mixture
from oracle import spans as ora

pytestmark = pytest.mark.gpu

ALPHA_FIELDS = STATE_FIELDS + ("alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid")


@pytest.mark.parametrize("beta", [False, True])
def test_span_scores_match_oracle(beta):
    rng = np.random.default_rng(3)
    Bt, G, D, W, T, K = 2, 8, 128, 24, 96, 12
    gen = torch.Generator().manual_seed(2)
    pool = (torch.randn(Bt, G, W, D, generator=gen) * 2).to(torch.bfloat16)
    pool_v = torch.randn(Bt, G, W, D, generator=gen).to(torch.bfloat16)
    flush = (torch.randn(Bt, G, T, D, generator=gen) * 3).to(torch.bfloat16)
    flush_v = torch.randn(Bt, G, T, D, generator=gen).to(torch.bfloat16)
    centers = torch.randn(Bt, G, K, D, generator=gen) * 2
    alive = torch.rand(Bt, G, K, generator=gen) < 0.7
    alive[1, 3] = False                                   # a group with no live center
    spans = [[(5, True), (7, True), (3, False)], [(10, True), (2, False)]]
    positions = [list(range(0, 15)), list(range(3, 15))]
    new_pos = [list(range(15, 15 + T)), list(range(15, 15 + T))]
    ends = [(rng.random(T) < 0.1).tolist() for _ in range(Bt)]
    cut = prod.cut_spans(spans, positions, new_pos, ends, W, 16)
    dev = torch.device("cuda")
    tensors = [x.to(dev) for x in (pool, pool_v, flush, flush_v, centers, alive)]
    got = prod.score_spans_split(*tensors[:4], W, cut, beta_novelty=beta, centroids=tensors[4],
                                 centroid_valid=tensors[5])
    torch.cuda.synchronize()
    keys = np.concatenate((pool.float().numpy(), flush.float().numpy()), axis=2)
    vals = np.concatenate((pool_v.float().numpy(), flush_v.float().numpy()), axis=2)
    ocut = ora.cut_spans(spans, positions, new_pos, ends, W, 16)
    want = ora.score_spans(keys, vals, ocut, beta, centers.numpy(), alive.numpy())
    np.testing.assert_array_equal(got.cpu().numpy(), want)


CASES = {
    # name: (batch, groups, dim, K, B, recent, flush, max_seq, s_h, exact, span, beta, blocks)
    "alpha_small": (2, 2, 64, 4, 8, 64, 64, 2048, 16.0, 32, 8, False, 6),
    "beta_small": (2, 2, 64, 4, 8, 64, 64, 2048, 16.0, 32, 8, True, 6),
    "beta_qwen_layer": (1, 8, 128, 12, 128, 2048, 2048, 32768, 64.0, 256, 64, True, 4),
}


@pytest.mark.parametrize("name", list(CASES))
def test_alpha_flush_matches_oracle(name):
    batch, groups, dim, K, B, recent, flush, max_seq, s_h, exact, span, beta, blocks = CASES[name]
    print(f"case {name}", flush=True)
    gpu, ora_c = make_pair(batch, groups, dim, K, B, recent, flush, max_seq, s_h, exact=exact, span=span,
                           beta_novelty=beta, beta_adaptive=beta)
    assert (gpu.B_prime, gpu.L_alloc) == (ora_c.B, ora_c.L)
    mix = Mixture(batch, groups, dim, clusters=K, seed=17)
    for blk in range(blocks):
        feed(gpu, ora_c, mix, blk * recent, recent, with_ends=True)
        torch.cuda.synchronize()
        assert gpu.alpha_count == ora_c.alpha_count, f"block {blk}: alpha_count"
        assert gpu._alpha_spans == ora_c.alpha_spans and gpu._alpha_positions == ora_c.alpha_positions
        bad = compare_state(gpu, ora_c, ALPHA_FIELDS)
        assert not bad, f"block {blk}: " + "; ".join(bad)
    # Coverage: without Beta, archived old exact rows that precede their cluster's
    # p_hi took the delayed-archive re-sort; with Beta some carry groups chose a
    # 2|2 or 3|1 cut.
    if not beta:
        assert ora_c.late_joins > 0
    else:
        cuts = np.concatenate([c for _, log in ora_c.beta_cuts for _, c in log])
        assert (cuts != 1).any()
