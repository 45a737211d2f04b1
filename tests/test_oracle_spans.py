"""Pins of the oracle's span scoring (oracle/spans.py) without the device.

* Beta novelty known answers (tests/test_beta_log_kv.py:21-42 of the reference):
  a singleton far from the live centers is rescued, an empty history scores
  no novelty, and the top-2 group mean keeps a sparse signal;
* closed forms (exact in float32 for small integer rows): a span of identical
  rows has no residual (score 0); a span of x and -x has residual equal to its
  energy (R = 1 per component);
* float64 restatement of the score formula on random spans.
"""

import numpy as np

from oracle import spans as ora


def select(k, v, old_spans, old_pos, new_pos, ends, old_width, budget, max_span, **kw):
    cut = ora.cut_spans(old_spans, old_pos, new_pos, ends, old_width, max_span)
    scores = ora.score_spans(k, v, cut, **kw)
    keep, archive, _, _ = ora.choose_spans(cut, scores, budget)
    return keep, archive


def test_novelty_rescues_singleton_and_handles_empty_history():
    k = np.broadcast_to(np.asarray([1.0, 3.0], np.float32).reshape(1, 1, 2, 1), (1, 4, 2, 2)).copy()
    centers = np.ones((1, 4, 2, 2), np.float32)
    valid = np.asarray([[[True, False]] * 4])
    args = (k, k, [[]], [[]], [[0, 1]], [[True, True]], 0, 1, 1)
    assert select(*args)[0] == [[0]]
    keep, archive = select(*args, beta_novelty=True, centroids=centers, centroid_valid=valid)
    assert keep == [[1]] and archive == [[0]]
    keep, _ = select(*args, beta_novelty=True, centroids=centers, centroid_valid=valid & False)
    assert keep == [[0]]


def test_top_groups_preserve_sparse_signal():
    k = np.ones((1, 4, 2, 1), np.float32)
    k[:, :2, 0] = 3.0
    k[:, :, 1] = 2.0
    keep, _ = select(k, k, [[]], [[]], [[0, 1]], [[True, True]], 0, 1, 1, beta_novelty=True,
                     centroids=np.ones((1, 4, 1, 1), np.float32), centroid_valid=np.ones((1, 4, 1), bool))
    assert keep == [[0]]


def test_score_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.integers(-4, 5, 16).astype(np.float32)                  # every sum and mean stays exact
    same = np.broadcast_to(x, (1, 2, 3, 16)).copy()               # three identical rows
    cut = ora.cut_spans([[]], [[]], [[0, 1, 2]], [[False, False, True]], 0, 8)
    assert ora.score_spans(same, same, cut).tolist() == [0.0]
    pm = np.stack([x, -x])[None, None].repeat(2, axis=1)            # x, -x: mean 0
    cut = ora.cut_spans([[]], [[]], [[0, 1]], [[False, True]], 0, 8)
    assert ora.score_spans(pm, pm, cut).tolist() == [2.0]


def test_score_matches_float64_formula():
    rng = np.random.default_rng(9)
    Bt, G, W, D, K = 1, 4, 30, 24, 3
    keys = rng.standard_normal((Bt, G, W, D)).astype(np.float32)
    vals = rng.standard_normal((Bt, G, W, D)).astype(np.float32) * 2
    cent = rng.standard_normal((Bt, G, K, D)).astype(np.float32)
    alive = np.asarray([[[True, False, True]] * G])
    ends = [(rng.random(W) < 0.2).tolist()]
    cut = ora.cut_spans([[]], [[]], [list(range(W))], ends, 0, 6)
    for beta in (False, True):
        got = ora.score_spans(keys, vals, cut, beta, cent, alive)
        (cands, _, tokens, lengths), = cut
        start, want = 0, []
        for n in lengths:
            idx = tokens[start:start + n]
            start += n
            r = []
            for x in (keys[0][:, idx].astype(np.float64), vals[0][:, idx].astype(np.float64)):
                mu = x.mean(1)                                   # [G, D]
                e = (x * x).mean(2).mean(1)                      # [G]
                msq = (mu * mu).mean(1)
                r.append((np.maximum(e - msq, 0) / np.maximum(e, 1e-12), mu, e, msq))
            if not beta:
                want.append(r[0][0].mean() + r[1][0].mean())
                continue
            mu, e, msq = r[0][1], r[0][2], r[0][3]
            c = cent[0].astype(np.float64)
            d = msq[:, None] + (c * c).mean(2) - 2 * (mu[:, None, :] * c).mean(2)
            near = np.where(alive[0], np.maximum(d, 0), np.inf).min(1)
            nov = near / np.maximum(e, 1e-12)
            q = (r[0][0] + r[1][0]) / 2 + nov / (1 + nov)
            want.append(np.sort(q)[::-1][:2].mean())
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)
