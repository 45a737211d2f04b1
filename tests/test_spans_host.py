"""Host span logic: product (one token scan, eviction queue) vs oracle (its own per-token and
per-span loops, pinned by the reference's known answers), and the known answers."""

import numpy as np
import pytest

from logkv_amd import alpha_log_kv as prod
from oracle import spans as ora


def test_one_row_runs_match_token_loop():
    """One row: an unfinished old span (of up to max_span + 1 tokens, so also one that disables
    the cap) continued or closed by a position jump, flush rows with jumps and boundaries."""
    rng = np.random.default_rng(11)
    for _ in range(600):
        count = int(rng.integers(0, 30))
        max_span = int(rng.integers(1, 6))
        pending = int(rng.integers(0, max_span + 2))
        steps = 1 + (rng.random(count) < 0.1) * rng.integers(1, 4, count)
        new_pos = (100 + np.cumsum(steps)).tolist()
        ends = (rng.random(count) < 0.2).tolist()
        last = (new_pos[0] if count else 100) - int(rng.integers(1, 3))
        spans = [[(pending, False)]] if pending else [[]]
        old_pos = [list(range(last - pending + 1, last + 1))]
        got = prod.cut_spans(spans, old_pos, [new_pos], [ends], pending, max_span)
        want = ora.cut_spans(spans, old_pos, [new_pos], [ends], pending, max_span)
        if want is None:
            assert got is None
            continue
        (cands, all_pos, tokens, lengths), = want
        assert got.candidates[0][0] == cands
        assert got.candidates[0][1].tolist() == list(all_pos)
        assert got.token_rows[0].tolist() == list(tokens) and got.length_rows[0] == list(lengths)


def _random_pool(rng, rows, max_span):
    """Random previous selection: closed old spans plus an optional unfinished tail."""
    spans, positions, pos = [], [], 0
    for _ in range(rows):
        row_spans, row_pos = [], []
        for _ in range(int(rng.integers(0, 4))):
            n = int(rng.integers(1, max_span + 1))
            row_spans.append((n, True))
            row_pos.extend(range(pos, pos + n))
            pos += n + int(rng.integers(0, 3))
        if rng.random() < 0.6:
            n = int(rng.integers(1, max_span + 1))
            row_spans.append((n, False))
            row_pos.extend(range(pos, pos + n))
            pos += n
        spans.append(row_spans)
        positions.append(row_pos)
    return spans, positions, pos


def test_cut_and_choose_match_oracle():
    rng = np.random.default_rng(5)
    for trial in range(200):
        rows, max_span = int(rng.integers(1, 4)), int(rng.integers(1, 9))
        spans, positions, pos = _random_pool(rng, rows, max_span)
        width = max((len(p) for p in positions), default=0)
        n = int(rng.integers(0, 40))
        new_pos = [list(range(pos + (1 if rng.random() < 0.3 else 0), pos + n + 1))[:n] for _ in range(rows)]
        ends = [(rng.random(n) < 0.15).tolist() for _ in range(rows)]
        got = prod.cut_spans(spans, positions, new_pos, ends, width, max_span)
        want = ora.cut_spans(spans, positions, new_pos, ends, width, max_span)
        if want is None:
            assert got is None
            continue
        for (cands, all_pos, tokens, lengths), g_c, g_t, g_l in zip(want, got.candidates, got.token_rows,
                                                                  got.length_rows):
            assert g_c[0] == cands and np.array_equal(g_c[1], all_pos)
            assert np.array_equal(g_t, tokens) and list(g_l) == list(lengths)
        scores = rng.random(sum(len(c[0]) for c in want)).astype(np.float32)
        scores[rng.random(len(scores)) < 0.2] = 0.0          # ties
        budget = int(rng.integers(1, 3 * max_span + 2))
        sel = prod.choose_spans(got, scores.tolist(), budget)
        keep, archive, sp, ps = ora.choose_spans(want, scores, budget)
        assert (sel.keep, sel.archive, sel.spans, sel.positions) == (keep, archive, sp, ps), trial


def test_known_answers_whole_spans_and_pending_tail():
    """litgpt tests/test_alpha_log_kv.py:81-93, through the oracle's scorer."""
    rng = np.random.default_rng(0)
    k = rng.standard_normal((1, 2, 7, 8)).astype(np.float32)
    cut = ora.cut_spans([[(2, False)]], [[0, 1]], [[2, 3, 4, 5, 6]], [[False, True, False, False, False]], 2, 4)
    keep, archive, sp, _ = ora.choose_spans(cut, ora.score_spans(k, k, cut), 7)
    assert keep == [list(range(7))] and sp == [[(4, True), (3, False)]] and archive == [[]]
    k[:, :, :4] = 1.0
    cut = ora.cut_spans([[(4, True)]], [[0, 1, 2, 3]], [[4, 5, 6]], [[False, False, True]], 4, 4)
    keep, archive, _, _ = ora.choose_spans(cut, ora.score_spans(k, k, cut), 4)
    assert keep == [[4, 5, 6]] and archive == [[0, 1, 2, 3]]


def test_known_answers_beta_novelty():
    """litgpt tests/test_beta_log_kv.py:21-42 through the oracle's scorer and greedy."""
    k = np.broadcast_to(np.asarray([1.0, 3.0], np.float32).reshape(1, 1, 2, 1), (1, 4, 2, 2)).copy()
    centers = np.ones((1, 4, 2, 2), np.float32)
    valid = np.asarray([[[True, False]] * 4])

    def select(beta, cvalid=None):
        cut = ora.cut_spans([[]], [[]], [[0, 1]], [[True, True]], 0, 1)
        s = ora.score_spans(k, k, cut, beta, centers, cvalid)
        return ora.choose_spans(cut, s, 1)

    assert select(False)[0] == [[0]]
    keep, archive, _, _ = select(True, valid)
    assert keep == [[1]] and archive == [[0]]
    assert select(True, valid & False)[0] == [[0]]
    # Span 0 unusual in two groups beats span 1 moderately unusual in all four.
    k2 = np.ones((1, 4, 2, 1), np.float32)
    k2[:, :2, 0] = 3.0
    k2[:, :, 1] = 2.0
    cut = ora.cut_spans([[]], [[]], [[0, 1]], [[True, True]], 0, 1)
    s = ora.score_spans(k2, k2, cut, True, np.ones((1, 4, 1, 1), np.float32), np.ones((1, 4, 1), bool))
    assert ora.choose_spans(cut, s, 1)[0] == [[0]]
