"""Alpha exact spans: candidate cutting, span scoring (Alpha and Beta novelty), greedy choice.

TEST INFRASTRUCTURE ONLY (the oracle). Written as per-token / per-span loops,
independently of the product's vectorised host code, so the two can check
each other.

* ``new_runs``: the per-token span rule (close after a boundary token or at the
  length cap - old pending tokens count toward the cap - and before a position
  jump) as stated by the reference's own loop form
  (tests/test_alpha_log_kv.py:44-62, vectorised at litgpt/alpha_log_kv.py:16-53);
* ``cut_spans``: candidates per row: closed old spans (old), a pending old span
  closed by a jump (new), the new runs with the pending span prepended to the
  first (litgpt/alpha_log_kv.py:84-122);
* ``score_spans``: ``R_X = max(E_X - mean_d mu_X^2, 0) / max(E_X, 1e-12)``;
  Alpha ``q = mean_g R_K + mean_g R_V``; Beta
  ``q_g = (R_K + R_V)/2 + N/(1+N)`` with
  ``N = min_alive (mean_d mu_K^2 + mean_d c^2 - 2 mean_d mu_K c)_+ / max(E_K, 1e-12)``
  and ``q`` the mean of the top two ``q_g`` (litgpt/alpha_log_kv.py:125-174);
* ``choose_spans``: bounded whole-span greedy (litgpt/alpha_log_kv.py:177-226).

Orders: token sums run sequentially in span order, feature sums use
``numerics.dsum``, group means sum the groups in index order.
"""

from __future__ import annotations

import numpy as np

from .numerics import dsum, f32


def new_runs(new_pos, ends, pending, pending_pos, max_span):
    """Per-token form: (pending_closed, [(start, stop, closed)]) over new-token indices."""
    current, out, pending_closed = list(range(-pending, 0)), [], False
    last = pending_pos
    for j, (pos, end) in enumerate(zip(new_pos, ends)):
        if current and pos != last + 1:
            if current[0] < 0 and current[-1] < 0:
                pending_closed = True
            else:
                out.append((max(current[0], 0), current[-1] + 1, True))
            current = []
        current.append(j)
        last = pos
        if end or len(current) == max_span:
            out.append((max(current[0], 0), current[-1] + 1, True))
            current = []
    if current and current[-1] >= 0:
        out.append((max(current[0], 0), current[-1] + 1, False))
    return pending_closed, out


def cut_spans(old_spans, old_positions, new_positions, ends, old_width, max_span):
    """Per row: list of candidates ``(ranges, old, closed)``, the row's ``[pool | flush]``
    positions, its flat token list and span lengths. ``None`` when no row has a span."""
    rows = []
    any_span = False
    for spans, old_pos, new_pos, boundaries in zip(old_spans, old_positions, new_positions, ends):
        cands, offset, pending = [], 0, None
        for length, closed in spans:
            if closed:
                cands.append(([(offset, offset + length)], True, True))
            else:
                pending = (offset, offset + length)
            offset += length
        all_pos = np.zeros(old_width + len(new_pos), dtype=np.int64)
        all_pos[:len(old_pos)] = old_pos
        all_pos[old_width:] = new_pos
        pending_len = 0 if pending is None else pending[1] - pending[0]
        pending_pos = int(all_pos[pending[1] - 1]) if pending_len else 0
        pending_closed, runs = new_runs(list(new_pos), list(boundaries), pending_len, pending_pos, max_span)
        if pending_closed:
            cands.append(([pending], False, True))
        for i, (start, stop, done) in enumerate(runs):
            ranges = [(start + old_width, stop + old_width)]
            if i == 0 and pending_len and not pending_closed:
                ranges.insert(0, pending)
            cands.append((ranges, False, done))
        if pending_len and not pending_closed and not runs:
            cands.append(([pending], False, False))
        tokens = [t for ranges, _, _ in cands for a, b in ranges for t in range(a, b)]
        lengths = [sum(b - a for a, b in ranges) for ranges, _, _ in cands]
        any_span = any_span or bool(lengths)
        rows.append((cands, all_pos, np.asarray(tokens, dtype=np.int64), lengths))
    return rows if any_span else None


def score_spans(keys, values, cut, beta_novelty=False, centroids=None, centroid_valid=None):
    """float32 score per candidate, rows concatenated in candidate order.

    ``keys``/``values``: ``[Bt, G, W, D]`` float32 views of ``[pool | flush]``.
    """
    keys, values = f32(keys), f32(values)
    n_groups, dim = keys.shape[1], keys.shape[-1]
    out = []
    for b, (cands, _, tokens, lengths) in enumerate(cut):
        start = 0
        for length in lengths:
            idx = tokens[start:start + length]
            start += length
            parts = []
            key_stats = None
            for x_all in (keys, values):
                x = x_all[b][:, idx]                                  # [G, n, D]
                n = np.float32(length)
                acc = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1]       # [G, D]
                means = acc / n
                ms = dsum(x * x) / np.float32(x.shape[-1])                        # [G, n]
                energy = np.add.accumulate(ms, axis=1, dtype=np.float32)[:, -1] / n  # [G]
                mean_square = dsum(means * means) / np.float32(x.shape[-1])       # [G]
                residual = np.maximum(energy - mean_square, np.float32(0.0))
                part = residual / np.maximum(energy, np.float32(1e-12))
                parts.append(part)
                if key_stats is None:
                    key_stats = (means, energy, mean_square)
            if not beta_novelty:
                total = np.float32(0.0)
                for p in parts:
                    s = p[0]
                    for g in range(1, n_groups):
                        s = np.float32(s + p[g])
                    total = np.float32(total + s / np.float32(n_groups))
                out.append(total)
                continue
            means, energy, mean_square = key_stats
            c = f32(centroids[b])                                              # [G, K, D]
            valid = np.asarray(centroid_valid[b], dtype=bool)                  # [G, K]
            dots = dsum(means[:, None, :] * c) / np.float32(dim)              # [G, K]
            cms = dsum(c * c) / np.float32(dim)
            dist = np.maximum((mean_square[:, None] + cms) - np.float32(2.0) * dots, np.float32(0.0))
            nearest = np.where(valid, dist, np.float32(np.inf)).min(axis=1)
            nearest = np.where(valid.any(axis=1), nearest, np.float32(0.0)).astype(np.float32)
            novelty = nearest / np.maximum(energy, np.float32(1e-12))
            q = (parts[0] + parts[1]) * np.float32(0.5) + novelty / (np.float32(1.0) + novelty)
            top = np.sort(q.astype(np.float32))[::-1][:min(2, n_groups)]
            s = top[0]
            for t in top[1:]:
                s = np.float32(s + t)
            out.append(np.float32(s / np.float32(len(top))))
    return np.asarray(out, dtype=np.float32)


def choose_spans(cut, host_scores, budget):
    """(keep, archive, spans, positions) per row; identical rule to the reference greedy."""
    keep, archive, out_spans, out_pos = [], [], [], []
    offset = 0
    for cands, positions, tokens, size in cut:
        n = len(cands)
        mandatory = {i for i in range(n) if not cands[i][2]}
        room = budget - sum(size[i] for i in mandatory)
        density = [float(host_scores[offset + i]) * (1.1 if cands[i][1] else 1.0) for i in range(n)]
        chosen = mandatory | {i for i in range(n) if cands[i][1]}
        room -= sum(size[i] for i in chosen - mandatory)

        def victims():
            return sorted(chosen - mandatory, key=lambda i: (density[i], -i))

        for i in victims():
            if room >= 0:
                break
            chosen.remove(i)
            room += size[i]
        ranked = sorted((i for i in range(n) if i not in chosen), key=lambda i: (-density[i], i))
        order = None
        for i in ranked:
            length = size[i]
            available, loss, remove = room, 0.0, []
            if available < length:
                if order is None:
                    order = victims()
                for j in order:
                    remove.append(j)
                    available += size[j]
                    loss += density[j] * size[j]
                    if available >= length:
                        break
            if available >= length and (not remove or density[i] * length > loss):
                chosen.difference_update(remove)
                chosen.add(i)
                room = available - length
                order = None
        selected = sorted(chosen)
        kept = np.repeat(np.isin(np.arange(n), selected), size).astype(bool) if n else np.zeros(0, bool)
        keep.append(tokens[kept].tolist())
        archive.append(tokens[~kept].tolist())
        out_spans.append([(size[i], cands[i][2]) for i in selected])
        out_pos.append(positions[tokens[kept]].tolist())
        offset += n
    return keep, archive, out_spans, out_pos
