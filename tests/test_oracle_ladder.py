"""Pins of the oracle's ladder rules (oracle/ladder.py) without the device.

* pair merges: the reference's compact() known answers
  (tests/test_log_kv_cache.py:349-410 of the reference);
* Beta: make_layout / merge_blocks known answers and the optimality property
  (tests/test_beta_log_kv.py:45-85 of the reference);
* Fenwick append: equal, entry for entry, to the reference's scalar
  one-entry-at-a-time rule (litgpt/log_kv_cache.py:1955-1976) applied row by
  row, including saturated top levels; mass and sum(w*p) conservation;
* centroid update: float64 closed form.
"""

import numpy as np
import pytest

from oracle import ladder as lad
from oracle.numerics import bf16_round


def rows_of(k, v, w, pos=None):
    n = len(w)
    pos = np.arange(n, dtype=np.int64) if pos is None else np.asarray(pos, dtype=np.int64)
    w = np.asarray(w, np.float32)
    return {"k": np.asarray(k, np.float32), "v": np.asarray(v, np.float32), "w": w, "p_lo": pos.copy(),
            "p_hi": pos.copy(), "sum_wp": pos * w.astype(np.int64), "order": pos.copy(),
            "pad": np.zeros(n, bool)}


def test_pair_merge_equal_weights_known_answer():
    k = np.concatenate([np.ones((4, 2)), np.full((4, 2), 3.0)])
    v = np.concatenate([np.full((4, 2), 2.0), np.full((4, 2), 6.0)])
    out = lad.merge_pairs(rows_of(k, v, [4.0] * 8))
    np.testing.assert_array_equal(out["k"], [[1, 1], [1, 1], [3, 3], [3, 3]])
    np.testing.assert_array_equal(out["v"], [[2, 2], [2, 2], [6, 6], [6, 6]])
    np.testing.assert_array_equal(out["w"], [8.0] * 4)


def test_pair_merge_unequal_weights_known_answer():
    out = lad.merge_pairs(rows_of([[1.0], [5.0], [3.0], [7.0]], [[2.0], [6.0], [4.0], [8.0]], [1, 3, 3, 1]))
    np.testing.assert_array_equal(out["k"][:, 0], [4.0, 4.0])
    np.testing.assert_array_equal(out["w"], [4.0, 4.0])
    # alpha weights the OLDER row: 0.25*2 + 0.75*6 = 5, 0.75*4 + 0.25*8 = 5
    np.testing.assert_array_equal(out["v"][:, 0], [5.0, 5.0])


def test_pair_merge_anchors_skip_massless_rows():
    a = rows_of([[0.0]], [[0.0]], [0.0], [7])
    b = rows_of([[1.0]], [[1.0]], [2.0], [3])
    out = lad.pair_merge(a, b)
    assert (out["p_lo"][0], out["p_hi"][0], out["w"][0]) == (3, 3, 2.0)
    out = lad.pair_merge(rows_of([[1.0]], [[1.0]], [1.0], [9]), b)
    assert (out["p_lo"][0], out["p_hi"][0], out["order"][0]) == (3, 9, 3)


def test_beta_layout_known_answer():
    assert lad.beta_layout([0, 6, 0, 2]).tolist() == [[0, 4, 0], [4, 2, 2], [6, 2, 3]]
    assert lad.beta_layout([]).shape == (0, 3)
    with pytest.raises(ValueError):
        lad.beta_layout([3])


def test_beta_merge_blocks_known_answer():
    values = np.asarray([10, 0, 0, 0, 7, 9, 20, 30], np.float32)
    weights = [1, 2, 3, 4, 1, 1, 2, 3]
    block = rows_of(np.ones((8, 8)), np.repeat(values[:, None], 8, axis=1), weights)
    out, cuts = lad.beta_merge(block, [6, 2])
    assert cuts.tolist() == [1, 1, 1]
    np.testing.assert_array_equal(out["w"], [1.0, 9.0, 2.0, 5.0])
    np.testing.assert_array_equal(out["v"][:, 0], [10.0, 0.0, 8.0, 26.0])
    assert out["sum_wp"].sum() == block["sum_wp"].sum()
    for f in ("k", "v"):
        np.testing.assert_allclose((out[f] * out["w"][:, None]).sum(0), (block[f] * block["w"][:, None]).sum(0))


def test_beta_cut_never_worse_than_fixed_pairs():
    rng = np.random.default_rng(83)
    n = 40
    block = rows_of(rng.standard_normal((n, 7)), rng.standard_normal((n, 11)), rng.integers(1, 10, n))
    _, cuts = lad.beta_merge(block, [n])
    for (start, width, _), cut in zip(lad.beta_layout([n]), cuts):
        if width < 4:
            continue
        w = block["w"][start:start + 4].astype(np.float64)

        def loss(split):
            total = 0.0
            for f in ("k", "v"):
                x = block[f][start:start + 4].astype(np.float64)
                energy = ((x * x).sum(-1) * w).sum() / w.sum()
                for part in (slice(0, split), slice(split, 4)):
                    mean = (x[part] * w[part, None]).sum(0) / w[part].sum()
                    total += (((x[part] - mean) ** 2).sum(-1) * w[part]).sum() / energy
            return total

        assert loss(int(cut)) <= loss(2) + 1e-5
        assert loss(int(cut)) <= min(loss(1), loss(3)) + 1e-5


def scalar_append(rows, count, entries, L, B):
    """The reference's scalar rule, one entry at a time (litgpt/log_kv_cache.py:1955-1976)."""
    def slot(ell, s):
        return lad.take(rows, slice(ell * B + s, ell * B + s + 1))

    def write(ell, s, e):
        for f in lad.FIELDS:
            rows[f][ell * B + s] = e[f][0]

    def clear(ell, s):
        for f in lad.FIELDS:
            rows[f][ell * B + s] = 0

    for i in range(len(entries["w"])):
        incoming = lad.to_storage(lad.take(entries, slice(i, i + 1)))
        ell = 0
        while True:
            if count[ell] < B:
                write(ell, int(count[ell]), incoming)
                count[ell] += 1
                break
            merged = lad.to_storage(lad.pair_merge(slot(ell, 0), slot(ell, 1)))
            tail = lad.take(rows, slice(ell * B + 2, ell * B + B))
            if ell == L - 1:
                write(ell, 0, merged)
                for s in range(B - 2):
                    write(ell, 1 + s, lad.take(tail, slice(s, s + 1)))
                write(ell, B - 1, incoming)
                count[ell] = B
                break
            for s in range(B - 2):
                write(ell, s, lad.take(tail, slice(s, s + 1)))
            write(ell, B - 2, incoming)
            clear(ell, B - 1)
            count[ell] = B - 1
            incoming = merged
            ell += 1


@pytest.mark.parametrize("seed,L,B,batches", [(0, 3, 4, [1, 3, 7, 2, 9]), (1, 2, 3, [5, 5, 5, 5, 5]),
                                              (2, 4, 5, [13, 1, 40, 2]), (3, 1, 4, [3, 6, 2])])
def test_fenwick_append_equals_scalar_rule(seed, L, B, batches):
    rng = np.random.default_rng(seed)
    dk, dv = 5, 3
    fields = lad.empty_rows(L * B, dk, dv)
    count = np.zeros(L, np.int64)
    ladder = lad.Ladder(fields, count, L, B)
    ref = lad.empty_rows(L * B, dk, dv)
    ref_count = np.zeros(L, np.int64)
    pos = 0
    for m in batches:
        k = bf16_round(rng.standard_normal((m, dk)).astype(np.float32))
        v = bf16_round(rng.standard_normal((m, dv)).astype(np.float32))
        staged = rows_of(k, v, np.ones(m), np.arange(pos, pos + m))
        pos += m
        ladder.append(staged, beta=False)
        scalar_append(ref, ref_count, staged, L, B)
        np.testing.assert_array_equal(count, ref_count)
        for f in lad.FIELDS:
            np.testing.assert_array_equal(fields[f], ref[f], err_msg=f)
        # conservation: every appended row's mass and weighted position is kept
        assert fields["w"].sum() == pos
        assert fields["sum_wp"].sum() == pos * (pos - 1) // 2


def test_fenwick_append_with_beta_conserves_mass_and_positions():
    rng = np.random.default_rng(7)
    L, B, dk, dv = 3, 6, 8, 8
    fields = lad.empty_rows(L * B, dk, dv)
    count = np.zeros(L, np.int64)
    ladder = lad.Ladder(fields, count, L, B)
    pos = 0
    for m in (4, 11, 23, 2, 17):
        staged = rows_of(bf16_round(rng.standard_normal((m, dk)).astype(np.float32)),
                         bf16_round(rng.standard_normal((m, dv)).astype(np.float32)), np.ones(m),
                         np.arange(pos, pos + m))
        pos += m
        cuts = ladder.append(staged, beta=True)
        assert all(set(np.unique(c).tolist()) <= {1, 2, 3} for _, c in cuts)
        assert fields["w"].sum() == pos
        assert fields["sum_wp"].sum() == pos * (pos - 1) // 2
        assert (count <= B).all()
        live = fields["w"] > 0
        assert (fields["p_lo"][live] <= fields["p_hi"][live]).all()


def test_centroid_update_matches_float64():
    rng = np.random.default_rng(5)
    mu = rng.standard_normal(64).astype(np.float32)
    keys = bf16_round(rng.standard_normal((37, 64)).astype(np.float32) * 3)
    got, n_eff = lad.centroid_update(mu, np.float32(12.0), keys)
    want = (12.0 * mu.astype(np.float64) + keys.astype(np.float64).sum(0)) / (12.0 + 37)
    assert n_eff == np.float32(49.0)
    np.testing.assert_allclose(got, want, rtol=5e-7 * 8, atol=3e-6)
    got0, n0 = lad.centroid_update(mu, np.float32(0.0), keys)
    np.testing.assert_allclose(got0, keys.astype(np.float64).mean(0), rtol=1e-6, atol=3e-6)
    assert n0 == np.float32(37.0)


def test_tiled_center_sum_hand_worked():
    """The parallel backend's order, worked by hand in float32: 2^24 followed by 32 ones. One row at
    a time every +1 rounds back to 2^24 (ties to even). In tiles of 32 the first tile's halving tree
    pairs 2^24 with a one (2^24 again), then adds 2 + 4 + 8 + 16 exactly: 2^24 + 30; the second tile
    is the last one, and 2^24 + 31 rounds to the even 2^24 + 32."""
    keys = np.asarray([[2.0 ** 24]] + [[1.0]] * 32, np.float32)
    assert lad.tiled_sum(keys[:32], 32)[0] == 2.0 ** 24 + 30
    assert lad.tiled_sum(keys, 32)[0] == 2.0 ** 24 + 32
    assert np.add.accumulate(keys, axis=0, dtype=np.float32)[-1][0] == 2.0 ** 24
    mu, n_eff = lad.centroid_update(np.zeros(1, np.float32), np.float32(0.0), keys, tile=32)
    assert n_eff == 33 and mu[0] == np.float32(np.float32(2.0 ** 24 + 32) / np.float32(33))
    seq, _ = lad.centroid_update(np.zeros(1, np.float32), np.float32(0.0), keys)
    assert seq[0] == np.float32(np.float32(2.0 ** 24) / np.float32(33))
    # Small integers sum exactly in any order: the tiles must then equal the float64 sum.
    rng = np.random.default_rng(3)
    ints = rng.integers(-50, 50, (75, 16)).astype(np.float32)
    np.testing.assert_array_equal(lad.tiled_sum(ints, 32), ints.astype(np.float64).sum(0))
