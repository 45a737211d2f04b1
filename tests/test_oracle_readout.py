"""Pins of the oracle's readout (oracle/readout.py) without the device.

* mid anchors: the reference's integer round-half-up known answers for entries
  whose weighted mean lies inside [p_lo, p_hi] (tests/test_log_kv_position.py:
  56-63 of the reference; the mid plan never clamps, litgpt/log_kv_cache.py:
  5979-5986);
* pack: the explicit rotate-half RoPE of exact rows at their positions and the
  -10000 mask of invalid rows (tests/test_alpha_log_kv.py:312-337 of the
  reference); plan order (clusters, then levels top first) and lane padding;
* attention: a slot of mass w behaves as w copies of its token
  (tests/test_log_kv_cache.py:2199-2226 of the reference), the causal tail, and
  the mass-biased softmax against a float64 evaluation with explicit masks.
"""

from types import SimpleNamespace

import numpy as np

from oracle import readout as ro
from oracle.numerics import bf16_round


def empty_state(Bt, G, K, L, B, dk, dv, P=0, recent=0):
    return SimpleNamespace(
        level_k=np.zeros((Bt, G, K, L, B, dk), np.float32), level_v=np.zeros((Bt, G, K, L, B, dv), np.float32),
        level_w=np.zeros((Bt, G, K, L, B), np.float32), level_sum_wp=np.zeros((Bt, G, K, L, B), np.int64),
        level_count=np.zeros((Bt, G, K, L), np.int64),
        alpha_k_raw=np.zeros((Bt, G, P, dk), np.float32), alpha_v=np.zeros((Bt, G, P, dv), np.float32),
        alpha_pos=np.zeros((Bt, P), np.int64), alpha_valid=np.zeros((Bt, P), bool), alpha_count=0,
        recent_k=np.zeros((Bt, G, recent, dk), np.float32), recent_v=np.zeros((Bt, G, recent, dv), np.float32),
        recent_count=0)


def test_mid_anchor_known_answers():
    s = empty_state(1, 1, 1, 1, 3, 2, 2)
    s.level_count[0, 0, 0, 0] = 3
    s.level_w[0, 0, 0, 0] = [2, 2, 2]
    s.level_sum_wp[0, 0, 0, 0] = [1, 2, 2_000_001]
    _, anchors, valid = ro.mid_plan(s.level_count, s.level_w, s.level_sum_wp)
    assert anchors.tolist() == [[[1, 1, 1_000_001]]]
    assert valid.all()


def test_plan_order_and_lane_padding():
    s = empty_state(1, 2, 2, 2, 3, 2, 2)
    s.level_count[0, 0] = [[1, 2], [0, 1]]          # lane 0: cluster 0 levels 0/1, cluster 1 level 1
    s.level_count[0, 1] = [[1, 0], [0, 0]]
    s.level_w[...] = 1.0
    idx, _, valid = ro.mid_plan(s.level_count, s.level_w, s.level_sum_wp)
    B, L = 3, 2
    flat = lambda c, ell, slot: (c * L + ell) * B + slot  # noqa: E731
    assert idx[0, 0].tolist() == [flat(0, 1, 0), flat(0, 1, 1), flat(0, 0, 0), flat(1, 1, 0)]
    assert idx[0, 1, :1].tolist() == [flat(0, 0, 0)] and valid[0, 1].tolist() == [True, False, False, False]


def test_pack_rope_and_mask_of_exact_rows():
    rng = np.random.default_rng(1)
    dk = dv = 8
    s = empty_state(2, 2, 1, 1, 1, dk, dv, P=4)
    s.alpha_count = 3
    s.alpha_valid[:, :3] = [[True, True, True], [True, False, False]]
    s.alpha_pos[:, :3] = [[7, 9, 11], [5, 0, 0]]
    s.alpha_k_raw[...] = bf16_round(rng.standard_normal(s.alpha_k_raw.shape).astype(np.float32))
    s.alpha_v[...] = bf16_round(rng.standard_normal(s.alpha_v.shape).astype(np.float32))
    phase = (np.arange(128, dtype=np.float32)[:, None] * np.float32(0.1)) * np.ones((1, 8), np.float32)
    cos, sin = np.cos(phase).astype(np.float32), np.sin(phase).astype(np.float32)
    ka, va = ro.pack(s, None, None, cos, sin)
    raw = s.alpha_k_raw[:, :, :3].astype(np.float64)
    c = cos[s.alpha_pos[:, :3]][:, None].astype(np.float64)
    sn = sin[s.alpha_pos[:, :3]][:, None].astype(np.float64)
    expected = c * raw + sn * np.concatenate((-raw[..., 4:], raw[..., :4]), -1)
    expected = np.where(s.alpha_valid[:, None, :3, None], expected, 0)
    pooled = ka.shape[2] - 3
    np.testing.assert_allclose(ka[:, :, pooled:, :8], expected, atol=2 ** -8 * np.abs(expected).max() + 1e-6)
    # -10000 stored in the bf16 workspace (the reference test compares in the tensor's dtype)
    assert (ka[1, :, pooled + 1:pooled + 3, 8] == bf16_round(np.float32(-10000.0))).all()
    assert (ka[0, :, pooled:pooled + 3, 8] == 0).all()
    np.testing.assert_array_equal(va[1, :, pooled + 1:pooled + 3], 0)


def packed_rows(rng, n, dk, dv, dim):
    ka = np.zeros((1, 1, n, dim), np.float32)
    va = np.zeros((1, 1, n, dim), np.float32)
    ka[..., :dk] = bf16_round(rng.standard_normal((1, 1, n, dk)).astype(np.float32))
    va[..., :dv] = bf16_round(rng.standard_normal((1, 1, n, dv)).astype(np.float32))
    return ka, va


def test_mass_slot_equals_duplicated_tokens():
    rng = np.random.default_rng(2)
    dk = dv = 16
    dim = ro.packed_dim(dk, dv)
    ka, va = packed_rows(rng, 5, dk, dv, dim)
    ka[0, 0, 2, dk] = np.log(np.float32(3.0))                      # slot 2 carries mass 3
    dup_k = np.concatenate([ka[:, :, :2], np.repeat(ka[:, :, 2:3], 3, 2), ka[:, :, 3:]], 2)
    dup_v = np.concatenate([va[:, :, :2], np.repeat(va[:, :, 2:3], 3, 2), va[:, :, 3:]], 2)
    dup_k[..., dk] = 0.0
    q = bf16_round(rng.standard_normal((1, 2, 1, dk)).astype(np.float32))
    scale = 0.25                                                     # 1/scale exact in bf16
    a = ro.attention(q, ka, va, scale, 0, dv)
    b = ro.attention(q, dup_k, dup_v, scale, 0, dv)
    # equal up to log(3) rounded to float32 (relative 2^-24 on the slot's weight)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-9)


def test_masked_softmax_with_causal_tail():
    rng = np.random.default_rng(4)
    dk = dv = 8
    dim = ro.packed_dim(dk, dv)
    n, tq = 9, 3
    ka, va = packed_rows(rng, n, dk, dv, dim)
    ka[0, 0, :6, dk] = bf16_round(np.log(rng.uniform(1, 64, 6)).astype(np.float32))
    ka[0, 0, 1, dk] = -10000.0                                       # an empty slot
    q = bf16_round(rng.standard_normal((1, 2, tq, dk)).astype(np.float32))
    scale = dk ** -0.5
    got = ro.attention(q, ka, va, scale, tq, dv)
    inv = float(bf16_round(np.float32(1.0 / scale)).reshape(-1)[0])
    for h in range(2):
        for i in range(tq):
            logits = scale * (ka[0, 0, :, :dk].astype(np.float64) @ q[0, h, i].astype(np.float64)) \
                + scale * inv * ka[0, 0, :, dk].astype(np.float64)
            visible = np.ones(n, bool)
            visible[n - tq + i + 1:] = False
            p = np.exp(logits[visible] - logits[visible].max())
            p /= p.sum()
            want = p @ va[0, 0, visible, :dv].astype(np.float64)
            np.testing.assert_allclose(got[0, h, i], want, rtol=1e-12, atol=1e-12)


def test_slot_encoding_equals_pack_of_the_materialized_state():
    """The reference packs a cache two ways that must agree on every visible row: the mid fast path
    (log(max(w, 1)) pooled, 0 exact / recent, -10000 invalid; litgpt/log_kv_pack.py:27-72) and the slot
    encoding of log_kv_slot_attention over the materialized state (lam*log(w), slot_valid;
    litgpt/log_kv_cache.py:6418-6464). Masses of valid pooled slots are integers >= 1."""
    rng = np.random.default_rng(12)
    Bt, G, K, L, B, dk, dv, P, R = 2, 2, 3, 3, 4, 16, 16, 5, 3
    s = empty_state(Bt, G, K, L, B, dk, dv, P=P, recent=R)
    s.level_count[:] = rng.integers(0, B + 1, size=s.level_count.shape)
    s.level_w[:] = rng.integers(0, 9, size=s.level_w.shape)          # some zero masses: invalid slots
    s.level_sum_wp[:] = s.level_w.astype(np.int64) * rng.integers(0, 500, size=s.level_w.shape)
    s.level_k[:] = bf16_round(rng.standard_normal(s.level_k.shape))
    s.level_v[:] = bf16_round(rng.standard_normal(s.level_v.shape))
    s.alpha_k_raw[:] = bf16_round(rng.standard_normal(s.alpha_k_raw.shape))
    s.alpha_v[:] = bf16_round(rng.standard_normal(s.alpha_v.shape))
    s.alpha_pos[:] = rng.integers(0, 500, size=s.alpha_pos.shape)
    s.alpha_valid[:] = rng.random(s.alpha_valid.shape) < 0.7
    s.alpha_count = P
    s.recent_k[:] = bf16_round(rng.standard_normal(s.recent_k.shape))
    s.recent_v[:] = bf16_round(rng.standard_normal(s.recent_v.shape))
    s.recent_count = R
    cos = rng.standard_normal((512, dk)).astype(np.float32)
    sin = rng.standard_normal((512, dk)).astype(np.float32)
    ka, va = ro.pack(s, None, None, cos, sin)
    idx, _, valid = ro.mid_plan(s.level_count, s.level_w, s.level_sum_wp)
    w_pooled = np.take_along_axis(s.level_w.reshape(Bt, G, -1), idx, axis=2)
    ev = np.broadcast_to(s.alpha_valid[:, None, :P], (Bt, G, P))
    slot_w = np.concatenate([np.where(valid, w_pooled, 1.0), ev.astype(np.float32),
                             np.ones((Bt, G, R), np.float32)], axis=-1)
    slot_valid = np.concatenate([valid, ev], axis=-1)
    sk, sv = ro.slot_pack(ka[..., :dk], va[..., :dv], slot_w, slot_valid=slot_valid)
    np.testing.assert_array_equal(sk, ka)
    np.testing.assert_array_equal(sv, va)


def test_slot_encoding_anchor_counts_and_lam():
    # M-expanded slots lose log(M) of mass whatever lam is (litgpt/log_kv_position.py:128-133).
    k = np.zeros((1, 1, 3, 8), np.float32)
    w = np.array([[[4.0, 0.5, 2.0]]], np.float32)
    ka, _ = ro.slot_pack(k, k, w, lam=0.0, slot_M=np.array([[[2, 0]]]))
    assert ka[0, 0, :, 8].tolist() == [bf16_round(np.float32(-np.log(2.0))).item(), 0.0, 0.0]
    ka, _ = ro.slot_pack(k, k, w, lam=1.0, slot_M=np.array([[[2, 0]]]))
    expect = [-np.log(np.float32(2)) + np.log(np.float32(4)), np.log(np.float32(1)), np.log(np.float32(2))]
    assert np.allclose(ka[0, 0, :, 8], bf16_round(np.asarray(expect, np.float32)))


def test_attention_gradient_matches_autograd():
    """The oracle's hand-written softmax backward against torch autograd of its own forward formula
    (float64, CPU): a dropped term, a transposed operand or a missed head sum fails here."""
    import torch

    rng = np.random.default_rng(4)
    Bt, G, rep, tq, total, dk, dv = 2, 2, 3, 5, 17, 8, 8
    dim = ro.packed_dim(dk, dv)
    q = bf16_round(rng.standard_normal((Bt, G * rep, tq, dk)))
    ka = bf16_round(rng.standard_normal((Bt, G, total, dim)))
    ka[..., dk + 1:] = 0
    va = bf16_round(rng.standard_normal((Bt, G, total, dim)))
    va[..., dv:] = 0
    dout = rng.standard_normal((Bt, G * rep, tq, dv)).astype(np.float32)
    scale = 0.3
    for causal in (0, tq):
        grads = ro.attention_grad(q, ka, va, scale, causal, dv, dout, grad_rows=7)
        qt = torch.tensor(q, dtype=torch.float64, requires_grad=True)
        kt = torch.tensor(ka, dtype=torch.float64, requires_grad=True)
        vt = torch.tensor(va, dtype=torch.float64, requires_grad=True)
        qa = torch.cat([qt, torch.full((Bt, G * rep, tq, 1), float(bf16_round(np.float32(1 / scale)).reshape(-1)[0]),
                                       dtype=torch.float64), torch.zeros(Bt, G * rep, tq, dim - dk - 1,
                                                                          dtype=torch.float64)], -1)
        s = scale * qa @ kt.repeat_interleave(rep, 1).transpose(-1, -2)
        if causal:
            for i in range(tq):
                s[:, :, i, total - causal + i + 1:] = float("-inf")
        out = torch.softmax(s, -1) @ vt.repeat_interleave(rep, 1)[..., :dv]
        out.backward(torch.tensor(dout))
        np.testing.assert_allclose(grads[0], qt.grad.numpy(), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(grads[1], kt.grad.numpy()[:, :, total - 7:, :dk], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(grads[2], vt.grad.numpy()[:, :, total - 7:, :dv], rtol=1e-10, atol=1e-12)
