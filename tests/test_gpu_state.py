"""Unpacked attention state and slot attention on the device: ``get_attention_state`` against the
oracle's plan and pack, ``log_kv_slot_attention`` over the state plus the in-flight chunk against the
packed chunk attention (the reference's two readouts of one cache) and against the oracle's float64
attention of the slot encoding; ``append_exact_tokens``; ``_convert_dtype``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import feed, make_pair, to_np
from logkv_amd import append_exact_tokens, log_kv_chunk_attention, log_kv_slot_attention
from oracle import readout as ro
from test_gpu_readout import assert_attention_close, state_of
from workloads import Mixture

pytestmark = pytest.mark.gpu


def _cache_after_flushes(exact, seed=3):
    gpu, ora = make_pair(batch=2, groups=2, dim=128, K=6, B=8, recent=64, flush=64, max_seq=4096, s_h=64.0,
                         exact=exact, span=8, beta_novelty=bool(exact), beta_adaptive=bool(exact))
    mix = Mixture(2, 2, 128, clusters=6, seed=seed)
    for blk in range(6):
        feed(gpu, ora, mix, blk * 48, 48, with_ends=bool(exact))
    torch.cuda.synchronize()
    return gpu


@pytest.mark.parametrize("exact", [0, 32])
def test_attention_state_matches_the_oracle(exact):
    cache = _cache_after_flushes(exact)
    st = cache.get_attention_state()
    state = state_of(cache)
    cos, sin = cache.cos_cache.cpu().numpy(), cache.sin_cache.cpu().numpy()
    ka, va = ro.pack(state, None, None, cos, sin)
    idx, _, valid = ro.mid_plan(state.level_count, state.level_w, state.level_sum_wp)
    Bt, G, width = idx.shape
    n_exact = cache.alpha_count
    rows = width + n_exact + cache.recent_count
    assert st.slot_k.shape == (Bt, G, rows, 128) and st.slot_w.shape == (Bt, G, rows)
    np.testing.assert_array_equal(to_np(st.slot_k), ka[..., :128])
    np.testing.assert_array_equal(to_np(st.slot_v), va[..., :128])
    w = np.take_along_axis(state.level_w.reshape(Bt, G, -1), idx, axis=2)
    ev = np.broadcast_to(state.alpha_valid[:, None, :n_exact], (Bt, G, n_exact)) if n_exact else \
        np.zeros((Bt, G, 0), bool)
    expect_valid = np.concatenate([valid, ev], axis=-1)
    np.testing.assert_array_equal(to_np(st.slot_valid), expect_valid)
    got_w = to_np(st.slot_w)
    np.testing.assert_array_equal(got_w[..., :width][valid], w[valid])
    np.testing.assert_array_equal(got_w[..., width:width + n_exact], ev.astype(np.float32))
    assert (got_w[..., width + n_exact:] == 1).all()
    assert st.M_s.shape == expect_valid.shape and bool((st.M_s == 1).all())


@pytest.mark.parametrize("heads,tq", [(4, 1), (4, 2), (8, 40)])
def test_slot_attention_equals_packed_chunk_attention(heads, tq):
    cache = _cache_after_flushes(32, seed=9)
    g = torch.Generator().manual_seed(heads * 100 + tq)
    dev = cache.level_k.device
    q = torch.randn(2, heads, tq, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(2, 2, tq, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(2, 2, tq, 128, generator=g).to(torch.bfloat16).to(dev)
    scale = 128 ** -0.5
    with torch.no_grad():
        fast = log_kv_chunk_attention(cache, q, k, v, scale, second_order_scale=0.0)
        st = append_exact_tokens(cache.get_attention_state(), k, v)
        slow = log_kv_slot_attention(q, st.slot_k, st.slot_v, st.slot_w, scale, causal_tail=tq,
                                     slot_valid=st.slot_valid, slot_M=st.M_s)
    # Both encode the same packed rows; the kernels may split the rows differently (the fast path's
    # buffer is sized for decode), so the two agree to the output's bf16 rounding and both meet the
    # float64 oracle's 2e-3 bar.
    ka, va = ro.pack(state_of(cache), to_np(k), to_np(v), cache.cos_cache.cpu().numpy(),
                     cache.sin_cache.cpu().numpy())
    ref = ro.attention(to_np(q), ka, va, scale, tq, 128)
    assert_attention_close(fast, ref)
    assert_attention_close(slow, ref)
    a, b = fast.float(), slow.float()
    assert bool(((a - b).abs() <= 2.0 ** -7 * torch.maximum(a.abs(), b.abs()) + 1e-6).all())


def test_slot_attention_matches_float64_oracle():
    g = torch.Generator().manual_seed(5)
    B, G, H, S, tq = 2, 2, 6, 300, 3
    sk = torch.randn(B, G, S, 64, generator=g).to(torch.bfloat16)
    sv = torch.randn(B, G, S, 64, generator=g).to(torch.bfloat16)
    sw = torch.randint(1, 40, (B, G, S), generator=g).float()
    sm = torch.randint(0, 3, (B, G, 100), generator=g)
    valid = torch.rand(B, G, 150, generator=g) < 0.8
    q = torch.randn(B, H, tq, 64, generator=g).to(torch.bfloat16)
    scale = 64 ** -0.5
    dev = torch.device("cuda")
    for lam, m in ((1.0, None), (0.5, sm), (0.0, sm)):
        with torch.no_grad():
            out = log_kv_slot_attention(q.to(dev), sk.to(dev), sv.to(dev), sw.to(dev), scale, lam=lam,
                                        causal_tail=tq, slot_M=None if m is None else m.to(dev),
                                        slot_valid=valid.to(dev))
        ka, va = ro.slot_pack(to_np(sk), to_np(sv), sw.numpy(), lam=lam,
                              slot_M=None if m is None else m.numpy(), slot_valid=valid.numpy())
        ref = ro.attention(to_np(q), ka, va, scale, tq, 64)
        assert_attention_close(out, ref)


def test_slot_attention_checks():
    dev = torch.device("cuda")
    sk = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16, device=dev)
    sw = torch.ones(1, 1, 4, device=dev)
    q = torch.zeros(1, 2, 1, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="no valid slot"):
        log_kv_slot_attention(q, sk, sk, sw, 0.125, slot_valid=torch.zeros(1, 1, 4, dtype=torch.bool, device=dev))
    with pytest.raises(ValueError, match="causal_tail"):
        log_kv_slot_attention(q, sk, sk, sw, 0.125, causal_tail=2)
    empty = log_kv_slot_attention(q, sk[:, :, :0], sk[:, :, :0], sw[:, :, :0], 0.125)
    assert empty.shape == (1, 2, 1, 64) and not bool(empty.any())


def test_append_exact_tokens_and_dtype_contract():
    cache = _cache_after_flushes(0)
    st = cache.get_attention_state()
    k = torch.ones(2, 2, 3, 128, dtype=torch.bfloat16, device=cache.level_k.device)
    grown = append_exact_tokens(st, k, 2 * k)
    S = st.slot_k.size(2)
    assert grown.slot_k.size(2) == S + 3 and torch.equal(grown.slot_v[:, :, S:], 2 * k)
    assert bool((grown.slot_w[:, :, S:] == 1).all()) and grown.slot_valid is st.slot_valid
    cache._convert_dtype(torch.bfloat16)           # no-op when the activations match
    cache._convert_dtype(torch.float32)            # entries stay bf16, readouts come back in float32
    assert cache.level_k.dtype == torch.bfloat16 and cache.get_attention_state().slot_k.dtype == torch.float32
    with pytest.raises(NotImplementedError):
        cache._convert_dtype(torch.float64)
