"""Activation dtypes other than bfloat16 (litgpt/log_kv_cache.py:6236-6268, ``_convert_dtype``; called
on every forward by litgpt/model.py:1096, :1197). The cache keeps bf16 entries; float16 / float32 rows
are rounded to bf16 (nearest even) where they enter and readouts return in the activation dtype. So a
cache run at float32 must hold, bit for bit, the state of a bf16 cache fed the same rows rounded to
bf16, and its outputs and gradients must equal that cache's, widened to float32. The constructor's
dtype also prices the Alpha budget, as the reference prices it (oracle ``budget`` with 4-byte
entries)."""

import pytest
import torch

from harness import make_pair
from logkv_amd import LogStructuredKVCache, append_exact_tokens, log_kv_chunk_attention, log_kv_slot_attention
from logkv_amd.log_kv_cache import LogKVStreamTrainingAttention
from oracle.cache import budget
from workloads import Mixture, rope_tables

pytestmark = pytest.mark.gpu


def _rows(mix, n, g, act):
    """Rows of the mixture in ``act`` with bits below bf16's mantissa, so the rounding is exercised."""
    x = mix.rows(n).float()
    return (x * (1.0 + 2.0 ** -10 * torch.rand(x.shape, generator=g))).to(act)


@pytest.mark.parametrize("act,exact", [(torch.float32, 0), (torch.float32, 32), (torch.float16, 32)])
def test_activation_dtype_matches_bf16_cache(act, exact):
    print(f"case activation dtype {act} exact={exact}", flush=True)
    kw = dict(batch=2, groups=2, dim=128, K=6, B=8, recent=64, flush=64, max_seq=64 * 10, s_h=16.0,
              exact=exact, span=8, beta_novelty=bool(exact), beta_adaptive=bool(exact))
    wide, _ = make_pair(**kw)
    ref, _ = make_pair(**kw)
    wide._convert_dtype(act)
    wide._convert_dtype(act)                      # idempotent
    dev = wide.level_k.device
    mix = Mixture(2, 2, 128, clusters=5, seed=23)
    g = torch.Generator().manual_seed(5)
    scale = 128 ** -0.5
    for blk in range(8):
        pos = torch.arange(blk * 64, blk * 64 + 64).unsqueeze(0).expand(2, -1).contiguous().to(dev)
        k, v, kr = (_rows(mix, 64, g, act).to(dev) for _ in range(3))
        q = torch.randn(2, 4, 64, 128, generator=g).to(act).to(dev)
        ends = mix.span_ends(blk * 64, 64, 8) if exact else None
        with torch.no_grad():
            out_w = log_kv_chunk_attention(wide, q, k, v, scale, second_order_scale=0.0)
            out_r = log_kv_chunk_attention(ref, q.bfloat16(), k.bfloat16(), v.bfloat16(), scale, second_order_scale=0.0)
        assert out_w.dtype == act and torch.equal(out_w, out_r.to(act)), f"block {blk}: attention"
        wide.add_recent(k, v, k_raw=kr, input_pos=pos, span_ends=ends)
        ref.add_recent(k.bfloat16(), v.bfloat16(), k_raw=kr.bfloat16(), input_pos=pos, span_ends=ends)
    assert wide._semantic_counts == ref._semantic_counts      # host reads run any pending (grouped) flush
    diff = [n for (n, a), (_, b) in zip(wide.named_buffers(), ref.named_buffers()) if not torch.equal(a, b)]
    assert not diff, diff
    assert wide.level_k.dtype == torch.bfloat16

    # Unpacked state and slot attention in the activation dtype.
    q = torch.randn(2, 4, 16, 128, generator=g).to(act).to(dev)
    k, v = (_rows(mix, 16, g, act).to(dev) for _ in range(2))
    st_w, st_r = wide.get_attention_state(), ref.get_attention_state()
    assert st_w.slot_k.dtype == act and torch.equal(st_w.slot_k, st_r.slot_k.to(act))
    assert torch.equal(st_w.slot_v, st_r.slot_v.to(act)) and torch.equal(st_w.slot_w, st_r.slot_w)
    st_w = append_exact_tokens(st_w, k, v)
    st_r = append_exact_tokens(st_r, k.bfloat16(), v.bfloat16())
    with torch.no_grad():
        s_w = log_kv_slot_attention(q, st_w.slot_k, st_w.slot_v, st_w.slot_w, scale, causal_tail=16,
                                    slot_valid=st_w.slot_valid, slot_M=st_w.M_s)
        s_r = log_kv_slot_attention(q.bfloat16(), st_r.slot_k, st_r.slot_v, st_r.slot_w, scale, causal_tail=16,
                                    slot_valid=st_r.slot_valid, slot_M=st_r.M_s)
    assert s_w.dtype == act and torch.equal(s_w, s_r.to(act))


def test_training_attention_in_float32():
    print("case stream training attention float32", flush=True)
    T, block = 192, 32
    kw = dict(batch=1, groups=2, dim=128, K=6, B=8, recent=64, flush=64, max_seq=4096, s_h=64.0)
    mix = Mixture(1, 2, 128, clusters=6, seed=41)
    g = torch.Generator().manual_seed(7)
    k_raw, v = _rows(mix, T, g, torch.float32).cuda(), _rows(mix, T, g, torch.float32).cuda()
    q = torch.randn(1, 4, T, 128, generator=g).cuda()
    k = k_raw.clone()
    dout = torch.randn(1, 4, T, 128, generator=g).cuda()
    scale = 128 ** -0.5
    wide, _ = make_pair(**kw)
    wide._convert_dtype(torch.float32)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v)]
    y = LogKVStreamTrainingAttention.apply(*xs, wide, scale, block, 0.0, k_raw, None)
    grads = torch.autograd.grad(y, xs, dout)
    ref, _ = make_pair(**kw)
    rs = [x.bfloat16().requires_grad_(True) for x in (q, k, v)]
    y_r = LogKVStreamTrainingAttention.apply(*rs, ref, scale, block, 0.0, k_raw.bfloat16(), None)
    grads_r = torch.autograd.grad(y_r, rs, dout.bfloat16())
    assert y.dtype == torch.float32 and torch.equal(y, y_r.float())
    # dout reaches the bf16 product rounded to bf16, the gradients come back widened.
    for a, b, name in zip(grads, grads_r, ("dq", "dk", "dv")):
        assert a.dtype == torch.float32 and torch.equal(a, b.float()), name
    for (n, a), (_, b) in zip(wide.named_buffers(), ref.named_buffers()):
        assert torch.equal(a, b), n


@pytest.mark.parametrize("max_seq,exact", [(32768, 256), (8192, 2048)])
def test_float32_constructor_prices_the_budget_at_four_bytes(max_seq, exact):
    print(f"case float32 constructor budget max_seq={max_seq} exact={exact}", flush=True)
    dim = 128
    cos, sin = rope_tables(max_seq, dim)
    caches = {}
    for dt in (torch.bfloat16, torch.float32):
        caches[dt] = LogStructuredKVCache(
            (1, 8, max_seq, dim), (1, 8, max_seq, dim), B=128, recent_size=2048, device="cuda", dtype=dt,
            semantic_clusters=True, cluster_k_max=12, semantic_s_h=64.0, semantic_flush_granularity=2048,
            semantic_anchor_mode="mid", allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dim,
            alpha_exact_tokens=exact, alpha_span_max_tokens=64)
    for dt, element in ((torch.bfloat16, 2), (torch.float32, 4)):
        c = caches[dt]
        want = budget(1, 8, max_seq, dim, dim, 128, 12, exact, element=element)
        assert (c.B_prime, c.max_levels) == want[:2], dt
        assert c.level_k.dtype == torch.bfloat16 and c.activation_dtype == dt
    if exact == 2048:          # here the 4-byte entries leave one slot per level fewer (79 -> 78)
        assert caches[torch.float32].B_prime == caches[torch.bfloat16].B_prime - 1
    with pytest.raises(NotImplementedError):
        caches[torch.bfloat16]._convert_dtype(torch.float64)


def test_module_casts_keep_bf16_entries():
    """``.float()`` / ``.to(dtype)`` on a module holding the cache (litgpt casts whole models) leave
    every buffer's dtype and contents alone and set the activation dtype; the cache then runs as after
    ``_convert_dtype``."""
    print("case module casts", flush=True)
    kw = dict(batch=1, groups=2, dim=128, K=6, B=8, recent=64, flush=64, max_seq=64 * 8, s_h=16.0)
    cache, _ = make_pair(**kw)
    ref, _ = make_pair(**kw)
    mix = Mixture(1, 2, 128, clusters=5, seed=3)
    dev = cache.level_k.device
    for blk in range(3):
        k, v = mix.rows(64).to(dev), mix.rows(64).to(dev)
        pos = torch.arange(blk * 64, blk * 64 + 64).unsqueeze(0).to(dev)
        for c in (cache, ref):
            c.add_recent(k, v, k_raw=k, input_pos=pos)
    assert cache._semantic_counts == ref._semantic_counts      # host reads run any pending (grouped) flush
    dtypes = {n: t.dtype for n, t in cache.named_buffers()}
    holder = torch.nn.Module()
    holder.kv_cache = cache
    holder.float()
    assert {n: t.dtype for n, t in cache.named_buffers()} == dtypes and cache.activation_dtype == torch.float32
    assert all(torch.equal(a, b) for (_, a), (_, b) in zip(cache.named_buffers(), ref.named_buffers()))
    q = torch.randn(1, 4, 16, 128, device=dev)
    k, v = mix.rows(16).to(dev), mix.rows(16).to(dev)
    with torch.no_grad():
        out = log_kv_chunk_attention(cache, q, k.float(), v.float(), 128 ** -0.5, second_order_scale=0.0)
        out_r = log_kv_chunk_attention(ref, q.bfloat16(), k, v, 128 ** -0.5, second_order_scale=0.0)
    assert out.dtype == torch.float32 and torch.equal(out, out_r.float())
    holder.to(torch.bfloat16)
    assert cache.activation_dtype == torch.bfloat16 and cache.level_k.dtype == torch.bfloat16
