"""Readout parity on the device: slot plan, packed K/V and mass-biased attention vs the oracle.

Packed rows are compared value-for-value (bf16), except the log-mass column,
which may differ by one bf16 ulp (device ``logf`` vs numpy ``log`` before
rounding). Attention is compared with the oracle's float64 evaluation on the
same bf16 operands: ``|out - ref| <= 2e-3 * max(1, |ref|) + ulp(ref) / 2``,
the last term being the rounding of the output to bf16 (up to 2^-8 relative,
so it is stated separately from the 2e-3 budget for the computation).
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from harness import feed, make_pair, to_np
from logkv_amd import LogStructuredKVCache, log_kv_chunk_attention, pack_mid_kv, packed_dim
from workloads import Mixture, fill_readout_state, rope_tables
from oracle import readout as ro
from oracle.numerics import bf16_round

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def state_of(cache):
    """Oracle-side view of a device cache's readout fields."""
    Bt, G = cache.batch_size, cache.n_groups
    ns = SimpleNamespace(
        level_k=to_np(cache.level_k), level_v=to_np(cache.level_v), level_w=to_np(cache.level_w),
        level_sum_wp=to_np(cache.level_sum_wp), level_count=to_np(cache.level_count).astype(np.int64),
        recent_k=to_np(cache.recent_k), recent_v=to_np(cache.recent_v), recent_count=cache.recent_count,
        alpha_count=cache.alpha_count)
    if cache.alpha_exact_tokens:
        ns.alpha_k_raw, ns.alpha_v = to_np(cache.alpha_k_raw), to_np(cache.alpha_v)
        ns.alpha_pos, ns.alpha_valid = to_np(cache.alpha_pos), to_np(cache.alpha_valid).astype(bool)
    else:
        ns.alpha_k_raw = np.zeros((Bt, G, 0, cache.k_dim), np.float32)
        ns.alpha_v = np.zeros((Bt, G, 0, cache.v_dim), np.float32)
        ns.alpha_pos, ns.alpha_valid = np.zeros((Bt, 0), np.int64), np.zeros((Bt, 0), bool)
    return ns


def assert_pack_equal(ka, va, ka_ref, va_ref, dk):
    ka, va = to_np(ka), to_np(va)
    assert ka.shape == ka_ref.shape and va.shape == va_ref.shape
    np.testing.assert_array_equal(va, va_ref)
    np.testing.assert_array_equal(np.delete(ka, dk, axis=-1), np.delete(ka_ref, dk, axis=-1))
    bias, bias_ref = ka[..., dk], ka_ref[..., dk]
    mag = np.abs(bias_ref.astype(np.float64))
    ulp = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 7), 0.0)
    assert (np.abs(bias - bias_ref) <= ulp).all(), "log-mass column off by more than 1 bf16 ulp"


def half_ulp_bf16(x):
    mag = np.abs(x)
    return np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 8), 0.0)


def assert_attention_close(out, ref):
    out = to_np(out).astype(np.float64)
    err = (np.abs(out - ref) - half_ulp_bf16(ref)) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= ATOL, f"attention error beyond output rounding {err.max():.3e} > {ATOL}"


def rand_bf16(g, *shape):
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def check_step(cache, cos, sin, q, k, v, scale, reuse=False, table_bf16=False):
    state = state_of(cache)
    ka_ref, va_ref = ro.pack(state, to_np(k), to_np(v), to_np(cos), to_np(sin), table_bf16=table_bf16)
    dev = cache.level_k.device
    with torch.no_grad():
        out = log_kv_chunk_attention(cache, q.to(dev), k.to(dev), v.to(dev), scale, second_order_scale=0.0,
                                     reuse_prefix=reuse)
    ref = ro.attention(to_np(q), ka_ref, va_ref, scale, q.size(2), cache.v_dim)
    assert_attention_close(out, ref)
    return ka_ref, va_ref


def test_plan_and_pack_after_flushes():
    gpu, ora = make_pair(batch=2, groups=2, recent=64, flush=64, max_seq=2048)
    mix = Mixture(2, 2, 128, 12, seed=5)
    start = 0
    for n in (64, 64, 64, 64, 64):
        feed(gpu, ora, mix, start, n)
        start += n
    torch.cuda.synchronize()
    plan = gpu._semantic_attention_plan()
    idx, anchors, valid = ro.mid_plan(ora.level_count, ora.level_w, ora.level_sum_wp)
    assert plan.width == idx.shape[-1]
    ref_counts = ora.level_count.reshape(4, -1).sum(1)
    assert to_np(plan.lane_counts()).tolist() == ref_counts.tolist()
    g = torch.Generator().manual_seed(1)
    k, v = rand_bf16(g, 2, 2, 3, 128), rand_bf16(g, 2, 2, 3, 128)
    dim = packed_dim(128, 128)
    ka, va = pack_mid_kv(gpu, plan, k.cuda(), v.cuda(), dim)
    ka_ref, va_ref = ro.pack(ora, to_np(k), to_np(v), ora.cos, ora.sin)
    assert_pack_equal(ka, va, ka_ref, va_ref, 128)


def test_chunk_attention_after_flushes_alpha_beta():
    gpu, ora = make_pair(batch=1, groups=2, recent=64, flush=64, max_seq=2048, exact=64, span=16,
                         beta_novelty=True, beta_adaptive=True)
    mix = Mixture(1, 2, 128, 12, seed=9)
    start = 0
    for n in (64,) * 6:
        feed(gpu, ora, mix, start, n, with_ends=True)
        start += n
    assert ora.alpha_count > 0
    g = torch.Generator().manual_seed(2)
    q = rand_bf16(g, 1, 4, 2, 128)
    k, v = rand_bf16(g, 1, 2, 2, 128), rand_bf16(g, 1, 2, 2, 128)
    ka_ref, va_ref = ro.pack(ora, to_np(k), to_np(v), ora.cos, ora.sin)
    with torch.no_grad():
        out = log_kv_chunk_attention(gpu, q.cuda(), k.cuda(), v.cuda(), 128 ** -0.5, second_order_scale=0.0)
    assert_attention_close(out, ro.attention(to_np(q), ka_ref, va_ref, 128 ** -0.5, 2, 128))
    ka, va = pack_mid_kv(gpu, gpu._semantic_attention_plan(), k.cuda(), v.cuda(), packed_dim(128, 128))
    assert_pack_equal(ka, va, ka_ref, va_ref, 128)


@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16])
def test_decode_reuse_synthetic_state(table_dtype):
    """Decode steps with prefix reuse over a synthetic state (masses ~ U(1, 64)); each step
    commits its token to the recent window, so the next one re-packs only new rows."""
    dk = 128
    cos, sin = rope_tables(4096, dk, dtype=table_dtype)
    cache = LogStructuredKVCache(
        (2, 4, 4096, dk), (2, 4, 4096, dk), B=32, recent_size=96, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=6, semantic_flush_granularity=32, semantic_anchor_mode="mid",
        allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dk, alpha_exact_tokens=32,
        alpha_span_max_tokens=8)
    fill_readout_state(cache, seed=3, recent=80)
    g = torch.Generator().manual_seed(4)
    scale = dk ** -0.5
    for step in range(4):
        q = rand_bf16(g, 2, 8, 1, dk)
        k, v = rand_bf16(g, 2, 4, 1, dk), rand_bf16(g, 2, 4, 1, dk)
        check_step(cache, cos, sin, q, k, v, scale, reuse=True, table_bf16=table_dtype == torch.bfloat16)
        if step < 3:
            pos = torch.full((2, 1), cache.token_count, dtype=torch.int64)
            cache.add_recent(k.cuda(), v.cuda(), k_raw=k.cuda(), input_pos=pos.cuda(),
                             span_ends=[[False], [False]])
    assert cache._mid_decode_state is not None


def test_decode_across_flush():
    """Reuse is dropped when a flush rewrites the ladders."""
    gpu, ora = make_pair(batch=1, groups=2, recent=32, flush=32, max_seq=1024)
    mix = Mixture(1, 2, 128, 12, seed=11)
    feed(gpu, ora, mix, 0, 32)
    feed(gpu, ora, mix, 32, 31)
    g = torch.Generator().manual_seed(5)
    start = 63
    for step in range(4):
        q = rand_bf16(g, 1, 4, 1, 128)
        k, v = rand_bf16(g, 1, 2, 1, 128), rand_bf16(g, 1, 2, 1, 128)
        ka_ref, va_ref = ro.pack(ora, to_np(k), to_np(v), ora.cos, ora.sin)
        with torch.no_grad():
            out = log_kv_chunk_attention(gpu, q.cuda(), k.cuda(), v.cuda(), 0.1, second_order_scale=0.0,
                                         reuse_prefix=True)
        assert_attention_close(out, ro.attention(to_np(q), ka_ref, va_ref, 0.1, 1, 128))
        feed(gpu, ora, mix, start, 1)
        start += 1


def test_decode_qwen_shape():
    """Qwen3-1.7B GQA readout (16 query / 8 KV heads x 128) over a 32K-token cache layout:
    recent 2048, exact pool 256, K=12 ladders; batch 2 to keep the oracle quick."""
    dk = 128
    cos, sin = rope_tables(32768, dk)
    cache = LogStructuredKVCache(
        (2, 8, 32768, dk), (2, 8, 32768, dk), B=128, recent_size=2048, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=12, semantic_flush_granularity=2048, semantic_anchor_mode="mid",
        allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dk, alpha_exact_tokens=256,
        alpha_span_max_tokens=64)
    fill_readout_state(cache, seed=7, fill=0.6)
    g = torch.Generator().manual_seed(6)
    q = rand_bf16(g, 2, 16, 1, dk)
    k, v = rand_bf16(g, 2, 8, 1, dk), rand_bf16(g, 2, 8, 1, dk)
    check_step(cache, cos, sin, q, k, v, dk ** -0.5, reuse=True)


@pytest.mark.parametrize("dk,dv,heads,groups,tq", [
    (128, 128, 8, 8, 1),    # one query per KV group; the bias column starts a 16-byte unit of its own
    (120, 120, 6, 2, 1),    # three queries per group (one idle query slot)
    (128, 128, 8, 2, 1),    # four queries per group
    (60, 60, 4, 2, 1),      # dk not a multiple of 8: the bias shares a unit with the last key features
    (200, 104, 2, 2, 1),    # two key units per lane, narrower values
    (132, 128, 2, 2, 2),    # two current rows (causal), bias sharing a unit, two key units per lane
])
def test_streaming_decode_shapes(dk, dv, heads, groups, tq):
    """Decode steps of up to 4 query rows per KV group take the streaming kernel; every variant of it
    (queries per group, key units per lane, bias column on its own or not) against the oracle."""
    print(f"case dk={dk} dv={dv} heads={heads} groups={groups} tq={tq}", flush=True)
    cos, sin = rope_tables(2048, dk)
    cache = LogStructuredKVCache(
        (2, groups, 2048, dk), (2, groups, 2048, dv), B=16, recent_size=128, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=4, semantic_flush_granularity=128, semantic_anchor_mode="mid",
        allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dk, alpha_exact_tokens=16,
        alpha_span_max_tokens=8)
    fill_readout_state(cache, seed=dk + tq, recent=100)
    g = torch.Generator().manual_seed(dk)
    q = rand_bf16(g, 2, heads, tq, dk)
    k, v = rand_bf16(g, 2, groups, tq, dk), rand_bf16(g, 2, groups, tq, dv)
    check_step(cache, cos, sin, q, k, v, dk ** -0.5)


def test_causal_chunk():
    """A multi-row chunk: row i sees the prefix and current rows 0..i only."""
    dk = 64
    cos, sin = rope_tables(1024, dk)
    cache = LogStructuredKVCache(
        (1, 2, 1024, dk), (1, 2, 1024, dk), B=16, recent_size=64, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=4, semantic_flush_granularity=16, semantic_anchor_mode="mid",
        allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dk)
    fill_readout_state(cache, seed=8, recent=40)
    g = torch.Generator().manual_seed(7)
    q = rand_bf16(g, 1, 4, 8, dk)
    k, v = rand_bf16(g, 1, 2, 8, dk), rand_bf16(g, 1, 2, 8, dk)
    check_step(cache, cos, sin, q, k, v, dk ** -0.5)


@pytest.mark.parametrize("dk,heads,groups,tq,recent", [
    (64, 4, 2, 128, 40),      # 256 query rows per KV group, packed width 72 (five 16-wide steps)
    (128, 16, 8, 300, 100),   # Qwen3-1.7B heads; query tiles that span two heads
])
def test_matrix_core_chunk_attention(dk, heads, groups, tq, recent):
    """Chunks of many query rows take the MFMA chunk kernel; same math, same tolerance."""
    print(f"case dk={dk} heads={heads} tq={tq}", flush=True)
    cos, sin = rope_tables(4096, dk)
    cache = LogStructuredKVCache(
        (1, groups, 4096, dk), (1, groups, 4096, dk), B=16, recent_size=512, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=4, semantic_flush_granularity=512, semantic_anchor_mode="mid",
        allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dk)
    fill_readout_state(cache, seed=9, recent=recent)
    g = torch.Generator().manual_seed(3)
    q = rand_bf16(g, 1, heads, tq, dk)
    k, v = rand_bf16(g, 1, groups, tq, dk), rand_bf16(g, 1, groups, tq, dk)
    check_step(cache, cos, sin, q, k, v, dk ** -0.5)


def test_matrix_core_chunk_attention_alpha_pool():
    """With an exact pool (masked rows) and after real flushes."""
    gpu, _ = make_pair(batch=2, groups=2, dim=64, K=4, B=16, recent=64, flush=64, max_seq=2048, s_h=16.0, exact=32,
                       span=8, beta_novelty=True, beta_adaptive=True)
    mix = Mixture(2, 2, 64, clusters=4, seed=5)
    dev = gpu.level_k.device
    for blk in range(5):
        k, v = mix.rows(64), mix.rows(64)
        pos = torch.arange(blk * 64, (blk + 1) * 64).unsqueeze(0).expand(2, -1).contiguous()
        gpu.add_recent(k.to(dev), v.to(dev), k_raw=k.to(dev), input_pos=pos.to(dev), span_ends=mix.span_ends(blk * 64, 64, 8))
    g = torch.Generator().manual_seed(4)
    q = rand_bf16(g, 2, 4, 96, 64)
    k, v = rand_bf16(g, 2, 2, 96, 64), rand_bf16(g, 2, 2, 96, 64)
    cos, sin = gpu.cos_cache.cpu(), gpu.sin_cache.cpu()
    check_step(gpu, cos, sin, q, k, v, 64 ** -0.5)


@pytest.mark.parametrize("max_seq", [4096, 65536])   # one key range per query block, and key-range splits
def test_chunk_attention_any_value_magnitude(max_seq):
    """The matrix-core chunk attention over values of any bf16 magnitude: lanes scaled by 1e10,
    by 1e-30 and by 1, and a lane whose first half of the features is scaled by 1e10 and second
    half by 1e-30 (a span no single fp16 scale covers, so that lane reads its bf16 rows). Attention
    is linear in V, so each output feature must be within 2e-3 of the float64 oracle relative to
    max(its column's scale, |ref|), beyond the output's bf16 rounding."""
    print(f"case value magnitudes max_seq={max_seq}", flush=True)
    dk, heads, groups, tq = 128, 8, 4, 200
    cos, sin = rope_tables(max_seq, dk)
    cache = LogStructuredKVCache(
        (1, groups, max_seq, dk), (1, groups, max_seq, dk), B=32, recent_size=256, device="cuda",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=4, semantic_flush_granularity=256,
        semantic_anchor_mode="mid", allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dk)
    fill_readout_state(cache, seed=21, recent=200)
    col = torch.ones(groups, dk, dtype=torch.float64)
    col[0], col[1] = 1e10, 1e-30
    col[3, : dk // 2], col[3, dk // 2:] = 1e10, 1e-30
    scale_v = col.to(torch.float32).view(1, groups, 1, 1, 1, dk).to(cache.level_v.device)
    cache.level_v.copy_((cache.level_v.float() * scale_v).to(torch.bfloat16))
    rscale = scale_v.view(1, groups, 1, dk)
    cache.recent_v.copy_((cache.recent_v.float() * rscale).to(torch.bfloat16))
    g = torch.Generator().manual_seed(8)
    q = rand_bf16(g, 1, heads, tq, dk)
    k = rand_bf16(g, 1, groups, tq, dk)
    v = (torch.randn(1, groups, tq, dk, generator=g) * rscale.cpu()).to(torch.bfloat16)
    state = state_of(cache)
    ka_ref, va_ref = ro.pack(state, to_np(k), to_np(v), to_np(cos), to_np(sin))
    dev = cache.level_k.device
    with torch.no_grad():
        out = log_kv_chunk_attention(cache, q.to(dev), k.to(dev), v.to(dev), dk ** -0.5, second_order_scale=0.0)
    ref = ro.attention(to_np(q), ka_ref, va_ref, dk ** -0.5, tq, dk)
    got = to_np(out).astype(np.float64)
    assert np.isfinite(got).all()
    rep = heads // groups
    colscale = np.repeat(col.numpy(), rep, axis=0)[None, :, None, :]      # [1, heads, 1, dk]
    err = (np.abs(got - ref) - half_ulp_bf16(ref)) / np.maximum(colscale, np.abs(ref))
    assert err.max() <= ATOL, f"error beyond output rounding {err.max():.3e} > {ATOL}"
