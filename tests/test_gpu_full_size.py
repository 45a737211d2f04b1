"""Parity at the benchmarked sizes, where the kernels take the geometry they run in the benchmark:

* decode at batch 8 over a 32K-token Qwen3-1.7B cache (64 lanes of about 8.8K packed rows, so the
  streaming kernel splits each lane 20 ways), every output against the oracle's float64 attention;
* chunk attention of one 2048-token prefill block, 16 query heads, over a state of more than 5K
  packed rows per lane (key ranges split over many blocks), sampled query rows of three KV groups
  against the oracle;
* one layer's Alpha + Beta stream of 11 flushes of 2048 rows (B'=125, L=7), every state field bit
  for bit after every flush, with carries reaching level 3 and beyond;
* the unified route at T = 4096 rows on two lanes (4108 nodes per lane: the reducer's largest LDS
  layout and a 4096-key sort), bit for bit after each of two flushes, old-old merges included.

The oracle runs on the CPU at these sizes, so each test takes up to a minute."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import STATE_FIELDS, compare_state, feed, make_pair, to_np
from logkv_amd import LogStructuredKVCache, log_kv_chunk_attention
from oracle import readout as ro
from test_gpu_readout import assert_attention_close, check_step, rand_bf16, state_of
from workloads import Mixture, fill_readout_state, rope_tables

pytestmark = pytest.mark.gpu

G, D, N, F, EXACT, SPAN = 8, 128, 32768, 2048, 256, 64


def qwen_cache(batch):
    cos, sin = rope_tables(N, D)
    cache = LogStructuredKVCache(
        (batch, G, N, D), (batch, G, N, D), B=128, recent_size=F, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=12, semantic_s_h=64.0, semantic_flush_granularity=F,
        semantic_anchor_mode="mid", allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D,
        alpha_exact_tokens=EXACT, alpha_span_max_tokens=SPAN, beta_novelty=True, beta_adaptive_merge=True)
    return cache, cos, sin


@pytest.mark.timeout(300)
def test_decode_batch8_full_context():
    print("case decode batch 8, 32K context", flush=True)
    cache, cos, sin = qwen_cache(8)
    fill_readout_state(cache, seed=21, recent=F - 9, archived=N - F - EXACT)
    rows = int(cache._semantic_attention_plan().width) + cache.alpha_count + cache.recent_count + 1
    assert rows > 8000, rows
    g = torch.Generator().manual_seed(31)
    q = rand_bf16(g, 8, 16, 1, D)
    k, v = rand_bf16(g, 8, G, 1, D), rand_bf16(g, 8, G, 1, D)
    check_step(cache, cos, sin, q, k, v, D ** -0.5, reuse=True)


@pytest.mark.timeout(300)
def test_chunk_prefill_block_full_size():
    print("case chunk attention, 2048 rows x 16 heads", flush=True)
    cache, cos, sin = qwen_cache(1)
    fill_readout_state(cache, seed=5, recent=F, archived=N - 2 * F - EXACT)
    g = torch.Generator().manual_seed(8)
    q = rand_bf16(g, 1, 16, F, D)
    k, v = rand_bf16(g, 1, G, F, D), rand_bf16(g, 1, G, F, D)
    with torch.no_grad():
        out = log_kv_chunk_attention(cache, q.cuda(), k.cuda(), v.cuda(), D ** -0.5, second_order_scale=0.0)
    torch.cuda.synchronize()
    ka, va = ro.pack(state_of(cache), to_np(k), to_np(v), to_np(cos), to_np(sin))
    start = ka.shape[2] - F
    assert start > 5000, start
    out = to_np(out.float())                     # [1, 16, F, D]
    qn = to_np(q)
    for grp in (0, 3, 7):
        for a, b in ((0, 128), (1000, 1128), (F - 128, F)):
            ref = ro.attention(qn[:, 2 * grp:2 * grp + 2, a:b], ka[:, grp:grp + 1, :start + b],
                               va[:, grp:grp + 1, :start + b], D ** -0.5, b - a, D)
            assert_attention_close(torch.from_numpy(out[:, 2 * grp:2 * grp + 2, a:b].copy()), ref)


@pytest.mark.timeout(300)
def test_alpha_beta_qwen_layer_stream_11_flushes():
    print("case Alpha + Beta Qwen layer, 11 flushes", flush=True)
    gpu, ora = make_pair(1, G, D, 12, 128, F, F, N, 64.0, exact=EXACT, span=SPAN, beta_novelty=True,
                         beta_adaptive=True)
    assert (gpu.B_prime, gpu.L_alloc) == (125, 7)
    fields = STATE_FIELDS + ("alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid")
    mix = Mixture(1, G, D, clusters=12, seed=29)
    for blk in range(12):
        print(f"block {blk}", flush=True)
        feed(gpu, ora, mix, blk * F, F, with_ends=True)
        torch.cuda.synchronize()
        assert gpu.alpha_count == ora.alpha_count, f"block {blk}: alpha_count"
        assert gpu._alpha_spans == ora.alpha_spans, f"block {blk}: spans"
        bad = compare_state(gpu, ora, fields)
        assert not bad, f"block {blk}: " + "; ".join(bad)
    assert int(ora.level_count[..., 3:].sum()) > 0, "no carry reached level 3"


@pytest.mark.timeout(300)
def test_unified_flush_4096_rows_two_lanes():
    from test_gpu_unified import _pair

    print("case unified route, T=4096, 2 lanes", flush=True)
    T = 4096
    gpu, ora = _pair(1, 2, D, 12, 128, T, 3 * T, 64.0)
    mix = Mixture(1, 2, D, clusters=14, seed=17, drift_every=T)
    dev = gpu.level_k.device
    for i in range(2):
        print(f"flush {i}", flush=True)
        k, v = mix.rows(T), mix.rows(T)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).contiguous()
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev))
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy(), None)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"flush {i}: " + "; ".join(bad)
    assert ora.ward_merges > 0, "no old-old merge was exercised"


@pytest.mark.timeout(300)
def test_unified_benched_geometry_sampled_lanes():
    """The unified-route benchmark's geometry on the device - batch 4 x 8 KV groups (32 lanes), 4096-row
    flushes, B=128, L=9 (131,072-token stream), s_h=64, the benchmark's drifting 12-Gaussian mixture -
    for five flushes (the centers drift before the fifth), with two lanes
    (first and last) checked after every flush against the oracle's reducer and commit (the Torch
    restatement, bit-identical to the numpy oracle) fed the same two lanes' rows: lanes are
    independent, so the sampled lanes see exactly what the whole batch saw."""
    from oracle.torch_cpu import TorchCpuCache
    from test_gpu_unified import _pair

    print("case unified route, benchmark geometry (32 lanes), lanes (0,0) and (3,7)", flush=True)
    Bt, T, N = 4, 4096, 131072
    gpu, _ = _pair(Bt, G, D, 12, 128, T, N, 64.0)
    assert gpu.L_alloc == 9
    cos, sin = rope_tables(N, D)
    ora = TorchCpuCache(2, 1, N, D, D, B=128, recent_size=T, K=12, s_h=64.0, flush=T, cos=cos.numpy(),
                        sin=sin.numpy(), unified=True)
    lanes = ((0, 0), (3, 7))
    mix = Mixture(Bt, G, D, clusters=12, seed=31, drift_every=2 * 16384)
    dev = gpu.level_k.device
    for i in range(5):
        print(f"flush {i}", flush=True)
        k, v = mix.rows(T), mix.rows(T)
        pos = torch.arange(i * T, (i + 1) * T).unsqueeze(0).expand(Bt, -1).contiguous()
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev))
        pick = lambda x: torch.stack([x[b, g] for b, g in lanes])[:, None].float().numpy()
        ora.flush_rows(pick(k), pick(v), pos[:2].numpy(), None)
        torch.cuda.synchronize()
        for f in STATE_FIELDS:
            a = to_np(getattr(gpu, f))
            got = np.stack([a[b, g] for b, g in lanes])[:, None]
            want = np.asarray(getattr(ora, f))
            if got.dtype == np.bool_ or want.dtype == np.bool_:
                same = got.astype(bool) == want.astype(bool)
            else:
                same = got.astype(want.dtype) == want
            assert same.all(), f"flush {i}: {f}: {int((~same).sum())} mismatches"
    assert int(ora.level_count[..., 1:].sum()) > 0 and ora.alive.sum() == 24
