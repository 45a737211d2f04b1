"""Streaming inference over the device cache (litgpt/model.py:1125-1361): the cache
state after a stream does not depend on how its tokens were split between block
prefill and pending-pair decode (bit for bit, every ladder / exact-pool / center
field), and outputs agree (within the attention tolerance) wherever the reference
states the semantics coincide: before any compaction, and for decode tokens."""

import numpy as np
import pytest
import torch

from harness import STATE_FIELDS, to_np
from logkv_amd import LogKVStreamingAttention, LogStructuredKVCache
from workloads import Mixture, rope_tables

pytestmark = pytest.mark.gpu

B, G, HQ, D, N, R = 2, 2, 4, 64, 512, 16


def new_engine(block):
    cos, sin = rope_tables(N, D)
    cache = LogStructuredKVCache(
        (B, G, N, D), (B, G, N, D), B=8, recent_size=R, device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=4, semantic_s_h=16.0, semantic_flush_granularity=R,
        semantic_anchor_mode="mid", allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D,
        alpha_exact_tokens=8, alpha_span_max_tokens=4, beta_novelty=True, beta_adaptive_merge=True)
    return LogKVStreamingAttention(cache, D ** -0.5, prefill_block=block)


def stream_inputs(T, seed=9):
    mix = Mixture(B, G, D, clusters=4, seed=seed)
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, HQ, T, D, generator=g)).to(torch.bfloat16).cuda()
    k, v, k_raw = mix.rows(T).cuda(), mix.rows(T).cuda(), mix.rows(T).cuda()
    ends = mix.span_ends(0, T, 5)
    return q, k, v, k_raw, ends


def run(engine, inputs, cuts):
    """Feed tokens [cuts[i], cuts[i + 1]) per call; returns outputs [B, T, HQ * D] as float."""
    q, k, v, k_raw, ends = inputs
    outs = []
    for a, b in zip(cuts[:-1], cuts[1:]):
        pos = torch.arange(a, b, device="cuda")
        outs.append(engine(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], k_raw[:, :, a:b], input_pos=pos,
                           span_ends=[row[a:b] for row in ends]))
    torch.cuda.synchronize()
    return torch.cat(outs, dim=1).float()


def assert_same_state(c1, c2):
    for f in STATE_FIELDS + ("recent_k", "recent_v", "alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid"):
        a, b = to_np(getattr(c1, f)), to_np(getattr(c2, f))
        assert np.array_equal(a, b, equal_nan=True), f"field {f} differs"
    assert c1.recent_count == c2.recent_count and c1.token_count == c2.token_count


def assert_close(a, b, what):
    """|a - b| <= 2e-3 * max(1, |b|) + one bf16 ulp of b: both outputs are rounded to bf16
    after computations that may differ in their last bits (different packed-row counts)."""
    mag = b.abs().clamp_min(1e-30)
    ulp = torch.where(b != 0, torch.exp2(torch.floor(torch.log2(mag)) - 7), torch.zeros_like(b))
    err = (((a - b).abs() - ulp) / b.abs().clamp_min(1.0)).max().item()
    assert err <= 2e-3, f"{what}: error beyond one bf16 ulp {err:.3e}"


def test_prefill_then_decode_matches_token_by_token_streaming():
    T = 48
    inputs = stream_inputs(T)
    blocky, single = new_engine(8), new_engine(8)
    # Stream 1: an odd prefill in blocks of 8 (its last token pending), then decode token by token.
    out1 = run(blocky, inputs, [0, 37] + list(range(38, T + 1)))
    # Stream 2: every token its own call (pending pairs throughout).
    out2 = run(single, inputs, list(range(0, T + 1)))
    assert blocky._log_kv_pending is None and single._log_kv_pending is None
    assert_same_state(blocky.cache, single.cache)
    # Before the first flush (the window holds R tokens) the block prefill is strict streaming.
    assert_close(out1[:, :R + 2], out2[:, :R + 2], "prefill before compaction")
    assert_close(out1[:, 37:], out2[:, 37:], "decode tokens")


def test_block_two_prefill_is_strict_streaming():
    T = 41
    inputs = stream_inputs(T, seed=4)
    pairs, single = new_engine(2), new_engine(2)
    out1 = run(pairs, inputs, [0, T])
    out2 = run(single, inputs, list(range(0, T + 1)))
    assert pairs._log_kv_pending is not None and single._log_kv_pending is not None
    assert_same_state(pairs.cache, single.cache)
    assert_close(out1, out2, "block-2 prefill vs token-by-token")
    # The pending token is part of the next call's first pair.
    q, k, v, k_raw, _ = stream_inputs(T + 1, seed=4)
    ends = [[False] for _ in range(B)]
    for e in (pairs, single):
        e(q[:, :, T:], k[:, :, T:], v[:, :, T:], k_raw[:, :, T:], input_pos=torch.tensor([T], device="cuda"),
          span_ends=ends)
        assert e._log_kv_pending is None
    assert_same_state(pairs.cache, single.cache)


def test_stream_matches_the_oracle():
    """Oracle evidence for the engine (litgpt/model.py:1219-1340): after an odd block prefill and
    token-by-token decode, the device cache equals an oracle cache fed the same tokens in 2-token
    commits, bit for bit; every decode output equals the float64 attention of its query over the
    oracle's state then plus the pending-and-current pair (non-causal among the two) or, for a
    token left pending, over the state plus itself."""
    from oracle import OracleCache
    from oracle import readout as ro

    T, prefill = 44, 29
    q, k, v, k_raw, ends = stream_inputs(T, seed=21)
    engine = new_engine(8)
    cache = engine.cache
    cos, sin = cache.cos_cache.cpu().numpy(), cache.sin_cache.cpu().numpy()
    ora = OracleCache(B, G, N, D, D, B=8, recent_size=R, K=4, s_h=16.0, flush=R, exact_tokens=8, span_max=4,
                      beta_novelty=True, beta_adaptive=True, cos=cos, sin=sin)
    qn, kn, vn, krn = to_np(q), to_np(k), to_np(v), to_np(k_raw)
    pos = np.arange(T)[None].repeat(B, 0)

    def commit(a, b):
        ora.add_recent(kn[:, :, a:b], vn[:, :, a:b], krn[:, :, a:b], pos[:, a:b], [row[a:b] for row in ends])

    run(engine, (q, k, v, k_raw, ends), [0, prefill])
    for a in range(0, prefill - 1, 2):        # the prefill commits every pair; its last token waits
        commit(a, a + 2)
    scale = D ** -0.5
    pending = prefill - 1
    for i in range(prefill, T):
        out = run(engine, (q, k, v, k_raw, ends), [i, i + 1])
        if pending is not None:
            ka, va = ora.pack(kn[:, :, pending:i + 1], vn[:, :, pending:i + 1])
            ref = ro.attention(qn[:, :, i:i + 1], ka, va, scale, 0, D)
            commit(pending, i + 1)
            pending = None
        else:
            ka, va = ora.pack(kn[:, :, i:i + 1], vn[:, :, i:i + 1])
            ref = ro.attention(qn[:, :, i:i + 1], ka, va, scale, 1, D)
            pending = i
        ref = torch.from_numpy(ref.transpose(0, 2, 1, 3).reshape(B, 1, HQ * D)).float()
        assert_close(out.cpu(), ref, f"decode token {i}")
    assert ora.token_count + (1 if pending is not None else 0) == T
    torch.cuda.synchronize()
    for f in STATE_FIELDS:
        a = to_np(getattr(cache, f))
        b = np.asarray(getattr(ora, f))
        assert np.array_equal(a.astype(np.float64), b.astype(np.float64)), f"field {f} differs from the oracle"
    assert cache.recent_count == ora.recent_count
    np.testing.assert_array_equal(to_np(cache.alpha_pos), ora.alpha_pos)
    np.testing.assert_array_equal(to_np(cache.alpha_valid).astype(bool), ora.alpha_valid)
