"""Training on the device: the matrix-core backward of the packed chunk attention against the
oracle's float64 gradient (within the reference's bf16 gradient tolerance, atol = rtol = 0.04 as in
its tests/test_log_kv_flash.py:45-66), slot-attention gradients (masked slots get exactly zero), and
LogKVStreamTrainingAttention: its forward and gradients equal a naive per-block autograd graph over
the same kernels bit for bit, and the backward's replay rebuilds the forward's cache state bit for bit
(op-log replay without Alpha; update tape with Alpha and Beta)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from harness import STATE_FIELDS, feed, make_pair, to_np
from logkv_amd import LogStructuredKVCache, log_kv_chunk_attention, log_kv_slot_attention
from logkv_amd.log_kv_cache import LogKVStreamTrainingAttention
from oracle import readout as ro
from test_gpu_readout import state_of
from workloads import Mixture, rope_tables

pytestmark = pytest.mark.gpu

TOL = 0.04


def assert_grad_close(got, ref, what):
    got = to_np(got).astype(np.float64)
    err = np.abs(got - ref) - (TOL + TOL * np.abs(ref))
    assert err.max() <= 0, f"{what}: gradient off by {err.max() + TOL:.3e} beyond {TOL} + {TOL}|ref|"


def _cache(exact=32, seed=3, blocks=6):
    gpu, ora = make_pair(batch=2, groups=2, dim=128, K=6, B=8, recent=64, flush=64, max_seq=4096, s_h=64.0,
                         exact=exact, span=8, beta_novelty=bool(exact), beta_adaptive=bool(exact))
    mix = Mixture(2, 2, 128, clusters=6, seed=seed)
    for blk in range(blocks):
        feed(gpu, ora, mix, blk * 48, 48, with_ends=bool(exact))
    torch.cuda.synchronize()
    return gpu


@pytest.mark.parametrize("heads,tq", [(4, 2), (4, 64), (8, 150)])
def test_chunk_backward_matches_float64_oracle(heads, tq):
    cache = _cache()
    g = torch.Generator().manual_seed(heads * 1000 + tq)
    dev = cache.level_k.device
    q = torch.randn(2, heads, tq, 128, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    k = torch.randn(2, 2, tq, 128, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    v = torch.randn(2, 2, tq, 128, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    dout = torch.randn(2, heads, tq, 128, generator=g).to(torch.bfloat16).to(dev)
    scale = 128 ** -0.5
    y = log_kv_chunk_attention(cache, q, k, v, scale, second_order_scale=0.0)
    dq, dk, dv = torch.autograd.grad(y, (q, k, v), dout)
    ka, va = ro.pack(state_of(cache), to_np(k), to_np(v), cache.cos_cache.cpu().numpy(), cache.sin_cache.cpu().numpy())
    rq, rk, rv = ro.attention_grad(to_np(q), ka, va, scale, tq, 128, to_np(dout), grad_rows=tq)
    assert_grad_close(dq, rq, "dq")
    assert_grad_close(dk, rk, "dk")
    assert_grad_close(dv, rv, "dv")


def test_slot_attention_gradients():
    g = torch.Generator().manual_seed(17)
    dev = torch.device("cuda")
    B, G, H, S, tq = 2, 2, 4, 90, 5
    sk = torch.randn(B, G, S, 64, generator=g).to(torch.bfloat16)
    sv = torch.randn(B, G, S, 64, generator=g).to(torch.bfloat16)
    valid = torch.rand(B, G, 40, generator=g) < 0.6
    sk[:, :, :40][~valid] = 1000            # payload of masked slots must not leak
    sw = torch.randint(1, 30, (B, G, S), generator=g).float()
    q = torch.randn(B, H, tq, 64, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, H, tq, 64, generator=g).to(torch.bfloat16)
    qd, kd, vd = (x.to(dev).requires_grad_(True) for x in (q, sk, sv))
    scale = 64 ** -0.5
    y = log_kv_slot_attention(qd, kd, vd, sw.to(dev), scale, causal_tail=tq, slot_valid=valid.to(dev))
    dq, dk, dv = torch.autograd.grad(y, (qd, kd, vd), dout.to(dev))
    ka, va = ro.slot_pack(to_np(sk), to_np(sv), sw.numpy(), slot_valid=valid.numpy())
    rq, rk, rv = ro.attention_grad(to_np(q), ka, va, scale, tq, 64, to_np(dout), grad_rows=S)
    assert_grad_close(dq, rq, "dq")
    assert_grad_close(dk, rk, "dk")
    assert_grad_close(dv, rv, "dv")
    masked = ~valid.to(dev)
    assert int(torch.count_nonzero(dk[:, :, :40][masked])) == 0
    assert int(torch.count_nonzero(dv[:, :, :40][masked])) == 0


def _training_cache(alpha, unified=False):
    cos, sin = rope_tables(1024, 128)
    return LogStructuredKVCache((1, 2, 1024, 128), (1, 2, 1024, 128), B=8, recent_size=64, device="cuda",
                                dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=6, semantic_s_h=64.0,
                                semantic_flush_granularity=32, semantic_anchor_mode="mid",
                                allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=128,
                                semantic_replay_updates=alpha, alpha_exact_tokens=32 if alpha else 0,
                                alpha_span_max_tokens=8, beta_novelty=alpha, beta_adaptive_merge=alpha,
                                semantic_unified_route=unified)


@pytest.mark.parametrize("alpha,unified", [(False, False), (True, False), (False, True)])
def test_stream_training_matches_naive_graph_and_replays_the_cache(alpha, unified):
    T, block, heads = 320, 32, 4
    mix = Mixture(1, 2, 128, clusters=6, seed=41)
    k_raw, v = mix.rows(T).cuda(), mix.rows(T).cuda()
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, heads, T, 128, generator=g).to(torch.bfloat16).cuda()
    k = k_raw.clone()                       # post-RoPE keys stand-in: any bf16 keys
    dout = torch.randn(1, heads, T, 128, generator=g).to(torch.bfloat16).cuda()
    ends = [[(p + 3) % 9 == 0 for p in range(T)]] if alpha else None
    scale = 128 ** -0.5

    # Naive graph: per block, attention with a gradient, then the detached commit.
    cache = _training_cache(alpha, unified)
    qn, kn, vn = (x.clone().requires_grad_(True) for x in (q, k, v))
    outs = []
    for s in range(0, T, block):
        outs.append(log_kv_chunk_attention(cache, qn[:, :, s:s + block], kn[:, :, s:s + block], vn[:, :, s:s + block],
                                           scale, 0.0))
        cache.add_recent(kn[:, :, s:s + block].detach(), vn[:, :, s:s + block].detach(),
                         k_raw=k_raw[:, :, s:s + block], span_ends=None if ends is None else
                         [row[s:s + block] for row in ends])
    naive = torch.cat(outs, dim=2)
    naive_state = {f: getattr(cache, f).clone() for f in STATE_FIELDS}
    gn = torch.autograd.grad(naive, (qn, kn, vn), dout)

    cache2 = _training_cache(alpha, unified)
    ql, kl, vl = (x.clone().requires_grad_(True) for x in (q, k, v))
    y = LogKVStreamTrainingAttention.apply(ql, kl, vl, cache2, scale, block, 0.0, k_raw, ends)
    assert torch.equal(y, naive)
    for f, x in naive_state.items():
        assert torch.equal(getattr(cache2, f), x), f"forward state {f}"
    gl = torch.autograd.grad(y, (ql, kl, vl), dout)
    for a, b, name in zip(gl, gn, ("dq", "dk", "dv")):
        assert torch.equal(a, b), name
    # The backward's replay rebuilt the forward's cache.
    for f, x in naive_state.items():
        assert torch.equal(getattr(cache2, f), x), f"replayed state {f}"
    if alpha:
        assert int(cache2.alpha_valid.sum()) > 0
