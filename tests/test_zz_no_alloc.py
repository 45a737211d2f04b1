"""The allocation-free decode entry point (logkv_decode_attention_static) against the
workspace one (logkv_decode_attention), both called through the C ABI: the same
kernels, so the outputs must be bit-identical, on two calls in a row - the second
smaller, with another kernel path - and a call beyond the static scratch is refused
before anything is launched."""

from __future__ import annotations

import ctypes as C

import pytest
import torch

from logkv_amd import LogStructuredKVCache, _lib, pack_mid_kv, packed_dim
from workloads import fill_readout_state, rope_tables

pytestmark = pytest.mark.gpu

STATIC_SCRATCH_BYTES = 16 << 20


def _inv_scale_bf16(scale):
    return torch.tensor(1.0 / scale, dtype=torch.float32).to(torch.bfloat16).item()


def _args(q, ka, va, width_rows, tail, scale, n_groups, out, exact=None):
    bt, hq, tq, dk = q.shape
    return _lib.AttentionArgs(
        q.data_ptr(), *q.stride()[:3], bt, hq, n_groups, tq, dk, out.size(-1), ka.size(3), ka.data_ptr(),
        va.data_ptr(), ka.size(2), tail, 0, float(scale), _inv_scale_bf16(scale), out.data_ptr(), *out.stride()[:3],
        None if exact is None else exact.data_ptr())


def _packed_case(batch, groups, heads, tq, seed, max_seq):
    dev = torch.device("cuda")
    cos, sin = rope_tables(max_seq, 128)
    cache = LogStructuredKVCache((batch, groups, max_seq, 128), (batch, groups, max_seq, 128), B=32,
                                 recent_size=128, device=dev, dtype=torch.bfloat16, semantic_clusters=True,
                                 cluster_k_max=12, semantic_s_h=64.0, semantic_flush_granularity=128,
                                 semantic_anchor_mode="mid", allocate_second_order=False, cos_cache=cos,
                                 sin_cache=sin, rope_n_elem=128, alpha_exact_tokens=64, alpha_span_max_tokens=16)
    fill_readout_state(cache, seed=seed)
    g = torch.Generator(device="cpu").manual_seed(seed + 1)
    k = torch.randn(batch, groups, tq, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(batch, groups, tq, 128, generator=g).to(torch.bfloat16).to(dev)
    q = torch.randn(batch, heads, tq, 128, generator=g).to(torch.bfloat16).to(dev)
    plan = cache._semantic_attention_plan()
    ka, va = pack_mid_kv(cache, plan, k, v, packed_dim(128, 128))
    ka, va = ka.contiguous(), va.contiguous()
    tail = cache.recent_count + tq
    return cache, plan, q, ka, va, tail


def _both(cache, plan, q, ka, va, tail):
    lib = _lib.lib()
    scale = 128 ** -0.5
    stream = torch.cuda.current_stream().cuda_stream
    out_ws = torch.full((*q.shape[:3], 128), float("nan"), dtype=torch.bfloat16, device=q.device)
    out_st = out_ws.clone()
    a_ws = _args(q, ka, va, plan.width, tail, scale, cache.n_groups, out_ws, cache.alpha_count_dev)
    a_st = _args(q, ka, va, plan.width, tail, scale, cache.n_groups, out_st, cache.alpha_count_dev)
    need = lib.logkv_attention_workspace_bytes(C.byref(a_ws))
    assert 0 < need <= STATIC_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.check(lib.logkv_decode_attention(C.byref(a_ws), plan.table.data_ptr(), plan.table.numel(), ws.data_ptr(),
                                          need, stream), "logkv_decode_attention")
    _lib.check(lib.logkv_decode_attention_static(C.byref(a_st), plan.table.data_ptr(), plan.table.numel(), stream),
               "logkv_decode_attention_static")
    torch.cuda.synchronize()
    return out_ws, out_st


def test_static_decode_equals_workspace_decode_twice():
    # First call: batch 8 x 8 KV groups, 16 query heads, one query row (streaming kernel).
    big = _packed_case(8, 8, 16, 1, seed=3, max_seq=8192)
    out_ws, out_st = _both(*big)
    assert not torch.isnan(out_ws.float()).any()
    assert torch.equal(out_ws, out_st)
    # Second call, smaller: batch 2 x 4 KV groups, 16 heads, two query rows (8 queries per KV
    # group: the tiled kernel). The scratch keeps the first call's partials; they must not leak.
    small = _packed_case(2, 4, 16, 2, seed=5, max_seq=4096)
    out_ws, out_st = _both(*small)
    assert not torch.isnan(out_ws.float()).any()
    assert torch.equal(out_ws, out_st)


def test_static_decode_refuses_more_than_its_scratch():
    lib = _lib.lib()
    dev = torch.device("cuda")
    # 64 lanes x 16 queries per KV group over 16896 rows: 33 splits of partials, 17.6 MB > 16 MiB.
    bt, G, heads, tq, cap, dim = 8, 8, 64, 2, 16896, 136
    ka = torch.zeros(bt, G, cap, dim, dtype=torch.bfloat16, device=dev)
    va = torch.zeros_like(ka)
    q = torch.zeros(bt, heads, tq, 128, dtype=torch.bfloat16, device=dev)
    out = torch.full((bt, heads, tq, 128), 7.0, dtype=torch.bfloat16, device=dev)
    table = torch.tensor([cap - 16], dtype=torch.int32, device=dev)
    a = _args(q, ka, va, cap - 16, 16, 128 ** -0.5, G, out)
    assert lib.logkv_attention_workspace_bytes(C.byref(a)) > STATIC_SCRATCH_BYTES
    rc = lib.logkv_decode_attention_static(C.byref(a), table.data_ptr(), 1, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.LOGKV_EINVAL
    assert "static scratch" in lib.logkv_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
