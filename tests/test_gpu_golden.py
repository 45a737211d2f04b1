"""The device path against the golden fixtures of the reference's own CPU Torch path (tests/golden,
written by make_fixtures.py): the same flush sequences fed to the HIP cache (every state field after
every block: integers bit for bit, payloads within one bf16 ulp, masses / centers within 1e-5
relative), the HIP Beta cut kernel on the fixture's blocks, and the HIP packer on a cache whose RoPE
tables are bf16."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_data import bf16_ulp, compare_state, config, from_bits, load, tables
from harness import to_np
from logkv_amd import LogStructuredKVCache
from logkv_amd.beta_log_kv import make_layout, merge_blocks, select_cuts
from logkv_amd.log_kv_pack import pack_mid_kv

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def device_cache(cfg, data):
    cos, sin = tables(data)
    shape = (cfg["batch"], cfg["groups"], cfg["max_seq"], cfg["dim"])
    return LogStructuredKVCache(
        shape, shape, B=cfg["B"], recent_size=cfg["recent"], device="cuda", dtype=torch.bfloat16,
        semantic_clusters=True, cluster_k_max=cfg["K"], semantic_s_h=cfg["s_h"],
        semantic_flush_granularity=cfg["flush"], semantic_anchor_mode="mid", allocate_second_order=False,
        cos_cache=cos, sin_cache=sin, rope_n_elem=cfg["dim"], alpha_exact_tokens=cfg["exact"],
        alpha_span_max_tokens=cfg["span"], beta_novelty=cfg["beta"], beta_adaptive_merge=cfg["beta"])


def bf16_rows(bits_array) -> torch.Tensor:
    return torch.from_numpy(from_bits(bits_array)).to(torch.bfloat16).to(DEV)


def device_get(cache):
    def get(name):
        if name == "alpha_spans":
            return cache._alpha_spans
        return to_np(getattr(cache, name))
    return get


@pytest.mark.parametrize("name,alpha", [("flush_alpha_beta.npz", True), ("flush_attach_seeded.npz", False)])
def test_device_flush_sequence_matches_reference(name, alpha):
    data = load(name)
    cfg = config(data)
    cache = device_cache(cfg, data)
    assert (cache.B_prime, cache.L_alloc) == (int(data["B_prime"]), int(data["levels"]))
    for i in range(int(data["blocks"])):
        print(f"{name}: block {i}", flush=True)
        k_raw, v, k = (bf16_rows(data[f"{f}_{i}"]) for f in ("k_raw", "v", "k"))
        pos = torch.from_numpy(data[f"pos_{i}"]).to(DEV)
        ends = data[f"ends_{i}"].astype(bool).tolist() if alpha else None
        cache.add_recent(k, v, k_raw=k_raw, input_pos=pos, span_ends=ends)
        torch.cuda.synchronize()
        bad = compare_state(device_get(cache), data, i, alpha)
        assert not bad, f"block {i}: " + "; ".join(bad)
        assert cache.recent_count == int(data[f"recent_count_{i}"])
        if alpha:
            assert cache.alpha_count == int(data[f"alpha_count_{i}"])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_device_beta_cuts_match_reference(dtype):
    data = load("select_cuts.npz")
    n = len(data["w"])
    k = torch.from_numpy(data["k"]).to(DEV)
    v = torch.from_numpy(data["v"]).to(DEV)
    w = torch.from_numpy(data["w"]).to(DEV)
    meta = torch.zeros(n, dtype=torch.int64, device=DEV)
    block = (k, v, w, None, None, None, None, None, meta, meta.clone(), meta.clone(), meta.clone(),
             torch.zeros(n, dtype=torch.bool, device=DEV))
    layout = make_layout(data["lengths"], DEV)
    np.testing.assert_array_equal(layout.cpu().numpy(), data["layout"])
    if dtype is torch.float32:
        np.testing.assert_array_equal(select_cuts(block, layout).cpu().numpy(), data["cuts"])
        return
    # bf16 payloads: the reference rounds them to float32 before the cost, so the fixture's float32
    # rows rounded to bf16 must give the cuts of the same rows rounded on the host.
    from oracle import ladder as ol

    kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)
    rows = {"k": kb.float().cpu().numpy(), "v": vb.float().cpu().numpy(), "w": data["w"],
            "p_lo": np.zeros(n, np.int64), "p_hi": np.zeros(n, np.int64), "sum_wp": np.zeros(n, np.int64),
            "order": np.zeros(n, np.int64), "pad": np.zeros(n, bool)}
    _, want = ol.beta_merge(rows, data["lengths"])
    _, got = merge_blocks((kb, vb) + block[2:], data["lengths"])
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_device_packer_with_bf16_tables_matches_reference():
    data = load("pack_torch.npz")
    cfg = dict(batch=1, groups=2, dim=32, max_seq=1024, K=4, B=8, recent=32, flush=32, exact=16, span=4, beta=False,
               s_h=16.0)
    cache = device_cache(cfg, data)
    assert cache.cos_cache.dtype is torch.bfloat16
    for i in range(int(data["blocks"])):
        cache.add_recent(bf16_rows(data[f"k_{i}"]), bf16_rows(data[f"v_{i}"]), k_raw=bf16_rows(data[f"k_raw_{i}"]),
                         input_pos=torch.from_numpy(data[f"pos_{i}"]).to(DEV),
                         span_ends=data[f"ends_{i}"].astype(bool).tolist())
    plan = cache._semantic_attention_plan()
    ka, va = pack_mid_kv(cache, plan, bf16_rows(data["cur_k"]), bf16_rows(data["cur_v"]), 40)
    ka, va = to_np(ka), to_np(va)
    want_k, want_v = from_bits(data["ka"]), from_bits(data["va"])
    assert ka.shape == want_k.shape
    np.testing.assert_array_equal(va, want_v)
    np.testing.assert_array_equal(np.delete(ka, 32, -1), np.delete(want_k, 32, -1))
    bias, ref = ka[..., 32], want_k[..., 32]
    assert (np.abs(bias - ref) <= bf16_ulp(ref)).all()
