"""Shared helpers: paired device cache / oracle cache and state comparison."""

from __future__ import annotations

import numpy as np
import torch

from workloads import Mixture, rope_tables

STATE_FIELDS = ("level_k", "level_v", "level_w", "level_p_lo", "level_p_hi", "level_sum_wp", "level_order",
                "pad_mask", "level_count", "centroid", "n_eff", "n_total", "p_hi_c", "level0_phase", "alive")


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


def make_pair(batch=1, groups=2, dim=128, K=12, B=128, recent=64, flush=64, max_seq=4096, s_h=64.0, exact=0,
              span=16, beta_novelty=False, beta_adaptive=False, centroid_backend="sequential", hard_cap_mult=0.0,
              lam=1.0):
    from logkv_amd import LogStructuredKVCache
    from oracle import OracleCache

    cos, sin = rope_tables(max_seq, dim)
    gpu = LogStructuredKVCache(
        (batch, groups, max_seq, dim), (batch, groups, max_seq, dim), B=B, recent_size=recent, device="cuda",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=s_h,
        semantic_flush_granularity=flush, semantic_anchor_mode="mid", allocate_second_order=False,
        cos_cache=cos, sin_cache=sin, rope_n_elem=dim, alpha_exact_tokens=exact, alpha_span_max_tokens=span,
        beta_novelty=beta_novelty, beta_adaptive_merge=beta_adaptive, semantic_centroid_backend=centroid_backend,
        semantic_capacity_hard_cap_mult=hard_cap_mult, cluster_lambda_rel=lam)
    ora = OracleCache(batch, groups, max_seq, dim, dim, B=B, recent_size=recent, K=K, s_h=s_h, flush=flush,
                      exact_tokens=exact, span_max=span, beta_novelty=beta_novelty, beta_adaptive=beta_adaptive,
                      cos=cos.numpy(), sin=sin.numpy(), centroid_tile=32 if centroid_backend == "parallel" else 1,
                      hard_cap_mult=hard_cap_mult, lam=lam)
    return gpu, ora


def feed(gpu, ora, mix: Mixture, start: int, n: int, with_ends=False):
    k_raw = mix.rows(n)
    v = mix.rows(n)
    k = mix.rows(n)
    pos = torch.arange(start, start + n).unsqueeze(0).expand(mix.batch, -1).contiguous()
    ends = mix.span_ends(start, n) if with_ends else None
    dev = gpu.level_k.device
    gpu.add_recent(k.to(dev), v.to(dev), k_raw=k_raw.to(dev), input_pos=pos.to(dev), span_ends=ends)
    ora.add_recent(k.float().numpy(), v.float().numpy(), k_raw.float().numpy(), pos.numpy(), ends)


def compare_state(gpu, ora, fields=STATE_FIELDS):
    """Bit-exact (value-equal) comparison; returns a list of mismatch descriptions."""
    bad = []
    for f in fields:
        a = to_np(getattr(gpu, f))
        b = np.asarray(getattr(ora, f))
        if a.shape != b.shape:
            bad.append(f"{f}: shape {a.shape} vs {b.shape}")
            continue
        if a.dtype == np.bool_ or b.dtype == np.bool_:
            eq = a.astype(bool) == b.astype(bool)
        elif np.issubdtype(b.dtype, np.floating):
            eq = (a == b) | (np.isnan(a) & np.isnan(b))
        else:
            eq = a.astype(np.int64) == b.astype(np.int64)
        if not eq.all():
            idx = np.argwhere(~eq)
            first = tuple(idx[0])
            bad.append(f"{f}: {int((~eq).sum())} mismatches, first at {first}: gpu={a[first]} oracle={b[first]}")
    return bad
