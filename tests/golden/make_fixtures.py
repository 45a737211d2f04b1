"""Write the golden fixtures of tests/golden from the reference's own CPU Torch path.

Run only where the reference tree is present (it is read from /root/reference; the tests read
the fixtures, never the reference): ``python tests/golden/make_fixtures.py``. It imports the reference's hot-path
modules through a bare namespace package, as the reference's own tools do
(unused/semantic_logkv_microbench.py:22-25), so neither ``litgpt/__init__.py`` nor anything
outside the LogKV modules is imported, and runs them on the CPU with seeded inputs:

* ``flush_alpha_beta.npz`` - a streamed sequence through ``LogStructuredKVCache`` with attach
  routing, the Alpha exact pool and Beta (litgpt/log_kv_cache.py:5847, :3904-4003): the inputs of
  every block and the whole cache state after it (integer fields, host mirrors, bf16 payloads,
  float32 masses / centers), which pins the driver's numbering (``level_order``,
  ``level0_phase``), the delayed archive and the Alpha / Beta choices end to end;
* ``flush_attach_seeded.npz`` - the same without Alpha, with orphans seeding new clusters
  (litgpt/log_kv_cache.py:4636-4680);
* ``choose_spans.json`` - random candidate sets cut by ``cut_spans`` and chosen by
  ``choose_spans`` with scores that tie (litgpt/alpha_log_kv.py:84-226);
* ``select_cuts.npz`` - Beta cuts of random blocks, near ties (identical rows) and two-row tails
  (litgpt/beta_log_kv.py:29-46);
* ``pack_torch.npz`` - the reference's Torch packer (``pack_mid_kv(..., backend="torch")``,
  litgpt/log_kv_pack.py:27-72) on a cache whose RoPE tables are bf16 (products rounded first).

Inputs are drawn from ``workloads.Mixture`` (bf16 values), so the product and the oracle can be
fed the same bytes; each file also holds the RoPE tables it used, so a host whose ``torch.cos``
rounds differently still replays the same arithmetic.
"""

from __future__ import annotations

import json
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REFERENCE = Path("/root/reference")
sys.path.insert(0, str(REPO / "tests"))

from workloads import Mixture, rope_tables  # noqa: E402


def reference_modules():
    pkg = types.ModuleType("litgpt")
    pkg.__path__ = [str(REFERENCE / "litgpt")]
    sys.modules.setdefault("litgpt", pkg)
    from litgpt import alpha_log_kv, beta_log_kv, log_kv_cache, log_kv_pack
    return log_kv_cache, alpha_log_kv, beta_log_kv, log_kv_pack


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> its uint16 bit patterns."""
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


STATE_INT = ("level_p_lo", "level_p_hi", "level_sum_wp", "level_order")
MIRRORS = {"level_count": "_semantic_counts", "alive": "_semantic_alive", "p_hi_c": "_semantic_p_hi_c",
           "level0_phase": "_semantic_level0_phase", "n_total": "_semantic_n_total"}


def record_state(cache, out: dict, step: int) -> None:
    for f in STATE_INT:
        out[f"{f}_{step}"] = getattr(cache, f).numpy().astype(np.int64)
    out[f"pad_mask_{step}"] = cache.pad_mask.numpy().astype(np.uint8)
    for f, mirror in MIRRORS.items():
        out[f"{f}_{step}"] = np.asarray(getattr(cache, mirror), dtype=np.int64)
    out[f"level_k_{step}"] = bits(cache.level_k)
    out[f"level_v_{step}"] = bits(cache.level_v)
    out[f"level_w_{step}"] = cache.level_w.numpy().astype(np.float32)
    out[f"centroid_{step}"] = cache.centroid.float().numpy().copy()
    out[f"n_eff_{step}"] = cache.n_eff.float().numpy().copy()
    out[f"recent_count_{step}"] = np.asarray(cache.recent_count)
    if cache.alpha_exact_tokens:
        out[f"alpha_count_{step}"] = np.asarray(cache.alpha_count)
        out[f"alpha_pos_{step}"] = cache.alpha_pos.numpy().astype(np.int64)
        out[f"alpha_valid_{step}"] = cache.alpha_valid.numpy().astype(np.uint8)
        out[f"alpha_k_raw_{step}"] = bits(cache.alpha_k_raw)
        out[f"alpha_v_{step}"] = bits(cache.alpha_v)
        spans = np.full((cache.batch_size, cache.alpha_exact_tokens, 2), -1, np.int64)
        for b, row in enumerate(cache._alpha_spans):
            for i, (length, closed) in enumerate(row):
                spans[b, i] = (length, int(closed))
        out[f"alpha_spans_{step}"] = spans


def stream(kv, config: dict, blocks: int, block: int, seed: int, with_ends: bool, name: str) -> None:
    batch, groups, dim = config["batch"], config["groups"], config["dim"]
    cos, sin = rope_tables(config["max_seq"], dim)
    cache = kv.LogStructuredKVCache(
        (batch, groups, config["max_seq"], dim), (batch, groups, config["max_seq"], dim), B=config["B"],
        recent_size=config["recent"], device="cpu", dtype=torch.bfloat16, semantic_clusters=True,
        cluster_k_max=config["K"], semantic_s_h=config["s_h"], semantic_flush_granularity=config["flush"],
        semantic_anchor_mode="mid", allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=dim,
        alpha_exact_tokens=config["exact"], alpha_span_max_tokens=config["span"],
        beta_novelty=config["beta"], beta_adaptive_merge=config["beta"])
    mix = Mixture(batch, groups, dim, clusters=config["clusters"], seed=seed, outlier=config["outlier"])
    out = {"config": np.asarray(json.dumps(config)), "blocks": np.asarray(blocks), "block": np.asarray(block),
           "B_prime": np.asarray(cache.B_prime), "levels": np.asarray(cache.L_alloc),
           "cos": cos.numpy().copy(), "sin": sin.numpy().copy()}
    for i in range(blocks):
        k_raw, v, k = mix.rows(block), mix.rows(block), mix.rows(block)
        pos = torch.arange(i * block, (i + 1) * block).unsqueeze(0).expand(batch, -1).contiguous()
        ends = mix.span_ends(i * block, block, config["span_stride"]) if with_ends else None
        cache.add_recent(k, v, k_raw=k_raw, input_pos=pos, span_ends=ends)
        out[f"k_raw_{i}"], out[f"v_{i}"], out[f"k_{i}"] = bits(k_raw), bits(v), bits(k)
        out[f"pos_{i}"] = pos.numpy().copy()
        if with_ends:
            out[f"ends_{i}"] = np.asarray(ends, dtype=np.uint8)
        record_state(cache, out, i)
    np.savez_compressed(HERE / name, **out)
    print(f"{name}: {blocks} blocks, B'={cache.B_prime}, L={cache.L_alloc}, "
          f"live ladder slots {int((cache.level_w > 0).sum())}")


def choose_cases(alpha, n_cases=300, seed=5) -> None:
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n_cases):
        rows, max_span = int(rng.integers(1, 4)), int(rng.integers(1, 9))
        spans, positions, pos = [], [], 0
        for _r in range(rows):
            row_spans, row_pos = [], []
            for _s in range(int(rng.integers(0, 5))):
                n = int(rng.integers(1, max_span + 1))
                row_spans.append((n, True))
                row_pos.extend(range(pos, pos + n))
                pos += n + int(rng.integers(0, 3))
            if rng.random() < 0.6:
                n = int(rng.integers(1, max_span + 1))
                row_spans.append((n, False))
                row_pos.extend(range(pos, pos + n))
                pos += n
            spans.append(row_spans)
            positions.append(row_pos)
        width = max((len(p) for p in positions), default=0)
        n = int(rng.integers(0, 60))
        new_pos = [list(range(pos + (1 if rng.random() < 0.3 else 0), pos + n + 1))[:n] for _ in range(rows)]
        ends = [(rng.random(n) < 0.15).tolist() for _ in range(rows)]
        cut = alpha.cut_spans(spans, positions, new_pos, ends, width, max_span)
        if cut is None:
            continue
        n_cand = sum(len(row) for row in cut.length_rows)
        scores = rng.random(n_cand).astype(np.float32)
        scores[rng.random(n_cand) < 0.25] = 0.5           # ties
        budget = int(rng.integers(1, 4 * max_span + 2))
        sel = alpha.choose_spans(cut, scores.tolist(), budget)
        cases.append({"spans": spans, "positions": positions, "new_positions": new_pos, "ends": ends,
                      "old_width": width, "max_span": max_span, "scores": scores.tolist(), "budget": budget,
                      "keep": sel.keep, "archive": sel.archive, "out_spans": [[list(s) for s in r] for r in sel.spans],
                      "out_positions": sel.positions})
    (HERE / "choose_spans.json").write_text(json.dumps(cases))
    print(f"choose_spans.json: {len(cases)} cases")


def select_cuts_cases(beta, seed=83) -> None:
    g = torch.Generator().manual_seed(seed)
    lengths = [4] * 40 + [2, 6, 10, 0, 8, 2]
    n = sum(lengths)
    k = torch.randn(n, 24, generator=g)
    v = torch.randn(n, 16, generator=g) * 3
    w = torch.randint(1, 12, (n,), generator=g).float()
    # Near ties: groups of four identical rows cost only the rounding of their side means under every cut.
    k[:16] = k[0]
    v[:16] = v[0]
    block = (k, v, w, None, None, None, None, None) + (torch.zeros(n, dtype=torch.int64),) * 4 + \
        (torch.zeros(n, dtype=torch.bool),)
    layout = beta.make_layout(lengths, "cpu")
    cuts = beta.select_cuts(block, layout)
    np.savez_compressed(HERE / "select_cuts.npz", k=k.numpy().copy(), v=v.numpy().copy(), w=w.numpy().copy(),
                        lengths=np.asarray(lengths), layout=layout.numpy().copy(), cuts=cuts.numpy().copy())
    print(f"select_cuts.npz: {len(layout)} groups, cuts {np.bincount(cuts.numpy(), minlength=4)[1:].tolist()}")


def pack_case(kv, pack) -> None:
    batch, groups, dim, max_seq = 1, 2, 32, 1024
    cos, sin = rope_tables(max_seq, dim, dtype=torch.bfloat16)
    cache = kv.LogStructuredKVCache(
        (batch, groups, max_seq, dim), (batch, groups, max_seq, dim), B=8, recent_size=32, device="cpu",
        dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=4, semantic_s_h=16.0,
        semantic_flush_granularity=32, semantic_anchor_mode="mid", allocate_second_order=False, cos_cache=cos,
        sin_cache=sin, rope_n_elem=dim, alpha_exact_tokens=16, alpha_span_max_tokens=4)
    mix = Mixture(batch, groups, dim, clusters=4, seed=61)
    out = {"cos": bits(cos), "sin": bits(sin)}
    for i in range(8):
        k_raw, v, k = mix.rows(24), mix.rows(24), mix.rows(24)
        pos = torch.arange(i * 24, (i + 1) * 24).unsqueeze(0)
        ends = mix.span_ends(i * 24, 24, 5)
        cache.add_recent(k, v, k_raw=k_raw, input_pos=pos, span_ends=ends)
        out[f"k_raw_{i}"], out[f"v_{i}"], out[f"k_{i}"], out[f"pos_{i}"] = bits(k_raw), bits(v), bits(k), pos.numpy()
        out[f"ends_{i}"] = np.asarray(ends, dtype=np.uint8)
    cur_k, cur_v = mix.rows(3), mix.rows(3)
    plan = cache._semantic_attention_plan()
    ka, va = pack.pack_mid_kv(cache, plan, cur_k, cur_v, 40, backend="torch")
    out.update(cur_k=bits(cur_k), cur_v=bits(cur_v), ka=bits(ka), va=bits(va), blocks=np.asarray(8),
               block=np.asarray(24), valid=plan[3].numpy().astype(np.uint8))
    np.savez_compressed(HERE / "pack_torch.npz", **out)
    print(f"pack_torch.npz: packed rows {ka.shape[2]}, pooled width {plan[0].shape[-1]}")


def main():
    kv, alpha, beta, pack = reference_modules()
    torch.manual_seed(0)
    stream(kv, dict(batch=2, groups=2, dim=32, max_seq=1024, K=4, B=8, recent=32, flush=32, exact=16, span=4,
                    beta=True, s_h=16.0, clusters=4, outlier=0.1, span_stride=5),
           blocks=12, block=16, seed=11, with_ends=True, name="flush_alpha_beta.npz")
    stream(kv, dict(batch=1, groups=2, dim=32, max_seq=1024, K=4, B=8, recent=32, flush=32, exact=0, span=4,
                    beta=False, s_h=4.0, clusters=6, outlier=0.2, span_stride=5),
           blocks=8, block=32, seed=13, with_ends=False, name="flush_attach_seeded.npz")
    choose_cases(alpha)
    select_cuts_cases(beta)
    pack_case(kv, pack)


if __name__ == "__main__":
    main()
