"""Benchmark of the SemanticLogKV flush path on one MI355X.

A step is one flush of 2048 rows into every layer cache of a 28-layer
Qwen3-1.7B-shaped KV stack (8 KV groups x 128, bf16, batch 1, K=12, B=128):
attach route + per-ladder commit (merges, carries, centers). Rows are seeded
synthetic Gaussian-mixture keys/values already resident in HBM. The caches are
first warmed with two flushes; steps then continue the same 32K-token stream.

Prints one JSON line: flushed tokens/s over the timed steps, the roofline of
the dominant kernel (the per-ladder commit) from HIP events on its stream, and
the oracle's CPU throughput on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def ladder_rows(counts, m, B, L):
    """(entry rows read, entry rows written, staged token rows read) of one Fenwick append.

    Count model of the reference append (litgpt/log_kv_cache.py:1815-1929): fill
    writes; a carry reads its pair rows and writes one carry row (read again at
    the next level); survivors are read and rewritten at the front; cleared
    slots are written; a saturated top level folds pool[0..mr] into slot 0 and
    rewrites slots 1..B-1.
    """
    counts = list(counts)
    rd = wr = tok = 0
    staged_is_tokens = True
    for ell in range(L):
        if m == 0:
            break
        take = min(B - counts[ell], m)
        wr += take
        if staged_is_tokens:
            tok += take
        else:
            rd += take
        mr = m - take
        if mr == 0:
            counts[ell] += take
            break
        if ell == L - 1:
            pool_staged = mr
            rd += B + pool_staged - 1   # fold reads pool[0..mr], tail reads the rest
            wr += B
            counts[ell] = B
            break
        n_carry = (mr + 1) // 2
        n_pair = 2 * n_carry
        stored_pairs = min(B, n_pair)
        staged_pairs = n_pair - stored_pairs
        rd += stored_pairs
        if staged_is_tokens:
            tok += staged_pairs
        else:
            rd += staged_pairs
        wr += n_carry
        n_surv = B + mr - n_pair
        stored_surv = max(0, B - n_pair)
        staged_surv = n_surv - stored_surv
        rd += stored_surv
        wr += stored_surv
        if staged_is_tokens:
            tok += staged_surv
        else:
            rd += staged_surv
        wr += staged_surv + (B - n_surv)
        counts[ell] = n_surv
        m = n_carry
        staged_is_tokens = False
    return rd, wr, tok


def commit_bytes(before_counts, before_alive, m_rows, B, L, dk, dv):
    """Algorithmic HBM bytes of one commit launch, from the state before it and rows per ladder."""
    import numpy as np

    entry = 2 * (dk + dv) + 4 + 4 * 8 + 1
    token = 2 * (dk + dv) + 8
    total = 0
    for idx in map(tuple, np.argwhere(m_rows > 0)):
        m = int(m_rows[idx])
        counts = before_counts[idx]
        if not before_alive[idx]:
            total += L * B * entry            # clear of the newly opened cluster
            counts = [0] * L
        rd, wr, tok = ladder_rows(counts, m, B, L)
        total += (rd + wr) * entry + tok * token + 2 * dk * 4   # + center read and write
    return total


def cpu_baseline(seconds: float):
    """Oracle (numpy restatement) flushes of one layer of the same workload on the host."""
    import numpy as np
    import torch

    from logkv_amd.workloads import Mixture
    from oracle import OracleCache

    torch.set_num_threads(1)
    mix = Mixture(1, 8, 128, clusters=12, seed=1)
    rows = lambda: mix.rows(2048).float().numpy()  # noqa: E731
    n, t, streams = 0, 0.0, 0
    while t < seconds:
        # One 32K-token stream per cache: two untimed warm-up flushes, then flushes 3..16.
        ora = OracleCache(1, 8, 32768, 128, 128, B=128, recent_size=2048, K=12, s_h=64.0, flush=2048)
        streams += 1
        for j in range(16):
            k, v = rows(), rows()
            pos = np.arange(j * 2048, (j + 1) * 2048)[None]
            t0 = time.perf_counter()
            ora.flush_rows(k, v, pos)
            if j >= 2:
                t += time.perf_counter() - t0
                n += 1
            if t >= seconds:
                break
    return {"value": 2048 * n / t, "unit": "flushed tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle (numpy) route+commit of {n} flushes (flushes 3..16 of {streams} 32K-token streams) "
                      f"of one layer, batch 1, 8 groups x 128, K=12, B=128, 2048 rows each, {t:.1f} s, 1 thread"}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box here has one MI355X, --gpus {args.gpus} is not run",
              file=sys.stderr)
        sys.exit(2)
    if 2 + args.warmup + args.steps > 16:
        print("warmup + steps must fit the 32K-token stream: at most 14 flushes after the two warm-up flushes",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from logkv_amd import LogStructuredKVCache
    from logkv_amd._lib import check, lib, ptr, stream_of
    from logkv_amd.workloads import rope_tables

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    G, D, K, B, F, N = 8, 128, 12, 128, 2048, 32768
    layers = args.layers
    cos, sin = rope_tables(N, D)
    caches = [LogStructuredKVCache((1, G, N, D), (1, G, N, D), B=B, recent_size=F, device=dev,
                                   dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=64.0,
                                   semantic_flush_granularity=F, semantic_anchor_mode="mid",
                                   allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D)
              for _ in range(layers)]
    n_flush = 2 + args.warmup + args.steps
    gen = torch.Generator(device=dev).manual_seed(1234)
    centers = torch.randn(layers, G, K, D, generator=gen, device=dev) * 4

    def mixture(layer):
        label = torch.randint(0, K, (1, G, F), generator=gen, device=dev)
        x = torch.gather(centers[layer][None].expand(1, -1, -1, -1), 2, label[..., None].expand(-1, -1, -1, D))
        x = x + torch.randn(1, G, F, D, generator=gen, device=dev) * 0.5
        far = torch.rand(1, G, F, generator=gen, device=dev) < 0.1
        return torch.where(far[..., None], torch.randn(x.shape, generator=gen, device=dev) * 12, x).to(torch.bfloat16)

    data = [[(mixture(li), mixture(li)) for li in range(layers)] for _ in range(n_flush)]
    positions = [torch.arange(j * F, (j + 1) * F, device=dev).unsqueeze(0).contiguous() for j in range(n_flush)]
    torch.cuda.synchronize()

    # Per-layer C views and workspaces, built once (the timed loop only launches).
    prepared = []
    for j in range(n_flush):
        row = []
        for li, cache in enumerate(caches):
            k, v = data[j][li]
            view = cache._ladder_view()
            rows = cache._rows_view(k, v, positions[j])
            ws = cache._workspace_for(view, F)
            row.append((view, rows, ws))
        prepared.append(row)
    L_ = lib()
    stream = torch.cuda.current_stream(dev)
    sp = stream_of(dev)

    def flush(j, events=None):
        for li, cache in enumerate(caches):
            view, rows, ws = prepared[j][li]
            if events is None:
                check(L_.logkv_route_commit(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws),
                                            ws.numel(), None, None, sp), "route_commit")
            else:
                check(L_.logkv_attach_assign(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws),
                                             ws.numel(), None, None, sp), "attach")
                events[li][0].record(stream)
                check(L_.logkv_commit_only(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws),
                                           ws.numel(), None, None, sp), "commit")
                events[li][1].record(stream)

    for j in range(2):
        flush(j)
    torch.cuda.synchronize()

    # Warm-up flushes double as the roofline accounting: per layer, the commit
    # launch is bracketed by HIP events on its stream and its algorithmic bytes
    # come from the count model over the state just before it.
    acc_bytes, acc_ms = [], []
    for j in range(2, 2 + args.warmup):
        for li, cache in enumerate(caches):
            before = (cache.level_count.long().cpu().numpy(), cache.alive.cpu().numpy(),
                      cache.n_total.long().cpu().numpy())
            view, rows, ws = prepared[j][li]
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            check(L_.logkv_attach_assign(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws),
                                         ws.numel(), None, None, sp), "attach")
            ev[0].record(stream)
            check(L_.logkv_commit_only(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws),
                                       ws.numel(), None, None, sp), "commit")
            ev[1].record(stream)
            torch.cuda.synchronize()
            m = cache.n_total.long().cpu().numpy() - before[2]
            acc_bytes.append(commit_bytes(before[0], before[1], m, B, cache.L_alloc, D, D))
            acc_ms.append(ev[0].elapsed_time(ev[1]))
    torch.cuda.synchronize()

    events = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in caches] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        flush(2 + args.warmup + s, events[s])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timed_commit_ms = float(np.mean([events[s][li][0].elapsed_time(events[s][li][1])
                                     for s in range(args.steps) for li in range(layers)]))
    avg_bytes = float(np.mean(acc_bytes)) if acc_bytes else 0.0
    avg_ms = float(np.mean(acc_ms)) if acc_ms else float("nan")
    achieved = float(np.mean([b / (t * 1e-3) / 1e9 for b, t in zip(acc_bytes, acc_ms)])) if acc_bytes else 0.0

    tokens = F * layers * args.steps
    result = {
        "metric": "flushed tokens/s (route+merge+pack) & decode ms/token at 32K ctx, 1 GPU",
        "value": tokens / elapsed,
        "unit": "flushed tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 storage, f32 math",
        "data": "synthetic seeded Gaussian mixture (12 centers N(0,1)*4, noise 0.5, 10% outliers N(0,1)*12)",
        "config": {"workload": f"{layers}-layer flush, Qwen3-1.7B KV shape (8x128 bf16), batch 1, flush 2048, "
                               f"K=12, B=128, attach route; Alpha/Beta off",
                   "layers": layers, "flush": F, "batch": 1, "kv_groups": G, "head_dim": D, "clusters": K,
                   "slots_per_level": caches[0].B_prime, "levels": caches[0].L_alloc,
                   "stream_flushes": f"{3 + args.warmup}..{2 + args.warmup + args.steps}"},
        "roofline": {"kernel": "commit_kernel", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes_per_launch": avg_bytes, "avg_launch_ms": avg_ms,
                     "accounting": f"{len(acc_ms)} commit launches of the warm-up flushes",
                     "timed_avg_launch_ms": timed_commit_ms},
        "decode_ms_per_token": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
