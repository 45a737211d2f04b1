"""Benchmark of the SemanticLogKV flush path and its decode readout on one MI355X.

Flush (the headline): a step is one flush of 2048 rows into every layer cache
of a 28-layer Qwen3-1.7B-shaped KV stack (8 KV groups x 128, bf16, batch 1,
K=12, B=128 with a 256-token Alpha exact pool and 64-token span cap, so
B'=125 and L=7; Beta novelty scoring and the 4->2 split on): Alpha span
scoring and choice, exact-pool partition, attach route of the archived rows,
per-ladder commit (merges, carries, centers), then the mid-anchor plan and the
pack of the new packed prefix that the next attention reads. Rows are seeded
synthetic Gaussian-mixture keys/values already resident in HBM; span ends are
seeded natural boundaries. The caches first take two untimed flushes; the
steps continue the same 32K-token stream.

Decode: one attention layer over a compressed 32K-token cache, batch 8,
Qwen3-1.7B GQA (16 query / 8 KV heads x 128): recent window 2048, exact pool
256, 12 clusters per lane with the ladder occupancy of 30,464 archived tokens,
masses ~ U(1, 64). A step attends one new token per sequence with the packed
prefix reused, as in the reference's decode loop.

Streaming prefill: 32,768 tokens in 2048-token blocks through 28 layer caches
with per-layer calls: the chunk attention of each block (matrix-core kernel)
and the flush it triggers; ms per block, the attention's TFLOP/s, and the
slots per cluster after each block (the O(log N) growth).

Unified-route control: the Ward / radius route at batch 4 x 8 KV groups with
4096-row flushes over a 131,072-token drifting stream (one layer), reported
beside the headline as flushed tokens/s and ms per flush.

Prints one JSON line: flushed tokens/s over the timed steps, the roofline of
the dominant stage (the ladder commit: its prepare, per-level carries and
finish launches) from HIP events on its stream over the timed region, decode ms/token with its own roofline, and the oracle's CPU
throughput on a bounded sample of the flush workload.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METER_EVERY = 7   # layers 0, 7, 14, 21 carry the commit-stage events
# HBM bytes of one stacked commit stage (28 layers) from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE runs scaled by a 1 GiB copy probe (profiles/commit_stage_traffic_28layer_
# stacked_qwen3_1.7b.md); counters cannot be read inside this process, so the figure is
# the profiled one and is re-measured whenever the commit kernels change.
STACKED_COMMIT_TRAFFIC_BYTES = 1582.0e6
G, D, K, B, F, N = 8, 128, 12, 128, 2048, 32768
EXACT, SPAN = 256, 64


def ladder_rows(counts, m, B, L, staged_tokens=True):
    """(entry rows read, entry rows written, staged token rows read) of one Fenwick append.

    Count model of the reference append (litgpt/log_kv_cache.py:1815-1929): fill
    writes; a carry reads its pair rows and writes one carry row (read again at
    the next level); survivors are read and rewritten at the front; cleared
    slots are written; a saturated top level folds pool[0..mr] into slot 0 and
    rewrites slots 1..B-1.
    """
    counts = list(counts)
    rd = wr = tok = 0
    staged_is_tokens = staged_tokens
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


def commit_bytes(counts, alive, p_hi, assign, order, positions, n_rows, B, L, dk, dv):
    """Algorithmic HBM bytes of one commit (all its launches), from the ladder state before it
    and the attach decisions.

    Entry = K and V bf16 + w f32 + p_lo, p_hi, sum_wp, order i64 + pad flag; token row =
    K and V bf16 + position i64. Per ladder with new rows: a dead cluster clears its L*B'
    entries and opens with one row; a delayed-archive ladder (first new position below
    its p_hi) reads its entries and the new rows into staging (written as entries),
    clears every slot and re-appends everything from level 0; otherwise the new rows
    are appended (count model above). Plus the center: new keys read, center read and
    written."""
    import numpy as np

    entry = 2 * (dk + dv) + 4 + 4 * 8 + 1
    token = 2 * (dk + dv) + 8
    n_batch, groups, K = alive.shape
    total = 0
    for b in range(n_batch):
        n = int(n_rows[b])
        rows_pos = positions[b][order[b][:n]]
        for g in range(groups):
            a = assign[b, g, :n]
            for c in range(K):
                sel = np.nonzero(a == c)[0]
                m = len(sel)
                if m == 0:
                    continue
                cnt = [int(x) for x in counts[b, g, c]]
                pos = rows_pos[sel]
                nn = m
                if not alive[b, g, c]:
                    total += L * B * entry + token + entry
                    cnt = [1] + [0] * (L - 1)
                    nn = m - 1
                    hi = int(pos[0])
                    first = 1
                else:
                    hi = int(p_hi[b, g, c])
                    first = 0
                total += nn * 2 * dk + 2 * dk * 4
                if nn == 0:
                    continue
                if int(pos[first]) < hi:
                    n_exist = sum(cnt)
                    staged = n_exist + nn
                    total += n_exist * entry + nn * token + staged * entry + L * B * entry
                    rd, wr, tok = ladder_rows([0] * L, staged, B, L, staged_tokens=False)
                else:
                    rd, wr, tok = ladder_rows(cnt, nn, B, L)
                total += (rd + wr) * entry + tok * token
    return total


def progress(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def span_ends_for(flush, batch=1):
    """Natural span boundaries of the stream's flush ``flush`` (same for every layer): row
    ``p`` of batch row ``b`` ends a span when ``(p + 7*b) % 32 == 0``, the rule of the
    reference's benchmark harness (unused/benchmark_log_kv_unified.py:36-40)."""
    return [[(p + 7 * b) % 32 == 0 for p in range(flush * F, (flush + 1) * F)] for b in range(batch)]


def cpu_baseline(seconds: float):
    """Oracle (numpy restatement) of the same flush for one layer on the host: Alpha/Beta, route,
    commit and the pack of the new prefix."""
    import numpy as np
    import torch

    from logkv_amd.workloads import Mixture, rope_tables
    from oracle import OracleCache

    torch.set_num_threads(1)
    cos, sin = (t.numpy() for t in rope_tables(N, D))
    mix = Mixture(1, G, D, clusters=K, seed=1)
    rows = lambda: mix.rows(F).float().numpy()  # noqa: E731
    n, t, streams = 0, 0.0, 0
    while t < seconds:
        # One 32K-token stream per cache: two untimed warm-up flushes, then flushes 3..16.
        ora = OracleCache(1, G, N, D, D, B=B, recent_size=F, K=K, s_h=64.0, flush=F, exact_tokens=EXACT,
                          span_max=SPAN, beta_novelty=True, beta_adaptive=True, cos=cos, sin=sin)
        streams += 1
        for j in range(16):
            k, v = rows(), rows()
            pos = np.arange(j * F, (j + 1) * F)[None]
            t0 = time.perf_counter()
            ora.flush_rows(k, v, pos, span_ends_for(j))
            ora.pack(None, None)
            if j >= 2:
                t += time.perf_counter() - t0
                n += 1
            if t >= seconds:
                break
    return {"value": F * n / t, "unit": "flushed tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle (numpy) Alpha/Beta + route + commit + pack of {n} flushes (flushes 3..16 of "
                      f"{streams} 32K-token streams) of one layer, batch 1, 8 groups x 128, K=12, B=128, "
                      f"exact pool 256, {F} rows each, {t:.1f} s, 1 thread"}


class CommitMeter:
    """Wraps a cache's route+commit so that the commit's launches are bracketed by HIP
    events on their stream, with the ladder state they start from copied aside on the
    device and the attach decisions kept (no host sync); algorithmic bytes are computed
    from those copies after the timed region."""

    def __init__(self, cache, torch):
        self.cache, self.torch = cache, torch
        self.records = []

    def __call__(self, k_raw, v, positions, counts=None, assign_out=None, order_out=None, record=False):
        from logkv_amd._lib import check, lib, ptr, stream_of

        if record:
            raise ValueError("the commit meter does not record op-logs")

        cache, torch = self.cache, self.torch
        dev = k_raw.device
        snap = (cache.level_count.clone(), cache.alive.clone(), cache.p_hi_c.clone())
        assign = torch.empty(cache.batch_size, cache.n_groups, k_raw.size(2), dtype=torch.int8, device=dev)
        order = torch.empty(cache.batch_size, k_raw.size(2), dtype=torch.int32, device=dev)
        view = cache._ladder_view()
        rows = cache._rows_view(k_raw, v, positions, counts)
        ws = cache._workspace_for(view, rows.tokens)
        sp = stream_of(dev)
        stream = torch.cuda.current_stream(dev)
        check(lib().logkv_attach_assign(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws), ws.numel(),
                                        ptr(assign), ptr(order), sp), "attach")
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(stream)
        check(lib().logkv_commit_only(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws), ws.numel(),
                                      ptr(assign), ptr(order), sp), "commit")
        ev[1].record(stream)
        n_rows = counts if counts is not None else torch.full((cache.batch_size,), k_raw.size(2), device=dev)
        self.records.append((snap, assign, order, positions, n_rows, ev))

    def results(self, B_, L_):
        out = []
        for (counts, alive, p_hi), assign, order, positions, n_rows, ev in self.records:
            nb = commit_bytes(counts.long().cpu().numpy(), alive.cpu().numpy(), p_hi.cpu().numpy(),
                              assign.cpu().numpy(), order.long().cpu().numpy(), positions.cpu().numpy(),
                              n_rows.cpu().numpy(), B_, L_, D, D)
            out.append((nb, ev[0].elapsed_time(ev[1])))
        return out


def flush_workload(args, torch, np):
    from logkv_amd import LogStructuredKVCache
    from logkv_amd.log_kv_pack import _decode_capacity, _launch_pack, packed_dim, readout_view
    from logkv_amd.workloads import rope_tables

    dev = torch.device("cuda", 0)
    layers = args.layers
    cos, sin = rope_tables(N, D)
    n_flush = 2 + args.warmup + args.steps
    gen = torch.Generator(device=dev).manual_seed(1234)
    centers = torch.randn(layers, G, K, D, generator=gen, device=dev) * 4

    def mixture():
        """[layers, G, F, D]: layer li's rows drawn around its own 12 centers."""
        label = torch.randint(0, K, (layers, G, F), generator=gen, device=dev)
        x = torch.gather(centers, 2, label[..., None].expand(-1, -1, -1, D))
        x = x + torch.randn(layers, G, F, D, generator=gen, device=dev) * 0.5
        far = torch.rand(layers, G, F, generator=gen, device=dev) < 0.1
        return torch.where(far[..., None], torch.randn(x.shape, generator=gen, device=dev) * 12, x).to(torch.bfloat16)

    # Flush j's rows of every layer, stacked [layers, G, F, D]; layer li's rows are
    # the batch-1 slice [li:li + 1]. Positions and boundary flags staged on the device.
    data = [(mixture(), mixture()) for _ in range(n_flush)]
    positions = [torch.arange(j * F, (j + 1) * F, device=dev).unsqueeze(0).expand(layers, -1).contiguous()
                 for j in range(n_flush)]
    ends = [torch.tensor(span_ends_for(j), dtype=torch.uint8, device=dev).expand(layers, -1).contiguous()
            for j in range(n_flush)]
    dim = packed_dim(D, D)
    torch.cuda.synchronize()

    def new_cache(batch):
        return LogStructuredKVCache((batch, G, N, D), (batch, G, N, D), B=B, recent_size=F, device=dev,
                                    dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K,
                                    semantic_s_h=64.0, semantic_flush_granularity=F, semantic_anchor_mode="mid",
                                    allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D,
                                    alpha_exact_tokens=EXACT, alpha_span_max_tokens=SPAN, beta_novelty=True,
                                    beta_adaptive_merge=True)

    def run_pass(stacked, n_streams, meter):
        """Fresh caches, 2 + warmup untimed flushes, then `steps` timed ones, each followed
        by the plan + pack of the next attention's packed prefix [pooled | exact | recent].
        stacked: one cache whose batch rows are the layers, one call per flush step.
        Otherwise one cache per layer, layer li's calls on stream li % n_streams (the
        layers' caches are independent, so their flushes may overlap; each layer's own
        flushes stay in order)."""
        caches = [new_cache(layers)] if stacked else [new_cache(1) for _ in range(layers)]
        workspaces = [tuple(torch.empty(c.batch_size, G, _decode_capacity(c, 2), dim, dtype=torch.bfloat16,
                                        device=dev) for _ in range(2)) for c in caches]
        empty = torch.empty(caches[0].batch_size, G, 0, D, dtype=torch.bfloat16, device=dev)
        streams = [torch.cuda.current_stream(dev)] + [torch.cuda.Stream(dev) for _ in range(n_streams - 1)]

        def flush(j):
            k, v = data[j]
            for li, cache in enumerate(caches):
                rows = slice(None) if stacked else slice(li, li + 1)
                with torch.cuda.stream(streams[li % n_streams]):
                    cache.route_and_flush_batch(k[rows], v[rows], positions[j][rows], span_ends=ends[j][rows])
                    view = readout_view(cache)
                    plan = cache._semantic_attention_plan()
                    _launch_pack(cache, view, plan, empty, empty, dim, *workspaces[li], False, 0)

        label = "stacked layers" if stacked else f"{n_streams} stream(s)"
        for j in range(2 + args.warmup):
            flush(j)
        torch.cuda.synchronize()
        progress(f"flush, {label}: {2 + args.warmup} untimed flushes done")
        # Commit launches of every METER_EVERY-th layer cache are bracketed by events.
        metered = caches[::METER_EVERY] if meter else []
        meters = [CommitMeter(c, torch) for c in metered]
        for c, m in zip(metered, meters):
            c._route_commit = m
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(args.steps):
            flush(2 + args.warmup + s)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        for c in metered:
            del c._route_commit
        progress(f"flush, {label}: {args.steps} timed flushes in {elapsed:.3f} s")
        rec = [r for m in meters for r in m.results(caches[0].B_prime, caches[0].L_alloc)]
        width = int(caches[0]._semantic_attention_plan().width)
        return elapsed, rec, caches[0].B_prime, caches[0].L_alloc, width

    tokens = F * layers * args.steps
    if args.flush_passes == "stacked" and args.mode == "stacked":
        one_stream = per_layer = None
    else:
        one_stream = run_pass(False, 1, args.mode == "layers")
        per_layer = run_pass(False, args.streams, False)[0] if args.streams > 1 else one_stream[0]
    if args.mode == "stacked":
        # The timed value comes from a pass without the commit meter (whose
        # state snapshots are copies inside the loop); a second pass over the
        # same flushes brackets the commit launches for the roofline.
        elapsed, _, B_, L_, width = run_pass(True, 1, False)
        rec = run_pass(True, 1, True)[1]
    else:
        _, rec, B_, L_, width = one_stream
        elapsed = per_layer
    launch_bytes = float(np.mean([b for b, _ in rec]))
    launch_ms = float(np.mean([t for _, t in rec]))
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    how = ("the layers' caches stacked as the batch rows of one cache, one flush call per step"
           if args.mode == "stacked" else f"one cache per layer, the layers' calls over {args.streams} streams")
    return {
        "value": tokens / elapsed,
        "ms_per_step": elapsed / args.steps * 1e3,
        "config": {"workload": f"{layers}-layer flush, Qwen3-1.7B KV shape (8x128 bf16), batch 1, flush {F}, "
                               f"K=12, B=128, Alpha exact pool {EXACT} / span cap {SPAN}, Beta novelty + 4->2 "
                               "split, attach route, mid-anchor plan + pack",
                   "layers": layers, "flush": F, "batch": 1, "kv_groups": G, "head_dim": D, "clusters": K,
                   "slots_per_level": B_, "levels": L_, "exact_tokens": EXACT,
                   "span_cap": SPAN, "stream_flushes": f"{3 + args.warmup}..{2 + args.warmup + args.steps}",
                   "pooled_width_after_last_flush": width, "mode": how,
                   **({} if one_stream is None else {
                       "per_layer_calls_one_stream_tokens_per_s": tokens / one_stream[0],
                       "per_layer_calls_one_stream_ms_per_layer_flush": one_stream[0] / args.steps / layers * 1e3,
                       f"per_layer_calls_{args.streams}_streams_tokens_per_s": tokens / per_layer})},
        "roofline": {"kernel": "commit stage: bucket_kernel + commit_kernel + units_kernel + carries_kernel per "
                               "level + finish_kernel" + (" (one launch sequence for all layers)" if args.mode == "stacked"
                                                  else " (one-stream pass)"),
                     "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": STACKED_COMMIT_TRAFFIC_BYTES if args.mode == "stacked" else None,
                     "algorithmic_bytes_per_launch": launch_bytes, "avg_launch_ms": launch_ms,
                     "launches": len(rec)},
    }


def decode_workload(args, torch, np):
    from logkv_amd import LogStructuredKVCache
    from logkv_amd.log_kv_pack import _launch_pack, packed_attention, packed_dim, readout_view
    from logkv_amd.workloads import fill_readout_state, rope_tables

    dev = torch.device("cuda", 0)
    Bt, HQ = 8, 16
    cos, sin = rope_tables(N, D)
    cache = LogStructuredKVCache((Bt, G, N, D), (Bt, G, N, D), B=B, recent_size=F, device=dev,
                                 dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=64.0,
                                 semantic_flush_granularity=F, semantic_anchor_mode="mid",
                                 allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D,
                                 alpha_exact_tokens=EXACT, alpha_span_max_tokens=SPAN, beta_novelty=True,
                                 beta_adaptive_merge=True)
    archived = N - F - EXACT
    fill_readout_state(cache, seed=21, recent=F, archived=archived)
    steps, warm = args.decode_steps, 8
    gen = torch.Generator(device=dev).manual_seed(77)
    qs = torch.randn(steps + warm, Bt, HQ, 1, D, generator=gen, device=dev).to(torch.bfloat16)
    ks = torch.randn(steps + warm, Bt, G, 1, D, generator=gen, device=dev).to(torch.bfloat16)
    vs = torch.randn(steps + warm, Bt, G, 1, D, generator=gen, device=dev).to(torch.bfloat16)
    dim = packed_dim(D, D)
    scale = D ** -0.5
    view = readout_view(cache)
    plan = cache._semantic_attention_plan()
    cap = cache.K_max * cache.L_alloc * cache.B_prime + EXACT + cache.recent_capacity + 2
    ka = torch.empty(Bt, G, cap, dim, dtype=torch.bfloat16, device=dev)
    va = torch.empty_like(ka)
    # Packed prefix once (the first decode step after a flush), then one new row per step.
    _launch_pack(cache, view, plan, ks[0], vs[0], dim, ka, va, False, 0)
    recent = cache.recent_count
    tail = recent + 1
    stream = torch.cuda.current_stream(dev)
    workspace = None
    events = []

    def step(i, timed):
        nonlocal workspace
        _launch_pack(cache, view, plan, ks[i], vs[i], dim, ka, va, True, recent)
        if timed:
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record(stream)
        _, workspace = packed_attention(qs[i], ka, va, plan, tail, scale, 1, D, G, workspace, cache.alpha_count_dev)
        if timed:
            ev[1].record(stream)
            events.append(ev)

    for i in range(warm):
        step(i, False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(warm + i, True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    progress(f"decode: {steps} steps in {elapsed:.3f} s")
    step_event_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in events]))
    # Launch durations apart from the host: the per-step events above also hold the
    # host's launch gaps whenever Python issues slower than the device runs (a serving
    # loop captures its step instead). One step (pack of the new row, then the
    # attention) and its attention alone are captured in HIP graphs from static
    # inputs, checked bit for bit against the eager calls, and replayed back to back.
    i_last = warm + steps - 1
    q_s, k_s, v_s = qs[i_last].clone(), ks[i_last].clone(), vs[i_last].clone()

    def full_step():
        _launch_pack(cache, view, plan, k_s, v_s, dim, ka, va, True, recent)
        return packed_attention(q_s, ka, va, plan, tail, scale, 1, D, G, workspace, cache.alpha_count_dev)[0]

    def attention_only():
        return packed_attention(q_s, ka, va, plan, tail, scale, 1, D, G, workspace, cache.alpha_count_dev)[0]

    def replayed_ms(fn, reps=64):
        eager = fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = fn()
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(out, eager):
            raise RuntimeError("graph replay of the decode step differs from the eager call")
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(stream)
        for _ in range(reps):
            graph.replay()
        ev[1].record(stream)
        torch.cuda.synchronize()
        if not torch.equal(out, eager):
            raise RuntimeError("graph replay of the decode step differs from the eager call")
        return ev[0].elapsed_time(ev[1]) / reps

    step_ms = replayed_ms(full_step)
    attn_ms = replayed_ms(attention_only)
    reps = 64
    width = plan.width
    rows = width + cache.alpha_count + tail
    lanes = Bt * G
    # Algorithmic bytes: every packed K and V row of every lane once, queries and outputs.
    attn_bytes = lanes * rows * dim * 2 * 2 + Bt * HQ * D * 2 * 2
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    eager_ms = elapsed / steps * 1e3
    return {
        "workload": "decode attention, one layer, batch 8, Qwen3-1.7B GQA (16 q / 8 KV heads x 128, bf16), "
                    f"32K-token cache: recent {F}, exact pool {EXACT}, 12 clusters holding {archived} archived "
                    "tokens per lane, masses ~ U(1,64); packed prefix reused, one new row per step; ms_per_token "
                    "= one step (pack of the new row + attention) replayed from a HIP graph, ms_per_token_eager = "
                    "the same steps launched from Python one by one",
        "ms_per_token": step_ms, "ms_per_token_28_layers": 28 * step_ms, "ms_per_token_eager": eager_ms,
        "steps": steps,
        "packed_rows_per_lane": rows, "pooled_width": width,
        "roofline": {"kernel": "stream_kernel + combine_kernel", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "algorithmic_bytes_per_launch": attn_bytes, "avg_launch_ms": attn_ms,
                     "timing": f"{reps} back-to-back replays of one step's attention launches (HIP graph)",
                     "avg_step_event_ms": step_event_ms},
    }


def prefill_workload(args, torch, np):
    """Streaming prefill of a 32,768-token sequence through 28 Qwen3-1.7B-shaped layer caches, one call per layer
    as a model makes them: per 2048-token block and layer, the chunk attention of the block's 16 query heads over
    [compressed cache | block] (causal within the block) and add_recent, which flushes 2048 rows into the ladders
    once the recent window is full. Queries, keys and values are seeded random bf16 (the model's projections are
    not on this path)."""
    from logkv_amd import LogStructuredKVCache, log_kv_chunk_attention
    from logkv_amd.workloads import Mixture, rope_tables

    dev = torch.device("cuda", 0)
    layers, HQ, blocks = args.layers, 16, N // F
    cos, sin = rope_tables(N, D)
    caches = [LogStructuredKVCache((1, G, N, D), (1, G, N, D), B=B, recent_size=F, device=dev, dtype=torch.bfloat16,
                                   semantic_clusters=True, cluster_k_max=K, semantic_s_h=64.0,
                                   semantic_flush_granularity=F, semantic_anchor_mode="mid",
                                   allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D,
                                   alpha_exact_tokens=EXACT, alpha_span_max_tokens=SPAN, beta_novelty=True,
                                   beta_adaptive_merge=True) for _ in range(layers)]
    gen = torch.Generator(device=dev).manual_seed(41)
    mix = Mixture(1, G, D, clusters=K, seed=43)
    q = torch.randn(1, HQ, F, D, generator=gen, device=dev).to(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    scale = D ** -0.5
    block_ms, attn_ms, slots, attn_flops = [], [], [], []
    for blk in range(blocks):
        k_raw, v = mix.rows(F).to(dev), mix.rows(F).to(dev)
        pos = torch.arange(blk * F, (blk + 1) * F, device=dev).unsqueeze(0)
        ends = torch.tensor([[(p + 7) % 32 == 0 for p in range(blk * F, (blk + 1) * F)]], dtype=torch.uint8,
                            device=dev)
        # Rows the block's attention reads in layer 0 (every layer holds the same counts):
        # the pooled width (largest lane), the exact pool, the recent window and the block.
        c0 = caches[0]
        rows = int(c0.level_count.long().sum((-1, -2)).max()) + c0.alpha_count + c0.recent_count + F
        attn_flops.append(layers * 4 * F * rows * D * HQ)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        events = []
        for cache in caches:
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record(stream)
            log_kv_chunk_attention(cache, q, k_raw, v, scale, second_order_scale=0.0)
            ev[1].record(stream)
            events.append(ev)
            cache.add_recent(k_raw, v, k_raw=k_raw, input_pos=pos, span_ends=ends)
        torch.cuda.synchronize()
        block_ms.append((time.perf_counter() - t0) * 1e3)
        attn_ms.append(float(np.sum([e[0].elapsed_time(e[1]) for e in events])))
        slots.append(float(c0.level_count.float().sum() / (G * K)))
    attn_s = float(np.sum(attn_ms)) * 1e-3
    tflops = float(np.sum(attn_flops)) / attn_s / 1e12
    progress(f"prefill: {blocks} blocks, {np.mean(block_ms):.1f} ms per block over {layers} layers")
    return {
        "workload": f"streaming prefill of {N} tokens through {layers} Qwen3-1.7B-shaped layer caches (16 q / 8 KV "
                    f"heads x 128, bf16), batch 1, {F}-token blocks, recent {F}, K={K}, B={B}, Alpha {EXACT}/{SPAN}, "
                    "Beta, mid anchor; per block and layer: chunk attention (matrix cores) + add_recent (flush)",
        "ms_per_block": float(np.mean(block_ms)), "ms_per_block_by_block": [round(x, 2) for x in block_ms],
        "attention_ms_per_block": float(np.mean(attn_ms)),
        "attention_roofline": {"kernel": "chunk_kernel", "bound": "mfma", "achieved": tflops, "peak": 2500.0,
                               "unit": "TFLOP/s", "frac": tflops / 2500.0,
                               "flops": "4 * T_q * S * D per query head (S = packed rows)"},
        "flushes": sum(1 for x in slots if x > 0),
        "slots_per_cluster_after_each_block": [round(x, 1) for x in slots],
    }


def unified_workload(args, torch, np):
    """The unified (Ward / radius) route control: batch 4 x 8 KV groups, recent = flush = 4096 rows, a
    131,072-token stream (31 flush events) of a 12-Gaussian mixture that drifts every 16K tokens."""
    from logkv_amd import LogStructuredKVCache
    from logkv_amd.workloads import Mixture, rope_tables

    dev = torch.device("cuda", 0)
    Bt, T, stream_tokens, s_h = 4, 4096, 131072, 64.0
    cos, sin = rope_tables(stream_tokens, D)
    cache = LogStructuredKVCache((Bt, G, stream_tokens, D), (Bt, G, stream_tokens, D), B=B, recent_size=T,
                                 device=dev, dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K,
                                 semantic_s_h=s_h, semantic_flush_granularity=T, semantic_anchor_mode="mid",
                                 allocate_second_order=False, semantic_unified_route=True, cos_cache=cos, sin_cache=sin,
                                 rope_n_elem=D)
    # Each flush draws T key rows and T value rows, so the centers move every 16K tokens.
    mix = Mixture(Bt, G, D, clusters=12, seed=31, drift_every=2 * 16384)
    flushes = stream_tokens // T - 1
    warm = 2
    stream = torch.cuda.current_stream(dev)
    times = []
    t_all = 0.0
    for i in range(flushes):
        k, v = mix.rows(T).to(dev), mix.rows(T).to(dev)
        pos = torch.arange(i * T, (i + 1) * T, device=dev).unsqueeze(0).expand(Bt, -1).contiguous()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev[0].record(stream)
        cache.route_and_flush_batch(k, v, pos)
        ev[1].record(stream)
        torch.cuda.synchronize()
        if i >= warm:
            t_all += time.perf_counter() - t0
            times.append(ev[0].elapsed_time(ev[1]))
    timed = flushes - warm
    ms = t_all / timed * 1e3
    progress(f"unified route: {timed} timed flushes, {ms:.1f} ms per flush")
    return {
        "workload": "unified Ward / radius route control, Qwen3-1.7B KV shape (8 x 128 bf16), batch 4, "
                    f"recent = flush = {T}, {stream_tokens}-token stream ({flushes} flush events), 12-Gaussian "
                    f"mixture drifting every 16K tokens, K={K}, B={B}, L={cache.L_alloc}, s_h={s_h}",
        "flushed_tokens_per_s": Bt * T / (ms * 1e-3), "ms_per_flush": ms,
        "device_ms_per_flush": float(np.mean(times)), "timed_flushes": timed, "warmup_flushes": warm,
        "live_clusters_per_lane": float(cache.alive.float().sum(-1).mean()),
        "note": "one layer; the reducer runs one workgroup per lane, all rounds of a stage in one launch",
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--mode", choices=("stacked", "layers"), default="stacked",
                    help="stacked: the layers' caches as batch rows of one cache (one call per flush step); "
                         "layers: one cache per layer")
    ap.add_argument("--streams", type=int, default=4,
                    help="HIP streams the per-layer calls are spread over (a one-stream pass always runs too)")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-unified", action="store_true", help="skip the unified-route control measurement")
    ap.add_argument("--no-prefill", action="store_true", help="skip the streaming-prefill measurement")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first copy this many MiB device to device (a plain copy of known size that scales "
                         "the FETCH_SIZE / WRITE_SIZE counters of a profiling run)")
    ap.add_argument("--flush-passes", choices=("all", "stacked"), default="all",
                    help="stacked: run only the stacked pass (profiling runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box here has one MI355X, --gpus {args.gpus} is not run",
              file=sys.stderr)
        sys.exit(2)
    if args.streams < 1:
        print("--streams must be at least 1", file=sys.stderr)
        sys.exit(2)
    if 2 + args.warmup + args.steps > 16:
        print("warmup + steps must fit the 32K-token stream: at most 14 flushes after the two warm-up flushes",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    torch.cuda.set_device(0)
    if args.copy_probe_mib:
        src = torch.ones(args.copy_probe_mib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        progress(f"copy probe: {args.copy_probe_mib} MiB copied")
        del src, dst
    fl = flush_workload(args, torch, np)
    result = {
        "metric": "flushed tokens/s (route+merge+pack) & decode ms/token at 32K ctx, 1 GPU",
        "value": fl["value"],
        "unit": "flushed tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": fl["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 storage, f32 math",
        "data": "synthetic seeded Gaussian mixture (12 centers N(0,1)*4, noise 0.5, 10% outliers N(0,1)*12), "
                "span ends where (p + 7b) % 32 == 0",
        "config": fl["config"],
        "roofline": fl["roofline"],
    }
    if not args.no_decode:
        result["decode"] = decode_workload(args, torch, np)
        result["decode_ms_per_token"] = result["decode"]["ms_per_token"]
    if not args.no_prefill and args.flush_passes == "all":
        result["prefill"] = prefill_workload(args, torch, np)
    if not args.no_unified and args.flush_passes == "all":
        result["unified"] = unified_workload(args, torch, np)
    if not args.no_cpu_baseline:
        progress("cpu baseline: oracle flushes on the host")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
