"""Benchmark of the SemanticLogKV flush path and its readout on one MI355X.

Headline (a step): one flush of 2048 rows into every layer cache of a
28-layer Qwen3-1.7B-shaped KV stack (8 KV groups x 128, bf16, batch 1, K=12,
B=128 with a 256-token Alpha exact pool and a 64-token span cap, so B'=125 and
L=7; Beta novelty scoring and the 4->2 split on): Alpha span scoring and
choice, exact-pool partition, attach route of the archived rows, per-ladder
commit (merges, carries, centers), then the mid-anchor plan and the pack of the
new packed prefix the next attention reads. Rows are seeded synthetic
Gaussian-mixture keys / values already resident in HBM, span ends follow the
reference harness's rule. A 32K-token stream holds 16 flushes: its first two
are untimed (they fill empty ladders), flushes 3..16 are steady-state steps.
Any --warmup / --steps is served by chaining fresh 32K-token streams: the
warm-up steps come first, then the timed ones; every stream's own two first
flushes run outside the timed region.

Beside the headline, each in its own guarded leg (a failing leg is recorded in
the line and never loses the headline): the one-layer flush of the CPU
reference configuration on the GPU, decode at 32K context (batch 8, GQA
16/8) through the streaming attention engine, streaming prefill of 32,768
tokens through 28 layer caches (chunk attention on the matrix cores + the
flushes), the unified Ward / radius route control, and the CPU baseline.

Prints one JSON line. ``roofline`` is the whole flush step: algorithmic bytes
of every stage (byte model below) over the step's duration from HIP events
on its stream over the timed region; ``roofline.stages`` splits it into the
Alpha selection + partition, the attach route, the ladder commit and the plan
+ pack, each timed by its own event pairs in a second pass over the same
flushes (the kernels are deterministic, so that pass reproduces the timed
pass's states).

``python bench.py --pmc-summary FETCH_DIR WRITE_DIR`` turns the counter
output of two ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` runs of
``bench.py --profile-flush`` into HBM bytes per step; ``--trace-summary CSV``
gives the kernel time per step of a ``--kernel-trace`` run of it and
``--kernel-counters DIR`` every kernel's mean counters of a ``--pmc`` run.
"""

from __future__ import annotations

import argparse
import ctypes as C
import gc
import json
import math
import os
import platform
import re
import sys
import time
import traceback
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
G, D, K, B, F, N = 8, 128, 12, 128, 2048, 32768
EXACT, SPAN = 256, 64
STREAM_FLUSHES = N // F          # 16 flushes per 32K-token stream
PREP_FLUSHES = 2                 # each stream's first two flushes: untimed
STEADY_FLUSHES = STREAM_FLUSHES - PREP_FLUSHES
MAX_LIVE_STREAMS = 6             # stacked caches alive at once (about 1.4 GB each)
ROPE_TABLE_BYTES = 4             # float32 cos / sin tables


def progress(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------------
# Schedule: warm-up and timed steps over chained 32K-token streams
# ----------------------------------------------------------------------

def flush_schedule(warmup: int, steps: int, max_live: int = MAX_LIVE_STREAMS):
    """Segments of the headline run for any warmup / steps.

    Step w (0-based over warm-up then timed steps) is flush 3 + (w % 14) of
    stream w // 14. A segment is a group of at most ``max_live`` streams whose
    caches are alive together: their two prep flushes, then their warm-up
    steps, then their timed steps (one bracketed region). Returns a list of
    segments ``{"streams": [...], "warm": [(stream, flush)], "timed": [...]}``
    whose timed lists, concatenated, hold exactly ``steps`` flushes."""
    if warmup < 0 or steps < 1:
        raise ValueError("--warmup must be >= 0 and --steps >= 1")
    total = warmup + steps
    n_streams = (total + STEADY_FLUSHES - 1) // STEADY_FLUSHES
    segments = []
    for first in range(0, n_streams, max_live):
        streams = list(range(first, min(n_streams, first + max_live)))
        warm, timed = [], []
        for s in streams:
            for j in range(STEADY_FLUSHES):
                w = s * STEADY_FLUSHES + j
                if w >= total:
                    break
                (warm if w < warmup else timed).append((s, PREP_FLUSHES + j))
        segments.append({"streams": streams, "warm": warm, "timed": timed})
    return segments


def span_ends_for(flush, batch=1):
    """Natural span boundaries of the stream's flush ``flush``: row ``p`` of batch row ``b`` ends a
    span when ``(p + 7*b) % 32 == 0``, the rule of the reference's benchmark harness
    (unused/benchmark_log_kv_unified.py:36-40)."""
    return [[(p + 7 * b) % 32 == 0 for p in range(flush * F, (flush + 1) * F)] for b in range(batch)]


# ----------------------------------------------------------------------
# Byte model (algorithmic HBM bytes)
# ----------------------------------------------------------------------

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
            rd += B + mr - 1   # fold reads pool[0..mr], tail reads the rest
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
    n_batch, groups, K_ = alive.shape
    total = 0
    for b in range(n_batch):
        n = int(n_rows[b])
        rows_pos = positions[b][order[b][:n]]
        for g in range(groups):
            a = assign[b * groups + g, :n] if assign.ndim == 2 else assign[b, g, :n]
            for c in range(K_):
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


def alpha_bytes(p0, keep, archived, T, P, groups, dk, dv, k_max):
    """Algorithmic bytes of the Alpha stage of one batch row: scoring reads the K and V rows of
    every candidate token of [exact pool | flush] (all p0 + T rows) plus positions, flags and the
    live centers; the partition reads each source row once and writes the P-row pool (kept rows,
    zero fill) and the archived rows, with their positions."""
    row = groups * 2 * (dk + dv)
    score = (p0 + T) * row + T * (8 + 1) + p0 * 8 + groups * k_max * (dk * 4 + 1)
    part = (keep + archived) * (row + 8) + P * (row + 8 + 1) + archived * (row + 8)
    return score, part


def route_bytes(archived, groups, dk, k_max):
    """Attach route of one batch row: positions read, every archived key read once per KV group,
    one decision byte written per (group, row), the centers read."""
    return archived * 8 + groups * archived * (2 * dk + 1) + groups * k_max * (dk * 4 + 1 + 8)


def pack_bytes(lane_slots, exact_rows, recent_rows, dk, dv, dim, rope_n):
    """Plan + pack of one batch row's packed prefix [pooled | exact | recent]: pooled slots read
    K, V, w, sum(w*p) and the cos / sin rows at their anchor; exact rows read K, V, position,
    valid flag and their table rows; recent rows read K and V; every lane writes K and V packed
    rows of width ``dim`` for the widest lane's pooled count plus the exact and recent rows."""
    table = 2 * rope_n * ROPE_TABLE_BYTES
    width = max(lane_slots) if lane_slots else 0
    rd = sum(lane_slots) * (2 * (dk + dv) + 4 + 8 + table)
    rd += len(lane_slots) * (exact_rows * (2 * (dk + dv) + 8 + 1 + table) + recent_rows * 2 * (dk + dv))
    wr = len(lane_slots) * (width + exact_rows + recent_rows) * 2 * dim * 2
    return rd + wr


def gbs(nbytes, ms):
    return nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0


# ----------------------------------------------------------------------
# Headline: 28-layer flush
# ----------------------------------------------------------------------

def new_flush_cache(torch, dev, batch, cos, sin, seq=N):
    from logkv_amd import LogStructuredKVCache

    return LogStructuredKVCache((batch, G, seq, D), (batch, G, seq, D), B=B, recent_size=F, device=dev,
                                dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K,
                                semantic_s_h=64.0, semantic_flush_granularity=F, semantic_anchor_mode="mid",
                                allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D,
                                alpha_exact_tokens=EXACT, alpha_span_max_tokens=SPAN, beta_novelty=True,
                                beta_adaptive_merge=True)


class FlushMeter:
    """A metered flush step of one stacked cache: HIP events around each stage's launches on the
    cache's stream and the state the byte model needs, copied aside on the device (no host sync
    inside the loop; bytes are computed afterwards)."""

    def __init__(self, cache, torch):
        self.cache, self.torch = cache, torch
        self.records = []
        self._cur = None

    def _event(self):
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record(self.torch.cuda.current_stream(self.cache.level_k.device))
        return ev

    def begin(self):
        c = self.cache
        self._cur = {"span_len": c.alpha_span_len.clone(), "span_count": c.alpha_span_count.clone()}
        self._cur["ev"] = [self._event()]

    def __call__(self, k_raw, v, positions, counts=None, assign_out=None, order_out=None, record=False):
        """Replaces the cache's route + commit for the metered pass: attach and commit as separate launches."""
        from logkv_amd._lib import check, lib, ptr, stream_of

        cache, torch, cur = self.cache, self.torch, self._cur
        if cur is None:   # an unmetered flush (the stream's prep and warm-up flushes)
            return type(cache)._route_commit(cache, k_raw, v, positions, counts, assign_out, order_out, record)
        cur["ev"].append(self._event())                      # end of the Alpha stage
        dev = k_raw.device
        cur["counts"] = cache.level_count.clone()
        cur["alive"] = cache.alive.clone()
        cur["p_hi"] = cache.p_hi_c.clone()
        cur["archived"] = counts.clone()
        cur["positions"] = positions.clone()
        assign = torch.empty(cache.batch_size * cache.n_groups, k_raw.size(2), dtype=torch.int8, device=dev)
        order = torch.empty(cache.batch_size, k_raw.size(2), dtype=torch.int32, device=dev)
        view = cache._ladder_view()
        rows = cache._rows_view(k_raw, v, positions, counts)
        ws = cache._workspace_for(view, rows.tokens)
        sp = stream_of(dev)
        cur["ev"].append(self._event())
        check(lib().logkv_attach_assign(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws), ws.numel(),
                                        ptr(assign), ptr(order), sp), "attach")
        cur["ev"].append(self._event())
        check(lib().logkv_commit_only(C.byref(view), C.byref(rows), C.byref(cache._params), ptr(ws), ws.numel(),
                                      ptr(assign), ptr(order), sp), "commit")
        cur["ev"].append(self._event())
        cur["assign"], cur["order"] = assign, order

    def before_pack(self):
        self._cur["ev"].append(self._event())

    def end(self):
        c, cur = self.cache, self._cur
        cur["ev"].append(self._event())
        cur["counts_after"] = c.level_count.clone()
        cur["new_span_len"] = c.alpha_span_len.clone()
        cur["new_span_count"] = c.alpha_span_count.clone()
        self.records.append(cur)
        self._cur = None

    def results(self):
        """Per metered step: bytes and milliseconds of each stage."""
        import numpy as np

        c = self.cache
        out = []
        for r in self.records:
            ev = r["ev"]
            ms = {"alpha": ev[0].elapsed_time(ev[1]), "route": ev[2].elapsed_time(ev[3]),
                  "commit": ev[3].elapsed_time(ev[4]), "pack": ev[5].elapsed_time(ev[6])}
            span_len, span_count = r["span_len"].cpu().numpy(), r["span_count"].cpu().numpy()
            new_len, new_count = r["new_span_len"].cpu().numpy(), r["new_span_count"].cpu().numpy()
            archived = r["archived"].cpu().numpy()
            counts_after = r["counts_after"].long().cpu().numpy()
            T = F
            by = {"alpha": 0, "route": 0, "commit": 0, "pack": 0}
            for b in range(c.batch_size):
                p0 = int(span_len[b, :span_count[b]].sum())
                keep = int(new_len[b, :new_count[b]].sum())
                if keep + int(archived[b]) != p0 + T:
                    raise RuntimeError(f"kept {keep} + archived {archived[b]} rows != pool {p0} + flush {T}")
                score, part = alpha_bytes(p0, keep, int(archived[b]), T, EXACT, G, D, D, K)
                by["alpha"] += score + part
                by["route"] += route_bytes(int(archived[b]), G, D, K)
                lanes = counts_after[b].sum(axis=(-1, -2)).tolist()
                by["pack"] += pack_bytes(lanes, keep, 0, D, D, 136, D)
            by["commit"] = commit_bytes(r["counts"].long().cpu().numpy(), r["alive"].cpu().numpy(),
                                        r["p_hi"].cpu().numpy(), r["assign"].cpu().numpy(),
                                        r["order"].long().cpu().numpy(), r["positions"].cpu().numpy(), archived,
                                        c.B_prime, c.L_alloc, D, D)
            out.append((by, ms))
        return out


STEP_TRAFFIC_PROFILE = Path(__file__).resolve().parent / "profiles" / "flush_step_traffic_28layer_stacked_qwen3_1.7b.md"


def profiled_step_traffic():
    """HBM bytes of one headline step as the committed FETCH_SIZE / WRITE_SIZE counter runs of
    ``--profile-flush`` measured them (the profile's "traffic ... MB per step" line), or (None, None)."""
    try:
        text = STEP_TRAFFIC_PROFILE.read_text()
    except OSError:
        return None, None
    m = re.search(r"traffic ([0-9.]+) MB per step", text)
    if not m:
        return None, None
    return float(m.group(1)) * 1e6, f"profiles/{STEP_TRAFFIC_PROFILE.name} (rocprofv3 FETCH_SIZE + WRITE_SIZE runs)"


def flush_workload(args, torch, np):
    from logkv_amd.log_kv_pack import _decode_capacity, _launch_pack, packed_dim, readout_view
    from workloads import rope_tables

    dev = torch.device("cuda", 0)
    layers = args.layers
    cos, sin = rope_tables(N, D)
    gen = torch.Generator(device=dev).manual_seed(1234)
    centers = torch.randn(layers, G, K, D, generator=gen, device=dev) * 4

    def mixture():
        """[layers, G, F, D]: layer li's rows drawn around its own 12 centers."""
        label = torch.randint(0, K, (layers, G, F), generator=gen, device=dev)
        x = torch.gather(centers, 2, label[..., None].expand(-1, -1, -1, D))
        x = x + torch.randn(layers, G, F, D, generator=gen, device=dev) * 0.5
        far = torch.rand(layers, G, F, generator=gen, device=dev) < 0.1
        return torch.where(far[..., None], torch.randn(x.shape, generator=gen, device=dev) * 12, x).to(torch.bfloat16)

    # Flush j of the stream for every layer, stacked [layers, G, F, D]; layer li's rows are the
    # batch-1 slice [li:li + 1]. Every chained stream replays the same rows into fresh caches.
    data = [(mixture(), mixture()) for _ in range(STREAM_FLUSHES)]
    positions = [torch.arange(j * F, (j + 1) * F, device=dev).unsqueeze(0).expand(layers, -1).contiguous()
                 for j in range(STREAM_FLUSHES)]
    ends = [torch.tensor(span_ends_for(j), dtype=torch.uint8, device=dev).expand(layers, -1).contiguous()
            for j in range(STREAM_FLUSHES)]
    dim = packed_dim(D, D)
    torch.cuda.synchronize()
    segments = flush_schedule(args.warmup, args.steps)

    def run_pass(stacked, n_streams, meter=False):
        """The schedule over fresh caches. stacked: one cache per stream whose batch rows are the
        layers (one call per flush step). Otherwise one cache per layer and stream, layer li's calls
        on HIP stream li % n_streams (the layers' caches are independent, so their flushes may
        overlap; each layer's own flushes stay in order)."""
        hip_streams = [torch.cuda.current_stream(dev)] + [torch.cuda.Stream(dev) for _ in range(n_streams - 1)]
        elapsed, step_ms, records, last = 0.0, [], [], None
        empty = torch.empty(layers if stacked else 1, G, 0, D, dtype=torch.bfloat16, device=dev)
        for seg in segments:
            live = {}
            for s in seg["streams"]:
                caches = [new_flush_cache(torch, dev, layers, cos, sin)] if stacked else \
                    [new_flush_cache(torch, dev, 1, cos, sin) for _ in range(layers)]
                packs = [tuple(torch.empty(c.batch_size, G, _decode_capacity(c, 2), dim, dtype=torch.bfloat16,
                                           device=dev) for _ in range(2)) for c in caches]
                meters = [FlushMeter(c, torch) for c in caches] if meter else None
                if meters:
                    for c, m in zip(caches, meters):
                        c._route_commit = m
                live[s] = (caches, packs, meters)

            def flush(s, j, events=None, metered=False):
                caches, packs, meters = live[s]
                k, v = data[j]
                if events is not None:
                    events[0].record(hip_streams[0])
                for li, cache in enumerate(caches):
                    rows = slice(None) if stacked else slice(li, li + 1)
                    with torch.cuda.stream(hip_streams[li % n_streams]):
                        m = meters[li] if metered else None
                        if m is not None:
                            m.begin()
                        cache.route_and_flush_batch(k[rows], v[rows], positions[j][rows], span_ends=ends[j][rows])
                        if m is not None:
                            m.before_pack()
                        view = readout_view(cache)
                        plan = cache._semantic_attention_plan()
                        _launch_pack(cache, view, plan, empty, empty, dim, *packs[li], False, 0)
                        if m is not None:
                            m.end()
                if events is not None:
                    events[1].record(hip_streams[0])

            for s in seg["streams"]:
                for j in range(PREP_FLUSHES):
                    flush(s, j)
            for s, j in seg["warm"]:
                flush(s, j)
            torch.cuda.synchronize()
            evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in seg["timed"]] \
                if stacked and n_streams == 1 else [None] * len(seg["timed"])
            t0 = time.perf_counter()
            for (s, j), ev in zip(seg["timed"], evs):
                flush(s, j, ev, metered=meter)
            torch.cuda.synchronize()
            elapsed += time.perf_counter() - t0
            step_ms += [ev[0].elapsed_time(ev[1]) for ev in evs if ev is not None]
            if meter:
                for caches, _, meters in live.values():
                    for c, m in zip(caches, meters):
                        del c._route_commit
                        records += m.results()
            s_last = seg["timed"][-1][0] if seg["timed"] else seg["streams"][-1]
            last = live[s_last][0][0]
            width = int(last._semantic_attention_plan().width)
            B_, L_ = last.B_prime, last.L_alloc
            del live
        label = "stacked layers" if stacked else f"{n_streams} stream(s)"
        progress(f"flush, {label}{' (metered)' if meter else ''}: {args.steps} timed flushes in {elapsed:.3f} s "
                 f"over {len(segments)} segment(s)")
        return {"elapsed": elapsed, "step_ms": step_ms, "records": records, "B": B_, "L": L_, "width": width}

    def add_recent_pass():
        """The layers driven as litgpt's model drives them: one cache per layer (batch 1, built as the
        model builds them, so they form one flush group), and per step, for every layer, the readout
        (plan + pack of the prefix the next attention reads) then add_recent of the step's 2048-row
        block. Each step's add_recent leaves the flush of the previous block pending; the first readout
        of the next step runs the 28 pending flushes as one stacked flush. Steps are blocks 3..15 of
        32K-token streams (the first three fill the window and the ladders), warm-up steps first."""
        total, done, elapsed = args.warmup + args.steps, 0, 0.0
        runs = [0, 0]
        empty = torch.empty(1, G, 0, D, dtype=torch.bfloat16, device=dev)
        while done < total:
            caches = [new_flush_cache(torch, dev, 1, cos, sin) for _ in range(layers)]
            packs = [tuple(torch.empty(1, G, _decode_capacity(c, 2), dim, dtype=torch.bfloat16, device=dev)
                           for _ in range(2)) for c in caches]
            t0 = None
            for blk in range(STREAM_FLUSHES):
                steady = blk >= 3
                if steady and done >= total:
                    break
                if steady and done >= args.warmup and t0 is None:
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                k, v = data[blk]
                for li, cache in enumerate(caches):
                    view = readout_view(cache)
                    plan = cache._semantic_attention_plan()
                    _launch_pack(cache, view, plan, empty, empty, dim, *packs[li], False, 0)
                    cache.add_recent(k[li:li + 1], v[li:li + 1], k_raw=k[li:li + 1],
                                     input_pos=positions[blk][li:li + 1], span_ends=ends[blk][li:li + 1])
                if steady:
                    done += 1
            if t0 is not None:
                torch.cuda.synchronize()
                elapsed += time.perf_counter() - t0
            for cache in caches:
                readout_view(cache)          # the last block's pending flush, outside the timed region
            group = caches[0]._group
            if group is not None:
                runs[0] += group.stacked_runs
                runs[1] += group.member_runs
            del caches, packs, group
        stacked, member = runs
        progress(f"flush, per-layer add_recent: {args.steps} timed steps in {elapsed:.3f} s "
                 f"({stacked} stacked group flushes, {member} member flushes)")
        return elapsed, stacked, member

    tokens = F * layers * args.steps
    timed = run_pass(True, 1)
    if args.profile_flush:
        # A counter run profiles the timed pass alone: its steps are the last cut_kernel ranges.
        return {"value": tokens / timed["elapsed"], "ms_per_step": timed["elapsed"] / args.steps * 1e3,
                "config": {"workload": "profiling run of the headline's timed stacked pass"},
                "roofline": {"avg_launch_ms": float(np.mean(timed["step_ms"]))}}
    metered = run_pass(True, 1, meter=True)
    per_layer = {}
    if args.flush_passes == "all":
        for n_streams in sorted({1, args.streams}):
            try:
                r = run_pass(False, n_streams)
                per_layer[f"per_layer_calls_{n_streams}_stream_tokens_per_s"] = tokens / r["elapsed"]
                per_layer[f"per_layer_calls_{n_streams}_stream_ms_per_layer_flush"] = \
                    r["elapsed"] / args.steps / layers * 1e3
            except Exception as e:   # a secondary pass never loses the headline
                per_layer[f"per_layer_calls_{n_streams}_stream_error"] = f"{type(e).__name__}: {e}"
        try:
            el, stacked_runs, member_runs = add_recent_pass()
            per_layer["per_layer_add_recent_tokens_per_s"] = tokens / el
            per_layer["per_layer_add_recent_ms_per_layer_flush"] = el / args.steps / layers * 1e3
            per_layer["per_layer_add_recent_note"] = (
                "one cache per layer driven as litgpt/model.py calls them (readout, then add_recent of the "
                "block); the caches form one flush group, so each step's 28 deferred flushes run as one "
                f"stacked flush ({stacked_runs} stacked, {member_runs} per-member flushes in the run); "
                "per_layer_calls_* time direct per-layer route_and_flush_batch calls, which are never deferred")
        except Exception as e:
            per_layer["per_layer_add_recent_error"] = f"{type(e).__name__}: {e}"
    recs = metered["records"]
    stage_bytes = {k: float(np.mean([by[k] for by, _ in recs])) for k in ("alpha", "route", "commit", "pack")}
    stage_ms = {k: float(np.mean([ms[k] for _, ms in recs])) for k in ("alpha", "route", "commit", "pack")}
    step_bytes = sum(stage_bytes.values())
    step_ms = float(np.mean(timed["step_ms"]))
    achieved = gbs(step_bytes, step_ms)
    stages = {k: {"bytes": stage_bytes[k], "ms": stage_ms[k], "achieved": gbs(stage_bytes[k], stage_ms[k]),
                  "frac": gbs(stage_bytes[k], stage_ms[k]) / HBM_PEAK_GBS} for k in stage_bytes}
    traffic, traffic_source = args.step_traffic, "--step-traffic" if args.step_traffic else None
    if traffic is None:
        traffic, traffic_source = profiled_step_traffic()
    return {
        "value": tokens / timed["elapsed"],
        "ms_per_step": timed["elapsed"] / args.steps * 1e3,
        "config": {"workload": f"{layers}-layer flush, Qwen3-1.7B KV shape (8x128 bf16), batch 1, flush {F}, "
                               f"K=12, B=128, Alpha exact pool {EXACT} / span cap {SPAN}, Beta novelty + 4->2 "
                               "split, attach route, mid-anchor plan + pack",
                   "layers": layers, "flush": F, "batch": 1, "kv_groups": G, "head_dim": D, "clusters": K,
                   "slots_per_level": timed["B"], "levels": timed["L"], "exact_tokens": EXACT, "span_cap": SPAN,
                   "steps_are": f"flushes 3..16 of chained 32K-token streams ({len(segments)} segment(s), "
                                f"{args.warmup} warm-up + {args.steps} timed steps)",
                   "pooled_width_after_last_flush": timed["width"],
                   "mode": "the layers' caches stacked as the batch rows of one cache, one flush call per step",
                   **per_layer},
        "roofline": {"kernel": "whole flush step: cut/score/choose + partition, order/attach/seed, "
                               "bucket/commit/units/carries x6/finishes (centers and the finishes of levels 0..2 "
                               "on a side stream), plan + pack (one launch sequence for all layers)",
                     "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic, "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": step_bytes, "avg_launch_ms": step_ms,
                     "launches": len(timed["step_ms"]),
                     "timing": "HIP events around each timed step on its stream",
                     "stages": stages},
    }


# ----------------------------------------------------------------------
# Config 1: one flush of one layer (the CPU reference configuration) on the GPU
# ----------------------------------------------------------------------

def config1_rows(torch, seed=7):
    """Qwen3-0.6B KV shape (8 x 128), batch 1: K=12 centers N(0,1)*4 (bf16) and the timed flush's 2048
    rows, 90% a center plus N(0, 0.5^2) noise, 10% outliers N(0,1)*12 (orphans); values N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    centers = torch.randn(1, G, K, D, generator=g) * 4
    label = torch.randint(0, K, (1, G, F), generator=g)
    x = torch.gather(centers, 2, label[..., None].expand(-1, -1, -1, D)) + torch.randn(1, G, F, D, generator=g) * 0.5
    far = torch.rand(1, G, F, generator=g) < 0.1
    k = torch.where(far[..., None], torch.randn(1, G, F, D, generator=g) * 12, x).to(torch.bfloat16)
    v = (torch.randn(1, G, F, D, generator=g)).to(torch.bfloat16)
    return centers.to(torch.bfloat16), k, v


def config1_setup(torch, dev, seed=7):
    """Qwen3-0.6B KV shape (8 x 128), batch 1, K=12 frozen centers N(0,1)*4 opened by a first flush of
    the 12 center rows at positions 0..11, then the timed flush: 2048 rows at positions 2048..4095,
    90% a center plus N(0, 0.5^2) noise, 10% outliers N(0,1)*12 (orphans). B=128, Alpha / Beta off,
    s_h = 64 (lambda * s_h separates noise, about 32, from outliers, about 2e4)."""
    from logkv_amd import LogStructuredKVCache
    from workloads import rope_tables

    cos, sin = rope_tables(N, D)
    cache = LogStructuredKVCache((1, G, N, D), (1, G, N, D), B=B, recent_size=F, device=dev, dtype=torch.bfloat16,
                                 semantic_clusters=True, cluster_k_max=K, semantic_s_h=64.0,
                                 semantic_flush_granularity=F, semantic_anchor_mode="mid",
                                 allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D)
    centers, k, v = config1_rows(torch, seed)
    return cache, centers, k, v


def config1_workload(args, torch, np):
    dev = torch.device("cuda", 0)
    cache, centers, k, v = config1_setup(torch, dev)
    seed_pos = torch.arange(K, device=dev).unsqueeze(0)
    cache.route_and_flush_batch(centers.to(dev), centers.to(dev), seed_pos)
    state = {n: b.clone() for n, b in cache.named_buffers()}
    kd, vd = k.to(dev), v.to(dev)
    pos = torch.arange(F, 2 * F, device=dev).unsqueeze(0)
    assign = torch.empty(G, F, dtype=torch.int8, device=dev)
    order = torch.empty(1, F, dtype=torch.int32, device=dev)
    snap = (cache.level_count.long().cpu().numpy(), cache.alive.cpu().numpy(), cache.p_hi_c.cpu().numpy())
    stream = torch.cuda.current_stream(dev)
    times = []
    reps = 50
    for i in range(reps + 5):
        for n, b in cache.named_buffers():
            b.copy_(state[n])
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(stream)
        cache.route_and_flush_batch(kd, vd, pos, assign_out=assign, order_out=order)
        ev[1].record(stream)
        torch.cuda.synchronize()
        if i >= 5:
            times.append(ev[0].elapsed_time(ev[1]))
    ms = float(np.median(times))
    nbytes = route_bytes(F, G, D, K) + commit_bytes(*snap, assign.cpu().numpy(), order.long().cpu().numpy(),
                                                    pos.cpu().numpy(), np.array([F]), cache.B_prime,
                                                    cache.L_alloc, D, D)
    orphans = int((~cache.alive.cpu()).sum())
    return {"workload": "one flush of one layer, Qwen3-0.6B KV shape (8 x 128 bf16), batch 1, 2048 rows, 12 live "
                        "clusters with frozen centers N(0,1)*4, 90% center + N(0,0.5^2), 10% outliers N(0,1)*12, "
                        "B=128, Alpha / Beta off, s_h=64; device time of the route + commit from HIP events, "
                        f"median of {reps} flushes from the same restored state",
            "ms_per_flush": ms, "flushed_tokens_per_s": F / (ms * 1e-3),
            "slots_per_level": cache.B_prime, "levels": cache.L_alloc, "clusters_alive_after": K * G - orphans,
            "roofline": {"kernel": "order/attach/seed + bucket/commit/units/carries/finish", "bound": "hbm",
                         "achieved": gbs(nbytes, ms), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs(nbytes, ms) / HBM_PEAK_GBS, "algorithmic_bytes_per_launch": nbytes,
                         "note": "a single small flush is launch- and latency-bound"}}


# ----------------------------------------------------------------------
# Config 4: decode at 32K context through the streaming engine
# ----------------------------------------------------------------------

def decode_workload(args, torch, np):
    from logkv_amd import LogKVStreamingAttention, LogStructuredKVCache
    from logkv_amd.log_kv_pack import _launch_pack, packed_attention, packed_dim, readout_view
    from workloads import fill_readout_state, rope_tables

    dev = torch.device("cuda", 0)
    Bt, HQ = 8, 16
    cos, sin = rope_tables(N, D)
    cache = LogStructuredKVCache((Bt, G, N, D), (Bt, G, N, D), B=B, recent_size=F, device=dev,
                                 dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=64.0,
                                 semantic_flush_granularity=F, semantic_anchor_mode="mid",
                                 allocate_second_order=False, cos_cache=cos, sin_cache=sin, rope_n_elem=D,
                                 alpha_exact_tokens=EXACT, alpha_span_max_tokens=SPAN, beta_novelty=True,
                                 beta_adaptive_merge=True)
    steps, warm = args.decode_steps, 8
    archived = N - F - EXACT
    # The recent window starts short by the decoded tokens, so it ends full and no flush falls inside.
    fill_readout_state(cache, seed=21, recent=F - steps - warm, archived=archived)
    scale = D ** -0.5
    engine = LogKVStreamingAttention(cache, scale)
    gen = torch.Generator(device=dev).manual_seed(77)
    n = steps + warm
    qs = torch.randn(n, Bt, HQ, 1, D, generator=gen, device=dev).to(torch.bfloat16)
    ks = torch.randn(n, Bt, G, 1, D, generator=gen, device=dev).to(torch.bfloat16)
    vs = torch.randn(n, Bt, G, 1, D, generator=gen, device=dev).to(torch.bfloat16)
    start = cache.token_count
    pos = torch.arange(start, start + n, device=dev)
    ends = (torch.rand(n, Bt, 1, generator=gen, device=dev) < 1 / 32).to(torch.uint8)
    for i in range(warm):
        engine(qs[i], ks[i], vs[i], ks[i], input_pos=pos[i:i + 1], span_ends=ends[i])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warm, n):
        engine(qs[i], ks[i], vs[i], ks[i], input_pos=pos[i:i + 1], span_ends=ends[i])
    torch.cuda.synchronize()
    eng_ms = (time.perf_counter() - t0) / steps * 1e3
    progress(f"decode: {steps} tokens through the streaming engine, {eng_ms:.4f} ms per token")
    if cache.recent_count != F and cache.recent_count + (1 if engine._log_kv_pending else 0) != F:
        raise RuntimeError(f"decode window ended at {cache.recent_count} rows, expected {F}")

    # The attention kernels apart from the host: one decode step (pack of the new row, attention)
    # and its attention alone captured in HIP graphs from static inputs, checked bit for bit
    # against the eager calls, and replayed back to back.
    dim = packed_dim(D, D)
    view = readout_view(cache)
    plan = cache._semantic_attention_plan()
    cap = cache.K_max * cache.L_alloc * cache.B_prime + EXACT + cache.recent_capacity + 2
    ka = torch.empty(Bt, G, cap, dim, dtype=torch.bfloat16, device=dev)
    va = torch.empty_like(ka)
    q_s, k_s, v_s = qs[-1].clone(), ks[-1].clone(), vs[-1].clone()
    recent = cache.recent_count
    tail = recent + 1
    _launch_pack(cache, view, plan, k_s, v_s, dim, ka, va, False, 0)
    _, workspace = packed_attention(q_s, ka, va, plan, tail, scale, 1, D, G, None, cache.alpha_count_dev)
    stream = torch.cuda.current_stream(dev)

    def full_step():
        _launch_pack(cache, view, plan, k_s, v_s, dim, ka, va, True, recent)
        return packed_attention(q_s, ka, va, plan, tail, scale, 1, D, G, workspace, cache.alpha_count_dev)[0]

    def attention_only():
        return packed_attention(q_s, ka, va, plan, tail, scale, 1, D, G, workspace, cache.alpha_count_dev)[0]

    def replayed_ms(fn, per_graph=8, replays=8):
        # per_graph calls captured back to back in one graph (as a model's layers issue them), the
        # graph replayed `replays` times; ms per call.
        eager = fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = [fn() for _ in range(per_graph)]
        graph.replay()
        torch.cuda.synchronize()
        if not all(torch.equal(o, eager) for o in outs):
            raise RuntimeError("graph replay of the decode step differs from the eager call")
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(stream)
        for _ in range(replays):
            graph.replay()
        ev[1].record(stream)
        torch.cuda.synchronize()
        if not all(torch.equal(o, eager) for o in outs):
            raise RuntimeError("graph replay of the decode step differs from the eager call")
        return ev[0].elapsed_time(ev[1]) / (per_graph * replays)

    step_ms = replayed_ms(full_step)
    attn_ms = replayed_ms(attention_only)
    width = plan.width
    rows = width + cache.alpha_count + tail
    lanes = Bt * G
    # Algorithmic bytes: every packed row of every lane once as the kernel needs it - the key's
    # D features and its bias column, the value's D features (2 * (D + 1) + 2 * D = 514 B) - plus
    # the queries and outputs.
    row_bytes = 2 * (D + 1) + 2 * D
    attn_bytes = lanes * rows * row_bytes + Bt * HQ * D * 2 * 2
    achieved = gbs(attn_bytes, attn_ms)
    # The packed rows the attention read, for the CPU baseline's slot attention over the same state.
    cpu_state = (q_s.cpu(), ka[:, :, :rows].float().cpu(), va[:, :, :rows].float().cpu(), scale)
    return {
        "_cpu_state": cpu_state,
        "workload": "decode, one layer, batch 8, Qwen3-1.7B GQA (16 q / 8 KV heads x 128, bf16), 32K-token cache: "
                    f"recent window ending at {F} rows, exact pool {EXACT}, 12 clusters holding {archived} archived "
                    "tokens per lane, masses ~ U(1,64); ms_per_token = wall time per token through "
                    "LogKVStreamingAttention (pending-token pairing, pack of the new rows, attention, add_recent "
                    "of every token pair), launched from Python",
        "ms_per_token": eng_ms, "ms_per_token_28_layers": 28 * eng_ms, "steps": steps,
        "device_ms_per_token": step_ms,
        "device_ms_per_token_note": "one step's pack + attention, 8 steps captured back to back in a HIP graph and "
                                    "replayed 8 times (no host work)",
        "packed_rows_per_lane": rows, "pooled_width": width,
        "roofline": {"kernel": "stream_kernel + combine_kernel", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "algorithmic_bytes_per_launch": attn_bytes, "bytes_per_packed_row": row_bytes,
                     "avg_launch_ms": attn_ms,
                     "timing": "HIP events around 8 replays of a HIP graph holding 8 back-to-back attention calls "
                               "(stream_kernel + combine_kernel each)"},
    }


# ----------------------------------------------------------------------
# Config 3: streaming prefill
# ----------------------------------------------------------------------

def prefill_workload(args, torch, np):
    """The streaming prefill on one stream (the line's figures and the attention roofline), then again with
    every cache's flushes on a side stream (``flush_stream``) beside the later layers' attention."""
    res = _prefill_pass(args, torch, np, False)
    if args.prefill_flush_stream:
        torch.cuda.empty_cache()
        side = _prefill_pass(args, torch, np, True)
        res["side_stream"] = {k: side[k] for k in ("ms_per_block", "ms_per_block_by_block", "tokens_per_s")}
        res["side_stream"]["note"] = ("flushes on a side stream: a layer's next attention waits for its own flush "
                                      "only; the attention kernels then share the GPU with flush kernels")
    return res


def _prefill_pass(args, torch, np, side_stream):
    """Streaming prefill of a 32,768-token sequence through 28 Qwen3-1.7B-shaped layer caches, one call per
    layer as a model makes them: per 2048-token block and layer, the chunk attention of the block's 16 query
    heads over [compressed cache | block] (causal within the block) and add_recent, which flushes 2048 rows
    into the ladders once the recent window is full. Queries, keys and values are seeded random bf16 (the
    model's projections are not on this path)."""
    from logkv_amd import LogStructuredKVCache, log_kv_chunk_attention
    from workloads import Mixture, rope_tables

    dev = torch.device("cuda", 0)
    layers, HQ, blocks = args.layers, 16, max(1, min(N // F, args.prefill_blocks))
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
    # Every layer's append + flush runs on a side stream beside the later layers' attention; a layer's
    # next attention waits for its own flush (the cache orders its readers after it).
    side = torch.cuda.Stream(dev) if side_stream else None
    for cache in caches:
        cache.flush_stream = side
    scale = D ** -0.5
    # Untimed warm-up on a spare cache: two blocks of attention + flush load every kernel of the path.
    spare = LogStructuredKVCache((1, G, 2 * F, D), (1, G, 2 * F, D), B=B, recent_size=F // 2, device=dev,
                                 dtype=torch.bfloat16, semantic_clusters=True, cluster_k_max=K, semantic_s_h=64.0,
                                 semantic_flush_granularity=F // 2, semantic_anchor_mode="mid",
                                 allocate_second_order=False, cos_cache=cos[:2 * F], sin_cache=sin[:2 * F],
                                 rope_n_elem=D, alpha_exact_tokens=EXACT, alpha_span_max_tokens=SPAN,
                                 beta_novelty=True, beta_adaptive_merge=True)
    warm = Mixture(1, G, D, clusters=K, seed=44)
    for blk in range(2):
        k_w, v_w = warm.rows(F // 2).to(dev), warm.rows(F // 2).to(dev)
        pos_w = torch.arange(blk * F // 2, (blk + 1) * F // 2, device=dev).unsqueeze(0)
        log_kv_chunk_attention(spare, q[:, :, :F // 2], k_w, v_w, scale, second_order_scale=0.0)
        ends_w = torch.tensor([[(p + 7) % 32 == 0 for p in range(blk * F // 2, (blk + 1) * F // 2)]],
                              dtype=torch.uint8, device=dev)
        spare.add_recent(k_w, v_w, k_raw=k_w, input_pos=pos_w, span_ends=ends_w)
    torch.cuda.synchronize()
    del spare
    block_ms, attn_ms, slots, attn_flops = [], [], [], []
    for blk in range(blocks):
        k_raw, v = mix.rows(F).to(dev), mix.rows(F).to(dev)
        pos = torch.arange(blk * F, (blk + 1) * F, device=dev).unsqueeze(0)
        ends = torch.tensor([[(p + 7) % 32 == 0 for p in range(blk * F, (blk + 1) * F)]], dtype=torch.uint8,
                            device=dev)
        # Rows the block's attention reads (every layer holds the same counts): the pooled width of the
        # widest lane, the exact pool, the recent window, then the block causally.
        c0 = caches[0]
        prefix = int(c0.level_count.long().sum((-1, -2)).max()) + c0.alpha_count + c0.recent_count
        attn_flops.append(layers * HQ * 4 * D * (F * prefix + F * (F + 1) // 2))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        events = []
        for cache in caches:
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            cache._await_flush(stream)   # the wait for the layer's last flush precedes the timed attention
            ev[0].record(stream)
            log_kv_chunk_attention(cache, q, k_raw, v, scale, second_order_scale=0.0)
            ev[1].record(stream)
            events.append(ev)
            cache.add_recent(k_raw, v, k_raw=k_raw, input_pos=pos, span_ends=ends)
        for cache in caches:
            cache._await_flush(stream)
        torch.cuda.synchronize()
        block_ms.append((time.perf_counter() - t0) * 1e3)
        attn_ms.append(float(np.sum([e[0].elapsed_time(e[1]) for e in events])))
        slots.append(float(c0.level_count.float().sum() / (G * K)))
    attn_s = float(np.sum(attn_ms)) * 1e-3
    tflops = float(np.sum(attn_flops)) / attn_s / 1e12
    progress(f"prefill: {blocks} blocks, {np.mean(block_ms):.1f} ms per block over {layers} layers")
    return {
        "workload": f"streaming prefill of {blocks * F} tokens through {layers} Qwen3-1.7B-shaped layer caches (16 q / 8 KV "
                    f"heads x 128, bf16), batch 1, {F}-token blocks, recent {F}, K={K}, B={B}, Alpha {EXACT}/{SPAN}, "
                    "Beta, mid anchor; per block and layer: chunk attention (matrix cores) + add_recent (flush)"
                    + (", flushes on a side stream beside the attention" if side is not None else ", one stream"),
        "ms_per_block": float(np.mean(block_ms)), "ms_per_block_by_block": [round(x, 2) for x in block_ms],
        "tokens_per_s": N / (float(np.sum(block_ms)) * 1e-3),
        "attention_ms_per_block": float(np.mean(attn_ms)),
        "attention_ms_by_block": [round(x, 2) for x in attn_ms],
        "attention_roofline": {"kernel": "chunk_kernel + chunk_combine_kernel", "bound": "mfma", "achieved": tflops,
                               "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tflops / BF16_PEAK_TFLOPS,
                               "flops": "4 * D per (query row, visible key) per query head: every prefix row and "
                                        "the block causally (T_q * (T_q + 1) / 2 pairs)"},
        "flushes": sum(1 for x in slots if x > 0),
        "slots_per_cluster_after_each_block": [round(x, 1) for x in slots],
    }


# ----------------------------------------------------------------------
# Config 5: unified route control
# ----------------------------------------------------------------------

def unified_workload(args, torch, np):
    """The unified (Ward / radius) route control: batch 4 x 8 KV groups, recent = flush = 4096 rows, a
    131,072-token stream (31 flush events) of a 12-Gaussian mixture that drifts every 16K tokens."""
    from logkv_amd import LogStructuredKVCache
    from workloads import Mixture, rope_tables

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
    reducer = np.zeros(4)   # summed over the timed flushes: dist, scan, Lance-Williams bytes; merges
    rounds = []
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
            reducer += unified_reducer_bytes(cache.unified_reduce_stats(T).numpy())
            rounds.append(int(cache.unified_reduce_stats(T)[:, 0, 1].max()))
    timed = flushes - warm
    ms = t_all / timed * 1e3
    dev_ms = float(np.mean(times))
    per_flush = reducer / timed
    alg = float(per_flush[:3].sum())
    achieved = gbs(alg, dev_ms)
    progress(f"unified route: {timed} timed flushes, {ms:.1f} ms per flush")
    return {
        "workload": "unified Ward / radius route control, Qwen3-1.7B KV shape (8 x 128 bf16), batch 4, "
                    f"recent = flush = {T}, {stream_tokens}-token stream ({flushes} flush events), 12-Gaussian "
                    f"mixture drifting every 16K tokens, K={K}, B={B}, L={cache.L_alloc}, s_h={s_h}",
        "flushed_tokens_per_s": Bt * T / (ms * 1e-3), "ms_per_flush": ms,
        "device_ms_per_flush": dev_ms, "timed_flushes": timed, "warmup_flushes": warm,
        "live_clusters_per_lane": float(cache.alive.float().sum(-1).mean()),
        "radius_stage_rounds_max": max(rounds), "merges_per_flush": float(per_flush[3]),
        "roofline": {"kernel": "whole unified flush: order, load nodes, distances, radius-stage and budget-stage "
                               "reducer rounds (plan / Lance-Williams / rescan / finish), labels, stage 2, final, "
                               "old-old merges, commit",
                     "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes_per_launch": alg,
                     "bytes_by_phase": {"distances": float(per_flush[0]), "scans": float(per_flush[1]),
                                        "lance_williams": float(per_flush[2])},
                     "avg_launch_ms": dev_ms,
                     "byte_model": "reducer distance-matrix traffic only (the commit's bytes are not counted): "
                                   "per lane and stage n^2 x 4 B written by the distance pass, 4 B per rescanned "
                                   "element (rescanned rows x live columns, the first scan n x n) and 16 B per "
                                   "Lance-Williams element (kept rows x live columns: both parents' entries read, "
                                   "the row and its mirror written), from the device reducer's counts",
                     "timing": "HIP events around each timed flush on its stream"},
    }


def unified_reducer_bytes(stats):
    """Algorithmic bytes of one unified flush's reducer from its per-lane, per-stage counts
    ``[lanes, 2, 8]`` (nodes, rounds, merges, Lance-Williams elements, rescanned elements): the
    distance pass writes n^2 f32 per stage, a rescan reads 4 B per element, a Lance-Williams update
    reads both parents' entries and writes the row and its mirror (16 B per element). Returns
    (distance, scan, Lance-Williams bytes, merges)."""
    import numpy as np

    n = stats[..., 0].astype(np.float64)
    return np.array([float((n * n * 4).sum()), float(stats[..., 4].astype(np.float64).sum() * 4),
                     float(stats[..., 3].astype(np.float64).sum() * 16), float(stats[..., 2].sum())])


# ----------------------------------------------------------------------
# CPU baseline
# ----------------------------------------------------------------------

def host_info():
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return model, cores


def _cpu_stream_flushes(cache_cls, seconds, threads):
    """Headline flushes (3..16 of fresh 32K-token streams) of one layer through ``cache_cls`` on the
    host with ``threads`` torch threads, until ``seconds`` of timed flush work: (tokens/s, flushes, s)."""
    import numpy as np
    import torch

    from workloads import Mixture, rope_tables

    torch.set_num_threads(threads)
    cos, sin = (t.numpy() for t in rope_tables(N, D))
    mix = Mixture(1, G, D, clusters=K, seed=1)
    n, t = 0, 0.0
    while t < seconds:
        cache = cache_cls(1, G, N, D, D, B=B, recent_size=F, K=K, s_h=64.0, flush=F, exact_tokens=EXACT,
                          span_max=SPAN, beta_novelty=True, beta_adaptive=True, cos=cos, sin=sin)
        for j in range(STREAM_FLUSHES):
            k, v = mix.rows(F).float().numpy(), mix.rows(F).float().numpy()
            pos = np.arange(j * F, (j + 1) * F)[None]
            t0 = time.perf_counter()
            cache.flush_rows(k, v, pos, span_ends_for(j))
            cache.pack(None, None)
            if j >= PREP_FLUSHES:
                t += time.perf_counter() - t0
                n += 1
            if t >= seconds:
                break
    return F * n / t, n, t


def _cpu_config1(threads, reps=5):
    """Config 1 on the host: the one-layer flush of ``config1_rows`` from its restored state (the 12
    centers opened by a first flush), median of ``reps`` flushes."""
    import copy

    import numpy as np
    import torch

    from oracle.torch_cpu import TorchCpuCache
    from workloads import rope_tables

    torch.set_num_threads(threads)
    centers, k, v = config1_rows(torch)
    cos, sin = (t.numpy() for t in rope_tables(N, D))
    base = TorchCpuCache(1, G, N, D, D, B=B, recent_size=F, K=K, s_h=64.0, flush=F, cos=cos, sin=sin)
    c = centers.float().numpy()
    base.flush_rows(c, c, np.arange(K)[None])
    times = []
    for _ in range(reps):
        cache = copy.deepcopy(base)
        t0 = time.perf_counter()
        cache.flush_rows(k.float().numpy(), v.float().numpy(), np.arange(F, 2 * F)[None])
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times)) * 1e3
    return {"ms_per_flush": ms, "flushed_tokens_per_s": F / (ms * 1e-3), "threads": threads,
            "clusters_alive_after": int(cache.alive.sum())}


def _cpu_decode(state, seconds, threads):
    """Decode attention on the host: the Torch-CPU slot attention (oracle/torch_cpu.py, the reference's
    SDPA over the Flash encoding, float32) over the packed rows the GPU's step read, one query per
    head for batch 8 x 16 heads; (ms per token per layer, steps timed)."""
    import torch

    from oracle.torch_cpu import slot_attention

    torch.set_num_threads(threads)
    q, ka, va, scale = state
    slot_attention(q, ka, va, scale, D)
    n, t = 0, 0.0
    while t < seconds or n < 3:
        t0 = time.perf_counter()
        slot_attention(q, ka, va, scale, D)
        t += time.perf_counter() - t0
        n += 1
    return t / n * 1e3, n


def _cpu_unified(threads, lanes, timed, warm):
    """The unified route's flush on the host for ``lanes`` sampled lanes (the first KV groups of batch
    row 0 of the GPU leg's stream, same generator and seed): the Torch-CPU reducer with the
    reference's Gram distances above 32 nodes and the batched commit (oracle/torch_cpu.py); flushes
    1..warm untimed, the next ``timed`` timed; (seconds per flush of the sampled lanes, flushes)."""
    import numpy as np
    import torch

    from oracle.torch_cpu import TorchCpuCache
    from workloads import Mixture, rope_tables

    torch.set_num_threads(threads)
    Bt, T, stream_tokens = 4, 4096, 131072
    cos, sin = (t.numpy() for t in rope_tables(stream_tokens, D))
    cache = TorchCpuCache(1, lanes, stream_tokens, D, D, B=B, recent_size=T, K=K, s_h=64.0, flush=T, cos=cos,
                          sin=sin, unified=True)
    cache.gram_distances = True
    mix = Mixture(Bt, G, D, clusters=12, seed=31, drift_every=2 * 16384)
    total = 0.0
    for i in range(warm + timed):
        k, v = mix.rows(T), mix.rows(T)
        k, v = k[:1, :lanes].float().numpy(), v[:1, :lanes].float().numpy()
        pos = np.arange(i * T, (i + 1) * T)[None]
        t0 = time.perf_counter()
        cache.flush_rows(k, v, pos)
        if i >= warm:
            total += time.perf_counter() - t0
    return total / timed, timed


def cpu_baseline(seconds: float, decode_state=None, unified=False):
    """The CPU baseline: the batched Torch-CPU port of the flush (oracle/torch_cpu.py, every ladder of
    a flush appended level by level, Beta groups as tensor operations, bit-identical to the oracle) on
    the host cores: the headline flush of one layer (Alpha / Beta, route, commit and the pack of the
    new prefix, flushes 3..16 of fresh 32K-token streams) with every available core and with one
    thread, and config 1's one-layer flush; the per-token numpy oracle is timed beside it."""
    import torch

    from oracle import OracleCache
    from oracle.torch_cpu import TorchCpuCache

    model, cores = host_info()
    all_rate, all_n, all_t = _cpu_stream_flushes(TorchCpuCache, seconds * 0.4, cores)
    one_rate, one_n, one_t = _cpu_stream_flushes(TorchCpuCache, seconds * 0.3, 1)
    ora_rate, ora_n, ora_t = _cpu_stream_flushes(OracleCache, seconds * 0.2, 1)
    config1 = _cpu_config1(cores)
    config1["1_thread"] = _cpu_config1(1)
    legs = {}
    if decode_state is not None:
        ms_all, n_all = _cpu_decode(decode_state, seconds * 0.1, cores)
        ms_one, n_one = _cpu_decode(decode_state, seconds * 0.1, 1)
        rows = decode_state[1].shape[2]
        legs["decode"] = {
            "value": ms_all, "unit": "ms per token per layer", "cores": cores, "kind": "port",
            "value_1_thread": ms_one, "higher_is_better": False,
            "sample": f"Torch-CPU slot attention (scaled_dot_product_attention over the packed Flash encoding, "
                      f"float32) of one decode step: batch 8 x 16 query heads over the GPU step's {rows} packed "
                      f"rows per lane; {n_all} steps on {cores} threads, {n_one} on 1 thread"}
    if unified:
        lanes_all, lanes_one, flush_tokens, all_lanes = 2, 1, 4 * 4096, 4 * G
        s_all, n_all = _cpu_unified(cores, lanes_all, timed=2, warm=1)
        s_one, n_one = _cpu_unified(1, lanes_one, timed=1, warm=1)
        legs["unified"] = {
            "value": flush_tokens / (s_all * all_lanes / lanes_all), "unit": "flushed tokens/s", "cores": cores,
            "kind": "port", "value_1_thread": flush_tokens / (s_one * all_lanes / lanes_one),
            "seconds_per_flush_sampled_lanes": s_all, "seconds_per_flush_sampled_lanes_1_thread": s_one,
            "sample": f"Torch-CPU unified route (the reducer restated on torch tensors with the reference's Gram "
                      f"distances, then the batched commit) of {lanes_all} of the {all_lanes} lanes (KV groups of "
                      f"batch row 0, same stream) for flushes 2..{1 + n_all} on {cores} threads and {lanes_one} lane "
                      f"for flush 2 on 1 thread; flushed tokens/s = 4 x 4096 / (seconds per flush x "
                      f"{all_lanes} / sampled lanes), lanes being independent"}
    torch.set_num_threads(cores)
    threads = torch.get_num_threads()
    return {"legs": legs, "value": all_rate, "unit": "flushed tokens/s", "cores": cores, "kind": "port",
            "value_1_thread": one_rate, "oracle_1_thread": ora_rate, "config1": config1,
            "host_cpu": model, "host_cores_available": cores, "torch_threads": threads,
            "sample": f"batched Torch-CPU port: Alpha/Beta + route + commit + pack of {all_n} flushes of one layer "
                      f"(flushes 3..16 of 32K-token streams; batch 1, 8 groups x 128, K=12, B=128, exact pool 256, "
                      f"{F} rows each) in {all_t:.1f} s on {cores} threads; {one_n} flushes in {one_t:.1f} s on 1 "
                      f"thread; the per-token numpy oracle: {ora_n} flushes in {ora_t:.1f} s on 1 thread"}


# ----------------------------------------------------------------------
# rocprofv3 counter summary
# ----------------------------------------------------------------------

def _counter_rows(path):
    import csv

    p = Path(path)
    files = [p] if p.is_file() else sorted(p.rglob("*counter_collection.csv"))
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {path}")
    rows = []
    for f in files:
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return rows


def _short(name):
    return name.replace("(anonymous namespace)::", "").split("(")[0].replace("logkv::", "").replace("void ", "")


def pmc_summary(fetch_dir, write_dir, steps, probe_mib):
    """HBM bytes per timed headline step from FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by
    its reading of the copy probe of ``probe_mib`` MiB; a step runs from one cut_kernel to the next."""
    out = {}
    for name, path in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _counter_rows(path)
        probe = [float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]]
        factor = probe_mib * 1024 / probe[0] if probe else 1.0
        starts = [i for i, r in enumerate(rows) if _short(r["Kernel_Name"]) == "cut_kernel"]
        bounds = list(zip(starts, starts[1:] + [len(rows)]))[-steps:]
        per_step, per_kernel = [], {}
        for a, b in bounds:
            total = 0.0
            for r in rows[a:b]:
                k = _short(r["Kernel_Name"])
                if "copyBuffer" in k or "elementwise" in k or "fill" in k.lower():
                    continue
                v = float(r["Counter_Value"]) * factor * 1024
                total += v
                per_kernel[k] = per_kernel.get(k, 0.0) + v / len(bounds)
            per_step.append(total)
        out[name] = {"bytes_per_step": sum(per_step) / len(per_step), "factor": factor,
                     "probe_kib": probe[0] if probe else None, "per_kernel": per_kernel}
    out["traffic_per_step"] = out["FETCH_SIZE"]["bytes_per_step"] + out["WRITE_SIZE"]["bytes_per_step"]
    return out


def trace_summary(trace_csv, steps):
    """Kernel time per headline step from a ``rocprofv3 --kernel-trace`` CSV of a ``--profile-flush`` run:
    the last ``steps`` ranges from one cut_kernel to the next, per kernel (mean us per step) and the span
    from the first kernel's start to the last kernel's end."""
    import csv

    with open(trace_csv) as fh:
        rows = sorted(csv.DictReader(fh), key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if _short(r["Kernel_Name"]) == "cut_kernel"]
    bounds = list(zip(starts, starts[1:] + [len(rows)]))[-steps:]
    per_kernel, spans = {}, []
    for a, b in bounds:
        keep = [r for r in rows[a:b] if "copyBuffer" not in r["Kernel_Name"]]
        for r in keep:
            k = _short(r["Kernel_Name"])
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            per_kernel[k] = per_kernel.get(k, 0.0) + us / len(bounds)
        spans.append((int(keep[-1]["End_Timestamp"]) - int(keep[0]["Start_Timestamp"])) / 1e3)
    return {"steps": len(bounds), "span_us": sum(spans) / len(spans), "kernel_us": sum(per_kernel.values()),
            "per_kernel_us": dict(sorted(per_kernel.items(), key=lambda kv: -kv[1]))}


def kernel_counters(counter_dir):
    """Mean of every counter per dispatch of each kernel in a ``rocprofv3 --pmc`` run, with the dispatch count."""
    out = {}
    for r in _counter_rows(counter_dir):
        k = _short(r["Kernel_Name"])
        e = out.setdefault(k, {"dispatches": set(), "counters": {}})
        e["dispatches"].add(r["Dispatch_Id"])
        e["counters"].setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: {"dispatches": len(e["dispatches"]),
                **{c: sum(v) / len(v) for c, v in sorted(e["counters"].items())}} for k, e in out.items()}


# ----------------------------------------------------------------------

def quiet_gc(fn, *args):
    """Run a measurement with Python's cycle collector paused (collected before): a collection
    inside a timed region stalls the host for milliseconds while the GPU waits for launches."""
    gc.collect()
    gc.disable()
    try:
        return fn(*args)
    finally:
        gc.enable()


def run_leg(result, key, fn, *args):
    """A secondary measurement: its failure is recorded in the line, never fatal."""
    try:
        result[key] = quiet_gc(fn, *args)
    except Exception as e:
        traceback.print_exc()
        result[key] = {"error": f"{type(e).__name__}: {e}"}
        progress(f"{key}: failed ({type(e).__name__}: {e})")


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--streams", type=int, default=4,
                    help="HIP streams the per-layer calls are spread over (a one-stream pass always runs too)")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-unified", action="store_true", help="skip the unified-route control measurement")
    ap.add_argument("--no-prefill", action="store_true", help="skip the streaming-prefill measurement")
    ap.add_argument("--no-config1", action="store_true", help="skip the one-layer flush of the CPU configuration")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first copy this many MiB device to device (a plain copy of known size that scales "
                         "the FETCH_SIZE / WRITE_SIZE counters of a profiling run)")
    ap.add_argument("--flush-passes", choices=("all", "stacked"), default="all",
                    help="stacked: only the stacked passes of the headline (profiling runs)")
    ap.add_argument("--profile-flush", action="store_true",
                    help="profiling run: the timed stacked pass of the headline only (no metered pass, no legs)")
    ap.add_argument("--only", choices=("config1", "decode", "prefill", "unified"),
                    help="profiling run: only this measurement, printed as its own JSON line")
    ap.add_argument("--prefill-flush-stream", type=int, default=1, choices=(0, 1),
                    help="1: also time the prefill with its flushes on a side stream (cache.flush_stream)")
    ap.add_argument("--prefill-blocks", type=int, default=N // F,
                    help="2048-token blocks of the streaming prefill (16 = the whole 32K-token sequence)")
    ap.add_argument("--step-traffic", type=float, default=None,
                    help="HBM bytes per headline step measured by counter runs (reported as roofline.traffic)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 --pmc runs of --profile-flush and exit")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="kernel time per headline step of a rocprofv3 --kernel-trace run of --profile-flush, and exit")
    ap.add_argument("--kernel-counters", metavar="PMC_DIR",
                    help="mean counter values per dispatch of each kernel of a rocprofv3 --pmc run, and exit")
    args = ap.parse_args(argv)
    if args.warmup < 0:
        ap.error("--warmup must be >= 0")
    if args.steps < 1:
        ap.error("--steps must be >= 1")
    if args.streams < 1:
        ap.error("--streams must be at least 1")
    return args


def main():
    args = parse_args()
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary, args.steps, args.copy_probe_mib or 1024), indent=1))
        return
    if args.trace_summary:
        print(json.dumps(trace_summary(args.trace_summary, args.steps), indent=1))
        return
    if args.kernel_counters:
        print(json.dumps(kernel_counters(args.kernel_counters), indent=1))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box here has one MI355X, so --gpus {args.gpus} is not run; the "
              "path shards by layer and lane with no exchange in the flush (see the sharding notes)", file=sys.stderr)
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
    if args.only:
        legs = {"config1": config1_workload, "decode": decode_workload, "prefill": prefill_workload,
                "unified": unified_workload}
        out = legs[args.only](args, torch, np)
        out.pop("_cpu_state", None)
        print(json.dumps(out), flush=True)
        return
    if args.profile_flush:
        args.flush_passes = "stacked"
    fl = quiet_gc(flush_workload, args, torch, np)
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
    if not args.profile_flush:
        if not args.no_config1:
            run_leg(result, "config1", config1_workload, args, torch, np)
        decode_state = None
        if not args.no_decode:
            run_leg(result, "decode", decode_workload, args, torch, np)
            decode_state = result["decode"].pop("_cpu_state", None)
            if "ms_per_token" in result["decode"]:
                result["decode_ms_per_token"] = result["decode"]["ms_per_token"]
        if not args.no_prefill and args.flush_passes == "all":
            run_leg(result, "prefill", prefill_workload, args, torch, np)
        if not args.no_unified and args.flush_passes == "all":
            run_leg(result, "unified", unified_workload, args, torch, np)
        run_leg(result, "hbm_copy", copy_peak, torch)
        if "gbs" in result["hbm_copy"]:
            result["hbm_copy_peak_gbs"] = result["hbm_copy"]["gbs"]
            for leg in (result, result.get("decode", {}), result.get("unified", {})):
                roof = leg.get("roofline") if isinstance(leg, dict) else None
                if roof and roof.get("unit") == "GB/s":
                    roof["frac_of_copy_peak"] = roof["achieved"] / result["hbm_copy_peak_gbs"]
        if not args.no_cpu_baseline:
            progress("cpu baseline: oracle flushes on the host")
            run_leg(result, "cpu_baseline", cpu_baseline, args.cpu_seconds, decode_state,
                    "flushed_tokens_per_s" in result.get("unified", {}))
            for name, leg in result["cpu_baseline"].pop("legs", {}).items():
                if isinstance(result.get(name), dict):
                    result[name]["cpu_baseline"] = leg
    print(json.dumps(result), flush=True)


def copy_peak(torch, mib=1024, reps=10):
    """A plain device-to-device copy of ``mib`` MiB timed with HIP events: the measured HBM ceiling
    (bytes read + bytes written per second) beside the 8 TB/s vendor figure."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    for _ in range(reps):
        dst.copy_(src)
    ev[1].record(stream)
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / reps
    del src, dst
    return {"gbs": 2 * n / ms * 1e-6, "bytes_per_copy": 2 * n, "ms_per_copy": ms,
            "how": f"{mib} MiB device-to-device copies (read + write bytes), mean of {reps} after 2 warm-up"}


if __name__ == "__main__":
    main()
