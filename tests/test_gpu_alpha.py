"""Alpha / Beta on the device against the oracle: span scores and whole flushes, bit for bit."""

import numpy as np
import pytest
import torch

from harness import STATE_FIELDS, compare_state, feed, make_pair, to_np
from logkv_amd import alpha_log_kv as prod
from workloads import Mixture
from oracle import spans as ora

pytestmark = pytest.mark.gpu

ALPHA_FIELDS = STATE_FIELDS + ("alpha_k_raw", "alpha_v", "alpha_pos", "alpha_valid")


@pytest.mark.parametrize("beta", [False, True])
def test_span_scores_match_oracle(beta):
    rng = np.random.default_rng(3)
    Bt, G, D, W, T, K = 2, 8, 128, 24, 96, 12
    gen = torch.Generator().manual_seed(2)
    pool = (torch.randn(Bt, G, W, D, generator=gen) * 2).to(torch.bfloat16)
    pool_v = torch.randn(Bt, G, W, D, generator=gen).to(torch.bfloat16)
    flush = (torch.randn(Bt, G, T, D, generator=gen) * 3).to(torch.bfloat16)
    flush_v = torch.randn(Bt, G, T, D, generator=gen).to(torch.bfloat16)
    centers = torch.randn(Bt, G, K, D, generator=gen) * 2
    alive = torch.rand(Bt, G, K, generator=gen) < 0.7
    alive[1, 3] = False                                   # a group with no live center
    spans = [[(5, True), (7, True), (3, False)], [(10, True), (2, False)]]
    positions = [list(range(0, 15)), list(range(3, 15))]
    new_pos = [list(range(15, 15 + T)), list(range(15, 15 + T))]
    ends = [(rng.random(T) < 0.1).tolist() for _ in range(Bt)]
    cut = prod.cut_spans(spans, positions, new_pos, ends, W, 16)
    dev = torch.device("cuda")
    tensors = [x.to(dev) for x in (pool, pool_v, flush, flush_v, centers, alive)]
    got = prod.score_spans_split(*tensors[:4], W, cut, beta_novelty=beta, centroids=tensors[4],
                                 centroid_valid=tensors[5])
    torch.cuda.synchronize()
    keys = np.concatenate((pool.float().numpy(), flush.float().numpy()), axis=2)
    vals = np.concatenate((pool_v.float().numpy(), flush_v.float().numpy()), axis=2)
    ocut = ora.cut_spans(spans, positions, new_pos, ends, W, 16)
    want = ora.score_spans(keys, vals, ocut, beta, centers.numpy(), alive.numpy())
    np.testing.assert_array_equal(got.cpu().numpy(), want)


CASES = {
    # name: (batch, groups, dim, K, B, recent, flush, max_seq, s_h, exact, span, beta, blocks)
    "alpha_small": (2, 2, 64, 4, 8, 64, 64, 2048, 16.0, 32, 8, False, 6),
    "beta_small": (2, 2, 64, 4, 8, 64, 64, 2048, 16.0, 32, 8, True, 6),
    "beta_qwen_layer": (1, 8, 128, 12, 128, 2048, 2048, 32768, 64.0, 256, 64, True, 4),
}


@pytest.mark.parametrize("name", list(CASES))
def test_alpha_flush_matches_oracle(name):
    batch, groups, dim, K, B, recent, flush, max_seq, s_h, exact, span, beta, blocks = CASES[name]
    print(f"case {name}", flush=True)
    gpu, ora_c = make_pair(batch, groups, dim, K, B, recent, flush, max_seq, s_h, exact=exact, span=span,
                           beta_novelty=beta, beta_adaptive=beta)
    assert (gpu.B_prime, gpu.L_alloc) == (ora_c.B, ora_c.L)
    mix = Mixture(batch, groups, dim, clusters=K, seed=17)
    for blk in range(blocks):
        feed(gpu, ora_c, mix, blk * recent, recent, with_ends=True)
        torch.cuda.synchronize()
        assert gpu.alpha_count == ora_c.alpha_count, f"block {blk}: alpha_count"
        assert gpu._alpha_spans == ora_c.alpha_spans and gpu._alpha_positions == ora_c.alpha_positions
        bad = compare_state(gpu, ora_c, ALPHA_FIELDS)
        assert not bad, f"block {blk}: " + "; ".join(bad)
    # Coverage: without Beta, archived old exact rows that precede their cluster's
    # p_hi took the delayed-archive re-sort; with Beta some carry groups chose a
    # 2|2 or 3|1 cut.
    if not beta:
        assert ora_c.late_joins > 0
    else:
        cuts = np.concatenate([c for _, log in ora_c.beta_cuts for _, c in log])
        assert (cuts != 1).any()


def _random_selection(rng, P, max_span, full=False):
    """Closed spans up to P - max_span rows and maybe a pending one; ``full``:
    closed spans filling all P rows (the next open candidate then forces
    evictions before the greedy); "long": closed spans and a pending span of
    max_span + 3 rows (a carry that does not split the first segment)."""
    if full == "long":
        spans, n = [], 0
        while n + max_span + 3 + max_span <= P:
            length = int(rng.integers(1, max_span + 1))
            spans.append((length, True))
            n += length
        return spans + [(max_span + 3, False)]
    spans, n = [], 0
    while True:
        length = int(rng.integers(1, max_span + 1))
        if full:
            length = min(length, P - n)
        elif n + length > P - max_span:
            break
        if length == 0:
            break
        spans.append((length, True))
        n += length
    if not full and rng.random() < 0.6:
        spans.append((int(rng.integers(1, max_span)), False))
    return spans


# (beta, seed, P, T, span cap, boundary rate, pool): small rows; a full
# pool (evictions before the greedy); 65-128 list entries (both register
# slots of the one-wave greedy); >128 closed candidates (the one-thread
# greedy); >512 candidates (the bitonic sort); a pending span longer than
# the cap.
SELECT_CASES = [(False, 0, 24, 40, 6, 0.2, False), (True, 1, 24, 40, 6, 0.2, False),
                (True, 2, 24, 40, 6, 0.2, False), (False, 3, 24, 40, 6, 0.2, True),
                (True, 4, 32, 48, 8, 0.25, True), (False, 7, 90, 60, 2, 0.5, True),
                (True, 8, 90, 60, 2, 0.5, False), (False, 5, 64, 600, 8, 0.5, False),
                (True, 6, 64, 1400, 8, 0.6, True), (False, 9, 40, 50, 6, 0.05, "long"),
                (True, 10, 40, 50, 6, 0.3, "long")]


@pytest.mark.parametrize("beta,seed,P,T,ms,rate,full", SELECT_CASES)
def test_device_selection_matches_oracle(beta, seed, P, T, ms, rate, full):
    """logkv_alpha_select (candidates, scores, greedy on the device) against the oracle's
    cut_spans / score_spans / choose_spans: pending spans closed by jumps or carried into
    the first run, caps, single-row spans (zero scores, ties), evictions."""
    import ctypes as C

    from logkv_amd import _lib

    rng = np.random.default_rng(seed)
    Bt, G, D, K = 2, 4, 64, 3
    dev = torch.device("cuda")
    spans = [_random_selection(rng, P, ms, full) for _ in range(Bt)]
    counts = [sum(n for n, _ in s) for s in spans]
    pool_pos = np.zeros((Bt, P), np.int64)
    new_pos = np.zeros((Bt, T), np.int64)
    for b in range(Bt):
        pool_pos[b, :counts[b]] = np.sort(rng.choice(max(60, 3 * P), counts[b], replace=False))
        start = int(pool_pos[b, counts[b] - 1]) + 1 + int(rng.random() < 0.5)
        steps = 1 + (rng.random(T) < 0.1) * rng.integers(1, 3, T)
        steps[0] = 0
        new_pos[b] = start + np.cumsum(steps)
    ends = rng.random((Bt, T)) < rate
    gen = torch.Generator().manual_seed(seed)
    pool_k = (torch.randn(Bt, G, P, D, generator=gen) * 2).to(torch.bfloat16)
    pool_v = torch.randn(Bt, G, P, D, generator=gen).to(torch.bfloat16)
    flush_k = (torch.randn(Bt, G, T, D, generator=gen) * 2).to(torch.bfloat16)
    flush_v = torch.randn(Bt, G, T, D, generator=gen).to(torch.bfloat16)
    single = rng.random(T) < 0.3                                    # constant rows: zero-score ties
    flush_k[:, :, single] = 1.0
    flush_v[:, :, single] = 1.0
    cent = torch.randn(Bt, G, K, D, generator=gen) * 2
    alive = torch.rand(Bt, G, K, generator=gen) < 0.7

    span_len = torch.zeros(Bt, P, dtype=torch.int32)
    span_closed = torch.zeros(Bt, P, dtype=torch.uint8)
    for b, s in enumerate(spans):
        for i, (n, c) in enumerate(s):
            span_len[b, i], span_closed[b, i] = n, int(c)
    t = {k: x.to(dev) for k, x in dict(
        span_len=span_len, span_closed=span_closed, span_count=torch.tensor([len(s) for s in spans], dtype=torch.int32),
        pool_pos=torch.from_numpy(pool_pos), new_pos=torch.from_numpy(new_pos),
        ends=torch.from_numpy(ends.astype(np.uint8)), pk=pool_k, pv=pool_v, fk=flush_k, fv=flush_v,
        cent=cent, alive=alive).items()}
    out = dict(keep=torch.empty(Bt, P, dtype=torch.int32, device=dev),
               archive=torch.empty(Bt, P + T, dtype=torch.int32, device=dev),
               acount=torch.empty(Bt, dtype=torch.int32, device=dev),
               nlen=torch.empty(Bt, P, dtype=torch.int32, device=dev),
               nclosed=torch.empty(Bt, P, dtype=torch.uint8, device=dev),
               ncount=torch.empty(Bt, dtype=torch.int32, device=dev),
               alpha=torch.empty(1, dtype=torch.int32, device=dev),
               scores=torch.empty(Bt * (P + T + 1), dtype=torch.float32, device=dev))
    pk, pv, fk, fv = t["pk"], t["pv"], t["fk"], t["fv"]
    rows = _lib.SpanArgs(_lib.ptr(pk), *pk.stride()[:3], _lib.ptr(pv), *pv.stride()[:3], _lib.ptr(fk),
                         *fk.stride()[:3], _lib.ptr(fv), *fv.stride()[:3], P, None, None, None, 0, G, D, D,
                         _lib.ptr(t["cent"]), _lib.ptr(t["alive"]), K, 1 if beta else 0, None)
    args = _lib.AlphaSelectArgs(
        _lib.ptr(t["span_len"]), _lib.ptr(t["span_closed"]), _lib.ptr(t["span_count"]), _lib.ptr(t["pool_pos"]),
        _lib.ptr(t["new_pos"]), T, _lib.ptr(t["ends"]), T, T, Bt, P, ms, rows, _lib.ptr(out["keep"]),
        _lib.ptr(out["archive"]), _lib.ptr(out["acount"]), _lib.ptr(out["nlen"]), _lib.ptr(out["nclosed"]),
        _lib.ptr(out["ncount"]), _lib.ptr(out["alpha"]), _lib.ptr(out["scores"]))
    ws = torch.empty(int(_lib.lib().logkv_alpha_select_workspace_bytes(C.byref(args))), dtype=torch.uint8,
                     device=dev)
    _lib.check(_lib.lib().logkv_alpha_select(C.byref(args), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev)),
               "select")
    torch.cuda.synchronize()

    width = max(counts)
    keys = np.concatenate((pool_k.float().numpy()[:, :, :width], flush_k.float().numpy()), axis=2)
    vals = np.concatenate((pool_v.float().numpy()[:, :, :width], flush_v.float().numpy()), axis=2)
    old_pos = [pool_pos[b, :counts[b]].tolist() for b in range(Bt)]
    cut = ora.cut_spans(spans, old_pos, new_pos.tolist(), ends.tolist(), width, ms)
    scores = ora.score_spans(keys, vals, cut, beta, cent.numpy(), alive.numpy())
    keep, archive, sp, _ = ora.choose_spans(cut, scores, P)
    n_cand = len(scores)
    np.testing.assert_array_equal(out["scores"].cpu().numpy()[:n_cand], scores)
    remap = lambda idx: [i if i < width else i - width + P for i in idx]  # noqa: E731
    for b in range(Bt):
        got_keep = [x for x in out["keep"][b].tolist() if x >= 0]
        got_arch = out["archive"][b].tolist()[:int(out["acount"][b])]
        assert got_keep == remap(keep[b]), b
        assert got_arch == remap(archive[b]), b
        n = int(out["ncount"][b])
        got_spans = list(zip(out["nlen"][b, :n].tolist(), [bool(x) for x in out["nclosed"][b, :n].tolist()]))
        assert got_spans == sp[b], b
    assert int(out["alpha"][0]) == max(len(k) for k in keep)
