"""Device flush (route + commit) against the oracle, bit for bit."""

import numpy as np
import pytest
import torch

from harness import compare_state, feed, make_pair, to_np
from workloads import Mixture

pytestmark = pytest.mark.gpu

CASES = {
    # name: (batch, groups, dim, K, B, recent, flush, max_seq, s_h, blocks)
    "small": (2, 2, 64, 4, 8, 32, 32, 1024, 16.0, 6),
    "mixture": (1, 4, 128, 12, 16, 128, 128, 4096, 64.0, 6),
    "qwen_layer": (1, 8, 128, 12, 128, 2048, 2048, 32768, 64.0, 3),
}


@pytest.mark.parametrize("name", list(CASES))
def test_flush_matches_oracle(name):
    batch, groups, dim, K, B, recent, flush, max_seq, s_h, blocks = CASES[name]
    print(f"case {name}", flush=True)
    gpu, ora = make_pair(batch, groups, dim, K, B, recent, flush, max_seq, s_h)
    mix = Mixture(batch, groups, dim, clusters=K, seed=7)
    for blk in range(blocks):
        feed(gpu, ora, mix, blk * recent, recent)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"block {blk}: " + "; ".join(bad)
    assert int(to_np(gpu.alive).sum()) > 0


def test_parallel_centroid_backend_matches_oracle():
    """semantic_centroid_backend="parallel": centers sum their new keys in 32-row tiles (each by a
    halving tree); the device equals an oracle cache with that order bit for bit, the sequential
    device run differs from it in some center's last bits (rows scaled by powers of two from 2^-6
    to 2^6, so float32 sums round and the order shows), and switching the backend on a live cache
    takes effect at the next flush."""
    print("case parallel centroid", flush=True)
    args = (1, 4, 128, 4, 16, 256, 256, 4096, 64.0)
    gpu, ora = make_pair(*args, centroid_backend="parallel")
    seq, _ = make_pair(*args)
    mix = Mixture(1, 4, 128, clusters=4, seed=12)
    g = torch.Generator().manual_seed(12)

    def block(start):
        scale = torch.exp2(torch.randint(-6, 7, (1, 1, 256, 1), generator=g).float())
        k_raw, v, k = ((mix.rows(256).float() * scale).to(torch.bfloat16) for _ in range(3))
        pos = torch.arange(start, start + 256).unsqueeze(0)
        return k_raw, v, k, pos

    def commit(caches, oracle, rows):
        k_raw, v, k, pos = rows
        for c in caches:
            c.add_recent(k.cuda(), v.cuda(), k_raw=k_raw.cuda(), input_pos=pos.cuda())
        oracle.add_recent(k.float().numpy(), v.float().numpy(), k_raw.float().numpy(), pos.numpy(), None)
        torch.cuda.synchronize()

    for blk in range(5):
        commit((gpu, seq), ora, block(blk * 256))
        bad = compare_state(gpu, ora)
        assert not bad, f"block {blk}: " + "; ".join(bad)
    assert not np.array_equal(to_np(gpu.centroid), to_np(seq.centroid))
    gpu.semantic_centroid_backend = "sequential"
    ora.centroid_tile = 1
    commit((gpu,), ora, block(5 * 256))
    bad = compare_state(gpu, ora)
    assert not bad, "after switching to sequential: " + "; ".join(bad)


@pytest.mark.parametrize("dim,flush,max_seq,sizes", [
    (64, 64, 64, (1, 40, 64, 64, 64, 64)),
    # 256-wide rows (two 8-byte units per lane in the fold) and, with three
    # levels, top folds of 70 and more rows (several weight batches)
    (256, 512, 8, (1, 300, 512, 512)),
])
def test_top_level_fold_and_skewed_cluster(dim, flush, max_seq, sizes):
    """One hot cluster saturates every level, so the top level folds."""
    batch, groups, K, B = 1, 2, 4, 4
    gpu, ora = make_pair(batch, groups, dim, K, B, recent=flush, flush=flush, max_seq=max_seq, s_h=1e9)
    assert gpu.L_alloc == ora.L
    mix = Mixture(batch, groups, dim, clusters=1, seed=3, outlier=0.0)
    dev = gpu.level_k.device
    start = 0
    for n in sizes:
        k, v = mix.rows(n), mix.rows(n)
        pos = torch.arange(start, start + n).unsqueeze(0).expand(batch, -1).contiguous()
        gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev))
        ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy())
        start += n
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"after {start} rows: " + "; ".join(bad)
    counts = to_np(gpu.level_count)
    assert (counts[..., -1] == B).any(), "top level never saturated"


def test_attach_decisions_with_seeds_and_ragged_rows():
    import ctypes as C

    from logkv_amd._lib import check, lib, ptr, stream_of
    from oracle import route

    batch, groups, dim, K = 2, 3, 128, 8
    gpu, ora = make_pair(batch, groups, dim, K, 16, recent=64, flush=64, max_seq=4096, s_h=40.0)
    mix = Mixture(batch, groups, dim, clusters=K, seed=11)
    dev = gpu.level_k.device
    # Warm up: one flush opens clusters; then kill some so seeds are needed again.
    k, v = mix.rows(64), mix.rows(64)
    pos = torch.arange(0, 64).unsqueeze(0).expand(batch, -1).contiguous()
    gpu.route_and_flush_batch(k.to(dev), v.to(dev), pos.to(dev))
    ora.flush_rows(k.float().numpy(), v.float().numpy(), pos.numpy())
    gpu.alive[0, 1, 2:5] = False
    ora.alive[0, 1, 2:5] = False
    T = 50
    k = mix.rows(T)
    perm = torch.stack([torch.randperm(T, generator=torch.Generator().manual_seed(b)) for b in range(batch)])
    pos = (100 + perm).contiguous()
    counts = torch.tensor([T, 37], dtype=torch.int32)
    view = gpu._ladder_view()
    # The view holds raw pointers: keep the device tensors alive until the kernels ran.
    k_dev, pos_dev, counts_dev = k.to(dev), pos.to(dev), counts.to(dev)
    rows = gpu._rows_view(k_dev, k_dev, pos_dev, counts_dev)
    ws = gpu._workspace_for(view, T)
    assign = torch.empty(batch, groups, T, dtype=torch.int8, device=dev)
    order = torch.empty(batch, T, dtype=torch.int32, device=dev)
    rc = lib().logkv_attach_assign(C.byref(view), C.byref(rows), C.byref(gpu._params), ptr(ws), ws.numel(),
                                   ptr(assign), ptr(order), stream_of(dev))
    check(rc, "attach")
    torch.cuda.synchronize()
    want, want_order = route.attach_assign(k.float().numpy(), pos.numpy(), counts.numpy(), ora.centroid, ora.alive,
                                           ora.p_hi_c, ora.s_h, ora.eta, ora.g0, ora.lam)
    for b in range(batch):
        n = int(counts[b])
        np.testing.assert_array_equal(to_np(order)[b, :n], want_order[b, :n])
        np.testing.assert_array_equal(to_np(assign)[b, :, :n], want[b, :, :n])
        assert (to_np(assign)[b, :, n:] == -1).all()


def test_beta_carries_keep_signed_zero_features():
    """Beta carries on 128-feature rows (four groups to a wave) whose feature
    columns are all -0, all +0, or mixed in sign across rows: the output
    means' zero signs follow the reference's term-by-term row sums, so the
    stored ladder rows are compared as bf16 bit patterns, not values."""
    print("case Beta carries, signed-zero columns", flush=True)
    gpu, ora = make_pair(1, 2, 128, 4, 8, 64, 64, 2048, 16.0, exact=16, span=4, beta_adaptive=True)
    mix = Mixture(1, 2, 128, clusters=4, seed=41)
    dev = gpu.level_k.device
    neg = torch.tensor(-0.0, dtype=torch.bfloat16)
    for blk in range(12):
        n = 64
        k_raw, v, k = mix.rows(n), mix.rows(n), mix.rows(n)
        for t in (k_raw, v, k):
            t[..., 0:8] = neg                     # every row -0
            t[..., 8:16] = 0.0                    # every row +0
            sign = torch.arange(n) % 3 == 0       # -0 on every third row, +0 elsewhere
            t[..., :, 16:24] = torch.where(sign[:, None], neg, torch.zeros((), dtype=torch.bfloat16))
        pos = torch.arange(blk * n, (blk + 1) * n).unsqueeze(0).contiguous()
        ends = mix.span_ends(blk * n, n)
        gpu.add_recent(k.to(dev), v.to(dev), k_raw=k_raw.to(dev), input_pos=pos.to(dev), span_ends=ends)
        ora.add_recent(k.float().numpy(), v.float().numpy(), k_raw.float().numpy(), pos.numpy(), ends)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"block {blk}: " + "; ".join(bad)
        for f in ("level_k", "level_v"):
            bits = getattr(gpu, f).view(torch.int16).cpu().numpy()
            ref = (np.asarray(getattr(ora, f), np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.int16)
            live = np.arange(bits.shape[-2])[None, None, None, None, :] < np.asarray(ora.level_count)[..., None]
            assert np.array_equal(np.where(live[..., None], bits, 0), np.where(live[..., None], ref, 0)), f"{f} bits"
    assert int(np.asarray(ora.level_count)[..., 1:].sum()) > 0, "no carry reached level 1"


def test_beta_carries_lattice_ties():
    """Beta carries whose groups tie: every token of a cluster is one of three lattice vectors (exact
    bf16), so 4-row groups often repeat rows (A A B B, A B A B, A A A A, ...), making cut costs tie
    exactly or up to the canonical evaluation's rounding (cuts 1 and 3 of A B A B are equal in exact
    arithmetic, their float costs differ only in rounding). The screened decision must defer every
    such group to the canonical evaluation: the ladders stay bit-identical to the oracle's."""
    print("case Beta carries, lattice ties", flush=True)
    gpu, ora = make_pair(1, 2, 128, 4, 8, 64, 64, 4096, 64.0, exact=16, span=4, beta_adaptive=True)
    g = torch.Generator().manual_seed(12)
    centers = (torch.randint(0, 2, (2, 4, 128), generator=g) * 2 - 1).float() * 2.0
    variants = torch.stack([torch.zeros(2, 128), (torch.randint(0, 2, (2, 128), generator=g) * 2 - 1) * 0.5,
                            (torch.randint(0, 3, (2, 128), generator=g) - 1) * 0.25], 1)   # [G, 3, D]
    dev = gpu.level_k.device
    for blk in range(24):
        n = 64
        rows = []
        for _ in range(3):
            c = torch.randint(0, 4, (2, n), generator=g)
            v = torch.randint(0, 3, (2, n), generator=g)
            x = torch.stack([centers[gi, c[gi]] + variants[gi, v[gi]] for gi in range(2)])
            rows.append(x.unsqueeze(0).to(torch.bfloat16))
        k_raw, v, k = rows
        pos = torch.arange(blk * n, (blk + 1) * n).unsqueeze(0).contiguous()
        ends = [[(p % 5) == 4 for p in range(blk * n, (blk + 1) * n)]]
        gpu.add_recent(k.to(dev), v.to(dev), k_raw=k_raw.to(dev), input_pos=pos.to(dev), span_ends=ends)
        ora.add_recent(k.float().numpy(), v.float().numpy(), k_raw.float().numpy(), pos.numpy(), ends)
        torch.cuda.synchronize()
        bad = compare_state(gpu, ora)
        assert not bad, f"block {blk}: " + "; ".join(bad)
    assert int(np.asarray(ora.level_count)[..., 2:].sum()) > 0, "no carry reached level 2"
    cuts = [int(x) for _, per in ora.beta_cuts for _, lvl in per for x in np.asarray(lvl).reshape(-1)]
    assert len(set(cuts)) >= 2, "the lattice produced a single cut only"


def test_attach_screen_ties_and_radius_edges():
    """Steady-state attach decisions (every cluster alive: the screened path) on rows built to sit on
    decision boundaries: midpoints of two lattice centers (equal costs, first cluster wins), rows at
    exactly the radius from their center and just past it, far rows equidistant from two centers
    (nearest-cluster ties), mixed with ordinary rows; every decision equals the oracle's."""
    import ctypes as C

    from logkv_amd._lib import check, lib, ptr, stream_of
    from oracle import route

    batch, groups, dim, K, T = 1, 2, 128, 8, 256
    s_h = 4.0
    gpu, ora = make_pair(batch, groups, dim, K, 16, recent=T, flush=T, max_seq=4096, s_h=s_h)
    g = torch.Generator().manual_seed(31)
    centers = (torch.randint(0, 2, (groups, K, dim), generator=g) * 2 - 1).float()       # +-1 lattice
    for dst in (gpu, ora):
        cen = centers.unsqueeze(0)
        if dst is gpu:
            dst.centroid.copy_(cen.to(dst.centroid.device))
            dst.alive.fill_(True)
            dst.p_hi_c.fill_(10)
            dst.n_total.fill_(5)
        else:
            dst.centroid[...] = cen.numpy()
            dst.alive[...] = True
            dst.p_hi_c[...] = 10
            dst.n_total[...] = 5
    rows = []
    for gi in range(groups):
        c = centers[gi]
        r = []
        for a in range(K):
            b = (a + 1 + gi) % K
            r.append((c[a] + c[b]) / 2)                           # equidistant from a and b
            e = torch.zeros(dim)
            e[a] = 2.0
            r.append(c[a] + e * torch.sign(c[a, a]))              # |x - c_a|^2 = 4 = lambda s_h exactly
            e[a] = 2.0078125                                      # just past the radius
            r.append(c[a] + e * torch.sign(c[a, a]))
            r.append((c[a] + c[b]) / 2 + 6.0 * torch.sign((c[a] + c[b]) / 2 + 0.5))   # far, equidistant
        while len(r) < T:
            a = int(torch.randint(0, K, (1,), generator=g))
            r.append(c[a] + torch.randn(dim, generator=g) * 0.3)
        rows.append(torch.stack(r[:T]))
    k = torch.stack(rows).unsqueeze(0).to(torch.bfloat16)
    pos = (100 + torch.arange(T)).unsqueeze(0).contiguous()
    dev = gpu.level_k.device
    view = gpu._ladder_view()
    k_dev, pos_dev = k.to(dev), pos.to(dev)
    rv = gpu._rows_view(k_dev, k_dev, pos_dev)
    ws = gpu._workspace_for(view, T)
    assign = torch.empty(batch, groups, T, dtype=torch.int8, device=dev)
    order = torch.empty(batch, T, dtype=torch.int32, device=dev)
    check(lib().logkv_attach_assign(C.byref(view), C.byref(rv), C.byref(gpu._params), ptr(ws), ws.numel(),
                                    ptr(assign), ptr(order), stream_of(dev)), "attach")
    torch.cuda.synchronize()
    want, _ = route.attach_assign(k.float().numpy(), pos.numpy(), np.array([T]), ora.centroid, ora.alive, ora.p_hi_c,
                                  ora.s_h, ora.eta, ora.g0, ora.lam)
    np.testing.assert_array_equal(to_np(assign), want)
    got = to_np(assign)
    assert (got[0, :, 0:4 * K:4] != -1).all()                     # midpoints decided (tie: the first)


def test_attach_screen_extreme_magnitudes():
    """Attach decisions on 128-feature rows where the matrix-core screen cannot decide: rows scaled
    by 2^31 (sums of squares far above 2^60), rows of magnitude 1e-30 (sums of squares underflow, so
    every cluster stays a candidate), and a lane with one center scaled by 2^40 (the whole lane takes
    the canonical trees); ordinary rows between them. Every decision equals the oracle's."""
    import ctypes as C

    from logkv_amd._lib import check, lib, ptr, stream_of
    from oracle import route

    print("case attach screen, extreme magnitudes", flush=True)
    batch, groups, dim, K, T = 1, 2, 128, 8, 192
    gpu, ora = make_pair(batch, groups, dim, K, 16, recent=T, flush=T, max_seq=4096, s_h=8.0)
    g = torch.Generator().manual_seed(53)
    centers = (torch.randint(0, 2, (groups, K, dim), generator=g) * 2 - 1).float()
    centers = centers + torch.randn(groups, K, dim, generator=g) * 0.25
    centers[1, 3] *= 2.0 ** 40
    for dst in (gpu, ora):
        if dst is gpu:
            dst.centroid.copy_(centers.unsqueeze(0).to(dst.centroid.device))
            dst.alive.fill_(True)
            dst.p_hi_c.fill_(10)
            dst.n_total.fill_(5)
        else:
            dst.centroid[...] = centers.unsqueeze(0).numpy()
            dst.alive[...] = True
            dst.p_hi_c[...] = 10
            dst.n_total[...] = 5
    a = torch.randint(0, K, (groups, T), generator=g)
    x = torch.stack([centers[gi, a[gi]] for gi in range(groups)]) + torch.randn(groups, T, dim, generator=g) * 0.4
    x[1, a[1] == 3] = torch.randn(int((a[1] == 3).sum()), dim, generator=g)
    kind = torch.arange(T) % 4
    x[:, kind == 1] *= 2.0 ** 31
    x[:, kind == 2] *= 1e-30
    k = x.unsqueeze(0).to(torch.bfloat16)
    pos = (100 + torch.arange(T)).unsqueeze(0).contiguous()
    dev = gpu.level_k.device
    view = gpu._ladder_view()
    k_dev, pos_dev = k.to(dev), pos.to(dev)
    rv = gpu._rows_view(k_dev, k_dev, pos_dev)
    ws = gpu._workspace_for(view, T)
    assign = torch.empty(batch, groups, T, dtype=torch.int8, device=dev)
    order = torch.empty(batch, T, dtype=torch.int32, device=dev)
    check(lib().logkv_attach_assign(C.byref(view), C.byref(rv), C.byref(gpu._params), ptr(ws), ws.numel(),
                                    ptr(assign), ptr(order), stream_of(dev)), "attach")
    torch.cuda.synchronize()
    want, _ = route.attach_assign(k.float().numpy(), pos.numpy(), np.array([T]), ora.centroid, ora.alive, ora.p_hi_c,
                                  ora.s_h, ora.eta, ora.g0, ora.lam)
    np.testing.assert_array_equal(to_np(assign), want)
    assert len(set(to_np(assign)[0, 0].tolist())) > 2
