"""The headline flush at its benchmarked geometry (28 Qwen3-1.7B-shaped layers stacked as the batch
rows of one cache: 8 groups x 128 features, 2048-row flushes, K = 12, B = 128 -> B' = 125, L = 7,
Alpha exact pool 256 / span cap 64, Beta novelty and 4 -> 2 split), the cache bench.py times, checked
through properties that hold at any size: every flushed token's mass is conserved (per lane, the
ladder's masses plus the lane's valid exact-pool rows equal the tokens flushed, as the oracle keeps
them), masses are whole non-negative numbers, payloads finite and the exact pool within its 256 rows. The oracle itself finishes this workload too slowly to compare state here; the same
kernels are compared with it bit for bit at smaller geometry and on single Qwen-shaped layers."""

import importlib.util
from pathlib import Path

import pytest
import torch

from workloads import rope_tables

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_geometry", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_benched_flush_conserves_mass_over_16_flushes():
    bench = _bench()
    layers, flushes = 28, 16
    print(f"case benched geometry: {layers} layers x {flushes} flushes of {bench.F} rows", flush=True)
    dev = torch.device("cuda", 0)
    cos, sin = rope_tables(bench.N, bench.D)
    cache = bench.new_flush_cache(torch, dev, layers, cos, sin)
    assert (cache.B_prime, cache.max_levels) == (125, 7)
    gen = torch.Generator(device=dev).manual_seed(99)
    shape = (layers, bench.G, bench.F, bench.D)
    centers = torch.randn(layers, bench.G, bench.K, bench.D, generator=gen, device=dev) * 4

    def rows():
        label = torch.randint(0, bench.K, shape[:3], generator=gen, device=dev)
        x = torch.gather(centers, 2, label[..., None].expand(*shape)) + torch.randn(shape, generator=gen, device=dev) * 0.5
        far = torch.rand(shape[:3], generator=gen, device=dev) < 0.1
        return torch.where(far[..., None], torch.randn(shape, generator=gen, device=dev) * 12, x).to(torch.bfloat16)

    for j in range(flushes):
        pos = torch.arange(j * bench.F, (j + 1) * bench.F, device=dev).unsqueeze(0).expand(layers, -1).contiguous()
        ends = torch.tensor(bench.span_ends_for(j), dtype=torch.uint8, device=dev).expand(layers, -1).contiguous()
        cache.route_and_flush_batch(rows(), rows(), pos, span_ends=ends)
        w = cache.level_w.double()
        lane_mass = w.reshape(layers, bench.G, -1).sum(-1)
        pool = cache.alpha_valid.reshape(layers, -1).sum(-1, dtype=torch.float64)
        assert pool.max().item() <= bench.EXACT
        want = float((j + 1) * bench.F)
        total = lane_mass + pool[:, None]
        assert torch.equal(total, torch.full_like(total, want)), \
            f"flush {j}: lane masses {total.min().item()}..{total.max().item()}, want {want}"
        assert torch.equal(w, w.round()) and bool((w >= 0).all()), f"flush {j}: masses"
    for name in ("level_k", "level_v", "alpha_k_raw", "alpha_v"):
        assert bool(torch.isfinite(getattr(cache, name).float()).all()), name
    assert int(cache.alpha_valid.sum()) > 0 and int((cache.level_w > 0).sum()) > 0
