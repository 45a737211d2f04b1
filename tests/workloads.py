"""Seeded synthetic workloads shaped like the benchmark configurations.

Keys and values are a Gaussian mixture around K frozen centers ``N(0,1)*4``:
90% of rows are a center plus ``N(0, 0.5^2)`` noise, 10% are far outliers
``N(0,1)*12``. Everything is drawn on the CPU from a ``torch.Generator`` so the
same bytes can be fed to the device and to the oracle.
"""

from __future__ import annotations

import torch


class Mixture:
    """``drift_every``: the centers are redrawn each time that many rows have
    been drawn (counted over every ``rows`` call, checked at call boundaries)."""

    def __init__(self, batch, groups, dim, clusters=12, seed=0, center_scale=4.0, noise=0.5, outlier=0.1,
                 outlier_scale=12.0, drift_every=0):
        self.g = torch.Generator().manual_seed(seed)
        self.batch, self.groups, self.dim = batch, groups, dim
        self.noise, self.outlier, self.outlier_scale = noise, outlier, outlier_scale
        self.center_scale, self.drift_every, self.drawn, self.epoch = center_scale, int(drift_every), 0, 0
        self.centers = torch.randn(batch, groups, clusters, dim, generator=self.g) * center_scale

    def rows(self, n):
        """bf16 rows ``[batch, groups, n, dim]``."""
        if self.drift_every and self.drawn // self.drift_every != self.epoch:
            self.epoch = self.drawn // self.drift_every
            self.centers = torch.randn(self.centers.shape, generator=self.g) * self.center_scale
        self.drawn += n
        k = self.centers.size(2)
        label = torch.randint(0, k, (self.batch, self.groups, n), generator=self.g)
        x = torch.gather(self.centers, 2, label[..., None].expand(-1, -1, -1, self.dim))
        x = x + torch.randn(self.batch, self.groups, n, self.dim, generator=self.g) * self.noise
        far = torch.rand(self.batch, self.groups, n, generator=self.g) < self.outlier
        x = torch.where(far[..., None], torch.randn(x.shape, generator=self.g) * self.outlier_scale, x)
        return x.to(torch.bfloat16)

    def span_ends(self, start, n, stride=32):
        """Synthetic natural boundaries: row ``p`` ends a span when ``(p + 7*b) % stride == 0``."""
        return [[(p + 7 * b) % stride == 0 for p in range(start, start + n)] for b in range(self.batch)]


def rope_tables(n_positions, n_elem, base=10000.0, dtype=torch.float32):
    """LitGPT-style rotate-half RoPE tables ``[n_positions, n_elem]``."""
    theta = 1.0 / (base ** (torch.arange(0, n_elem, 2, dtype=torch.float32) / n_elem))
    idx = torch.outer(torch.arange(n_positions, dtype=torch.float32), theta)
    idx = torch.cat((idx, idx), dim=-1)
    return torch.cos(idx).to(dtype), torch.sin(idx).to(dtype)


def fenwick_counts(tokens, chunk, B, L):
    """Per-level slot counts of one ladder after appending ``tokens`` rows in
    ``chunk``-row batches: fill free slots, pair-merge the overflow into carries
    for the next level, keep the survivors; a saturated top level stays full
    (the count rule of litgpt/log_kv_cache.py:1815-1929)."""
    counts = [0] * L
    left = int(tokens)
    while left > 0:
        m = min(chunk, left)
        left -= m
        for ell in range(L):
            take = min(B - counts[ell], m)
            mr = m - take
            if mr == 0:
                counts[ell] += take
                break
            if ell == L - 1:
                counts[ell] = B
                break
            n_carry = (mr + 1) // 2
            counts[ell] = B + mr - 2 * n_carry
            m = n_carry
    return counts


@torch.no_grad()
def fill_readout_state(cache, seed=0, fill=0.75, recent=None, exact=None, mass=(1.0, 64.0), archived=None,
                       flushes=15):
    """Synthetic compressed-cache state for readout: random bf16 keys / values, masses ~ U(mass),
    position sums inside the cache's span, a full recent window and exact pool unless given.

    Slot counts: with ``archived`` tokens per lane, each cluster holds the ladder
    occupancy of its share (a random split over the clusters) appended over
    ``flushes`` flushes; otherwise about ``fill`` of each level, at random."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    Bt, G, K, L, S = cache.level_w.shape
    dk, dv = cache.k_dim, cache.v_dim
    if archived is None:
        counts = torch.binomial(torch.full((Bt, G, K, L), float(S)), torch.full((Bt, G, K, L), fill), generator=g)
    else:
        share = torch.rand(Bt, G, K, generator=g) + 0.5
        share = (share / share.sum(-1, keepdim=True) * archived).long()
        counts = torch.tensor([[[fenwick_counts(int(t), max(1, int(t) // flushes), S, L) for t in lane]
                                for lane in row] for row in share.tolist()])
    counts = counts.to(torch.int16)
    occupied = torch.arange(S).view(1, 1, 1, 1, S) < counts.unsqueeze(-1)
    w = torch.empty(Bt, G, K, L, S).uniform_(*mass, generator=g).floor() * occupied
    horizon = max(cache.max_seq_length - cache.recent_capacity, 1)
    anchor = torch.randint(0, horizon, (Bt, G, K, L, S), generator=g)
    cache.level_count.copy_(counts)
    cache.level_w.copy_(w)
    cache.level_sum_wp.copy_((w.long() * anchor) * occupied)
    cache.level_k.copy_((torch.randn(cache.level_k.shape, generator=g) * occupied.unsqueeze(-1)).to(torch.bfloat16))
    cache.level_v.copy_((torch.randn(cache.level_v.shape, generator=g) * occupied.unsqueeze(-1)).to(torch.bfloat16))
    n_recent = cache.recent_size if recent is None else recent
    cache.recent_k[:, :, :n_recent].copy_(torch.randn(Bt, G, n_recent, cache.recent_k.size(-1), generator=g))
    cache.recent_v[:, :, :n_recent].copy_(torch.randn(Bt, G, n_recent, dv, generator=g))
    cache.recent_count = n_recent
    if cache.alpha_exact_tokens:
        P = cache.alpha_exact_tokens
        n_exact = P if exact is None else exact
        cache.alpha_k_raw[:, :, :n_exact].copy_(torch.randn(Bt, G, n_exact, dk, generator=g))
        cache.alpha_v[:, :, :n_exact].copy_(torch.randn(Bt, G, n_exact, dv, generator=g))
        cache.alpha_pos[:, :n_exact].copy_(torch.randint(0, horizon, (Bt, n_exact), generator=g))
        cache.alpha_valid[:, :n_exact].copy_(torch.rand(Bt, n_exact, generator=g) < 0.95)
        cache.alpha_count = n_exact
    cache.token_count = horizon + n_recent
    cache._mid_decode_state = None
