"""Seeded synthetic workloads shaped like the benchmark configurations.

Keys and values are a Gaussian mixture around K frozen centers ``N(0,1)*4``:
90% of rows are a center plus ``N(0, 0.5^2)`` noise, 10% are far outliers
``N(0,1)*12``. Everything is drawn on the CPU from a ``torch.Generator`` so the
same bytes can be fed to the device and to any CPU checker.
"""

from __future__ import annotations

import torch


class Mixture:
    def __init__(self, batch, groups, dim, clusters=12, seed=0, center_scale=4.0, noise=0.5, outlier=0.1,
                 outlier_scale=12.0):
        self.g = torch.Generator().manual_seed(seed)
        self.batch, self.groups, self.dim = batch, groups, dim
        self.noise, self.outlier, self.outlier_scale = noise, outlier, outlier_scale
        self.centers = torch.randn(batch, groups, clusters, dim, generator=self.g) * center_scale

    def rows(self, n):
        """bf16 rows ``[batch, groups, n, dim]``."""
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
