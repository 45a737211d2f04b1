"""Loading and comparison helpers for the golden fixtures written by tests/golden/make_fixtures.py
from the reference's CPU Torch path. The bar: integer fields, decisions and indices bit for bit;
merged keys / values and masses within 1e-5 relative or one bf16 ulp."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

INT_FIELDS = ("level_count", "level_p_lo", "level_p_hi", "level_sum_wp", "level_order", "pad_mask", "alive",
              "n_total", "p_hi_c", "level0_phase")


def load(name: str):
    return np.load(GOLDEN / name, allow_pickle=False)


def config(data) -> dict:
    return json.loads(str(data["config"]))


def from_bits(x: np.ndarray) -> np.ndarray:
    return (np.asarray(x, np.uint16).astype(np.uint32) << 16).view(np.float32)


def tables(data):
    """The RoPE tables a fixture was written with, as torch tensors (bf16 tables are stored as bits)."""
    import torch

    out = []
    for name in ("cos", "sin"):
        x = data[name]
        out.append(torch.from_numpy(from_bits(x)).to(torch.bfloat16) if x.dtype == np.uint16
                   else torch.from_numpy(np.asarray(x, np.float32)))
    return tuple(out)


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    mag = np.abs(np.asarray(x, np.float64))
    return np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-38))) - 7), 2.0 ** -133)


def compare_state(get, data, step: int, alpha: bool) -> list[str]:
    """Mismatches between a cache state (``get(name)`` -> numpy array) and the fixture after ``step``."""
    bad = []
    for f in INT_FIELDS:
        a = np.asarray(get(f)).astype(np.int64)
        b = data[f"{f}_{step}"].astype(np.int64)
        if a.shape != b.shape or not np.array_equal(a, b):
            n = int((a != b).sum()) if a.shape == b.shape else -1
            bad.append(f"{f}: {n} mismatches")
    for f in ("level_k", "level_v"):
        a = np.asarray(get(f), np.float64)
        b = from_bits(data[f"{f}_{step}"]).astype(np.float64)
        if np.any(np.abs(a - b) > bf16_ulp(b)):
            bad.append(f"{f}: beyond one bf16 ulp")
    for f, tol in (("level_w", 1e-5), ("centroid", 1e-5), ("n_eff", 1e-5)):
        a = np.asarray(get(f), np.float64)
        b = data[f"{f}_{step}"].astype(np.float64)
        if np.any(np.abs(a - b) > tol * np.maximum(np.abs(b), 1e-30)):
            bad.append(f"{f}: beyond {tol} relative (max {np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-30)):.2e})")
    if alpha:
        for f in ("alpha_pos", "alpha_valid"):
            if not np.array_equal(np.asarray(get(f)).astype(np.int64), data[f"{f}_{step}"].astype(np.int64)):
                bad.append(f"{f}: mismatch")
        for f in ("alpha_k_raw", "alpha_v"):
            if not np.array_equal(np.asarray(get(f), np.float32), from_bits(data[f"{f}_{step}"])):
                bad.append(f"{f}: mismatch")
        spans = data[f"alpha_spans_{step}"]
        got = get("alpha_spans")
        want = [[(int(n), bool(c)) for n, c in row if n >= 0] for row in spans]
        if got != want:
            bad.append("alpha spans differ")
    return bad
