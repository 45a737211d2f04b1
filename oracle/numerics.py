"""Exact float32 building blocks shared by every oracle function.

TEST INFRASTRUCTURE ONLY: nothing in the product package imports this module.

The reference leaves its reduction orders to PyTorch (GEMM, ``segment_reduce``,
``sum``) and Triton (``tl.sum``); none of them is specified. The oracle pins one
order, chosen so that a 64-wide wavefront reproduces it exactly:

* ``dsum``: a reduction over the feature axis. Lane ``l`` of a 64-lane wave
  accumulates ``t[l], t[l+64], t[l+128], ...`` sequentially; the 64 partial
  sums are then folded by a halving tree (``p[i] += p[i+32]``, then ``+16`` ...
  ``+1``), which is also what an xor-butterfly leaves in every lane.
* ``seqsum``: a sequential float32 sum along an axis in index order, used for
  token-order sums (centroids, span means), matching the reference's
  "increasing-token sum order" comment (litgpt/log_kv_cache.py:4323-4325).

Every operation is a single IEEE float32 add, multiply or divide; no fused
multiply-add appears anywhere, matching ``enable_fp_fusion=False`` in every
reference kernel (litgpt/log_kv_updates_triton.py:87, log_kv_route_triton.py:915).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
WAVE = 64


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), as float32.

    Same rule as ``tensor.to(torch.bfloat16)`` on the reference's storage casts
    (litgpt/log_kv_cache.py:1906, log_kv_updates_triton.py:23). NaN stays NaN.
    """
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32).reshape(a.shape)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.float32("nan")
    return out


def dsum(t) -> np.ndarray:
    """Canonical feature-axis sum of the last axis (see module docstring)."""
    t = np.asarray(t, dtype=np.float32)
    d = t.shape[-1]
    chunks = max(1, -(-d // WAVE))
    if d != chunks * WAVE:
        pad = np.zeros(t.shape[:-1] + (chunks * WAVE - d,), dtype=np.float32)
        t = np.concatenate((t, pad), axis=-1)
    s = t[..., 0:WAVE].copy()
    for j in range(1, chunks):
        s = s + t[..., j * WAVE:(j + 1) * WAVE]
    width = WAVE
    while width > 1:
        width //= 2
        s = s[..., :width] + s[..., width:2 * width]
    return s[..., 0]


def seqsum(t, axis: int = 0) -> np.ndarray:
    """Sequential float32 sum along ``axis`` in index order (first term unadded)."""
    t = np.asarray(t, dtype=np.float32)
    t = np.moveaxis(t, axis, 0)
    if t.shape[0] == 0:
        return np.zeros(t.shape[1:], dtype=np.float32)
    return np.add.accumulate(t, axis=0, dtype=np.float32)[-1]


def argmin_first(x, axis: int = -1) -> np.ndarray:
    """Index of the minimum, lowest index on ties (``torch.argmin`` / ``tie_break_left``)."""
    return np.argmin(np.asarray(x), axis=axis)


def argmax_first(x, axis: int = -1) -> np.ndarray:
    return np.argmax(np.asarray(x), axis=axis)
