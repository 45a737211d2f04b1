"""Beta compaction: four ordered entries become two contiguous weighted-mean entries.

Call surface of the reference module (litgpt/beta_log_kv.py): ``make_layout``,
``select_cuts``, ``apply_cuts``, ``merge_blocks``. A *block* is the 13-field
entry tuple of the reference (``k, v, w``, five second-order fields that must be
``None``, ``p_lo, p_hi, sum_wp, order, pad``) with one row per entry; the lanes
of a block are consecutive runs of even length. Cut choice and merges run in the
HIP library (``logkv_beta_merge``) with the arithmetic of the ladder's own Beta
carries; the layout is host data, as in the reference.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib

_N_FIELDS = 13
_META = (8, 9, 10, 11)   # p_lo, p_hi, sum_wp, order


def make_layout(lengths, device):
    """Rows ``(input start, width, output start)`` of every group, int64 ``[groups, 3]`` on ``device``.

    Each lane of even length ``n`` contributes groups at offsets 0, 4, 8, ... of
    its run, of width ``min(4, n - offset)`` (so 4, or 2 for a tail); a group's
    outputs start at half its input start (litgpt/beta_log_kv.py:7-18).
    """
    lengths = [int(n) for n in np.asarray(lengths, dtype=np.int64).reshape(-1)]
    if any(n < 0 or n % 2 for n in lengths):
        raise ValueError("Beta compaction requires even nonnegative lane lengths")
    table = []
    base = 0
    for n in lengths:
        table.extend((base + off, min(4, n - off), (base + off) // 2) for off in range(0, n, 4))
        base += n
    return torch.tensor(table, dtype=torch.int64).reshape(-1, 3).to(device)


def _check_block(block):
    if len(block) != _N_FIELDS:
        raise ValueError(f"a Beta block has {_N_FIELDS} entry fields")
    if any(block[f] is not None for f in range(3, 8)):
        raise ValueError("Beta compaction only supports first-order entries")
    k, v, w = block[0], block[1], block[2]
    if k is None or v is None or w is None:
        raise ValueError("Beta compaction needs the K, V and mass fields")
    n = k.size(0)
    if k.dim() != 2 or v.dim() != 2 or w.dim() != 1 or v.size(0) != n or w.size(0) != n:
        raise ValueError("Beta block fields must be [rows, d] payloads and [rows] masses")
    for f, x in enumerate(block):
        if x is None:
            continue
        _lib.require_device(x, "Beta block field")
        if x.device != k.device:
            raise ValueError("Beta block fields must share one device")
        if f >= 8 and (x.dim() != 1 or x.size(0) != n):
            raise ValueError("Beta block metadata must be [rows]")
    for x in (k, v, w):
        if not x.dtype.is_floating_point:
            raise ValueError("Beta payloads and masses must be floating point")
    for f in _META:
        if block[f] is not None and block[f].dtype != torch.int64:
            raise ValueError("Beta anchors and order must be int64")
    if block[12] is not None and block[12].dtype != torch.bool:
        raise ValueError("Beta padding flags must be bool")


def _contig(x):
    return None if x is None else x.contiguous()


def _payload(x):
    """K / V rows as the kernel reads them: bfloat16 or float32 with contiguous features; other
    floating dtypes are upcast to float32 first, as the reference's ``.float()`` reads them
    (exact for float16)."""
    if x.dtype in (torch.bfloat16, torch.float32):
        return x if x.stride(-1) == 1 else x.contiguous()
    return x.float().contiguous()


def _run(block, layout, cuts, apply, outputs):
    k, v, w = _payload(block[0]), _payload(block[1]), block[2].float().contiguous()
    if layout.dtype != torch.int64 or layout.dim() != 2 or layout.size(1) != 3 or layout.device != k.device:
        raise ValueError("Beta layout must be int64 [groups, 3] on the block's device")
    layout = layout.contiguous()
    meta = [_contig(block[f]) for f in _META]
    pad = _contig(block[12])
    status = torch.zeros(1, dtype=torch.int32, device=k.device)
    ptr = _lib.ptr
    args = _lib.BetaArgs(
        ptr(k), k.stride(0), int(k.dtype == torch.float32), ptr(v), v.stride(0), int(v.dtype == torch.float32),
        ptr(w), *(ptr(m) for m in meta), None if pad is None else pad.view(torch.uint8).data_ptr(),
        k.size(0), k.size(1), v.size(1), ptr(layout), layout.size(0), ptr(cuts), int(apply))
    if outputs is not None:
        out = outputs
        args.out_k, args.out_v = ptr(out[0]), ptr(out[1])
        # Side masses are summed in float32; a block of another mass dtype gets them cast below.
        out_w = out[2] if out[2].dtype == torch.float32 else torch.empty_like(out[2], dtype=torch.float32)
        args.out_w = ptr(out_w)
        args.out_p_lo, args.out_p_hi, args.out_sum_wp, args.out_order = (ptr(out[f]) for f in _META)
        args.out_pad = None if out[12] is None else out[12].view(torch.uint8).data_ptr()
    _lib.check(_lib.lib().logkv_beta_merge(C.byref(args), ptr(status), _lib.stream_of(k.device)), "logkv_beta_merge")
    if int(status.item()):
        raise ValueError("Beta layout or recorded cuts out of range for this block")
    if outputs is not None and out_w is not outputs[2]:
        outputs[2].copy_(out_w)


def select_cuts(block, layout):
    """One byte per group: the cut in (2, 1, 3) of least normalised distortion (ties prefer 2|2);
    a two-entry tail has the sentinel 1 (litgpt/beta_log_kv.py:29-46)."""
    _check_block(block)
    cuts = torch.empty(layout.size(0), dtype=torch.uint8, device=block[0].device)
    if layout.size(0):
        _run(block, layout, cuts, apply=False, outputs=None)
    return cuts


def _outputs_like(block):
    n = block[0].size(0) // 2
    return tuple(None if x is None else torch.empty((n, *x.shape[1:]), device=x.device,
                                                    dtype=torch.float32 if i < 2 else x.dtype)
                 for i, x in enumerate(block))


def apply_cuts(block, layout, cuts):
    """Apply recorded cuts without evaluating candidate costs (litgpt/beta_log_kv.py:49-92): per group the
    side masses, float32 weighted-mean K / V, anchors over rows of positive mass, summed w*p, smallest
    order and the AND of the padding flags."""
    _check_block(block)
    if cuts.dtype != torch.uint8 or cuts.shape != (layout.size(0),) or cuts.device != block[0].device:
        raise ValueError("recorded Beta cuts do not match the compaction layout")
    out = _outputs_like(block)
    if layout.size(0):
        _run(block, layout, cuts.contiguous(), apply=True, outputs=out)
    return out


def merge_blocks(block, lengths, cuts=None):
    """Compact every lane of ``block`` (lane lengths ``lengths``): choose the cuts unless recorded ones are
    given, then merge; returns ``(merged block, cuts)`` (litgpt/beta_log_kv.py:95-105)."""
    if sum(int(n) for n in lengths) != block[0].size(0):
        raise ValueError("Beta lane lengths must cover the compaction input")
    layout = make_layout(lengths, block[0].device)
    if cuts is not None and (cuts.shape != (len(layout),) or cuts.dtype != torch.uint8
                             or cuts.device != layout.device):
        raise ValueError("recorded Beta cuts do not match the compaction layout")
    if not len(layout):
        empty = torch.empty(0, dtype=torch.uint8, device=layout.device) if cuts is None else cuts
        return tuple(None if x is None else x[:0] for x in block), empty
    _check_block(block)
    out = _outputs_like(block)
    if cuts is None:
        cuts = torch.empty(layout.size(0), dtype=torch.uint8, device=layout.device)
        _run(block, layout, cuts, apply=False, outputs=out)
    else:
        _run(block, layout, cuts.contiguous(), apply=True, outputs=out)
    return out, cuts
