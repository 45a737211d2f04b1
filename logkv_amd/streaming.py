"""Inference streaming over a LogStructuredKVCache: block prefill and pending-token decode
pairing of CausalSelfAttention's LogKV path (litgpt/model.py:1125-1361, inference:
``defer_last_single=True``, no gradient).

The model's projections, RoPE and output projection are not on this path: the caller
hands over post-RoPE queries and keys, values and the pre-RoPE keys that routing uses,
and gets the attention output. Every attention runs in the HIP library
(``log_kv_chunk_attention``: pack + streaming / matrix-core kernels) and every commit
is the cache's ``add_recent`` (the flush kernels).
"""

from __future__ import annotations

import torch

from .log_kv_pack import log_kv_chunk_attention


def _cols(rows, start, end):
    """Columns [start, end) of per-row span flags (host lists or a [B, T] tensor)."""
    if rows is None:
        return None
    if isinstance(rows, torch.Tensor):
        return rows[:, start:end]
    return [row[start:end] for row in rows]


def _join(a, b):
    """Span flags of a block followed by another (lists or tensors)."""
    if isinstance(a, torch.Tensor) or isinstance(b, torch.Tensor):
        dev = (a if isinstance(a, torch.Tensor) else b).device
        return torch.cat([torch.as_tensor(x, dtype=torch.uint8, device=dev) for x in (a, b)], dim=1)
    return [list(x) + list(y) for x, y in zip(a, b)]


class LogKVStreamingAttention:
    """The streaming engine of one attention layer over ``cache``.

    ``__call__(q, k, v, k_raw, input_pos, span_ends)`` processes T new tokens
    (q ``[B, n_head, T, d]`` post-RoPE, k / v ``[B, n_groups, T, d]`` post-RoPE keys and
    values, k_raw the pre-RoPE keys, input_pos ``[T]`` or ``[B, T]``, span_ends per-row
    flags when the cache has an Alpha exact pool) and returns ``[B, T, n_head * dv]``:

    * a token left pending by the previous call is paired with the first new token: that
      token's query attends to the cache plus both (non-causal among the two), then both
      are committed (litgpt/model.py:1226-1250);
    * the rest runs in blocks of ``max(2, min(prefill_block, recent_size))`` tokens: the
      block's queries attend to the cache state at the block's start plus the block's own
      tokens causally, then the block is committed; a lone final token of odd length is
      attended but kept pending (litgpt/model.py:1252-1340), so prefill and decode keep
      the 2-token commit boundaries of the concatenated sequence.

    The pending tuple is ``_log_kv_pending`` (keys, values, pre-RoPE keys, positions,
    span flags), the attribute the compression accounting reads.
    """

    def __init__(self, cache, scale: float, prefill_block: int = 2048):
        if not cache.semantic_clusters:
            raise NotImplementedError("streaming runs on the semantic LogKV cache")
        self.cache = cache
        self.scale = float(scale)
        self.prefill_block = int(prefill_block)
        self._log_kv_pending = None

    @property
    def kv_cache(self):
        return self.cache

    def reset(self) -> None:
        """Empty the cache and drop the pending token (a new request)."""
        self.cache.reset_parameters()
        self._log_kv_pending = None

    @torch.no_grad()
    def __call__(self, q, k, v, k_raw, input_pos=None, span_ends=None):
        cache = self.cache
        B, _, T, _ = q.shape
        if T < 1:
            raise ValueError("at least one token per call")
        if cache.alpha_exact_tokens and span_ends is None:
            raise ValueError("an Alpha exact pool needs span boundary flags for every streamed token")

        def pos_slice(a, b):
            if input_pos is None:
                return None
            return input_pos[a:b] if input_pos.dim() == 1 else input_pos[:, a:b]

        outputs, start = [], 0
        pending = self._log_kv_pending
        if pending is not None:
            pk, pv, pk_raw, ppos, pends = pending
            # The pair's keys and values serve the attention and the commit.
            kk, vv = torch.cat([pk, k[:, :, :1]], dim=2), torch.cat([pv, v[:, :, :1]], dim=2)
            outputs.append(log_kv_chunk_attention(cache, q[:, :, :1], kk, vv, self.scale, 0.0, causal_tail=0,
                                                  reuse_prefix=True))
            pos0 = pos_slice(0, 1)
            pos = None if ppos is None or pos0 is None else torch.cat([ppos.to(pos0.device), pos0], dim=-1)
            ends = None if pends is None else _join(pends, _cols(span_ends, 0, 1))
            cache.add_recent(kk, vv, k_raw=torch.cat([pk_raw, k_raw[:, :, :1]], dim=2), input_pos=pos,
                             span_ends=ends)
            self._log_kv_pending = None
            start = 1

        blk_size = max(2, min(self.prefill_block, cache.recent_size))
        while start < T:
            end = min(T, start + blk_size)
            defer_tail = end == T and (end - start) % 2 == 1
            commit_end = end - 1 if defer_tail else end
            outputs.append(log_kv_chunk_attention(cache, q[:, :, start:end], k[:, :, start:end], v[:, :, start:end],
                                                  self.scale, 0.0, reuse_prefix=True))
            if commit_end > start:
                cache.add_recent(k[:, :, start:commit_end], v[:, :, start:commit_end],
                                 k_raw=k_raw[:, :, start:commit_end], input_pos=pos_slice(start, commit_end),
                                 span_ends=_cols(span_ends, start, commit_end))
            if defer_tail:
                self._log_kv_pending = (k[:, :, commit_end:end], v[:, :, commit_end:end],
                                        k_raw[:, :, commit_end:end], pos_slice(commit_end, end),
                                        _cols(span_ends, commit_end, end))
            start = end
        y = outputs[0] if len(outputs) == 1 else torch.cat(outputs, dim=2)   # [B, n_head, T, dv]
        return y.transpose(1, 2).reshape(B, T, -1)
