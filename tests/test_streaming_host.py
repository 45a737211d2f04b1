"""Host logic of the streaming engine that needs no device: span-flag slicing and
joining (host lists and tensors alike) and the constructor's checks."""

from types import SimpleNamespace

import pytest
import torch

from logkv_amd.streaming import LogKVStreamingAttention, _cols, _join


def test_span_flag_columns_and_join_lists():
    rows = [[True, False, True], [False, False, True]]
    assert _cols(rows, 1, 3) == [[False, True], [False, True]]
    assert _cols(None, 0, 1) is None
    assert _join([[True]], [[False, True]]) == [[True, False, True]]


def test_span_flag_join_mixes_tensors_and_lists():
    t = torch.tensor([[1, 0], [0, 1]], dtype=torch.uint8)
    assert torch.equal(_cols(t, 1, 2), torch.tensor([[0], [1]], dtype=torch.uint8))
    joined = _join([[True], [False]], t)
    assert joined.dtype == torch.uint8 and joined.tolist() == [[1, 1, 0], [0, 0, 1]]
    assert _join(t, [[False], [True]]).tolist() == [[1, 0, 0], [0, 1, 1]]


def test_engine_needs_the_semantic_cache():
    with pytest.raises(NotImplementedError):
        LogKVStreamingAttention(SimpleNamespace(semantic_clusters=False), 0.125)
    engine = LogKVStreamingAttention(SimpleNamespace(semantic_clusters=True), 0.125, prefill_block=64)
    assert engine.kv_cache is engine.cache and engine._log_kv_pending is None
