"""Host side of beta_log_kv: the layout schedule and the argument checks that run before any
device work (no GPU needed)."""

from __future__ import annotations

import pytest
import torch

from logkv_amd.beta_log_kv import make_layout, merge_blocks, select_cuts


def test_layout_known_answers():
    # litgpt tests/test_beta_log_kv.py:48-49
    assert make_layout([0, 6, 0, 2], "cpu").tolist() == [[0, 4, 0], [4, 2, 2], [6, 2, 3]]
    assert make_layout([], "cpu").shape == (0, 3)
    assert make_layout([8, 4], "cpu").tolist() == [[0, 4, 0], [4, 4, 2], [8, 4, 4]]
    assert make_layout([10], "cpu").tolist() == [[0, 4, 0], [4, 4, 2], [8, 2, 4]]


def test_layout_groups_cover_each_lane_once():
    lengths = [2, 0, 14, 6, 4, 0, 22]
    layout = make_layout(lengths, "cpu").tolist()
    covered = [i for start, width, _ in layout for i in range(start, start + width)]
    assert covered == list(range(sum(lengths)))
    assert all(width in (2, 4) for _, width, _ in layout)
    # Outputs are half the inputs and contiguous.
    outs = [o + s for start, width, o in layout for s in range(2 if width == 4 else 1)]
    assert outs == list(range(sum(lengths) // 2))


@pytest.mark.parametrize("lengths", [[3], [2, -2], [1, 1]])
def test_layout_rejects_odd_or_negative_lanes(lengths):
    with pytest.raises(ValueError):
        make_layout(lengths, "cpu")


def test_block_checks_run_before_the_device():
    k = torch.zeros(4, 8)
    block = (k, k, torch.ones(4), torch.zeros(4, 8), None, None, None, None, None, None, None, None, None)
    with pytest.raises(ValueError, match="first-order"):
        select_cuts(block, make_layout([4], "cpu"))
    plain = (k, k, torch.ones(4)) + (None,) * 10
    with pytest.raises(ValueError, match="cover"):
        merge_blocks(plain, [2])
    # A CPU block reaches the device check: the HIP library has no CPU path.
    with pytest.raises(ValueError, match="ROCm"):
        select_cuts(plain, make_layout([4], "cpu"))
