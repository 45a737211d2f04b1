"""The standalone Beta compaction (beta_log_kv) on the device: the reference's known answers,
cut optimality against fixed pairs (float64 losses), and bit-exact agreement with the oracle's
Beta merge on random blocks of bf16 and float32 payloads."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from logkv_amd.beta_log_kv import apply_cuts, make_layout, merge_blocks, select_cuts
from oracle import ladder as ol

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def entry_block(values, weights, dtype=torch.float32):
    """The reference test's block (tests/test_beta_log_kv.py:13-18): V rows constant per entry."""
    v = torch.tensor(values, dtype=dtype)[:, None].repeat(1, 8).to(DEV)
    w = torch.tensor(weights, dtype=torch.float32, device=DEV)
    pos = torch.arange(len(values), device=DEV, dtype=torch.int64)
    return (torch.ones_like(v), v, w, None, None, None, None, None,
            pos, pos.clone(), pos * w.long(), pos.clone(), torch.zeros_like(pos, dtype=torch.bool))


def test_known_answer_and_replay():
    # litgpt tests/test_beta_log_kv.py:45-63: two lanes of 6 and 2 entries never merge across lanes.
    assert make_layout([0, 6, 0, 2], DEV).tolist() == [[0, 4, 0], [4, 2, 2], [6, 2, 3]]
    block = entry_block([10, 0, 0, 0, 7, 9, 20, 30], [1, 2, 3, 4, 1, 1, 2, 3])
    result, cuts = merge_blocks(block, [6, 2])
    assert cuts.tolist() == [1, 1, 1]
    assert result[2].tolist() == [1.0, 9.0, 2.0, 5.0]
    assert result[1][:, 0].tolist() == [10.0, 0.0, 8.0, 26.0]
    assert int(result[10].sum()) == int(block[10].sum())
    for f in (0, 1):
        torch.testing.assert_close((result[f] * result[2][:, None]).sum(0), (block[f] * block[2][:, None]).sum(0))
    replay, _ = merge_blocks(block, [6, 2], cuts=cuts)
    for first, second in zip(result, replay):
        if first is not None:
            assert torch.equal(first, second)
    assert torch.equal(select_cuts(block, make_layout([6, 2], DEV)), cuts)


def test_cut_loss_never_exceeds_fixed_pairs():
    # litgpt tests/test_beta_log_kv.py:66-85, losses evaluated in float64 on the host.
    g = torch.Generator().manual_seed(83)
    block = list(entry_block([0] * 40, torch.randint(1, 10, (40,), generator=g).tolist()))
    block[0] = torch.randn(40, 7, generator=g).to(DEV)
    block[1] = torch.randn(40, 11, generator=g).to(DEV)
    layout = make_layout([40], DEV)
    _, cuts = merge_blocks(tuple(block), [40])
    xs = [block[0].double().cpu(), block[1].double().cpu()]
    w_all = block[2].double().cpu()
    for start, cut in zip(layout[:, 0].tolist(), cuts.tolist()):
        w = w_all[start:start + 4]

        def loss(split):
            total = 0.0
            for x in xs:
                x = x[start:start + 4]
                energy = (x.square().sum(-1) * w).sum() / w.sum()
                for part in (slice(0, split), slice(split, 4)):
                    mean = (x[part] * w[part, None]).sum(0) / w[part].sum()
                    total += float(((x[part] - mean).square().sum(-1) * w[part]).sum() / energy)
            return total

        assert loss(cut) <= loss(2) + 1e-5


def _random_block(g, lengths, dk, dv, dtype):
    n = sum(lengths)
    k = (torch.randn(n, dk, generator=g) * 3).to(dtype)
    v = (torch.randn(n, dv, generator=g) * 3).to(dtype)
    w = torch.randint(0, 9, (n,), generator=g).float()        # some zero masses
    lo = torch.randint(0, 10000, (n,), generator=g)
    hi = lo + torch.randint(0, 50, (n,), generator=g)
    swp = lo * w.long()
    order = torch.randint(0, 1 << 40, (n,), generator=g)
    pad = torch.rand(n, generator=g) < 0.3
    return tuple(x.to(DEV) if x is not None else None for x in
                 (k, v, w, None, None, None, None, None, lo, hi, swp, order, pad))


def _as_oracle(block):
    return {"k": block[0].float().cpu().numpy(), "v": block[1].float().cpu().numpy(),
            "w": block[2].cpu().numpy(), "p_lo": block[8].cpu().numpy(), "p_hi": block[9].cpu().numpy(),
            "sum_wp": block[10].cpu().numpy(), "order": block[11].cpu().numpy(), "pad": block[12].cpu().numpy()}


@pytest.mark.parametrize("dk,dv,dtype", [(128, 128, torch.bfloat16), (64, 96, torch.bfloat16),
                                         (7, 11, torch.float32), (200, 256, torch.float32)])
def test_matches_oracle_bit_for_bit(dk, dv, dtype):
    g = torch.Generator().manual_seed(dk * 1000 + dv)
    lengths = [0, 6, 2, 40, 4, 18, 0, 10]
    block = _random_block(g, lengths, dk, dv, dtype)
    out, cuts = merge_blocks(block, lengths)
    ref, ref_cuts = ol.beta_merge(_as_oracle(block), lengths)
    np.testing.assert_array_equal(cuts.cpu().numpy(), ref_cuts)
    for f, name in ((0, "k"), (1, "v"), (2, "w"), (8, "p_lo"), (9, "p_hi"), (10, "sum_wp"), (11, "order"),
                    (12, "pad")):
        np.testing.assert_array_equal(out[f].cpu().numpy(), ref[name], err_msg=name)
    assert out[0].dtype == torch.float32 and out[12].dtype == torch.bool
    # Recorded cuts reproduce the merge without re-selection.
    again = apply_cuts(block, make_layout(lengths, DEV), cuts)
    for a, b in zip(out, again):
        if a is not None:
            assert torch.equal(a, b)


def test_recorded_cuts_are_validated():
    block = entry_block([1, 2, 3, 4], [1, 1, 1, 1])
    layout = make_layout([4], DEV)
    with pytest.raises(ValueError):
        apply_cuts(block, layout, torch.tensor([0], dtype=torch.uint8, device=DEV))
    with pytest.raises(ValueError):
        merge_blocks(block, [4], cuts=torch.tensor([2, 2], dtype=torch.uint8, device=DEV))
    bad_layout = torch.tensor([[2, 4, 0]], dtype=torch.int64, device=DEV)   # runs past the block
    with pytest.raises(ValueError):
        select_cuts(block, bad_layout)


def test_other_float_dtypes_are_upcast():
    """float16 payloads and bfloat16 masses are read as float32, as the reference's ``.float()``
    reads them: the merge equals that of the same block upcast beforehand, and the merged masses
    keep the block's mass dtype."""
    g = torch.Generator().manual_seed(23)
    lengths = [6, 4, 10]
    base = _random_block(g, lengths, 64, 64, torch.float32)
    half = (base[0].half(), base[1].half(), base[2].bfloat16()) + base[3:]
    upcast = (half[0].float(), half[1].float(), half[2].float()) + base[3:]
    out, cuts = merge_blocks(half, lengths)
    want, want_cuts = merge_blocks(upcast, lengths)
    assert torch.equal(cuts, want_cuts)
    assert out[2].dtype == torch.bfloat16 and torch.equal(out[2], want[2].bfloat16())
    for f in (0, 1, 8, 9, 10, 11, 12):
        assert torch.equal(out[f], want[f]), f
