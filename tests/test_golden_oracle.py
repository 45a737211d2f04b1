"""The oracle against the golden fixtures of the reference's own CPU Torch path (tests/golden,
written by make_fixtures.py): flush sequences with attach routing, Alpha, Beta, delayed archival
and seeding (every state field after every block), span choices on large random cases, Beta cuts
with near ties and tails, and the Torch packer with bf16 RoPE tables. Integers bit for bit,
payloads within one bf16 ulp, masses and centers within 1e-5 relative."""

from __future__ import annotations

import json

import numpy as np
import pytest

from golden_data import GOLDEN, bf16_ulp, compare_state, config, from_bits, load, tables
from logkv_amd import alpha_log_kv as prod_spans
from oracle import OracleCache
from oracle import ladder as ol
from oracle import spans as ora_spans


def oracle_for(cfg, data):
    import torch

    cos, sin = tables(data)
    table_dtype = cos.dtype
    cos, sin = cos.float().numpy(), sin.float().numpy()
    return OracleCache(cfg["batch"], cfg["groups"], cfg["max_seq"], cfg["dim"], cfg["dim"], B=cfg["B"],
                       recent_size=cfg["recent"], K=cfg["K"], s_h=cfg["s_h"], flush=cfg["flush"],
                       exact_tokens=cfg["exact"], span_max=cfg["span"], beta_novelty=cfg["beta"],
                       beta_adaptive=cfg["beta"], cos=cos, sin=sin, table_bf16=table_dtype is torch.bfloat16)


def oracle_get(ora):
    def get(name):
        if name == "alpha_spans":
            return [list(row) for row in ora.alpha_spans]
        return getattr(ora, name)
    return get


@pytest.mark.parametrize("name,alpha", [("flush_alpha_beta.npz", True), ("flush_attach_seeded.npz", False)])
def test_oracle_flush_sequence_matches_reference(name, alpha):
    data = load(name)
    cfg = config(data)
    ora = oracle_for(cfg, data)
    assert (ora.B, ora.L) == (int(data["B_prime"]), int(data["levels"]))
    for i in range(int(data["blocks"])):
        k_raw, v, k = (from_bits(data[f"{f}_{i}"]) for f in ("k_raw", "v", "k"))
        ends = data[f"ends_{i}"].astype(bool).tolist() if alpha else None
        ora.add_recent(k, v, k_raw, data[f"pos_{i}"], ends)
        bad = compare_state(oracle_get(ora), data, i, alpha)
        assert not bad, f"block {i}: " + "; ".join(bad)
        assert ora.recent_count == int(data[f"recent_count_{i}"])
    # The sequence exercised what it pins: several flushes, carries past level 0, Alpha keeps.
    assert int(data["level_count_" + str(int(data["blocks"]) - 1)][..., 1:].sum()) > 0
    if alpha:
        assert ora.late_joins > 0 or int(data[f"alpha_count_{int(data['blocks']) - 1}"]) > 0


def _cases():
    return json.loads((GOLDEN / "choose_spans.json").read_text())


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_span_choice_matches_reference(impl):
    for i, c in enumerate(_cases()):
        spans = [[tuple(s) for s in row] for row in c["spans"]]
        args = (spans, c["positions"], c["new_positions"], c["ends"], c["old_width"], c["max_span"])
        if impl == "oracle":
            cut = ora_spans.cut_spans(*args)
            keep, archive, out_spans, out_pos = ora_spans.choose_spans(cut, np.asarray(c["scores"], np.float32),
                                                                       c["budget"])
        else:
            sel = prod_spans.choose_spans(prod_spans.cut_spans(*args), c["scores"], c["budget"])
            keep, archive, out_spans, out_pos = sel.keep, sel.archive, sel.spans, sel.positions
        assert keep == c["keep"] and archive == c["archive"], i
        assert [[list(s) for s in r] for r in out_spans] == c["out_spans"], i
        assert out_pos == c["out_positions"], i


def test_beta_cuts_match_reference():
    data = load("select_cuts.npz")
    k, v, w = data["k"], data["v"], data["w"]
    rows = {"k": k, "v": v, "w": w, "p_lo": np.zeros(len(w), np.int64), "p_hi": np.zeros(len(w), np.int64),
            "sum_wp": np.zeros(len(w), np.int64), "order": np.zeros(len(w), np.int64),
            "pad": np.zeros(len(w), bool)}
    np.testing.assert_array_equal(ol.beta_layout(data["lengths"]), data["layout"])
    _, cuts = ol.beta_merge(rows, data["lengths"])
    np.testing.assert_array_equal(cuts, data["cuts"])
    # The first four groups hold identical rows: every cut costs only the rounding of its side means,
    # so those decisions pin the order of the weighted sums, not just the cost formula.
    assert len(set(data["cuts"][:4].tolist())) > 1


def test_torch_packer_with_bf16_tables_matches_reference():
    import torch

    data = load("pack_torch.npz")
    cfg = dict(batch=1, groups=2, dim=32, max_seq=1024, K=4, B=8, recent=32, flush=32, exact=16, span=4, beta=False,
               s_h=16.0)
    ora = oracle_for(cfg, data)
    assert tables(data)[0].dtype is torch.bfloat16
    for i in range(int(data["blocks"])):
        ora.add_recent(from_bits(data[f"k_{i}"]), from_bits(data[f"v_{i}"]), from_bits(data[f"k_raw_{i}"]),
                       data[f"pos_{i}"], data[f"ends_{i}"].astype(bool).tolist())
    ka, va = ora.pack(from_bits(data["cur_k"]), from_bits(data["cur_v"]))
    want_k, want_v = from_bits(data["ka"]), from_bits(data["va"])
    assert ka.shape == want_k.shape
    np.testing.assert_array_equal(va, want_v)
    np.testing.assert_array_equal(np.delete(ka, 32, -1), np.delete(want_k, 32, -1))
    bias, ref = ka[..., 32], want_k[..., 32]
    assert (np.abs(bias - ref) <= bf16_ulp(ref)).all()
