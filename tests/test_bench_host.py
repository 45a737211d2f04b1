"""Host-side checks of bench.py: argument parsing and the flush schedule for any warmup / steps
(no GPU touched)."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("argv", [["--gpus", "1", "--steps", "20", "--warmup", "5"], [],
                                  ["--steps", "1", "--warmup", "0"], ["--steps", "200", "--warmup", "30"]])
def test_driver_arguments_parse(bench, argv):
    args = bench.parse_args(argv)
    assert args.steps >= 1 and args.warmup >= 0


@pytest.mark.parametrize("warmup,steps", [(5, 20), (0, 1), (2, 12), (13, 1), (14, 14), (30, 200), (0, 1000)])
def test_schedule_serves_any_steps(bench, warmup, steps):
    segs = bench.flush_schedule(warmup, steps)
    timed = [x for s in segs for x in s["timed"]]
    warm = [x for s in segs for x in s["warm"]]
    assert len(timed) == steps and len(warm) == warmup
    order = warm + timed
    # Steps walk flushes 3..16 (indices 2..15) of successive streams, in order, each used once.
    expect = [(w // bench.STEADY_FLUSHES, bench.PREP_FLUSHES + w % bench.STEADY_FLUSHES)
              for w in range(warmup + steps)]
    assert sorted(order) == expect
    for seg in segs:
        assert len(seg["streams"]) <= bench.MAX_LIVE_STREAMS
        assert all(s in seg["streams"] for s, _ in seg["warm"] + seg["timed"])
        assert all(bench.PREP_FLUSHES <= j < bench.STREAM_FLUSHES for _, j in seg["warm"] + seg["timed"])
    # Warm-up steps precede every timed step.
    first_timed = next(i for i, s in enumerate(segs) if s["timed"])
    assert not any(s["warm"] for s in segs[first_timed + 1:])


def test_schedule_rejects_nonsense(bench):
    with pytest.raises(ValueError):
        bench.flush_schedule(0, 0)
    with pytest.raises(ValueError):
        bench.flush_schedule(-1, 3)


def test_ladder_count_model_known_cases(bench):
    # Fill only: 3 new rows into an empty 4-slot level 0 of a 3-level ladder are written once.
    assert bench.ladder_rows([0, 0, 0], 3, 4, 3) == (0, 3, 3)
    # Full level 0 (B=4) plus 2 new rows: the oldest 2 of [4 stored | 2 staged] pair into 1 carry,
    # 2 stored survivors move to the front, the 2 staged rows survive behind them.
    rd, wr, tok = bench.ladder_rows([4, 0, 0], 2, 4, 3)
    # level 0: pairs read 2 stored, survivors read 2 stored + 2 staged tokens; writes: carry 1,
    # survivors 2 + 2, cleared 0; level 1: the carry fills one slot (read 1, write 1).
    assert (rd, wr, tok) == (2 + 2 + 1, 1 + 2 + 2 + 1, 2)
