"""The oracle: a CPU (numpy) restatement of SemanticLogKV's flush and readout path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only to check results or
as the timed CPU baseline - the product package ``logkv_amd`` never imports it and
has no CPU fallback.

Modules and what pins them (the tests named in brackets):
* ``numerics`` - bf16 rounding and the canonical float32 reduction orders
  [tests/test_oracle_numerics.py: torch's bf16 cast, the 64-lane xor
  butterfly, float64 sums];
* ``route`` - attach decisions and seeding [tests/test_oracle_route.py: float64
  brute force on rows with a clear decision margin, farthest-point seeds,
  invariants];
* ``ladder`` - pair / Beta / fold merges, Fenwick append, centroid update
  [tests/test_oracle_ladder.py: the reference's known answers, the reference's
  scalar one-entry-at-a-time rule, mass and position conservation, Beta
  optimality, float64 centroid];
* ``spans`` - Alpha span cutting, scoring and greedy choice
  [tests/test_spans_host.py and tests/test_oracle_spans.py: the reference's
  known answers (whole spans, pending tails, novelty rescue, top-2 groups),
  exact closed forms, float64 scores];
* ``readout`` - attention plan, pack, attention, slot encoding, attention gradients
  [tests/test_oracle_readout.py: known anchors, explicit RoPE and mask rows, mass
  slot = duplicated tokens, float64 masked softmax, the slot encoding against the
  pack, gradients against torch autograd in float64];
* ``cache`` - one layer's cache and flush driver [tests/test_oracle_cache.py:
  delayed-archive known answer, budget closed form, streaming invariants];
* ``unified`` - the unified Ward / radius route [tests/test_oracle_unified.py:
  hand-worked reducer answers (Ward cost, Lance-Williams update, radius
  bound, xor tie rule, budget order), incremental rounds equal to a full
  recompute, labels and Ward entry order, route invariants, an old-old merge];
* ``oplog`` - op-log rows of a flush and the replay parse
  [tests/test_oracle_oplog.py: hand-derived logs of small flushes, replay
  reproducing the recorded state bit for bit, the reference's parse errors].

Golden fixtures from the reference's own CPU Torch path (tests/golden, written by
tests/golden/make_fixtures.py in the build container) pin ``cache``, ``ladder``,
``spans`` and ``readout`` end to end [tests/test_golden_oracle.py: two streamed flush
sequences with every state field after every block, 299 span choices with tied scores,
Beta cuts with near ties and tails, the packer with bf16 RoPE tables]; the centroid's
tiled ("parallel") order is pinned by a hand-worked float32 case
[tests/test_oracle_ladder.py].

Parity unpinned: last-ulp agreement with the reference's own float traces on inputs
beyond the fixtures, where it leaves the order to a library (Torch GEMM / cdist /
segment_reduce summation orders, Triton ``tl.sum``, Flash SDPA): the oracle fixes one
order that the device reproduces bit for bit, and the fixtures show it giving the
reference's values and decisions on their inputs.
"""

from .cache import OracleCache, budget  # noqa: F401
