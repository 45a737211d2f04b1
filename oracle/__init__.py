"""The oracle: a CPU (numpy) restatement of SemanticLogKV's flush and readout path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
the timed CPU baseline - the product package ``logkv_amd`` never imports it and
has no CPU fallback.

Modules and what pins them (the tests named in brackets):
* ``numerics`` - bf16 rounding and the canonical float32 reduction orders
  [tests/test_oracle_numerics.py: torch's bf16 cast, float64 sums];
* ``route`` - attach decisions and commit grouping [tests/test_oracle_route.py:
  float64 brute force with decision margins, invariants];
* ``ladder`` - pair / Beta / fold merges, Fenwick append, centroid update
  [tests/test_oracle_ladder.py: the reference's known answers, the scalar
  one-entry-at-a-time rule, mass and position conservation, float64 centroid];
* ``spans`` - Alpha span cutting, scoring and greedy choice
  [tests/test_oracle_spans.py: the reference's known answers, closed forms];
* ``readout`` - attention plan, pack, attention [tests/test_oracle_readout.py:
  known anchors, textbook softmax, duplicated-token equivalence];
* ``cache`` - one layer's cache and flush driver [tests/test_oracle_cache.py].
"""

from .cache import OracleCache, budget  # noqa: F401
