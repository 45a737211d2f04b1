"""Pins of the oracle's float32 building blocks (oracle/numerics.py).

* ``bf16_round`` equals torch's float32 -> bfloat16 cast (round to nearest
  even) on random values, ties, subnormals, huge values and infinities;
* ``dsum`` equals the value a 64-lane xor butterfly leaves in lane 0 (the
  device's wave sum), for widths that are and are not multiples of 64, and
  stays within float32 error of the float64 sum;
* ``seqsum`` is the left-to-right float32 sum.
"""

import numpy as np
import torch

from oracle.numerics import WAVE, bf16_round, dsum, seqsum


def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * 10,
        (rng.integers(0, 2 ** 16, 2048).astype(np.uint32) << 16 | 0x8000).view(np.float32),   # exact ties
        np.asarray([0.0, -0.0, 1e-40, -1e-42, 3.4e38, -3.4e38, np.inf, -np.inf], np.float32),
    ])
    x = x[np.isfinite(x) | np.isinf(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = bf16_round(x)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all(), x[~same][:8]
    assert np.isnan(bf16_round(np.asarray([np.nan], np.float32))).all()


def butterfly_lane0(t):
    """xor-butterfly over 64 lanes, lane l first adding its features l, l+64, ..."""
    d = t.shape[-1]
    lanes = np.zeros(WAVE, np.float32)
    for l in range(WAVE):
        acc = None
        for j in range(l, d, WAVE):
            acc = t[j] if acc is None else np.float32(acc + t[j])
        lanes[l] = np.float32(0.0) if acc is None else acc
    for off in (32, 16, 8, 4, 2, 1):
        lanes = (lanes + lanes[np.arange(WAVE) ^ off]).astype(np.float32)
    assert (lanes == lanes[0]).all()
    return lanes[0]


def test_dsum_is_the_wave_butterfly():
    rng = np.random.default_rng(1)
    for d in (1, 8, 64, 100, 128, 136, 256):
        for _ in range(5):
            t = (rng.standard_normal(d) * rng.uniform(0.1, 100)).astype(np.float32)
            assert dsum(t) == butterfly_lane0(t), d
            assert abs(float(dsum(t)) - t.astype(np.float64).sum()) <= 1e-5 * np.abs(t).sum() + 1e-30


def test_dsum_batched_shape():
    t = np.random.default_rng(2).standard_normal((3, 4, 136)).astype(np.float32)
    out = dsum(t)
    assert out.shape == (3, 4)
    assert out[2, 1] == dsum(t[2, 1])


def test_seqsum_is_left_to_right():
    t = np.asarray([1e8, 1.0, -1e8, 1.0], np.float32)
    assert seqsum(t) == np.float32(np.float32(np.float32(1e8 + 1.0) - 1e8) + 1.0)
    assert seqsum(np.zeros((0, 3), np.float32)).tolist() == [0.0, 0.0, 0.0]


def test_division_through_double_reciprocal_is_ieee_float_division():
    """The kernels divide by a weight mass as float(double(a) * (1 / double(b))):
    the double product is within 2^-52 of a / b and a float quotient that is not
    a float lies at least 2^-50 from any rounding boundary, so the result must
    equal IEEE float division. Checked here on random pairs over the whole
    exponent range, subnormal numerators and quotients, integer masses (the
    kernels' denominators) and exact quotients."""
    rng = np.random.default_rng(7)
    n = 2_000_000
    bits = rng.integers(0, 0x7F800000, n, dtype=np.int64).astype(np.uint32)
    a = bits.view(np.float32) * np.where(rng.random(n) < 0.5, -1, 1).astype(np.float32)
    b = rng.integers(1, 0x7F800000, n, dtype=np.int64).astype(np.uint32).view(np.float32)
    masses = rng.integers(1, 1 << 20, n).astype(np.float32)
    small = (rng.standard_normal(n) * 1e-40).astype(np.float32)          # subnormal numerators
    exact = (rng.integers(-1000, 1000, n) * masses).astype(np.float32)   # exact quotients
    for num, den in ((a, b), (a, masses), (small, masses), (exact, masses),
                     (rng.standard_normal(n).astype(np.float32), np.float32(1e-12) + masses * 0)):
        with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
            want = num / den
            got = (num.astype(np.float64) * (1.0 / den.astype(np.float64))).astype(np.float32)
        same = (got == want) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (num[~same][:5], den[~same][:5])
        assert (np.signbit(got) == np.signbit(want))[~np.isnan(want)].all()
