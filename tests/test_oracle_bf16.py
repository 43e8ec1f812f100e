"""Pins oracle.bf16 (the RNE cast the reference gets from ml_dtypes,
npu_llm/runtime/cpu_backend.py:7-8) against the definition of
round-to-nearest-even, evaluated independently in float64, and against
torch's bfloat16 cast."""

import numpy as np

from oracle import bf16


def _rne_by_definition(f32):
    """Nearest bf16 by exact float64 distance; ties to even mantissa."""
    f = np.asarray(f32, dtype=np.float32)
    u = f.view(np.uint32)
    sign = u & np.uint32(0x80000000)
    mag = u & np.uint32(0x7FFFFFFF)
    lo = (mag >> np.uint32(16)).astype(np.uint32)          # truncated toward zero
    hi = lo + np.uint32(1)

    def value(bits16):
        as32 = (bits16.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)
        # the step past the largest finite bf16 rounds to infinity; give it
        # its unbounded-exponent value 2**128 when measuring distances
        return np.where(bits16 == 0x7F80, 2.0**128, as32)

    x = mag.view(np.float32).astype(np.float64)
    dlo = x - value(lo)
    dhi = value(hi) - x
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo & np.uint32(1)) == 1))
    out = np.where(pick_hi, hi, lo).astype(np.uint32)
    return (out | (sign >> np.uint32(16))).astype(np.uint16)


def test_rne_matches_definition_on_dense_sweep():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    np.testing.assert_array_equal(bf16.to_bits(f), _rne_by_definition(f))


def test_rne_ties_and_specials():
    cases = [
        (1.0, 0x3F80),
        (-2.0, 0xC000),
        (0.0, 0x0000),
        (-0.0, 0x8000),
        (np.inf, 0x7F80),
        (-np.inf, 0xFF80),
        # halfway between 1.0 (even) and 1.0078125 (odd): stays at even 1.0
        (float(np.uint32(0x3F808000).view(np.float32)), 0x3F80),
        # halfway between 1.0078125 (odd) and 1.015625 (even): rounds up to even
        (float(np.uint32(0x3F818000).view(np.float32)), 0x3F82),
        # just above halfway rounds up
        (float(np.uint32(0x3F808001).view(np.float32)), 0x3F81),
        # largest finite float32 overflows to +inf under RNE
        (float(np.finfo(np.float32).max), 0x7F80),
        # smallest subnormal rounds to zero; a subnormal near the top keeps bits
        (float(np.uint32(0x00000001).view(np.float32)), 0x0000),
        (float(np.uint32(0x007F8000).view(np.float32)), 0x0080),
    ]
    values = np.array([v for v, _ in cases], dtype=np.float32)
    expected = np.array([b for _, b in cases], dtype=np.uint16)
    np.testing.assert_array_equal(bf16.to_bits(values), expected)


def test_nan_stays_quiet_nan_with_sign():
    nan_bits = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0xFF812345], dtype=np.uint32)
    out = bf16.to_bits(nan_bits.view(np.float32))
    assert np.all(np.isnan(bf16.from_bits(out)))
    np.testing.assert_array_equal(out & 0x8000, np.array([0, 0x8000, 0, 0x8000], np.uint16))


def test_widening_is_exact_and_round_trips():
    bits = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16)
    f = bf16.from_bits(bits)
    finite = np.isfinite(f)
    np.testing.assert_array_equal(bf16.to_bits(f[finite]), bits[finite])


def test_agrees_with_torch_cast():
    import torch  # CPU only; imported here so GPU test processes never load it

    rng = np.random.default_rng(2)
    f = (rng.standard_normal(200_000) * np.exp(rng.uniform(-60, 60, 200_000))).astype(np.float32)
    t = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16.to_bits(f), t)


def test_planted_truncation_is_caught():
    """A cast that truncates instead of rounding fails the definition check."""
    rng = np.random.default_rng(3)
    f = rng.standard_normal(10_000).astype(np.float32)
    truncated = (f.view(np.uint32) >> 16).astype(np.uint16)
    assert np.any(truncated != _rne_by_definition(f))
