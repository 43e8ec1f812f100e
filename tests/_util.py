"""Helpers shared by the tests (not a test module)."""

import sys

import numpy as np


def announce(message):
    """Print and flush a line naming the case about to run on the GPU."""
    sys.stdout.write(message + "\n")
    sys.stdout.flush()
    sys.stderr.write(message + "\n")
    sys.stderr.flush()


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def near_tie(logits, rel=2.0**-7):
    """True when the top-2 gap is below ``rel`` relative to |top1| (the
    exemption for greedy-token agreement)."""
    lg = np.asarray(logits, dtype=np.float64)
    top2 = np.partition(lg, -2)[-2:]
    hi, lo = max(top2), min(top2)
    return (hi - lo) < rel * max(abs(hi), 1e-30)


def bf16_ulp_diff(a_bits, b_bits):
    """Distance in bf16 representable steps between two uint16 arrays."""
    def ordered(bits):
        b = np.asarray(bits, dtype=np.uint16).astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(ordered(a_bits) - ordered(b_bits))
