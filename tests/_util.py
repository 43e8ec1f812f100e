"""Helpers shared by the tests (not a test module)."""

import json
import sys
from pathlib import Path

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


def fwd_bound(w64, x64):
    """Forward error bound of a float32 dot product of length K (rows of w64)."""
    k = w64.shape[-1]
    gamma = k * 2.0**-24 / (1 - k * 2.0**-24)
    return 1.01 * gamma * (np.abs(w64) @ np.abs(x64)) + 1e-30


def ulp_bf16(x):
    x = np.abs(np.asarray(x, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(x, 2.0**-126))) - 7)


def check_bf16(y_bits, ref_bits, sum_bound, exact_frac=0.97):
    """Two float32 sums, each within `sum_bound` of exact, rounded to bf16 may
    differ by both errors plus one bf16 step; most should agree exactly."""
    from oracle import bf16

    y = bf16.from_bits(y_bits).astype(np.float64)
    ref = bf16.from_bits(ref_bits).astype(np.float64)
    excess = np.abs(y - ref) - (ulp_bf16(ref) + 2 * sum_bound)
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert np.all(excess <= 0), (f"{int((excess > 0).sum())} outside the bound; worst at {worst}: "
                                 f"got {y[worst]!r}, want {ref[worst]!r}")
    exact = (np.asarray(y_bits) == np.asarray(ref_bits)).mean()
    assert exact >= exact_frac, f"only {exact:.4f} bit-exact"


def check_kv_slot(engine, stage, layer, slot, tol):
    """KV slot `slot` of `layer` holds the oracle's key and value rows: each
    KV head within rel-L2 `tol` of the oracle's same head and far from every
    other head (a head written to the wrong place fails), nothing zero."""
    from oracle import bf16

    k, v = engine.read_kv(layer, slot)
    worst = 0.0
    for got_bits, want_bits in ((k, stage.key_cache[layer][:, slot]), (v, stage.value_cache[layer][:, slot])):
        got, want = bf16.from_bits(got_bits), bf16.from_bits(want_bits)
        assert np.all(np.any(got_bits != 0, axis=-1)), f"layer {layer} slot {slot}: a head row is empty"
        for h in range(got.shape[0]):
            err = rel_l2(got[h], want[h])
            worst = max(worst, err)
            assert err <= tol, f"layer {layer} slot {slot} head {h}: rel-L2 {err:.3e}"
            for h2 in range(got.shape[0]):
                if h2 != h:
                    assert rel_l2(got[h], want[h2]) > 0.5, f"layer {layer} slot {slot}: head {h} looks like {h2}"
    return worst


_FLOORS = {row["label"]: row["rel_l2"] for row in json.loads(
    (Path(__file__).resolve().parent / "golden" / "order_sensitivity.json").read_text())}


def full_depth_tol(label):
    """1.3 times the oracle's own summation-order floor for this workload
    (the oracle against itself with exactly rounded projections)."""
    return 1.3 * _FLOORS[label]
