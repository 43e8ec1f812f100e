"""bfloat16 <-> float32 conversion on uint16 bit patterns (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, smoke() and bench's CPU baseline.

The reference casts with ``ml_dtypes.bfloat16`` (``runtime/cpu_backend.py:7-8``),
which rounds to nearest, ties to even.  The same integer formula appears in
the reference's device code (``kernels/qwen_engine_common.h:35-46``) and its
Colibri backend (``colibri-xdna/backend/backend_xdna.cpp:35-40``).  NaN maps
to a quiet NaN that keeps the sign bit.

Pinned by ``tests/test_oracle_bf16.py``: exhaustive agreement with
``torch.Tensor.to(torch.bfloat16)`` on a dense sweep of bit patterns, plus the
textbook special cases (ties to even in both directions, overflow to inf,
subnormals, signed zeros, NaN).
"""

import numpy as np

__all__ = ["to_bits", "from_bits", "round_f32"]


def to_bits(values):
    """Return the RNE bfloat16 bit patterns (uint16) of ``float32(values)``."""
    f = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    rounded = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    bits = rounded.astype(np.uint16)
    nan = np.isnan(f)
    if np.any(nan):
        quiet = ((u >> np.uint64(16)) & np.uint64(0x8000)).astype(np.uint16) | np.uint16(0x7FC0)
        bits = np.where(nan, quiet, bits)
    return bits


def from_bits(bits):
    """Widen bfloat16 bit patterns (uint16) to float32 exactly."""
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_f32(values):
    """``float32(bfloat16(values))``: the value the reference's ``_bf16`` keeps."""
    return from_bits(to_bits(values))
