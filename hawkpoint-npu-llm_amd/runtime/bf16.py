"""Host-side bfloat16 helpers: values travel as uint16 bit patterns.

Round-to-nearest-even with a quiet-NaN branch, the rounding the reference
gets from ml_dtypes (npu_llm/runtime/cpu_backend.py:7-8).
"""

import numpy as np

__all__ = ["to_bits", "from_bits"]


def to_bits(values):
    """float32 -> bfloat16 bits (uint16), round to nearest even."""
    f = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    u = f.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    out = ((u.astype(np.uint64) + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        out[nan] = ((u[nan] >> np.uint32(16)) & np.uint32(0x8000)).astype(np.uint16) | np.uint16(0x7FC0)
    return out


def from_bits(bits):
    """bfloat16 bits (uint16) -> float32, exact."""
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)
