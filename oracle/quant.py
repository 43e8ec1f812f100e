"""int8 per-output-row quantisation and the W8 projection formula (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, smoke() and bench's CPU baseline.

``quantize_per_output_channel`` follows ``npu_llm/tools/convert_smollm2.py:81-86``:
``s = max(absmax_row / 127, float32.tiny)``, ``q = clip(rint(w / s), -127, 127)``.
``project_w8`` follows the device formula of ``kernels/project_w8bf16.cc:14-38``:
FP32 accumulation of ``f32(q) * f32(bf16 x)``, then ``bf16(acc * scale[row])``.

Pinned by ``tests/test_oracle_quant.py``: the reference test's bound
(``tests/test_converter.py:15-24``: ``|q*s - w| <= s/2 + 1e-6`` per row, seed 7,
N(0, 0.2), 32x64), exactness of the int8 extremes (every row holds +-127),
and the W8 projection against a float64 brute force.
"""

import numpy as np

from oracle.bf16 import round_f32

__all__ = ["quantize_per_output_channel", "project_w8"]


def quantize_per_output_channel(weight):
    weight = np.asarray(weight, dtype=np.float32)
    max_abs = np.max(np.abs(weight), axis=1)
    scale = np.maximum(max_abs / 127.0, np.finfo(np.float32).tiny)
    q = np.clip(np.rint(weight / scale[:, None]), -127, 127).astype(np.int8)
    return q, scale.astype(np.float32)


def project_w8(q, scale, activation, *, round_bf16=True):
    """``bf16((f32(q) @ f32(bf16(x))) * scale)``; FP32 result when not rounding."""
    acc = np.asarray(q, dtype=np.float32) @ round_f32(activation)
    out = acc * np.asarray(scale, dtype=np.float32)
    return round_f32(out) if round_bf16 else out
