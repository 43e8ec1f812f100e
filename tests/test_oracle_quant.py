"""Pins oracle.quant: the reference quantiser (npu_llm/tools/convert_smollm2.py:81-86)
and the W8 projection formula (npu_llm/kernels/project_w8bf16.cc:14-38)."""

import numpy as np

from oracle import bf16
from oracle.quant import project_w8, quantize_per_output_channel
from runtime.synthetic import quantize_rows


def test_quantiser_bound_of_reference_test():
    # npu_llm/tests/test_converter.py:15-24: seed 7, N(0, 0.2), 32 x 64
    rng = np.random.default_rng(7)
    weight = rng.normal(0, 0.2, (32, 64)).astype(np.float32)
    q, scale = quantize_per_output_channel(weight)
    restored = q.astype(np.float32) * scale[:, None]
    assert q.dtype == np.int8 and scale.dtype == np.float32
    assert np.all(np.abs(restored - weight).max(axis=1) <= scale / 2 + 1e-6)


def test_quantiser_uses_full_range_and_handles_zero_rows():
    rng = np.random.default_rng(8)
    weight = rng.normal(0, 0.02, (16, 896)).astype(np.float32)
    weight[3] = 0.0
    q, scale = quantize_per_output_channel(weight)
    live = np.ones(16, bool)
    live[3] = False
    assert np.all(np.abs(q[live]).max(axis=1) == 127)
    assert np.all(q[3] == 0) and scale[3] == np.finfo(np.float32).tiny


def test_product_quantiser_matches_oracle():
    rng = np.random.default_rng(9)
    weight = bf16.round_f32(rng.normal(0, 0.02, (64, 896)).astype(np.float32))
    q1, s1 = quantize_per_output_channel(weight)
    q2, s2 = quantize_rows(weight)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)


def test_project_w8_matches_float64():
    rng = np.random.default_rng(10)
    q = rng.integers(-127, 128, (40, 896)).astype(np.int8)
    scale = rng.uniform(1e-4, 1e-3, 40).astype(np.float32)
    x = bf16.round_f32(rng.normal(size=896).astype(np.float32))
    y = project_w8(q, scale, x)
    exact = (q.astype(np.float64) @ x.astype(np.float64)) * scale.astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.abs(exact))) - 7)
    gamma = 896 * 2.0**-24
    bound = 0.5 * ulp * 1.001 + gamma * (np.abs(q.astype(np.float64)) @ np.abs(x)) * scale + 2e-7 * np.abs(exact)
    assert np.all(np.abs(y - exact) <= bound)
    # dequantising before rounding the sum, or forgetting the scale, is caught
    assert np.any(np.abs(bf16.round_f32(q.astype(np.float32) @ x) - exact) > bound)
