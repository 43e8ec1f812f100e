"""Pins the expert-offload oracle (oracle/experts.py) on the CPU.

- the reference's own tests (colibri-xdna/backend/test_backend_xdna.cpp, its
  three cases and tolerances; ollama-xdna/backend/test_experts.cpp's pattern
  at a reduced size here, full size in the GPU test);
- each upload format's decode on hand-built bytes (nibble order, bias 8, the
  ragged last scale group);
- ties to even in the requantisation, and the scale of an all-zero row;
- a two-tile row whose per-tile rounding gives 1.0 where one rounding of the
  whole row gives 1.96875;
- SwiGLU through identity projections, with gate and up distinguishable.
A planted mistake in the oracle (round half away from zero, one rounding per
row, silu applied to up) fails at least one of these; the last test shows it.
"""

import math

import numpy as np
import pytest

from oracle import experts as ox
from oracle.bf16 import round_f32
from tests._expert_cases import (colibri_expert_group_case, colibri_grouped_int4_case, colibri_matmul_case,
                                 tile_rounding_row)

F = np.float32


def _project_upload(case):
    w = ox.decode_colibri(case["weights"], case["scales"], case["fmt"], case["input_size"], case["output_size"],
                          case["group"])
    return ox.project(*ox.requantize_rows(w), case["x"])


@pytest.mark.parametrize("build", [colibri_matmul_case, colibri_grouped_int4_case])
def test_reference_matmul_cases(build):
    case = build()
    got = _project_upload(case)
    assert np.max(np.abs(got - case["expected"])) < case["tol"]


def test_reference_expert_group_case():
    case = colibri_expert_group_case()
    got = ox.expert_group(case["gates"], case["ups"], case["downs"], case["x"])
    assert got.shape == case["expected"].shape
    assert np.max(np.abs(got - case["expected"])) < case["tol"]


def test_reference_expert_pattern_reduced():
    # test_experts.cpp's pattern, 2 experts x 256 x 512, as float32 weights
    e = np.arange(2)[:, None, None]
    r = np.arange(256)[None, :, None]
    c = np.arange(512)[None, None, :]
    q = (((e * 7 + r * 3 + c * 5) % 31) - 15).astype(F)
    s = (F(0.0005) * (1 + np.arange(256) % 5)).astype(F)
    w = q * s[None, :, None]
    x = (F(0.002) * (((np.arange(2)[:, None] + np.arange(512)[None, :]) % 17) - 8)).astype(F)
    got = ox.mul_mat_id(w, x, [0, 1])
    want = np.stack([(q[i].astype(np.float64) @ x[i]) * s for i in range(2)])
    assert np.max(np.abs(got - want)) < 0.03


def test_decode_formats_closed_form():
    # fmt 1: int8 x row scale
    q = np.array([[1, -2, 127], [0, 5, -127]], np.int8)
    s = np.array([0.5, 0.25], F)
    assert np.array_equal(ox.decode_colibri(q, s, 1, 3, 2), [[0.5, -1.0, 63.5], [0.0, 1.25, -31.75]])
    # fmt 2: byte 0x3A -> column 0 (low nibble 10) = 2, column 1 (high nibble 3) = -5;
    # odd width: the last byte's high nibble is unused
    packed = np.array([0x3A, 0xF0, 0x08, 0x0F], np.uint8)  # 2 rows of 3 columns, 2 bytes each
    d = ox.decode_colibri(packed, np.array([1.0, 2.0], F), 2, 3, 2)
    assert np.array_equal(d, [[2.0, -5.0, -8.0], [0.0, -16.0, 14.0]])
    # fmt 4: 5 columns, group 2 -> 3 groups, the last holding one column
    packed = np.array([0x99, 0x99, 0x09], np.uint8)  # every nibble 9 -> value 1
    scales = np.array([1.0, 10.0, 100.0], F)
    assert np.array_equal(ox.decode_colibri(packed, scales, 4, 5, 1, group=2), [[1.0, 1.0, 10.0, 10.0, 100.0]])
    with pytest.raises(ValueError):
        ox.decode_colibri(packed, scales, 3, 5, 1)


def test_requantize_ties_to_even_and_zero_rows():
    q, s = ox.requantize_rows(np.array([[127, 2.5, 3.5, -2.5, 0.5, -0.5], [0, 0, 0, 0, 0, 0]], F))
    assert s.tolist() == [1.0, 1.0]
    assert q.tolist() == [[127, 2, 4, -2, 0, 0], [0, 0, 0, 0, 0, 0]]
    # every nonzero row reaches +-127 exactly, and the error is at most half a step
    w = np.random.default_rng(5).normal(0, 0.3, (16, 100)).astype(F)
    q, s = ox.requantize_rows(w)
    assert np.all(np.max(np.abs(q.astype(int)), axis=1) == 127)
    assert np.all(np.abs(q * s[:, None] - w) <= s[:, None] / 2 + 1e-6)
    assert np.array_equal(s, (np.max(np.abs(w), axis=1) / F(127)).astype(F))


def test_per_tile_rounding():
    w, x = tile_rounding_row()
    q, s = ox.requantize_rows(w)
    assert s[0] == 1.0 and q[0, 0] == 127 and q[0, 2049] == -1
    assert ox.project(q, s, x)[0] == 1.0
    # one rounding over the whole row would keep the fraction
    assert round_f32(np.float32(q[0].astype(np.float64) @ x))[()] == 1.96875


def _silu(v):
    return v / (1 + math.exp(-v))


def test_swiglu_through_identity_projections():
    n = 4
    x = np.array([1.0, 2.0, -1.0, 3.0], F)
    eye = np.eye(n, dtype=F)
    got = ox.expert_group([eye], [2 * eye], [eye], x)
    want = np.array([_silu(v) * 2 * v for v in x.tolist()])
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want))
    swapped = np.array([_silu(2 * v) * v for v in x.tolist()])
    assert np.any(np.abs(got - swapped) > 2.0 ** -7 * np.abs(swapped))
    # a zero gate silences the expert whatever up holds
    assert np.array_equal(ox.expert_group([0 * eye], [eye], [eye], x), np.zeros(n, F))


def test_planted_mistakes_fail_the_pins(monkeypatch):
    # one rounding per row instead of per 2048-column tile
    w, x = tile_rounding_row()
    q, s = ox.requantize_rows(w)
    assert ox.project(q, s, x, tile=1 << 20)[0] != 1.0
    # round half away from zero instead of half to even
    away = lambda v: np.sign(v) * np.floor(np.abs(v) + 0.5)
    row = np.array([127, 2.5, 3.5, -2.5], F)
    assert away(row).tolist() != ox.requantize_rows(row[None])[0][0].tolist()
    # silu applied to up instead of gate
    monkeypatch.setattr(ox, "silu_times", lambda g, u: ((u / (1 + np.exp(-u))) * g).astype(F))
    eye = np.eye(4, dtype=F)
    x = np.array([1.0, 2.0, -1.0, 3.0], F)
    got = ox.expert_group([eye], [2 * eye], [eye], x)
    want = np.array([_silu(v) * 2 * v for v in x.tolist()])
    assert not np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want))
