"""Pins the oracle's GGML Q4_K / Q6_K and dense W8-tile restatements
(oracle/experts.py) on the CPU.

No reference fixture holds Q4_K or Q6_K data, so the pins are:
- blocks written column by column from ggml's published layouts
  (tests/_expert_cases.py) and read back through the oracle, on random
  quants and scales;
- single-quant probes that put one nibble or one high-bit pair in a zero
  block and find the one weight that moves, at the column the layout names;
- scale/min probes for each sub-block, including the top-2-bit packing of
  pairs 4..7;
- fp16 special values against numpy's float16;
- per-tile rounding: two tiles built from Q4_K blocks whose per-tile bf16
  results sum to 1.0 where one rounding would give 1.96875;
- dense W8 tiles: one scale per (row, 2048-column tile).
"""

import numpy as np
import pytest

from oracle import experts as ox
from oracle.bf16 import round_f32
from tests._expert_cases import q4k_block, q6k_block

F = np.float32


def test_f16_special_values():
    raw = np.array([0x3C00, 0xC000, 0x0001, 0x8001, 0x03FF, 0x7BFF, 0x7C00, 0x0000, 0x8000], np.uint16)
    got = ox._f16(raw & 0xFF, raw >> 8)
    want = raw.view(np.float16).astype(F)
    assert np.array_equal(got, want)
    assert got[0] == 1.0 and got[1] == -2.0 and got[2] == 2.0 ** -24 and got[5] == 65504.0 and np.isinf(got[6])


def test_q4k_round_trip_through_the_writer():
    rng = np.random.default_rng(1)
    for _ in range(20):
        d, dmin = rng.uniform(0.01, 1), rng.uniform(0.01, 1)
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        w = ox.dequant_q4k(q4k_block(d, dmin, sc, mn, q), 1, 256)[0]
        d16, m16 = F(np.float16(d)), F(np.float16(dmin))
        sub = np.arange(256) // 32  # sub-block of each column
        want = (d16 * sc[sub].astype(F)).astype(F) * q.astype(F) - (m16 * mn[sub].astype(F)).astype(F)
        assert np.array_equal(w, want.astype(F))


def test_q4k_single_nibble_probes():
    zero = np.zeros(8, int)
    for c in range(256):
        q = np.zeros(256, int)
        q[c] = 1
        w = ox.dequant_q4k(q4k_block(1.0, 0.0, np.ones(8, int), zero, q), 1, 256)[0]
        assert np.flatnonzero(w).tolist() == [c] and w[c] == 1.0


def test_q4k_scale_and_min_of_each_sub_block():
    for j in range(8):
        sc = np.ones(8, int)
        mn = np.zeros(8, int)
        sc[j], mn[j] = 63, 45  # top bits set: exercises the packed high bits of pairs 4..7
        w0 = ox.dequant_q4k(q4k_block(1.0, 1.0, sc, mn, np.zeros(256, int)), 1, 256)[0]
        w1 = ox.dequant_q4k(q4k_block(1.0, 1.0, sc, mn, np.ones(256, int)), 1, 256)[0]
        cols = np.arange(32 * j, 32 * j + 32)
        assert np.all(w0[cols] == -45) and np.all(np.delete(w0, cols) == 0)
        assert np.all(w1[cols] == 63 - 45) and np.all(np.delete(w1, cols) == 1)


def test_q6k_round_trip_through_the_writer():
    rng = np.random.default_rng(2)
    for _ in range(20):
        d = rng.uniform(0.01, 1)
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(0, 64, 256)
        w = ox.dequant_q6k(q6k_block(d, sc, q), 1, 256)[0]
        d16 = F(np.float16(d))
        idx = 8 * (np.arange(256) // 128) + (np.arange(256) % 128) // 16
        want = (d16 * sc[idx].astype(F)).astype(F) * (q - 32).astype(F)
        assert np.array_equal(w, want.astype(F))


def test_q6k_single_bit_probes():
    base = np.full(256, 32)  # q - 32 = 0 everywhere
    for c in range(256):
        for v in (1, 16, 48):  # a low-nibble value, a high-bit value, both high bits
            q = base.copy()
            q[c] = v
            w = ox.dequant_q6k(q6k_block(1.0, np.ones(16, int), q), 1, 256)[0]
            assert np.flatnonzero(w).tolist() == [c] and w[c] == v - 32


def test_q6k_scale_of_each_16_columns():
    for m in range(16):
        sc = np.ones(16, int)
        sc[m] = -3
        w = ox.dequant_q6k(q6k_block(1.0, sc, np.full(256, 33)), 1, 256)[0]
        cols = 128 * (m // 8) + 16 * (m % 8) + np.arange(16)
        assert np.all(w[cols] == -3) and np.all(np.delete(w, cols) == 1)


def test_quant_per_tile_rounding():
    blocks = []
    for blk in range(16):  # one row of 4096 columns: two tiles of 8 blocks
        q = np.zeros(256, int)
        if blk == 0:
            q[0] = q[1] = 1
        if blk == 8:
            q[0] = 1
        blocks.append(q4k_block(1.0, 0.0, np.ones(8, int), np.zeros(8, int), q))
    w = ox.dequant_q4k(np.concatenate(blocks), 1, 4096)
    x = np.zeros(4096, F)
    x[0], x[1], x[2048] = 256, 0.96875, -255
    assert ox.project_dequantized(w, x)[0] == 1.0
    assert ox.project_dequantized(w, x, tile=4096)[0] == 1.96875  # one rounding keeps the fraction


def test_dense_tiles_scale_each_tile_on_its_own():
    w = np.zeros((2, 5000), F)
    w[0, 0], w[0, 2048 + 7], w[0, 4096 + 3] = 127.0, 1.0, -0.5
    w[1, :] = 0.0
    q, s = ox.dense_w8_tiles(w)
    assert s.shape == (2, 3)
    assert s[0].tolist() == [1.0, F(1.0) / F(127), F(0.5) / F(127)] and s[1].tolist() == [1.0, 1.0, 1.0]
    assert q[0, 0] == 127 and q[0, 2048 + 7] == 127 and q[0, 4096 + 3] == -127
    x = np.zeros(5000, F)
    x[0], x[2048 + 7], x[4096 + 3] = 1.0, 1.0, 2.0
    got = ox.project_tiles(q, s, x)
    # tile results: 127, bf16(127 * (1/127)) = 1, bf16(-127 * 2 * (0.5/127)) = -1
    assert got[0] == 127.0 and got[1] == 0.0
    # a single per-row scale (1) flushes the last tile's -0.5 to 0 instead
    q1, s1 = ox.requantize_rows(w)
    assert q1[0, 4096 + 3] == 0 and ox.project(q1, s1, x)[0] == 128.0
