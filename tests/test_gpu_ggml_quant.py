"""GGML Q4_K / Q6_K dequant-fused GEMVs and the dense W8-tile MUL_MAT on the
GPU, through the C ABI (include/hk_experts.h), against oracle/experts.py.

Tolerance: one tile is bf16(sum_c w_c * bf16(x_c)); the GPU sums in float32
in its own order where the oracle sums exactly, so a tile may land one bf16
step (at most 2^-7 of its magnitude) away.  A row agrees with the oracle to
within 2^-7 of the sum of its tiles' magnitudes, and most rows exactly.
"""

import numpy as np
import pytest

from _util import announce
from oracle import experts as ox
from tests._expert_cases import q4k_block, random_q4k, random_q6k

pytestmark = pytest.mark.gpu
F = np.float32
Q4K, Q6K = 12, 14


def _dequant(kind, blocks, rows, cols):
    return (ox.dequant_q4k if kind == Q4K else ox.dequant_q6k)(blocks, rows, cols)


def _random_blocks(kind, rng, rows, cols):
    return (random_q4k if kind == Q4K else random_q6k)(rng, rows, cols)


def _tile_bound(w, x):
    total = np.zeros(w.shape[0], np.float64)
    for t0 in range(0, w.shape[1], ox.TILE):
        total += np.abs(ox.project_dequantized(w[:, t0:t0 + ox.TILE], x[t0:t0 + ox.TILE]))
    return total * 2.0 ** -7


def _check(got, want, bound):
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound), (float(err.max()), int(np.argmax(err - bound)))
    return float(np.mean(got == want))


@pytest.mark.parametrize("kind", [Q4K, Q6K])
@pytest.mark.parametrize("input_rows", [1, 6])
def test_quant_mul_mat_id(hk_lib, kind, input_rows):
    from runtime.experts import GgmlExperts

    n_experts, out_dim, in_dim = 10, 300, 2048
    announce(f"ggml quant mul_mat_id type={kind} {n_experts}x{out_dim}x{in_dim} input_rows={input_rows}")
    rng = np.random.default_rng(kind * 10 + input_rows)
    blocks = _random_blocks(kind, rng, n_experts * out_dim, in_dim)
    x = rng.normal(0, 1, (input_rows, in_dim)).astype(F)
    ids = np.array([9, 0, 4, 4, 7, 2], np.int32)
    set_ = GgmlExperts.quant(kind, blocks, n_experts, out_dim, in_dim)
    got = set_.mul_mat_id(x, ids)
    per_expert = blocks.reshape(n_experts, -1)
    exact = []
    for slot, e in enumerate(ids):
        w = _dequant(kind, per_expert[e], out_dim, in_dim)
        row = x[0 if input_rows == 1 else slot]
        exact.append(_check(got[slot], ox.project_dequantized(w, row), _tile_bound(w, row)))
    print(f"exact fraction {np.mean(exact):.3f}")
    assert np.mean(exact) >= 0.9
    set_.close()


@pytest.mark.parametrize("kind", [Q4K, Q6K])
@pytest.mark.parametrize("out_dim,in_dim", [(333, 5120), (37, 256), (2049, 2304)])
def test_quant_dense_mul_mat(hk_lib, kind, out_dim, in_dim):
    from runtime.experts import GgmlExperts

    announce(f"ggml quant dense type={kind} {out_dim}x{in_dim}")
    rng = np.random.default_rng(out_dim + in_dim + kind)
    blocks = _random_blocks(kind, rng, out_dim, in_dim)
    x = rng.normal(0, 1, in_dim).astype(F)
    set_ = GgmlExperts.quant(kind, blocks, 1, out_dim, in_dim)
    got = set_.mul_mat(x)
    w = _dequant(kind, blocks, out_dim, in_dim)
    exact = _check(got, ox.project_dequantized(w, x), _tile_bound(w, x))
    assert exact >= 0.9, exact
    if in_dim > 2048 or out_dim > 2048:
        with pytest.raises(ValueError):
            set_.mul_mat_id(x, np.array([0], np.int32))  # wider than MUL_MAT_ID allows
    set_.close()


def test_quant_per_tile_rounding(hk_lib):
    from runtime.experts import GgmlExperts

    announce("ggml quant per-tile rounding row")
    blocks = []
    for blk in range(16):
        q = np.zeros(256, int)
        if blk == 0:
            q[0] = q[1] = 1
        if blk == 8:
            q[0] = 1
        blocks.append(q4k_block(1.0, 0.0, np.ones(8, int), np.zeros(8, int), q))
    set_ = GgmlExperts.quant(Q4K, np.concatenate(blocks), 1, 1, 4096)
    x = np.zeros(4096, F)
    x[0], x[1], x[2048] = 256, 0.96875, -255
    assert set_.mul_mat(x)[0] == 1.0
    set_.close()


@pytest.mark.parametrize("out_dim,in_dim", [(77, 5000), (4100, 896)])
def test_dense_w8_tiles(hk_lib, out_dim, in_dim):
    from runtime.experts import GgmlExperts

    announce(f"ggml dense w8 {out_dim}x{in_dim}")
    rng = np.random.default_rng(out_dim)
    w = rng.normal(0, 0.05, (out_dim, in_dim)).astype(F)
    w[:, 2048:] *= 0.01  # later tiles on a much smaller range: their own scales matter
    x = rng.normal(0, 1, in_dim).astype(F)
    set_ = GgmlExperts.dense(w)
    got = set_.mul_mat(x)
    q, s = ox.dense_w8_tiles(w)
    want = ox.project_tiles(q, s, x)
    bound = np.zeros(out_dim)
    for t, t0 in enumerate(range(0, in_dim, ox.TILE)):
        bound += np.abs(ox.project_tiles(q[:, t0:t0 + ox.TILE], s[:, t:t + 1], x[t0:t0 + ox.TILE]))
    exact = _check(got, want, bound * 2.0 ** -7)
    assert exact >= 0.9, exact
    with pytest.raises(ValueError):
        set_.mul_mat_id(x, np.array([0], np.int32))  # a dense set is not a MUL_MAT_ID set
    set_.close()


def test_quant_rejections(hk_lib):
    from runtime.experts import GgmlExperts

    announce("ggml quant rejections")
    with pytest.raises(ValueError):
        GgmlExperts.quant(13, np.zeros(144, np.uint8), 1, 1, 256)  # Q5_K is not a native type
    with pytest.raises(ValueError):
        GgmlExperts.quant(Q4K, np.zeros(144, np.uint8), 1, 1, 200)  # not a whole block
    rng = np.random.default_rng(0)
    e = GgmlExperts(rng.normal(0, 1, (8, 4, 32)).astype(F))
    with pytest.raises(ValueError):
        e.mul_mat(np.zeros(32, F))  # a MUL_MAT_ID set has no dense form
    e.close()
    two = GgmlExperts.quant(Q6K, random_q6k(rng, 2 * 4, 256), 2, 4, 256)
    with pytest.raises(ValueError):
        two.mul_mat(np.zeros(256, F))  # dense needs exactly one matrix
    two.close()
