"""Routed-expert block on the GPU against oracle/moe.py, and the W8 expert
GEMV against the reference's own expert test pattern
(ollama-xdna/backend/test_experts.cpp:58-182)."""

import numpy as np
import pytest

from _util import announce, rel_l2
from oracle import bf16
from oracle.moe import moe_forward, route

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def moe_weights():
    from runtime.moe import synthetic_moe

    return synthetic_moe(seed=0)


@pytest.fixture(scope="module")
def block(moe_weights):
    from runtime.moe import MoEBlock

    router, gate_up, down = moe_weights
    b = MoEBlock(router, gate_up, down, top_k=6, shared=2, max_tokens=16)
    yield b
    b.close()


def _tie_gap(probs, k):
    """Gap between the k-th and (k+1)-th largest router probabilities."""
    s = np.sort(probs)[::-1]
    return float(s[k - 1] - s[k])


@pytest.mark.parametrize("tokens", [1, 2, 4, 8, 16])
def test_moe_block_matches_oracle(block, moe_weights, tokens):
    router, gate_up, down = moe_weights
    announce(f"moe block T={tokens}")
    rng = np.random.default_rng(100 + tokens)
    x = bf16.to_bits(rng.normal(0, 1, (tokens, 2048)).astype(np.float32))
    y, ids, w = block.forward(x)
    ref_y, ref_ids, ref_w = moe_forward(x, router, gate_up, down, top_k=6, shared=2)
    for t in range(tokens):
        _, _, probs = route(router, bf16.from_bits(x[t]), 6)
        if not np.array_equal(ids[t], ref_ids[t]):
            # only a float32 near-tie of the router may reorder or swap experts
            gaps = [_tie_gap(probs, k) for k in range(1, 7)]
            assert min(gaps) < 1e-6, (t, ids[t], ref_ids[t], gaps)
            continue
        np.testing.assert_allclose(w[t], ref_w[t], rtol=1e-5, atol=1e-7)
        err = rel_l2(bf16.from_bits(y[t]), bf16.from_bits(ref_y[t]))
        assert err <= 1e-2, (t, err)


def test_moe_block_beyond_16_tokens_matches_oracle(moe_weights):
    """24 tokens: groups of more than 16 rows run on the grouped tile GEMM
    (up to 16 on the expert slabs), and the top-k waves take two tokens each."""
    from runtime.moe import MoEBlock

    router, gate_up, down = moe_weights
    announce("moe block T=24 (grouped tile GEMM)")
    b = MoEBlock(router, gate_up, down, top_k=6, shared=2, max_tokens=32)
    try:
        rng = np.random.default_rng(124)
        x = bf16.to_bits(rng.normal(0, 1, (24, 2048)).astype(np.float32))
        y, ids, w = b.forward(x)
    finally:
        b.close()
    ref_y, ref_ids, ref_w = moe_forward(x, router, gate_up, down, top_k=6, shared=2)
    for t in range(24):
        if not np.array_equal(ids[t], ref_ids[t]):
            _, _, probs = route(router, bf16.from_bits(x[t]), 6)
            assert min(_tie_gap(probs, k) for k in range(1, 7)) < 1e-6, (t, ids[t], ref_ids[t])
            continue
        np.testing.assert_allclose(w[t], ref_w[t], rtol=1e-5, atol=1e-7)
        assert rel_l2(bf16.from_bits(y[t]), bf16.from_bits(ref_y[t])) <= 1e-2, t


def test_moe_experts_with_given_routing(block, moe_weights):
    """The MUL_MAT_ID form with caller ids equals the routed forward."""
    announce("moe experts with given ids")
    rng = np.random.default_rng(7)
    x = bf16.to_bits(rng.normal(0, 1, (5, 2048)).astype(np.float32))
    y, ids, w = block.forward(x)
    y2 = block.experts(x, ids, w)
    np.testing.assert_array_equal(y, y2)
    bad = ids.copy()
    bad[0, 0] = 64
    with pytest.raises(ValueError):
        block.experts(x, bad, w)


def test_moe_experts_repeated_ids_beyond_16_rows(block, moe_weights):
    """Caller ids may name one expert several times per token: 3 tokens x 6
    times expert 3 is 18 rows for one expert, more than the expert slabs
    take, so the grouped tile GEMM runs; against the oracle's experts and
    combine (oracle/moe.py moe_forward's order)."""
    from oracle.moe import expert_forward

    router, gate_up, down = moe_weights
    announce("moe experts, one expert named 18 times")
    rng = np.random.default_rng(9)
    x = bf16.to_bits(rng.normal(0, 1, (3, 2048)).astype(np.float32))
    ids = np.full((3, 6), 3, dtype=np.int32)
    w = rng.uniform(0.05, 0.3, (3, 6)).astype(np.float32)
    y = block.experts(x, ids, w)
    for t in range(3):
        xt = bf16.from_bits(x[t])
        e3 = expert_forward(gate_up[3], down[3], xt)
        acc = np.zeros(2048, dtype=np.float32)
        for k in range(6):
            acc = acc + w[t, k] * e3
        for s_ in range(2):
            acc = acc + expert_forward(gate_up[64 + s_], down[64 + s_], xt)
        assert rel_l2(bf16.from_bits(y[t]), bf16.from_bits(bf16.to_bits(acc))) <= 1e-2, t


def test_w8_expert_gemv_reference_pattern(hk_lib):
    """8 experts x 2048x2048 int8 with the reference test's pattern, scales and
    inputs; max error against the float-accumulated expectation < 0.03 (the
    reference's bound) and within one bf16 rounding."""
    from runtime import hip

    announce("w8 expert gemv, reference pattern")
    E, R, C = 8, 2048, 2048
    r = np.arange(R)[:, None]
    c = np.arange(C)[None, :]
    worst = 0.0
    out_buf = hip.DeviceBuffer(2 * R)
    for e in range(E):
        wq = (((e * 7 + r * 3 + c * 5) % 31) - 15).astype(np.int8)
        scale = (0.0005 * (1 + (np.arange(R) % 5))).astype(np.float32)
        x = bf16.to_bits(np.float32(0.002) * ((((e + np.arange(C)) % 17) - 8).astype(np.float32)))
        Q, S, X = (hip.DeviceBuffer.from_array(a) for a in (wq, scale, x))
        hip.check(hk_lib.hk_gemv_w8(Q.ptr, S.ptr, X.ptr, None, None, out_buf.ptr, None, R, C, None), "w8")
        hip.check(hk_lib.hk_stream_sync(None), "sync")
        got = bf16.from_bits(out_buf.read(np.uint16, R))
        expected = (wq.astype(np.float32) @ bf16.from_bits(x)) * scale
        worst = max(worst, float(np.abs(got - expected).max()))
        # a float32 sum in another order may land on the other side of a
        # bf16 rounding boundary: one bf16 step
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(expected), 2.0**-126))) - 7)
        assert np.all(np.abs(got - expected) <= ulp * 1.0001 + 1e-6)
    assert worst < 0.03
