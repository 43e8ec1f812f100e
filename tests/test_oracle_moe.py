"""Pins oracle.moe and the W8 expert projection.

- The reference's own expert test (ollama-xdna/backend/test_experts.cpp:58-182):
  8 experts of 2048x2048 int8 weights with the pattern
  ((e*7 + r*3 + c*5) % 31) - 15, row scales 0.0005*(1 + r%5), inputs
  bf16(0.002*(((e + c) % 17) - 8)); the device output must be within 0.03 of
  the float-accumulated expectation.  Restated here for oracle.quant.project_w8.
- Router: softmax invariants, rank order, ties to the lower expert id.
- Expert and block: float64 evaluations without intermediate rounding;
  planted mistakes (renormalised weights, a dropped shared expert, swapped
  gate/up) are caught.
"""

import numpy as np

from oracle import bf16
from oracle.moe import expert_forward, moe_forward, route
from oracle.quant import project_w8

EXPERTS, ROWS, COLS = 8, 2048, 2048


def _reference_pattern():
    e = np.arange(EXPERTS)[:, None, None]
    r = np.arange(ROWS)[None, :, None]
    c = np.arange(COLS)[None, None, :]
    weights = (((e * 7 + r * 3 + c * 5) % 31) - 15).astype(np.int8)
    scales = (0.0005 * (1 + (np.arange(ROWS) % 5))).astype(np.float32)
    scales = np.broadcast_to(scales, (EXPERTS, ROWS))
    inputs = np.stack([
        bf16.round_f32(np.float32(0.002) * ((((x + np.arange(COLS)) % 17) - 8).astype(np.float32)))
        for x in range(EXPERTS)
    ])
    return weights, scales, inputs


def test_w8_expert_projection_meets_reference_test():
    weights, scales, inputs = _reference_pattern()
    worst = 0.0
    for ex in range(EXPERTS):
        out = project_w8(weights[ex], scales[ex], inputs[ex])
        expected = (weights[ex].astype(np.float32) @ inputs[ex]) * scales[ex]
        worst = max(worst, float(np.abs(out - expected).max()))
        # tighter than the reference's 0.03: one bf16 rounding of the result
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(expected), 2.0**-126))) - 7)
        assert np.all(np.abs(out - expected) <= ulp * 0.5 * 1.0001 + 1e-6)
    assert worst < 0.03


def test_router_softmax_topk_and_ties():
    rng = np.random.default_rng(3)
    router = bf16.to_bits(rng.normal(0, 0.02, (64, 256)).astype(np.float32))
    x = bf16.round_f32(rng.normal(0, 1, 256).astype(np.float32))
    ids, w, p = route(router, x, 6)
    assert abs(float(p.sum()) - 1.0) < 1e-5 and np.all(p > 0)
    assert list(ids) == list(np.argsort(-p.astype(np.float64), kind="stable")[:6])
    assert np.all(np.diff(w) <= 0)
    # two experts with identical rows tie exactly: the lower id ranks first
    router2 = router.copy()
    best = int(ids[0])
    twin = 63 if best != 63 else 62
    router2[twin] = router2[best]
    ids2, _, _ = route(router2, x, 6)
    lo, hi = sorted((best, twin))
    assert list(ids2[:2]) == [lo, hi]


def _f64_expert(gu_bits, d_bits, x):
    gu = bf16.from_bits(gu_bits).astype(np.float64) @ x.astype(np.float64)
    g, u = np.split(gu, 2)
    return bf16.from_bits(d_bits).astype(np.float64) @ (g / (1 + np.exp(-g)) * u)


def _model(rng, n_exp=8, shared=2, H=128, inter=64, std=0.1):
    router = bf16.to_bits(rng.normal(0, 0.05, (n_exp, H)).astype(np.float32))
    gate_up = bf16.to_bits(rng.normal(0, std, (n_exp + shared, 2 * inter, H)).astype(np.float32))
    down = bf16.to_bits(rng.normal(0, std, (n_exp + shared, H, inter)).astype(np.float32))
    return router, gate_up, down


def test_expert_tracks_float64():
    rng = np.random.default_rng(4)
    _, gate_up, down = _model(rng)
    x = bf16.round_f32(rng.normal(0, 1, 128).astype(np.float32))
    out = expert_forward(gate_up[0], down[0], x)
    ref = _f64_expert(gate_up[0], down[0], x)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-2


def test_block_tracks_float64_and_catches_planted_mistakes():
    rng = np.random.default_rng(5)
    router, gate_up, down = _model(rng)
    x_bits = bf16.to_bits(rng.normal(0, 1, (4, 128)).astype(np.float32))
    y, ids, w = moe_forward(x_bits, router, gate_up, down, top_k=3, shared=2)
    x = bf16.from_bits(x_bits)
    for t in range(4):
        r = bf16.from_bits(router).astype(np.float64) @ x[t].astype(np.float64)
        p = np.exp(r - r.max())
        p /= p.sum()
        top = np.argsort(-p, kind="stable")[:3]
        assert list(top) == list(ids[t])
        ref = sum(p[e] * _f64_expert(gate_up[e], down[e], x[t]) for e in top)
        ref = ref + sum(_f64_expert(gate_up[8 + s], down[8 + s], x[t]) for s in range(2))
        got = bf16.from_bits(y[t]).astype(np.float64)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2
        renorm = sum(p[e] / p[top].sum() * _f64_expert(gate_up[e], down[e], x[t]) for e in top)
        renorm = renorm + sum(_f64_expert(gate_up[8 + s], down[8 + s], x[t]) for s in range(2))
        no_shared = ref - _f64_expert(gate_up[9], down[9], x[t])
        for wrong in (renorm, no_shared):
            assert np.linalg.norm(got - wrong) / np.linalg.norm(wrong) > 2e-2
