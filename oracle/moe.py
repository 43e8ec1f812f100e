"""Routed-expert (MoE) decode block (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, smoke() and bench's CPU baseline.

The reference offloads only the expert projections given expert ids (the GGML
``MUL_MAT_ID`` path, ``ollama-xdna/backend/ggml-xdna.cpp:1301-1441``, and the
Colibri expert group, ``colibri-xdna/backend/backend_xdna.cpp:316-348``: gate,
up, ``silu(g) * u``, down).  The router, top-k and the weighted combine live in
upstream ggml / Colibri, which the reference does not vendor, so the block is
defined here, with the decode layer's rounding points
(``npu_llm/runtime/cpu_backend.py:151-171``):

    r     = f32(W_router) @ f32(bf16(x))                   (64 float32 logits)
    p     = exp(r - max r) / sum(exp(r - max r))            (float32 softmax)
    top-k = the k largest p, ties to the lower expert id; weights = p (no renormalisation)
    e(x)  = bf16(W_down @ bf16((g / (1 + exp(-clip(g, -80, 80)))) * u)),
            g, u = bf16(W_gate @ x), bf16(W_up @ x)
    y     = bf16( sum_k p_k * e_k(x)  +  sum_s e_shared_s(x) )   (float32, k in rank
            order, then the shared experts in order; each product and sum rounded)

Expert weights: ``gate_up`` [E, 2 I, H] (gate rows then up rows, as the dense
layers store them) and ``down`` [E, H, I], all bf16 bits; the shared experts
follow the routed ones in the same arrays.

Pinning: the router/top-k/combine definition is this build's own (parity with
the reference is unpinned -- the reference has no router).  The expert
projection arithmetic is pinned by the reference's expert test pattern
(``ollama-xdna/backend/test_experts.cpp:58-182``, restated in
``tests/test_oracle_moe.py``), the float64 expert check and softmax / top-k
invariants in the same file.
"""

import numpy as np

from oracle.bf16 import from_bits, round_f32

__all__ = ["route", "expert_forward", "moe_forward"]


def route(router_bits, x, top_k):
    """Softmax router and top-k: returns (ids [k], weights [k], probs [E])."""
    r = from_bits(router_bits) @ round_f32(x)
    p = np.exp(r - np.max(r))
    p = p / np.sum(p)
    order = sorted(range(p.shape[0]), key=lambda e: (-float(p[e]), e))[:top_k]
    return np.array(order, dtype=np.int32), p[order].astype(np.float32), p


def expert_forward(gate_up_bits, down_bits, x):
    """One SwiGLU expert on one token: bf16 output (as float32 values)."""
    gu = round_f32(from_bits(gate_up_bits) @ round_f32(x))
    g, u = np.split(gu, 2)
    act = round_f32((g / (1.0 + np.exp(-np.clip(g, -80.0, 80.0)))) * u)
    return round_f32(from_bits(down_bits) @ act)


def moe_forward(x_bits, router_bits, gate_up_bits, down_bits, *, top_k=6, shared=2):
    """The block for T tokens: returns (y bf16 bits [T, H], ids [T, k], weights [T, k])."""
    from oracle.bf16 import to_bits

    x = from_bits(x_bits)
    n_routed = router_bits.shape[0]
    T, H = x.shape
    y = np.empty((T, H), dtype=np.uint16)
    ids = np.empty((T, top_k), dtype=np.int32)
    weights = np.empty((T, top_k), dtype=np.float32)
    for t in range(T):
        ids[t], weights[t], _ = route(router_bits, x[t], top_k)
        acc = np.zeros(H, dtype=np.float32)
        for e, w in zip(ids[t], weights[t]):
            acc = acc + w * expert_forward(gate_up_bits[e], down_bits[e], x[t])
        for s in range(shared):
            e = n_routed + s
            acc = acc + expert_forward(gate_up_bits[e], down_bits[e], x[t])
        y[t] = to_bits(acc)
    return y, ids, weights
