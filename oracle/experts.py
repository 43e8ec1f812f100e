"""Expert-projection offload contracts of the GGML and Colibri backends (oracle).

TEST INFRASTRUCTURE ONLY: imported by tests, never by the product.

Both reference backends hand a CPU-resident MoE model's expert projections to
an accelerator.  Their host code fixes everything but the accelerator's inner
sum:

``decode_colibri``
    Colibri's upload formats, ``colibri-xdna/backend/backend_xdna.cpp:122-136``:
    0 float32, 1 int8 x per-row scale, 2 int4 (low nibble is the even column,
    bias 8) x per-row scale, 4 int4 x per-(row, column // group) scale.
``requantize_rows``
    ``ggml-xdna.cpp:712-731`` (pack_expert) and ``backend_xdna.cpp:138-157``
    (pack_tensor): ``s = max|w| / 127`` (1 for an all-zero row),
    ``q = nearbyint(w / s)`` (round half to even), clamped to +-127.
``project``
    ``backend_xdna.cpp:159-206``: the columns go in 2048-wide tiles; each
    tile's accelerator result is a bf16 and the tiles are summed in float32 in
    tile order.  The accelerator computes ``bf16((sum_c q[r][c] * bf16(x[c]))
    * s[r])`` per tile (the W8 kernel both backends load; its source is not
    in the reference, so the inner sum is taken exactly here, in float64,
    and rounded once to float32).
``mul_mat_id``
    ``ggml-xdna.cpp:1301-1441`` (compute_experts): slot i uses expert
    ``ids[i]`` and input row ``0`` when there is one input row, else row i;
    the dims are at most 2048, so one tile.
``expert_group``
    ``backend_xdna.cpp:316-348``: gate and up projections, ``silu(g) * u`` in
    float32 with ``silu(g) = g / (1 + exp(-g))``, then the down projection.

Pinned by ``tests/test_oracle_experts.py``: the reference's own test
(``colibri-xdna/backend/test_backend_xdna.cpp``: its three cases and
tolerances against float32 sums of the unquantised weights), closed forms of
each format's decode on hand-built bytes (nibble order, bias, ragged last
group), ties-to-even of the requantisation, a constructed two-tile case whose
per-tile rounding differs from one rounding of the whole row, and SwiGLU
identities with identity projections (gate and up not interchangeable).
"""

import numpy as np

from oracle.bf16 import round_f32

__all__ = ["TILE", "decode_colibri", "requantize_rows", "project", "mul_mat_id", "expert_group"]

TILE = 2048


def decode_colibri(weights, scales, fmt, input_size, output_size, group=0):
    """float32 [output][input] values of a Colibri upload (backend_xdna.cpp:122-136)."""
    n, m = int(input_size), int(output_size)
    if fmt == 0:
        return np.asarray(weights, dtype=np.float32).reshape(m, n).copy()
    scales = np.asarray(scales, dtype=np.float32)
    if fmt == 1:
        q = np.asarray(weights, dtype=np.int8).reshape(m, n).astype(np.float32)
        return q * scales[:m, None]
    if fmt not in (2, 4):
        raise ValueError(f"unsupported format {fmt}")
    row_bytes = (n + 1) // 2
    packed = np.asarray(weights, dtype=np.uint8).reshape(m, row_bytes)
    cols = np.arange(n)
    byte = packed[:, cols // 2]
    nib = np.where(cols % 2 == 1, byte >> 4, byte & 15).astype(np.int32) - 8
    if fmt == 2:
        return nib.astype(np.float32) * scales[:m, None]
    groups = (n + group - 1) // group
    s = scales.reshape(m, groups)[:, cols // group]
    # int * float in float32, as the C++ `value * scales[...]`
    return nib.astype(np.float32) * s


def requantize_rows(w):
    """int8 rows and float32 row scales (ggml-xdna.cpp:712-731, backend_xdna.cpp:138-157)."""
    w = np.asarray(w, dtype=np.float32)
    peak = np.max(np.abs(w), axis=1) if w.shape[1] else np.zeros(w.shape[0], np.float32)
    scale = np.where(peak > 0, peak / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w / scale[:, None]), -127, 127).astype(np.int8)
    return q, scale


def project(q, scale, x, tile=TILE):
    """float32 [out]: per-tile bf16 results summed in float32 (backend_xdna.cpp:159-206)."""
    q = np.asarray(q, dtype=np.int8)
    xb = round_f32(np.asarray(x, dtype=np.float32)).astype(np.float64)
    scale = np.asarray(scale, dtype=np.float32)
    total = np.zeros(q.shape[0], dtype=np.float32)
    for t0 in range(0, q.shape[1], tile):
        part = (q[:, t0:t0 + tile].astype(np.float64) @ xb[t0:t0 + tile]).astype(np.float32)
        total = (total + round_f32(part * scale)).astype(np.float32)
    return total


def mul_mat_id(weights, inputs, ids):
    """GGML MUL_MAT_ID (ggml-xdna.cpp:1301-1441): float32 [len(ids)][out]."""
    weights = np.asarray(weights, dtype=np.float32)
    inputs = np.asarray(inputs, dtype=np.float32).reshape(-1, weights.shape[2])
    out = np.empty((len(ids), weights.shape[1]), dtype=np.float32)
    for slot, e in enumerate(ids):
        q, s = requantize_rows(weights[e])
        out[slot] = project(q, s, inputs[0 if inputs.shape[0] == 1 else slot])
    return out


def silu_times(g, u):
    """``(g / (1 + exp(-g))) * u`` in float32 (backend_xdna.cpp:341-342)."""
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return ((g / (np.float32(1.0) + np.exp(-g))) * np.asarray(u, dtype=np.float32)).astype(np.float32)


def expert_group(gates, ups, downs, x):
    """Colibri expert group (backend_xdna.cpp:316-348).

    ``gates``/``ups``/``downs`` are float32 weight matrices (already decoded),
    ``x`` the experts' inputs back to back; returns their outputs back to back.
    """
    n = len(gates)
    x = np.asarray(x, dtype=np.float32).reshape(n, -1)
    out = []
    for i in range(n):
        g = project(*requantize_rows(gates[i]), x[i])
        u = project(*requantize_rows(ups[i]), x[i])
        out.append(project(*requantize_rows(downs[i]), silu_times(g, u)))
    return np.concatenate(out).astype(np.float32)
