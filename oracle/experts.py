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

``dense_w8_tiles`` / ``project_tiles``
    The dense GGML MUL_MAT (``ggml-xdna.cpp:768-832`` pack_dense_tile,
    ``:1444-1538``): one int8 scale per (row, 2048-column tile).
``dequant_q4k`` / ``dequant_q6k`` / ``project_dequantized``
    GGML's Q4_K and Q6_K blocks as the reference's native kernels read them
    (``npu_llm/kernels/project_q4k_bf16.cc:76-117``,
    ``project_q6k_bf16.cc:53-99``; the formats are upstream ggml's, from the
    ggml bundled with Ollama v0.33.3, which is not in the reference tree):
    per tile ``bf16(sum_c w_c * bf16(x_c))`` with no scale, tiles summed in
    float32.  Q4_K: ``w = (d * sc) * q - dmin * m`` per 32-column sub-block,
    6-bit (sc, m) pairs packed in 12 bytes; Q6_K: ``w = (d * sc) * (q - 32)``
    per 16 columns, 6-bit q from a low nibble and a 2-bit high part.

Pinned by ``tests/test_oracle_experts.py``: the reference's own test
(``colibri-xdna/backend/test_backend_xdna.cpp``: its three cases and
tolerances against float32 sums of the unquantised weights), closed forms of
each format's decode on hand-built bytes (nibble order, bias, ragged last
group), ties-to-even of the requantisation, a constructed two-tile case whose
per-tile rounding differs from one rounding of the whole row, and SwiGLU
identities with identity projections (gate and up not interchangeable);
the dense tiles' scales on a row whose tiles differ in range; for Q4_K and
Q6_K, single-quant probes that locate every nibble and high-bit pair in its
column, scale/min probes for every sub-block with the 6-bit pairs packed by
the published layout written out in the test, fp16 special values against
numpy's float16, and the two-tile rounding case built from Q4_K blocks.  No
reference fixture holds Q4_K or Q6_K data.
"""

import numpy as np

from oracle.bf16 import round_f32

__all__ = ["TILE", "decode_colibri", "requantize_rows", "project", "mul_mat_id", "expert_group",
           "dense_w8_tiles", "project_tiles", "dequant_q4k", "dequant_q6k", "project_dequantized",
           "Q4K_BYTES", "Q6K_BYTES"]

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


# ---- dense W8 tiles ----

def dense_w8_tiles(w, tile=TILE):
    """int8 [out][in] and float32 [out][tiles]: one scale per (row, tile) (ggml-xdna.cpp:800-826)."""
    w = np.asarray(w, dtype=np.float32)
    tiles = -(-w.shape[1] // tile)
    q = np.zeros(w.shape, np.int8)
    s = np.zeros((w.shape[0], tiles), np.float32)
    for t in range(tiles):
        qt, st = requantize_rows(w[:, t * tile:(t + 1) * tile])
        q[:, t * tile:(t + 1) * tile] = qt
        s[:, t] = st
    return q, s


def project_tiles(q, scales, x, tile=TILE):
    """Like ``project`` with the scale of each tile from ``scales[:, t]``."""
    q = np.asarray(q, dtype=np.int8)
    xb = round_f32(np.asarray(x, dtype=np.float32)).astype(np.float64)
    total = np.zeros(q.shape[0], dtype=np.float32)
    for t, t0 in enumerate(range(0, q.shape[1], tile)):
        part = (q[:, t0:t0 + tile].astype(np.float64) @ xb[t0:t0 + tile]).astype(np.float32)
        total = (total + round_f32(part * scales[:, t])).astype(np.float32)
    return total


# ---- GGML Q4_K / Q6_K ----

QK = 256
Q4K_BYTES = 144
Q6K_BYTES = 210


def _f16(lo, hi):
    """IEEE half from two bytes (little endian), widened exactly to float32."""
    bits = (np.asarray(lo, np.uint16) | (np.asarray(hi, np.uint16) << 8)).astype(np.uint16)
    return bits.view(np.float16).astype(np.float32)


def _q4k_scale_min(sb):
    """6-bit (scale, min) of the 8 sub-blocks from the 12 packed bytes [..., 12]
    (project_q4k_bf16.cc:54-68, GGML's get_scale_min_k4)."""
    sb = sb.astype(np.uint32)
    sc = np.empty(sb.shape[:-1] + (8,), np.uint32)
    mn = np.empty_like(sc)
    for j in range(4):
        sc[..., j] = sb[..., j] & 63
        mn[..., j] = sb[..., j + 4] & 63
    for j in range(4, 8):
        sc[..., j] = (sb[..., j + 4] & 0x0F) | ((sb[..., j - 4] >> 6) << 4)
        mn[..., j] = (sb[..., j + 4] >> 4) | ((sb[..., j] >> 6) << 4)
    return sc, mn


def dequant_q4k(blocks, out_dim, in_dim):
    """float32 [out][in] of Q4_K rows (project_q4k_bf16.cc:88-114)."""
    nb = in_dim // QK
    b = np.asarray(blocks, np.uint8).reshape(out_dim, nb, Q4K_BYTES)
    d = _f16(b[..., 0], b[..., 1])
    dmin = _f16(b[..., 2], b[..., 3])
    sc, mn = _q4k_scale_min(b[..., 4:16])
    dsc = (d[..., None] * sc.astype(np.float32)).astype(np.float32)  # [out][nb][8]
    msc = (dmin[..., None] * mn.astype(np.float32)).astype(np.float32)
    qs = b[..., 16:].reshape(out_dim, nb, 4, 32)  # group g of 64 columns: 32 bytes
    w = np.empty((out_dim, nb, 4, 64), np.float32)
    lo = (qs & 15).astype(np.float32)
    hi = (qs >> 4).astype(np.float32)
    for g in range(4):
        w[:, :, g, :32] = (dsc[:, :, 2 * g, None] * lo[:, :, g]).astype(np.float32) - msc[:, :, 2 * g, None]
        w[:, :, g, 32:] = (dsc[:, :, 2 * g + 1, None] * hi[:, :, g]).astype(np.float32) - msc[:, :, 2 * g + 1, None]
    return w.reshape(out_dim, in_dim)


def dequant_q6k(blocks, out_dim, in_dim):
    """float32 [out][in] of Q6_K rows (project_q6k_bf16.cc:66-96)."""
    nb = in_dim // QK
    b = np.asarray(blocks, np.uint8).reshape(out_dim, nb, Q6K_BYTES)
    d = _f16(b[..., 208], b[..., 209])
    w = np.empty((out_dim, nb, 2, 128), np.float32)
    idx = np.arange(32) // 16
    for half in range(2):
        ql = b[..., half * 64:half * 64 + 64].astype(np.int32)
        qh = b[..., 128 + half * 32:128 + half * 32 + 32].astype(np.int32)
        sc = b[..., 192 + half * 8:192 + half * 8 + 8].view(np.int8).astype(np.float32)
        q = [
            ((ql[..., :32] & 15) | ((qh & 3) << 4)) - 32,
            ((ql[..., 32:] & 15) | (((qh >> 2) & 3) << 4)) - 32,
            ((ql[..., :32] >> 4) | (((qh >> 4) & 3) << 4)) - 32,
            ((ql[..., 32:] >> 4) | (((qh >> 6) & 3) << 4)) - 32,
        ]
        for k in range(4):
            ds = (d[..., None] * sc[..., idx + 2 * k]).astype(np.float32)  # [out][nb][32]
            w[:, :, half, 32 * k:32 * k + 32] = (ds * q[k].astype(np.float32)).astype(np.float32)
    return w.reshape(out_dim, in_dim)


def project_dequantized(w, x, tile=TILE):
    """float32 [out]: per tile bf16(sum_c w_c * bf16(x_c)) (exact sum, rounded once
    to float32), tiles summed in float32."""
    w = np.asarray(w, dtype=np.float32).astype(np.float64)
    xb = round_f32(np.asarray(x, dtype=np.float32)).astype(np.float64)
    total = np.zeros(w.shape[0], dtype=np.float32)
    for t0 in range(0, w.shape[1], tile):
        part = (w[:, t0:t0 + tile] @ xb[t0:t0 + tile]).astype(np.float32)
        total = (total + round_f32(part)).astype(np.float32)
    return total
