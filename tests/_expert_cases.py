"""Inputs of the reference's own expert-offload tests, restated as arrays.

``colibri-xdna/backend/test_backend_xdna.cpp`` builds its three cases from
closed-form patterns (sin/cos of float32 arguments, integer patterns for the
int4 case); ``ollama-xdna/backend/test_experts.cpp:58-87`` builds an 8 x 2048
x 2048 int8 pattern with per-row scales.  Each builder returns the inputs and
the reference test's expected values, computed as that test computes them
(float32 sums of the unquantised weights), and the tolerance it asserts.
"""

import numpy as np

F = np.float32


def colibri_matmul_case():
    """test_backend_xdna.cpp:23-45: fmt 0, 32 -> 16, max error < 0.15."""
    n, m = 32, 16
    x = np.sin(np.arange(1, n + 1, dtype=F) * F(0.17)).astype(F)
    rows = np.arange(m, dtype=F)[:, None] + F(3)
    cols = np.arange(n, dtype=F)[None, :] + F(1)
    w = np.cos((rows * cols).astype(F) * F(0.013)).astype(F)
    expected = np.zeros(m, F)
    for c in range(n):  # float32 accumulation in column order
        expected = (expected + w[:, c] * x[c]).astype(F)
    return dict(weights=w, scales=None, fmt=0, input_size=n, output_size=m, group=0, x=x,
                expected=expected, tol=0.15)


def colibri_grouped_int4_case():
    """test_backend_xdna.cpp:47-76: fmt 4, 33 -> 3, group 16, max error < 0.08."""
    n, m, group = 33, 3, 16
    row_bytes = (n + 1) // 2
    groups = (n + group - 1) // group
    packed = np.zeros((m, row_bytes), np.uint8)
    scales = np.zeros((m, groups), F)
    x = ((np.arange(n) % 7 - 3) * 0.125).astype(F)
    expected = np.zeros(m, F)
    for r in range(m):
        for b in range(groups):
            scales[r, b] = F(0.02) * F(r + b + 1)
        for c in range(n):
            value = (r * 5 + c * 3) % 16 - 8
            if c & 1:
                packed[r, c // 2] |= np.uint8((value + 8) << 4)
            else:
                packed[r, c // 2] |= np.uint8(value + 8)
            expected[r] = F(expected[r] + F(F(value) * scales[r, c // group]) * x[c])
    return dict(weights=packed.reshape(-1), scales=scales.reshape(-1), fmt=4, input_size=n, output_size=m,
                group=group, x=x, expected=expected, tol=0.08)


def colibri_expert_group_case():
    """test_backend_xdna.cpp:78-139: two experts, 32 -> 24 -> 32, max error < 0.15."""
    experts, n, hidden = 2, 32, 24
    gates, ups, downs, xs, expected = [], [], [], [], []
    for e in range(experts):
        col = np.arange(n, dtype=F)
        x = np.sin((F(e + 1) * (col + F(2))).astype(F) * F(0.09)).astype(F)
        r = np.arange(hidden, dtype=F)[:, None]
        c = np.arange(n, dtype=F)[None, :]
        g = (np.cos((F(e + 2) * (r + F(1)) + c).astype(F) * F(0.031)) * F(0.2)).astype(F)
        u = (np.sin((F(e + 1) * (c + F(1)) + r).astype(F) * F(0.027)) * F(0.2)).astype(F)
        dr = np.arange(n, dtype=F)[:, None]
        dc = np.arange(hidden, dtype=F)[None, :]
        d = (np.cos(((dr + F(1)) * (dc + F(3)) + F(e)).astype(F) * F(0.019)) * F(0.1)).astype(F)
        g_ref = np.zeros(hidden, F)
        u_ref = np.zeros(hidden, F)
        for k in range(n):
            g_ref = (g_ref + g[:, k] * x[k]).astype(F)
            u_ref = (u_ref + u[:, k] * x[k]).astype(F)
        silu = (g_ref / (F(1) + np.exp(-g_ref))).astype(F)
        y = np.zeros(n, F)
        for k in range(hidden):
            y = (y + (d[:, k] * silu[k]).astype(F) * u_ref[k]).astype(F)
        gates.append(g), ups.append(u), downs.append(d), xs.append(x), expected.append(y)
    return dict(gates=gates, ups=ups, downs=downs, x=np.concatenate(xs), expected=np.concatenate(expected),
                tol=0.15, input_size=n, hidden=hidden)


def ggml_expert_pattern_case():
    """test_experts.cpp:58-87,155-182: 8 experts x 2048 x 2048, every 17th row, max error < 0.03.

    The reference test feeds its int8 pattern and scales to the accelerator
    directly; through the MUL_MAT_ID contract the weights arrive as float32
    (``q * s``) and are requantised, as ``pack_expert`` does.
    """
    experts, rows, cols = 8, 2048, 2048
    e = np.arange(experts)[:, None, None]
    r = np.arange(rows)[None, :, None]
    c = np.arange(cols)[None, None, :]
    q = (((e * 7 + r * 3 + c * 5) % 31) - 15).astype(np.int8)
    scales = (F(0.0005) * (1 + np.arange(rows) % 5).astype(F)).astype(F)
    weights = (q.astype(F) * scales[None, :, None]).astype(F)
    x = (F(0.002) * (((np.arange(experts)[:, None] + np.arange(cols)[None, :]) % 17) - 8).astype(F)).astype(F)
    check_rows = np.arange(0, rows, 17)
    expected = np.empty((experts, check_rows.size), F)
    for i in range(experts):
        # float32 sums of q * bf16(x) (x is bf16-exact here), then * scale
        acc = (q[i][check_rows].astype(np.float64) @ x[i].astype(np.float64)).astype(F)
        expected[i] = acc * scales[check_rows]
    return dict(weights=weights, x=x, ids=np.arange(experts, dtype=np.int32), check_rows=check_rows,
                expected=expected, tol=0.03)


def tile_rounding_row():
    """One row over two 2048-column tiles whose per-tile bf16 results sum to
    1.0, while one rounding of the whole row would give 1.96875.

    Tile 0: 127*2 + 1*2 + 1*0.96875 = 256.96875 -> bf16 256 (spacing 2 there).
    Tile 1: -127*2 - 1*1 = -255, exact.  Row max |w| = 127, so the scale is 1
    and the requantisation keeps the integers.
    """
    w = np.zeros((1, 4096), F)
    x = np.zeros(4096, F)
    w[0, 0], x[0] = 127, 2
    w[0, 1], x[1] = 1, 2
    w[0, 2], x[2] = 1, 0.96875
    w[0, 2048], x[2048] = -127, 2
    w[0, 2049], x[2049] = -1, 1
    return w, x


# ---- GGML Q4_K / Q6_K block writers ----
#
# Written from ggml's published block layouts (the reader under test is
# oracle/experts.py), column by column:
#   Q4_K (144 bytes): fp16 d, fp16 dmin, 12 bytes of 6-bit (scale, min) pairs
#     for the eight 32-column sub-blocks, then 128 bytes of nibbles; column c
#     sits in byte 16 + 32 * (c // 64) + c % 32, in the low nibble when
#     c % 64 < 32, else the high nibble, and belongs to sub-block c // 32.
#     Pairs 0..3 take the low 6 bits of bytes j (scale) and j + 4 (min);
#     pairs 4..7 keep their low 4 bits in byte j + 4 (scale low, min high) and
#     their top 2 bits in the top bits of bytes j - 4 (scale) and j (min).
#   Q6_K (210 bytes): ql[128], qh[64], int8 scales[16], fp16 d; 6-bit q (the
#     weight is d * scale * (q - 32)); column c in half h = c // 128, quarter
#     k = (c % 128) // 32, l = c % 32: low 4 bits in ql[64 h + l + 32 (k & 1)]
#     (low nibble for k < 2, else high), top 2 bits in bits 2k, 2k + 1 of
#     qh[32 h + l]; scale index 8 h + (c % 128) // 16.

def f16_bytes(value):
    return np.frombuffer(np.float16(value).tobytes(), np.uint8)


def q4k_block(d, dmin, sc, mn, q):
    """One Q4_K block: sc, mn 8 values in 0..63, q 256 values in 0..15."""
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = f16_bytes(d), f16_bytes(dmin)
    s = np.zeros(12, np.uint32)
    for j in range(4):
        s[j] |= sc[j] & 63
        s[j + 4] |= mn[j] & 63
    for j in range(4, 8):
        s[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (mn[j] >> 4) << 6
    b[4:16] = s.astype(np.uint8)
    for c in range(256):
        i = 16 + 32 * (c // 64) + c % 32
        b[i] |= (q[c] & 15) if c % 64 < 32 else (q[c] & 15) << 4
    return b


def q6k_block(d, sc, q):
    """One Q6_K block: sc 16 int8 values, q 256 values in 0..63."""
    b = np.zeros(210, np.uint8)
    for c in range(256):
        h, k, l = c // 128, (c % 128) // 32, c % 32
        i = 64 * h + l + 32 * (k & 1)
        b[i] |= (q[c] & 15) if k < 2 else (q[c] & 15) << 4
        b[128 + 32 * h + l] |= (q[c] >> 4) << (2 * k)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = f16_bytes(d)
    return b


def _f16_pairs(values):
    return np.asarray(values, np.float16).view(np.uint8).reshape(np.shape(values) + (2,))


def random_q4k(rng, rows, cols):
    """Random valid Q4_K rows: random quants, scales and mins; d, dmin small."""
    nb = cols // 256
    b = rng.integers(0, 256, (rows, nb, 144), dtype=np.uint8)
    b[..., 0:2] = _f16_pairs(rng.uniform(0.002, 0.01, (rows, nb)))
    b[..., 2:4] = _f16_pairs(rng.uniform(0.001, 0.01, (rows, nb)))
    return b.reshape(-1)


def random_q6k(rng, rows, cols):
    nb = cols // 256
    b = rng.integers(0, 256, (rows, nb, 210), dtype=np.uint8)
    b[..., 208:210] = _f16_pairs(rng.uniform(0.0005, 0.002, (rows, nb)))
    return b.reshape(-1)
