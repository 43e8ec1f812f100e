"""The expert-offload shims (include/hk_experts.h) on the GPU, through the C
ABI, against oracle/experts.py and the reference's own tests
(colibri-xdna/backend/test_backend_xdna.cpp, ollama-xdna/backend/test_experts.cpp).

Tolerances.  One projection tile is ``bf16((sum q * bf16(x)) * s)``: the GPU
sums in float32 in its own order where the oracle sums exactly, so a tile may
land on the neighbouring bf16 value, one bf16 step (at most 2^-7 of the
value) away.  A projection therefore agrees with the oracle to within 2^-7 of
the sum of its tiles' magnitudes.  Expert groups chain three projections and a
SwiGLU, so they are held to rel-L2 <= 1e-2 against the oracle (the float
tolerance of the decode path) and to the reference test's absolute bounds.
"""

import numpy as np
import pytest

from _util import announce, rel_l2
from oracle import experts as ox
from tests._expert_cases import (colibri_expert_group_case, colibri_grouped_int4_case, colibri_matmul_case,
                                 ggml_expert_pattern_case, tile_rounding_row)

pytestmark = pytest.mark.gpu
F = np.float32


@pytest.fixture(scope="module")
def coli(hk_lib):
    from runtime import experts

    experts.coli_init(0)
    yield experts
    experts.coli_shutdown()


def _tile_bound(q, s, x):
    """2^-7 x the sum over tiles of |tile result| (the oracle's own tiles)."""
    total = np.zeros(q.shape[0], np.float64)
    for t0 in range(0, q.shape[1], ox.TILE):
        total += np.abs(ox.project(q[:, t0:t0 + ox.TILE], s, x[t0:t0 + ox.TILE]))
    return total * 2.0 ** -7


def _assert_projection(got, w, x):
    q, s = ox.requantize_rows(w)
    want = ox.project(q, s, x)
    err = np.abs(got.astype(np.float64) - want)
    bound = _tile_bound(q, s, x)
    assert np.all(err <= bound), (float(err.max()), int(np.argmax(err - bound)))
    return float(np.mean(got == want))


# ---- Colibri ----

@pytest.mark.parametrize("build", [colibri_matmul_case, colibri_grouped_int4_case])
def test_colibri_reference_matmul_cases(coli, build):
    case = build()
    announce(f"coli matmul reference case fmt={case['fmt']}")
    got = coli.coli_matmul(case["weights"], case["scales"], case["fmt"], case["x"], case["input_size"],
                           case["output_size"], case["group"])
    assert np.max(np.abs(got - case["expected"])) < case["tol"]
    w = ox.decode_colibri(case["weights"], case["scales"], case["fmt"], case["input_size"], case["output_size"],
                          case["group"])
    _assert_projection(got, w, case["x"])


def test_colibri_reference_expert_group(coli):
    announce("coli expert group reference case")
    case = colibri_expert_group_case()
    n, hid = case["input_size"], case["hidden"]
    g = [coli.ColiTensor(w, None, 0, n, hid) for w in case["gates"]]
    u = [coli.ColiTensor(w, None, 0, n, hid) for w in case["ups"]]
    d = [coli.ColiTensor(w, None, 0, hid, n) for w in case["downs"]]
    got = coli.expert_group(g, u, d, case["x"])
    assert np.max(np.abs(got - case["expected"])) < case["tol"]
    want = ox.expert_group(case["gates"], case["ups"], case["downs"], case["x"])
    assert rel_l2(got, want) <= 1e-2
    for t in g + u + d:
        t.close()


def _random_upload(rng, fmt, n, m, group):
    if fmt == 0:
        return rng.normal(0, 0.2, (m, n)).astype(F), None
    if fmt == 1:
        return rng.integers(-127, 128, (m, n)).astype(np.int8), rng.uniform(1e-3, 2e-3, m).astype(F)
    packed = rng.integers(0, 256, (m, (n + 1) // 2)).astype(np.uint8)
    if fmt == 2:
        return packed, rng.uniform(1e-2, 2e-2, m).astype(F)
    return packed, rng.uniform(1e-2, 2e-2, (m, (n + group - 1) // group)).astype(F)


@pytest.mark.parametrize("fmt", [0, 1, 2, 4])
def test_colibri_formats_over_ragged_tiles(coli, fmt):
    n, m, group = 4100, 37, 32  # three tiles, the last of 4 columns
    announce(f"coli matmul fmt={fmt} {n}->{m}")
    rng = np.random.default_rng(40 + fmt)
    w, s = _random_upload(rng, fmt, n, m, group)
    x = rng.normal(0, 1, n).astype(F)
    got = coli.coli_matmul(w, s, fmt, x, n, m, group)
    dense = ox.decode_colibri(w, s, fmt, n, m, group)
    exact = _assert_projection(got, dense, x)
    assert exact >= 0.5, exact


def test_colibri_tile_rounding_row(coli):
    announce("coli per-tile rounding row")
    w, x = tile_rounding_row()
    got = coli.coli_matmul(w, None, 0, x, w.shape[1], 1)
    assert got[0] == 1.0


@pytest.mark.parametrize("count,n,mid", [(8, 2048, 1408), (3, 2500, 2100), (1, 40, 24)])
def test_colibri_expert_group_matches_oracle(coli, count, n, mid):
    announce(f"coli expert group count={count} {n}->{mid}->{n}")
    rng = np.random.default_rng(count * 1000 + n)
    gw = [rng.normal(0, 0.05, (mid, n)).astype(F) for _ in range(count)]
    uw = [rng.normal(0, 0.05, (mid, n)).astype(F) for _ in range(count)]
    dw = [rng.normal(0, 0.05, (n, mid)).astype(F) for _ in range(count)]
    x = rng.normal(0, 1, count * n).astype(F)
    g = [coli.ColiTensor(w, None, 0, n, mid) for w in gw]
    u = [coli.ColiTensor(w, None, 0, n, mid) for w in uw]
    d = [coli.ColiTensor(w, None, 0, mid, n) for w in dw]
    got = coli.expert_group(g, u, d, x)
    want = ox.expert_group(gw, uw, dw, x)
    err = rel_l2(got, want)
    print(f"rel_l2={err:.2e} max_abs={np.max(np.abs(got - want)):.3e} exact={np.mean(got == want):.3f}")
    assert err <= 1e-2
    if count == 1:
        single = coli.expert_mlp(g[0], u[0], d[0], x)
        assert np.array_equal(single, got)
    for t in g + u + d:
        t.close()


def test_colibri_rejections_and_update(coli):
    import ctypes

    announce("coli rejections and update")
    rng = np.random.default_rng(7)
    n, mid = 64, 48
    mk = lambda shape: rng.normal(0, 0.1, shape).astype(F)
    g = [coli.ColiTensor(mk((mid, n)), None, 0, n, mid) for _ in range(9)]
    u = [coli.ColiTensor(mk((mid, n)), None, 0, n, mid) for _ in range(9)]
    dw = [mk((n, mid)) for _ in range(9)]
    d = [coli.ColiTensor(w, None, 0, mid, n) for w in dw]
    x = rng.normal(0, 1, 9 * n).astype(F)
    with pytest.raises(RuntimeError):
        coli.expert_group(g, u, d, x)  # 9 experts: more than a group holds
    odd = coli.ColiTensor(mk((mid, n + 1)), None, 0, n + 1, mid)
    with pytest.raises(RuntimeError):
        coli.expert_group([g[0], odd], u[:2], d[:2], x[:2 * n])  # gate and up disagree
    with pytest.raises(RuntimeError):
        coli.expert_group(g[:1], u[:1], [g[1]], x[:n])  # down is not mid -> n
    with pytest.raises(RuntimeError):
        coli.ColiTensor(np.zeros(16, np.uint8), np.ones(1, F), 3, 32, 1)  # format 3 is not accepted
    with pytest.raises(RuntimeError):
        coli.ColiTensor(mk((4, 4)), None, 0, 4, 4, device=1)
    lib = coli.lib()
    arr = lambda ts: (ctypes.c_void_p * len(ts))(*[t.handle for t in ts])
    out = np.zeros(n, F)
    rows = (ctypes.c_int * 1)(2)
    assert lib.coli_cuda_expert_group(arr(g[:1]), arr(u[:1]), arr(d[:1]), rows, 1, out.ctypes.data,
                                      x.ctypes.data) == 0
    # update replaces the weights in place
    new = mk((n, mid))
    d[0].update(new, None)
    got = coli.expert_group(g[:1], u[:1], d[:1], x[:n])
    gw0 = ox.decode_colibri(_host(g[0]), None, 0, n, mid)
    uw0 = ox.decode_colibri(_host(u[0]), None, 0, n, mid)
    assert rel_l2(got, ox.expert_group([gw0], [uw0], [new], x[:n])) <= 1e-2
    assert d[0].device() == 0
    for t in g + u + d + [odd]:
        t.close()


def _host(tensor):
    return tensor._w


def test_colibri_shutdown_refuses_then_reinit(coli):
    announce("coli shutdown and re-init")
    w = np.eye(8, dtype=F)
    t = coli.ColiTensor(w, None, 0, 8, 8)
    coli.coli_shutdown()
    assert coli.lib().coli_cuda_device_count() == 0
    with pytest.raises(RuntimeError):
        coli.expert_mlp(t, t, t, np.ones(8, F))
    coli.coli_init(0)
    assert coli.lib().coli_cuda_device_count() == 1 and coli.lib().coli_cuda_device_at(0) == 0
    y = coli.expert_mlp(t, t, t, np.ones(8, F))
    assert rel_l2(y, ox.expert_group([w], [w], [w], np.ones(8, F))) <= 1e-2
    t.close()


# ---- GGML MUL_MAT_ID ----

def test_ggml_reference_expert_pattern(hk_lib):
    from runtime.experts import GgmlExperts

    announce("ggml mul_mat_id reference pattern 8x2048x2048")
    case = ggml_expert_pattern_case()
    set_ = GgmlExperts(case["weights"])
    got = set_.mul_mat_id(case["x"], case["ids"])
    err = np.abs(got[:, case["check_rows"]] - case["expected"])
    assert err.max() < case["tol"], float(err.max())
    want = ox.mul_mat_id(case["weights"], case["x"], case["ids"])
    for i in range(8):
        q, s = ox.requantize_rows(case["weights"][i])
        assert np.all(np.abs(got[i] - want[i]) <= _tile_bound(q, s, case["x"][i]))
    # the timing hook re-runs the launch with other id rows; a call afterwards is unchanged
    assert set_.repeat_ms(np.stack([np.roll(case["ids"], k) for k in range(3)])) > 0
    assert np.array_equal(set_.mul_mat_id(case["x"], case["ids"]), got)
    set_.close()


@pytest.mark.parametrize("input_rows", [1, 4])
def test_ggml_ids_repeat_and_broadcast(hk_lib, input_rows):
    from runtime.experts import GgmlExperts

    announce(f"ggml mul_mat_id ragged 12x77x1000 input_rows={input_rows}")
    rng = np.random.default_rng(input_rows)
    w = rng.normal(0, 0.1, (12, 77, 1000)).astype(F)
    x = rng.normal(0, 1, (input_rows, 1000)).astype(F)
    ids = np.array([3, 3, 11, 0], np.int32)
    a = GgmlExperts(w)
    b = GgmlExperts(w[:8] * 2)  # a second set alive at the same time
    got = a.mul_mat_id(x, ids)
    other = b.mul_mat_id(x[:1], ids[:1])
    for slot, e in enumerate(ids):
        row = x[0 if input_rows == 1 else slot]
        _assert_projection(got[slot], w[e], row)
    _assert_projection(other[0], w[3] * 2, x[0])
    if input_rows == 4:
        assert not np.array_equal(got[0], got[1])  # same expert, different rows
    else:
        assert np.array_equal(got[0], got[1])
    with pytest.raises(ValueError):
        b.repeat_ms(np.zeros((0, 1), np.int32))
    with pytest.raises(ValueError):
        b.repeat_ms(np.array([[8]], np.int32))  # b holds 8 experts
    for bad_ids, rows in (([12], 1), ([-1], 1), (list(range(9)), 1), ([0, 1, 2, 3], 2)):
        with pytest.raises(ValueError):
            a.mul_mat_id(np.zeros((rows, 1000), F), np.array(bad_ids, np.int32))
    a.close()
    b.close()
