"""Per-operation parity on the GPU through libhk.so's C ABI.

Each kernel is compared with the oracle (oracle/) on the same seeded inputs.
GEMV sums are float32 in a different order from BLAS sgemv, so bf16 outputs
may differ from the oracle by one bf16 step where the exact sum sits near a
rounding boundary; float32 outputs are held to the forward error bound of a
float64 brute force.  RoPE, the KV append and argmax are bit-exact.
"""

import ctypes

import numpy as np
import pytest

from _util import announce, bf16_ulp_diff
from oracle import bf16
from oracle.cpu_backend import CPUDecoderStage
from oracle.quant import project_w8, quantize_per_output_channel

pytestmark = pytest.mark.gpu

# (M, K, bias) of the Qwen2.5-0.5B projections and the SmolLM2-135M ones
QWEN_SHAPES = [(1152, 896, True), (896, 896, False), (9728, 896, False), (896, 4864, False),
               (151936, 896, False)]
SMOL_SHAPES = [(960, 576, False), (576, 576, False), (3072, 576, False), (576, 1536, False)]


def _dev(array):
    from runtime import hip

    return hip.DeviceBuffer.from_array(np.ascontiguousarray(array))


def _read(buf, dtype, n):
    return buf.read(dtype, n)


def _bound(w64, x64, exact):
    k = w64.shape[1]
    gamma = k * 2.0**-24 / (1 - k * 2.0**-24)
    return 1.01 * gamma * (np.abs(w64) @ np.abs(x64)) + 1e-30


def _ulp(x):
    x = np.abs(np.asarray(x, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(x, 2.0**-126))) - 7)


def _check_bf16(y_bits, ref_bits, sum_bound):
    """GPU and oracle each round a float32 sum carrying at most `sum_bound`
    error; their bf16 results may differ by the two sum errors plus one bf16
    step, and should agree exactly almost everywhere."""
    y = bf16.from_bits(y_bits).astype(np.float64)
    ref = bf16.from_bits(ref_bits).astype(np.float64)
    assert np.all(np.abs(y - ref) <= _ulp(ref) + 2 * sum_bound)
    assert (y_bits == ref_bits).mean() >= 0.97


@pytest.mark.parametrize("m,k,bias", QWEN_SHAPES + SMOL_SHAPES)
def test_gemv_bf16_matches_oracle(hk_lib, m, k, bias):
    from runtime import hip

    announce(f"gemv_bf16 M={m} K={k} bias={bias}")
    rng = np.random.default_rng(m + 7 * k)
    w_bits = bf16.to_bits(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    x_bits = bf16.to_bits(rng.normal(0, 1, k).astype(np.float32))
    b = rng.normal(0, 0.02, m).astype(np.float32) if bias else None
    W, X = _dev(w_bits), _dev(x_bits)
    Yf = hip.DeviceBuffer(4 * m)
    hip.check(hk_lib.hk_gemv_bf16(W.ptr, X.ptr, None, None, None, Yf.ptr, m, k, None), "gemv f32")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    yf = _read(Yf, np.float32, m)
    w64 = bf16.from_bits(w_bits).astype(np.float64)
    x64 = bf16.from_bits(x_bits).astype(np.float64)
    exact = w64 @ x64
    assert np.all(np.abs(yf - exact) <= _bound(w64, x64, exact))

    # bf16 output with the reference's rounding points
    Y = hip.DeviceBuffer(2 * m)
    B = _dev(b) if bias else None
    hip.check(hk_lib.hk_gemv_bf16(W.ptr, X.ptr, B.ptr if B else None, None, Y.ptr, None, m, k, None),
              "gemv bf16")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    y = _read(Y, np.uint16, m)
    ref = bf16.round_f32(bf16.from_bits(w_bits) @ bf16.from_bits(x_bits))
    if bias:
        ref = bf16.round_f32(ref + b)
    _check_bf16(y, bf16.to_bits(ref), _bound(w64, x64, exact))


# every Qwen2.5-0.5B projection shape with W8 weights (the QKV with its bias),
# the LM head shape included, and one SmolLM2-135M shape
W8_SHAPES = [(m, k, bias) for m, k, bias in QWEN_SHAPES] + [(576, 1536, False)]


@pytest.mark.parametrize("m,k,bias", W8_SHAPES)
def test_gemv_w8_matches_oracle(hk_lib, m, k, bias):
    from runtime import hip

    announce(f"gemv_w8 M={m} K={k} bias={bias}")
    rng = np.random.default_rng(3 * m + k)
    w = bf16.round_f32(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    q, s = quantize_per_output_channel(w)
    x_bits = bf16.to_bits(rng.normal(0, 1, k).astype(np.float32))
    b = rng.normal(0, 0.02, m).astype(np.float32) if bias else None
    Q, S, X = _dev(q), _dev(s), _dev(x_bits)
    B = _dev(b) if bias else None
    Yf = hip.DeviceBuffer(4 * m)
    Y = hip.DeviceBuffer(2 * m)
    hip.check(hk_lib.hk_gemv_w8(Q.ptr, S.ptr, X.ptr, None, None, None, Yf.ptr, m, k, None), "w8 f32")
    hip.check(hk_lib.hk_gemv_w8(Q.ptr, S.ptr, X.ptr, B.ptr if B else None, None, Y.ptr, None, m, k, None),
              "w8 bf16")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    x = bf16.from_bits(x_bits)
    q64 = q.astype(np.float64)
    exact = (q64 @ x.astype(np.float64)) * s
    bound = _bound(q64, x.astype(np.float64), exact) * s + 2e-7 * np.abs(exact)
    assert np.all(np.abs(_read(Yf, np.float32, m) - exact) <= bound)
    ref = project_w8(q, s, x)
    if bias:
        ref = bf16.round_f32(ref + b)
        bound = bound + _ulp(exact)  # the bias add rounds once more
    _check_bf16(_read(Y, np.uint16, m), bf16.to_bits(ref), bound)


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_gemv_repeat_graph_replays_match_direct_launches(hk_lib, w8):
    """hk_gemv_repeat (the GEMV microbenchmark): its captured graph, replayed
    twice, leaves the output of the last launch's weight copy, the same
    float32 bits as a direct GEMV of that copy."""
    import ctypes

    from runtime import hip

    announce(f"gemv repeat graph w8={w8}")
    m, k, copies, count = 896, 896, 3, 5
    rng = np.random.default_rng(21)
    x = _dev(bf16.to_bits(rng.normal(0, 1, k).astype(np.float32)))
    ws, ss = [], []
    for _ in range(copies):
        w = bf16.round_f32(rng.normal(0, 0.02, (m, k)).astype(np.float32))
        if w8:
            q, sc = quantize_per_output_channel(w)
            ws.append(_dev(q))
            ss.append(_dev(sc))
        else:
            ws.append(_dev(bf16.to_bits(w)))
    ptrs = (ctypes.c_void_p * copies)(*[b.ptr for b in ws])
    sptrs = (ctypes.c_void_p * copies)(*[b.ptr for b in ss]) if w8 else None
    y, want = hip.DeviceBuffer(4 * m), hip.DeviceBuffer(4 * m)
    last = (count - 1) % copies
    if w8:
        hip.check(hk_lib.hk_gemv_w8(ws[last].ptr, ss[last].ptr, x.ptr, None, None, None, want.ptr, m, k, None), "w8")
    else:
        hip.check(hk_lib.hk_gemv_bf16(ws[last].ptr, x.ptr, None, None, None, want.ptr, m, k, None), "bf16")
    for _ in range(2):  # the capture, then a replay
        y.zero()
        hip.check(hk_lib.hk_gemv_repeat(ptrs, sptrs, copies, x.ptr, y.ptr, m, k, count, None), "repeat")
        hip.check(hk_lib.hk_stream_sync(None), "sync")
        np.testing.assert_array_equal(_read(y, np.uint32, m), _read(want, np.uint32, m))


def test_gemv_residual_epilogue(hk_lib):
    from runtime import hip

    announce("gemv residual 896x4864")
    rng = np.random.default_rng(12)
    m, k = 896, 4864
    w_bits = bf16.to_bits(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    x_bits = bf16.to_bits(rng.normal(0, 1, k).astype(np.float32))
    r_bits = bf16.to_bits(rng.normal(0, 1, m).astype(np.float32))
    W, X, R = _dev(w_bits), _dev(x_bits), _dev(r_bits)
    Y = hip.DeviceBuffer(2 * m)
    hip.check(hk_lib.hk_gemv_bf16(W.ptr, X.ptr, None, R.ptr, Y.ptr, None, m, k, None), "gemv")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    proj = bf16.round_f32(bf16.from_bits(w_bits) @ bf16.from_bits(x_bits))
    ref = bf16.to_bits(proj + bf16.from_bits(r_bits))
    w64 = bf16.from_bits(w_bits).astype(np.float64)
    x64 = bf16.from_bits(x_bits).astype(np.float64)
    # a one-step difference in the rounded projection carries into the sum
    bound = _bound(w64, x64, None) + _ulp(proj)
    _check_bf16(_read(Y, np.uint16, m), ref, bound)


def test_gemv_rejects_bad_shapes(hk_lib):
    from runtime import hip

    W = hip.DeviceBuffer(64)
    with pytest.raises(ValueError):
        hip.check(hk_lib.hk_gemv_bf16(W.ptr, W.ptr, None, None, W.ptr, None, 4, 12, None), "gemv")
    with pytest.raises(ValueError):
        hip.check(hk_lib.hk_gemv_w8(W.ptr, None, W.ptr, None, None, W.ptr, None, 4, 16, None), "w8")


@pytest.mark.parametrize("n,eps", [(576, 1e-5), (896, 1e-6), (2048, 1e-6)])
def test_rmsnorm_matches_oracle(hk_lib, n, eps):
    from runtime import hip

    announce(f"rmsnorm n={n}")
    rng = np.random.default_rng(n)
    x_bits = bf16.to_bits(rng.normal(0, 0.5, n).astype(np.float32))
    g_bits = bf16.to_bits((1 + rng.normal(0, 0.05, n)).astype(np.float32))
    X, G, O = _dev(x_bits), _dev(g_bits), hip.DeviceBuffer(2 * n)
    hip.check(hk_lib.hk_rmsnorm(X.ptr, G.ptr, ctypes.c_float(np.float32(eps)), O.ptr, n, None), "rmsnorm")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    stage = object.__new__(CPUDecoderStage)
    stage.epsilon = eps
    stage._raw = {"g": bf16.from_bits(g_bits)}
    ref = bf16.to_bits(stage.norm(bf16.from_bits(x_bits), "g"))
    diff = bf16_ulp_diff(_read(O, np.uint16, n), ref)
    assert diff.max() <= 1 and (diff == 0).mean() >= 0.99


def test_swiglu_matches_oracle(hk_lib):
    from runtime import hip

    announce("swiglu 4864")
    rng = np.random.default_rng(13)
    inter = 4864
    gu_bits = bf16.to_bits(rng.normal(0, 3, 2 * inter).astype(np.float32))
    gu_bits[:4] = bf16.to_bits(np.array([-100.0, 100.0, 0.0, -80.0], np.float32))
    GU, A = _dev(gu_bits), hip.DeviceBuffer(2 * inter)
    hip.check(hk_lib.hk_swiglu(GU.ptr, A.ptr, inter, None), "swiglu")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    g, u = np.split(bf16.from_bits(gu_bits), 2)
    ref = bf16.to_bits((g / (1.0 + np.exp(-np.clip(g, -80.0, 80.0)))) * u)
    diff = bf16_ulp_diff(_read(A, np.uint16, inter), ref)
    assert diff.max() <= 1 and (diff == 0).mean() >= 0.99


@pytest.mark.parametrize("n", [1, 1000, 151936])
def test_argmax_first_maximum(hk_lib, n):
    from runtime import hip

    announce(f"argmax n={n}")
    rng = np.random.default_rng(n)
    x = rng.normal(size=n).astype(np.float32)
    if n > 10:
        x[n // 3] = x[n // 2] = x.max() + 1.0  # tie: the lower index wins
        x[7] = -0.0
    X, I = _dev(x), hip.DeviceBuffer(4)
    for _ in range(3):  # the reduction state must reset itself between calls
        hip.check(hk_lib.hk_argmax_f32(X.ptr, n, I.ptr, None), "argmax")
        hip.check(hk_lib.hk_stream_sync(None), "sync")
        assert int(_read(I, np.int32, 1)[0]) == int(np.argmax(x))


def _attention_case(hk_lib, q_heads, kv_heads, ctx, position, seed):
    from runtime import hip
    from runtime.qwen_engine import rope_tables

    rng = np.random.default_rng(seed)
    theta = 1e6
    cos, sin = rope_tables(theta, 64, ctx)
    kc = np.zeros((kv_heads, ctx, 64), np.uint16)
    vc = np.zeros((kv_heads, ctx, 64), np.uint16)
    kc[:, :position] = bf16.to_bits(rng.normal(0, 1, (kv_heads, position, 64)).astype(np.float32))
    vc[:, :position] = bf16.to_bits(rng.normal(0, 1, (kv_heads, position, 64)).astype(np.float32))
    qkv_bits = bf16.to_bits(rng.normal(0, 1, (q_heads + 2 * kv_heads) * 64).astype(np.float32))
    QKV, COS, SIN, KC, VC = _dev(qkv_bits), _dev(cos), _dev(sin), _dev(kc), _dev(vc)
    OUT = hip.DeviceBuffer(2 * q_heads * 64)
    hip.check(hk_lib.hk_attention_decode(QKV.ptr, COS.ptr, SIN.ptr, KC.ptr, VC.ptr, position, ctx,
                                         q_heads, kv_heads, 64, OUT.ptr, None), "attention")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    out = _read(OUT, np.uint16, q_heads * 64)
    kc_gpu = _read(KC, np.uint16, kc.size).reshape(kc.shape)
    vc_gpu = _read(VC, np.uint16, vc.size).reshape(vc.shape)

    stage = object.__new__(CPUDecoderStage)
    stage.q_heads, stage.kv_heads, stage.head_dim = q_heads, kv_heads, 64
    stage.q_per_kv = q_heads // kv_heads
    stage._rope_inv_frequency = (1.0 / (theta ** (np.arange(32, dtype=np.float32) / np.float32(32))))
    stage.key_cache = {0: kc.copy()}
    stage.value_cache = {0: vc.copy()}
    ref = stage.attention(bf16.from_bits(qkv_bits), 0, position)
    return out, ref, kc_gpu, vc_gpu, stage


@pytest.mark.parametrize(
    "q_heads,kv_heads,ctx,position",
    [(14, 2, 128, 0), (14, 2, 128, 70), (9, 3, 64, 50), (14, 2, 4096, 255), (14, 2, 4096, 256),
     (14, 2, 4096, 1000), (14, 2, 4096, 4095), (16, 1, 512, 300)],
)
def test_attention_decode_matches_oracle(hk_lib, q_heads, kv_heads, ctx, position):
    announce(f"attention Hq={q_heads} Hkv={kv_heads} ctx={ctx} p={position}")
    out, ref, kc_gpu, vc_gpu, stage = _attention_case(hk_lib, q_heads, kv_heads, ctx, position, position + 1)
    # the KV append is bit-exact: same RoPE tables, same rounding points
    np.testing.assert_array_equal(kc_gpu, stage.key_cache[0])
    np.testing.assert_array_equal(vc_gpu, stage.value_cache[0])
    # softmax-weighted sums in a different float32 order: one bf16 step plus
    # an absolute term for outputs near zero (values are O(1))
    got = bf16.from_bits(out).astype(np.float64)
    assert np.all(np.abs(got - ref) <= _ulp(ref) + 1e-5)
    assert (out == bf16.to_bits(ref)).mean() >= 0.95
