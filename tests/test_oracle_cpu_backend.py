"""Pins oracle.cpu_backend (restatement of npu_llm/runtime/cpu_backend.py).

Each check is an independent computation, not the oracle's formula retyped:
the reference test's per-head attention loop (tests/test_cpu_backend.py:17-52),
float64 brute force with a forward error bound for projections, float64 closed
forms for RMSNorm / SwiGLU, complex-number rotation for RoPE, NumPy's argmax
semantics, and a float64 model written without intermediate rounding for the
whole step.  Planted mistakes (on the CPU, in copies of the oracle) show the
checks are sensitive to them.
"""

import numpy as np
import pytest

from oracle import bf16
from oracle.cpu_backend import CPUDecoderStage, OracleDecoder, decode_result
from runtime.synthetic import SyntheticModel

TINY = {
    "model_family": "qwen2",
    "hidden_size": 64,
    "intermediate_size": 128,
    "attention_heads": 4,
    "kv_heads": 2,
    "head_dim": 16,
    "layers": 2,
    "vocab_size": 97,
    "rope_theta": 10000.0,
    "rms_norm_eps": 1e-6,
    "qkv_bias": True,
}


def _bf16_vec(rng, n, scale=1.0):
    return bf16.round_f32(rng.normal(0, scale, n).astype(np.float32))


def _ulp_bf16(x):
    x = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0**-126)))
    return 2.0 ** (e - 7)


# -- attention ---------------------------------------------------------------

def _bare_stage(q_heads, kv_heads, head_dim, context, inv):
    stage = object.__new__(CPUDecoderStage)
    stage.q_heads, stage.kv_heads, stage.head_dim = q_heads, kv_heads, head_dim
    stage.q_per_kv = q_heads // kv_heads
    stage._rope_inv_frequency = np.asarray(inv, np.float32)
    stage.key_cache = {0: np.zeros((kv_heads, context, head_dim), np.uint16)}
    stage.value_cache = {0: np.zeros((kv_heads, context, head_dim), np.uint16)}
    return stage


def _loop_attention(stage, qkv, position):
    """Per-head loop of the reference test, over the caches after the append."""
    q_size = stage.q_heads * stage.head_dim
    query = stage.rotate(np.asarray(qkv[:q_size]).reshape(stage.q_heads, stage.head_dim), position)
    scale = stage.head_dim ** -0.5
    expected = np.empty((stage.q_heads, stage.head_dim), np.float32)
    for kv_head in range(stage.kv_heads):
        keys = bf16.from_bits(stage.key_cache[0][kv_head, : position + 1])
        values = bf16.from_bits(stage.value_cache[0][kv_head, : position + 1])
        for g in range(stage.q_per_kv):
            q_head = kv_head * stage.q_per_kv + g
            scores = keys @ query[q_head] * scale
            scores -= np.max(scores)
            p = np.exp(scores)
            p /= np.sum(p)
            expected[q_head] = p @ values
    return expected.reshape(-1)


def test_attention_matches_reference_loop_with_zero_history():
    stage = _bare_stage(4, 2, 4, 5, [1.0, 0.5])
    rng = np.random.default_rng(42)
    qkv = bf16.round_f32(rng.normal(size=32).astype(np.float32))
    actual = stage.attention(qkv, 0, 3)
    np.testing.assert_allclose(actual, _loop_attention(stage, qkv, 3), atol=2e-2, rtol=2e-2)


def test_attention_matches_reference_loop_with_history():
    rng = np.random.default_rng(5)
    stage = _bare_stage(6, 2, 8, 12, rng.uniform(0.1, 1.0, 4))
    for kvh in range(2):
        stage.key_cache[0][kvh, :9] = bf16.to_bits(rng.normal(size=(9, 8)))
        stage.value_cache[0][kvh, :9] = bf16.to_bits(rng.normal(size=(9, 8)))
    qkv = bf16.round_f32(rng.normal(size=(6 + 4) * 8).astype(np.float32))
    actual = stage.attention(qkv, 0, 9)
    expected = _loop_attention(stage, qkv, 9)
    np.testing.assert_allclose(actual, expected, atol=1e-2, rtol=1e-2)
    # slot 9 was written, slots above it were not
    assert np.any(stage.key_cache[0][:, 9] != 0)
    assert np.all(stage.key_cache[0][:, 10:] == 0)


def test_attention_position_zero_returns_value():
    """At position 0 softmax over one slot is 1, so the output is V (bf16)."""
    rng = np.random.default_rng(25)
    stage = _bare_stage(4, 2, 8, 4, rng.uniform(0.1, 1.0, 4))
    qkv = bf16.round_f32(rng.normal(size=(4 + 4) * 8).astype(np.float32))
    out = stage.attention(qkv, 0, 0)
    v = qkv[(4 + 2) * 8:].reshape(2, 8)
    np.testing.assert_array_equal(out.reshape(2, 2, 8), np.repeat(v[:, None, :], 2, axis=1))


# -- projections ---------------------------------------------------------------

class _OneTensorModel:
    def __init__(self, name, bits, meta):
        self.metadata = meta
        self.tensors = {name: {}}
        self._bits = {name: bits}

    def bf16_projection(self, name):
        return self._bits[name]


def _meta(h=64):
    m = dict(TINY)
    m["hidden_size"] = h
    return m


@pytest.mark.parametrize("m,k", [(37, 96), (5, 896), (64, 4864)])
def test_project_within_forward_error_bound_of_float64(m, k):
    rng = np.random.default_rng(m * 1000 + k)
    w_bits = bf16.to_bits(rng.normal(0, 0.02, (m, k)))
    x = _bf16_vec(rng, k)
    stage = object.__new__(CPUDecoderStage)
    stage.model = _OneTensorModel("w", w_bits, _meta())
    stage._weights, stage.w8 = {}, False
    y = stage.project("w", x)
    w64 = bf16.from_bits(w_bits).astype(np.float64)
    exact = w64 @ x.astype(np.float64)
    gamma = k * 2.0**-24 / (1 - k * 2.0**-24)
    bound = gamma * (np.abs(w64) @ np.abs(x.astype(np.float64))) + 0.5 * _ulp_bf16(exact) * 1.0001
    assert np.all(np.abs(y.astype(np.float64) - exact) <= bound)
    # a transposed operand (wrong index order) is far outside the bound
    if m == k:
        wrong = bf16.round_f32(bf16.from_bits(w_bits).T @ x)
        assert np.any(np.abs(wrong - exact) > bound)


def _norm_stage(eps):
    stage = object.__new__(CPUDecoderStage)
    stage.epsilon = eps
    stage._raw = {}
    return stage


@pytest.mark.parametrize("n,eps", [(576, 1e-5), (896, 1e-6)])
def test_norm_matches_float64_closed_form(n, eps):
    rng = np.random.default_rng(n)
    x = _bf16_vec(rng, n, 0.3)
    gamma = _bf16_vec(rng, n, 0.05) + np.float32(1.0)
    stage = _norm_stage(eps)
    stage._raw["g"] = bf16.round_f32(gamma)
    out = stage.norm(x, "g")
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + eps) * bf16.round_f32(gamma).astype(np.float64)
    ulps = np.abs(out - ref) / _ulp_bf16(ref)
    assert np.max(ulps) <= 1.0
    # a dropped epsilon would still pass; a dropped gamma must not
    assert np.max(np.abs(bf16.round_f32(x64 / np.sqrt(np.mean(x64 * x64) + eps)) - ref) / _ulp_bf16(ref)) > 1.0


def test_rotate_is_complex_rotation():
    rng = np.random.default_rng(9)
    stage = object.__new__(CPUDecoderStage)
    stage.head_dim = 64
    stage._rope_inv_frequency = (1.0 / (1e6 ** (np.arange(32, dtype=np.float32) / np.float32(32)))).astype(np.float32)
    heads = bf16.round_f32(rng.normal(size=(5, 64)).astype(np.float32))
    # position 0: cos 1, sin 0 -> identity on bf16 inputs, bit for bit
    np.testing.assert_array_equal(stage.rotate(heads, 0), heads)
    for position in (1, 7, 63, 4095):
        angle = np.float64(np.float32(position) * stage._rope_inv_frequency)
        z = (heads[:, :32].astype(np.float64) + 1j * heads[:, 32:].astype(np.float64)) * np.exp(1j * angle)
        ref = np.concatenate([z.real, z.imag], axis=1)
        out = stage.rotate(heads, position)
        # f32 angle evaluation differs from f64 in the last bits; allow 2 bf16 ulps
        # plus the absolute error of cos/sin at large angles
        err = np.abs(out - ref)
        assert np.all(err <= 2 * _ulp_bf16(ref) + 1e-5 * np.abs(heads).max())


def test_rotate_sign_mistake_is_caught():
    rng = np.random.default_rng(10)
    heads = rng.normal(size=(3, 64))
    angle = 0.7 * np.ones(32)
    z = (heads[:, :32] + 1j * heads[:, 32:]) * np.exp(1j * angle)
    wrong = np.concatenate(
        [heads[:, :32] * np.cos(angle) + heads[:, 32:] * np.sin(angle),
         heads[:, 32:] * np.cos(angle) - heads[:, :32] * np.sin(angle)], axis=1)
    assert np.max(np.abs(wrong - np.concatenate([z.real, z.imag], axis=1))) > 0.1


def test_swiglu_matches_float64():
    rng = np.random.default_rng(11)
    g = bf16.round_f32(rng.normal(0, 3, 4096).astype(np.float32))
    u = bf16.round_f32(rng.normal(0, 3, 4096).astype(np.float32))
    g[:4] = [-100.0, 100.0, 0.0, -80.0]
    act = bf16.round_f32((g / (1.0 + np.exp(-np.clip(g, -80.0, 80.0)))) * u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = g64 / (1.0 + np.exp(-g64)) * u64
    ok = np.abs(act - ref) <= _ulp_bf16(ref) + 1e-30
    assert np.all(ok)


def test_argmax_first_maximum_wins():
    logits = np.array([0.5, 2.0, -1.0, 2.0, 1.9], np.float32)
    assert decode_result(logits) == 1
    token, diag = decode_result(logits, diagnostics=True)
    assert token == 1 and diag["top_token_ids"][0] in (1, 3)
    assert diag["top_logit_margin"] == 0.0


# -- whole step against a float64 model --------------------------------------

def _f64_model_logits(model, tokens, positions_to_keep):
    """Float64 decoder without intermediate rounding (complex RoPE, loop
    attention), written independently of the oracle."""
    m = model.metadata
    H, D = m["hidden_size"], m["head_dim"]
    nq, nkv, inter = m["attention_heads"], m["kv_heads"], m["intermediate_size"]
    eps = m["rms_norm_eps"]
    w = lambda n: bf16.from_bits(model.bf16_projection(n)).astype(np.float64)  # noqa: E731
    r = lambda n: model.raw_f32(n).astype(np.float64)  # noqa: E731
    E = r("token_embedding").reshape(m["vocab_size"], H)
    inv = 1.0 / (m["rope_theta"] ** (np.arange(D // 2) / (D // 2)))
    K = {l: [] for l in range(m["layers"])}
    V = {l: [] for l in range(m["layers"])}

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x) + eps) * g

    def rope(x, pos):
        z = (x[..., : D // 2] + 1j * x[..., D // 2:]) * np.exp(1j * pos * inv)
        return np.concatenate([z.real, z.imag], axis=-1)

    out = {}
    for pos, tok in enumerate(tokens):
        h = E[tok].copy()
        for l in range(m["layers"]):
            p = f"layer{l:02d}"
            qkv = w(f"{p}.qkv") @ rms(h, r(f"{p}.input_norm")) + r(f"{p}.qkv_bias")
            q = rope(qkv[: nq * D].reshape(nq, D), pos)
            k = rope(qkv[nq * D:(nq + nkv) * D].reshape(nkv, D), pos)
            v = qkv[(nq + nkv) * D:].reshape(nkv, D)
            K[l].append(k)
            V[l].append(v)
            att = np.zeros((nq, D))
            for hq in range(nq):
                kvh = hq // (nq // nkv)
                s = np.array([K[l][t][kvh] @ q[hq] for t in range(pos + 1)]) / np.sqrt(D)
                pr = np.exp(s - s.max())
                pr /= pr.sum()
                att[hq] = sum(pr[t] * V[l][t][kvh] for t in range(pos + 1))
            h = h + w(f"{p}.o_proj") @ att.reshape(-1)
            gu = w(f"{p}.gate_up") @ rms(h, r(f"{p}.post_attn_norm"))
            g, u = gu[:inter], gu[inter:]
            h = h + w(f"{p}.down_proj") @ (g / (1 + np.exp(-g)) * u)
        if pos in positions_to_keep:
            out[pos] = w("lm_head") @ rms(h, r("final_norm"))
    return out


def test_whole_step_tracks_float64_model():
    model = SyntheticModel(TINY, seed=3, std=0.15)
    rng = np.random.default_rng(4)
    tokens = [int(t) for t in rng.integers(0, TINY["vocab_size"], 12)]
    oracle = OracleDecoder(model, 16)
    got = {}
    for pos, tok in enumerate(tokens):
        _, lg = oracle.decode_token(tok, pos, compute_logits=pos in (0, 5, 11))
        if lg is not None:
            got[pos] = lg
    ref = _f64_model_logits(model, tokens, {0, 5, 11})
    for pos in ref:
        err = np.linalg.norm(got[pos] - ref[pos]) / np.linalg.norm(ref[pos])
        assert err < 2e-2, (pos, err)


def test_whole_step_check_catches_planted_mistakes(monkeypatch):
    """Swapping gate and up, or dropping the attention residual, in a copy of
    the oracle moves the logits far from the float64 model."""
    model = SyntheticModel(TINY, seed=3, std=0.15)
    tokens = [5, 17, 42, 8, 90, 1]
    ref = _f64_model_logits(model, tokens, {5})[5]

    def run(stage_cls):
        dec = OracleDecoder(model, 8)
        dec.stage.__class__ = stage_cls
        lg = None
        for pos, tok in enumerate(tokens):
            _, lg = dec.decode_token(tok, pos, compute_logits=pos == 5)
        return lg

    class NoResidual(CPUDecoderStage):
        def layer(self, hidden, layer, position):
            out = super().layer(hidden, layer, position)
            return bf16.round_f32(out - np.asarray(hidden, np.float32))

    class SwappedGateUp(CPUDecoderStage):
        def project(self, name, activation):
            y = super().project(name, activation)
            if name.endswith("gate_up"):
                g, u = np.split(y, 2)
                return np.concatenate([u, g])
            return y

    for cls in (NoResidual, SwappedGateUp):
        lg = run(cls)
        assert np.linalg.norm(lg - ref) / np.linalg.norm(ref) > 0.1, cls.__name__


# -- batched prefill (rows at once) -------------------------------------------

def _per_position(model, tokens, context, *, w8=False):
    dec = OracleDecoder(model, context, w8=w8)
    lg = None
    for pos, tok in enumerate(tokens):
        _, lg = dec.decode_token(tok, pos, compute_logits=pos == len(tokens) - 1)
    return dec, lg


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_prefill_rows_matches_per_position_decode(w8):
    """The batched prefill equals the reference's position-by-position prefill
    up to float32 summation order: KV caches agree to one bf16 step (nearly
    all bit for bit), the last logits to rel-L2 1e-3, and both track the
    float64 model."""
    model = SyntheticModel(TINY, seed=3, std=0.15)
    rng = np.random.default_rng(21)
    tokens = [int(t) for t in rng.integers(0, TINY["vocab_size"], 13)]
    ref, ref_logits = _per_position(model, tokens, 16, w8=w8)
    dec = OracleDecoder(model, 16, w8=w8)
    tok, logits = dec.prefill(tokens)
    assert tok == int(np.argmax(logits))
    assert np.linalg.norm(logits - ref_logits) / np.linalg.norm(ref_logits) < 1e-3
    for layer in range(TINY["layers"]):
        for got, want in ((dec.stage.key_cache[layer], ref.stage.key_cache[layer]),
                          (dec.stage.value_cache[layer], ref.stage.value_cache[layer])):
            from _util import bf16_ulp_diff
            diff = bf16_ulp_diff(got, want)
            assert diff.max() <= 1 and (diff == 0).mean() >= 0.97
            assert np.all(got[:, len(tokens):] == 0)
    if not w8:
        f64 = _f64_model_logits(model, tokens, {len(tokens) - 1})[len(tokens) - 1]
        assert np.linalg.norm(logits - f64) / np.linalg.norm(f64) < 2e-2


def test_prefill_rows_blas_products_agree_with_the_einsum():
    """From CPUDecoderStage.BLAS_ROWS rows the batched attention takes BLAS
    matrix products instead of the einsum contractions; on the same 300 rows
    (two KV blocks of scores, a nonzero start) the two agree to one bf16 step
    per output or, where P @ V cancels to almost nothing, to 1e-5 absolute
    (values are ~0.5 here); nearly all bit for bit; and the KV caches they
    write are identical (the append precedes the scores)."""
    model = SyntheticModel(TINY, seed=9, std=0.15)
    rng = np.random.default_rng(23)
    outs, caches = [], []
    for blas_rows in (10 ** 9, 1):
        dec = OracleDecoder(model, 320)
        st = dec.stage
        st.BLAS_ROWS = blas_rows
        qkv = np.asarray(rng.normal(size=(300, (st.q_heads + 2 * st.kv_heads) * st.head_dim)) * 0.5, np.float32)
        rng = np.random.default_rng(23)  # the same rows for both
        outs.append(st.attention_rows(qkv, 0, 7, block=256))
        caches.append((st.key_cache[0].copy(), st.value_cache[0].copy()))
    from _util import bf16_ulp_diff
    from oracle.bf16 import to_bits
    diff = bf16_ulp_diff(to_bits(outs[0]), to_bits(outs[1]))
    assert np.all((diff <= 1) | (np.abs(outs[0] - outs[1]) <= 1e-5)) and (diff == 0).mean() >= 0.99
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])


def test_prefill_rows_blocks_and_offset_start():
    """Rows scored in several blocks, a prompt starting at a nonzero slot, and
    a continuation after an earlier prefill give the per-position result."""
    model = SyntheticModel(TINY, seed=5, std=0.15)
    rng = np.random.default_rng(22)
    tokens = [int(t) for t in rng.integers(0, TINY["vocab_size"], 11)]
    ref, ref_logits = _per_position(model, tokens, 12)
    dec = OracleDecoder(model, 12)
    block_rows = CPUDecoderStage.attention_rows.__defaults__
    CPUDecoderStage.attention_rows.__defaults__ = (3,)
    try:
        dec.prefill(tokens[:4], 0, compute_logits=False)
        _, logits = dec.prefill(tokens[4:], 4)
    finally:
        CPUDecoderStage.attention_rows.__defaults__ = block_rows
    assert np.linalg.norm(logits - ref_logits) / np.linalg.norm(ref_logits) < 1e-3
    from _util import bf16_ulp_diff
    for layer in range(TINY["layers"]):
        assert bf16_ulp_diff(dec.stage.key_cache[layer], ref.stage.key_cache[layer]).max() <= 1


def test_prefill_rows_check_catches_a_non_causal_mask():
    """A planted mistake in a copy of the oracle -- every row also attends to
    the later prompt slots -- moves the last logits far from the float64
    model, which the correct batched prefill tracks."""
    model = SyntheticModel(TINY, seed=3, std=0.15)
    tokens = [5, 17, 42, 8, 90, 1, 33, 60]
    ref = _f64_model_logits(model, tokens, {7})[7]

    class SeesTheFuture(CPUDecoderStage):
        def attention_rows(self, qkv_rows, layer, start, block=256):
            n = np.asarray(qkv_rows).shape[0]
            saved = self._rope_inv_frequency
            out = super().attention_rows(qkv_rows, layer, start, block)
            # recompute each row over all n slots, keeping its own rotation
            keys = bf16.from_bits(self.key_cache[layer][:, :start + n])
            values = bf16.from_bits(self.value_cache[layer][:, :start + n])
            d = self.head_dim
            for i in range(n):
                angle = np.float32(start + i) * saved
                c, s_ = np.cos(angle), np.sin(angle)
                q = np.asarray(qkv_rows[i, :self.q_heads * d], np.float32).reshape(self.q_heads, d)
                q = bf16.round_f32(np.concatenate([q[:, :d // 2] * c - q[:, d // 2:] * s_,
                                                   q[:, d // 2:] * c + q[:, :d // 2] * s_], axis=-1))
                g = q.reshape(self.kv_heads, self.q_per_kv, d)
                sc = np.einsum("kqd,ksd->kqs", g, keys) * d**-0.5
                pr = np.exp(sc - sc.max(axis=-1, keepdims=True))
                pr /= pr.sum(axis=-1, keepdims=True)
                out[i] = bf16.round_f32(np.einsum("kqs,ksd->kqd", pr, values).reshape(-1))
            return out

    good = OracleDecoder(model, 8)
    _, lg_good = good.prefill(tokens)
    bad = OracleDecoder(model, 8)
    bad.stage.__class__ = SeesTheFuture
    _, lg_bad = bad.prefill(tokens)
    assert np.linalg.norm(lg_good - ref) / np.linalg.norm(ref) < 2e-2
    assert np.linalg.norm(lg_bad - ref) / np.linalg.norm(ref) > 5e-2


def test_w8_stage_branch_is_project_w8():
    """The W8 stage multiplies through oracle.quant.project_w8 (pinned against
    float64 in test_oracle_quant.py), and the rows form agrees with it."""
    from oracle.quant import project_w8

    model = SyntheticModel(TINY, seed=6, std=0.15)
    stage = CPUDecoderStage(model, 0, 8, w8=True)
    rng = np.random.default_rng(23)
    for name in ("layer00.qkv", "layer01.down_proj"):
        q = model.quantized(name)
        k = q.weight.shape[1]
        x = bf16.round_f32(rng.normal(size=(3, k)).astype(np.float32))
        for i in range(3):
            np.testing.assert_array_equal(stage.project(name, x[i]), project_w8(q.weight, q.scale, x[i]))
        from _util import bf16_ulp_diff
        rows = stage.project_rows(name, x)
        want = np.stack([project_w8(q.weight, q.scale, x[i]) for i in range(3)])
        assert bf16_ulp_diff(bf16.to_bits(rows), bf16.to_bits(want)).max() <= 1
    # the LM head stays bf16 in W8 mode
    x = bf16.round_f32(rng.normal(size=TINY["hidden_size"]).astype(np.float32))
    np.testing.assert_array_equal(stage.project("lm_head", x),
                                  CPUDecoderStage(model, 0, 8).project("lm_head", x))


def test_teacher_forced_rows_match_per_position_logits_with_random_gains():
    """``teacher_forced`` (every row of a batched prefill through the final
    norm and LM head) gives the per-position decode's logits at every
    position up to float32 summation order, and tracks the float64 model,
    on a model whose RMSNorm gains are random (layer gains U(0.5, 1.5), final
    gains 8 U(0.5, 1.5)) so a gain applied wrongly or not at all shows."""
    model = SyntheticModel(TINY, seed=6, std=0.15, norm_gains=8.0)
    assert not np.all(model.raw_f32("layer00.input_norm") == 1.0)
    rng = np.random.default_rng(23)
    tokens = [int(t) for t in rng.integers(0, TINY["vocab_size"], 9)]
    rows = OracleDecoder(model, 12).teacher_forced(tokens)
    assert rows.shape == (9, TINY["vocab_size"]) and rows.dtype == np.float32
    dec = OracleDecoder(model, 12)
    for pos, tok in enumerate(tokens):
        _, lg = dec.decode_token(tok, pos)
        assert np.linalg.norm(rows[pos] - lg) / np.linalg.norm(lg) < 1e-3, pos
    ref = _f64_model_logits(model, tokens, set(range(9)))
    for pos in ref:
        assert np.linalg.norm(rows[pos] - ref[pos]) / np.linalg.norm(ref[pos]) < 2e-2, pos
    # the same weights with unit gains are far away: the gains are in use
    plain = _f64_model_logits(SyntheticModel(TINY, seed=6, std=0.15), tokens, {8})[8]
    assert np.linalg.norm(rows[8] - plain) / np.linalg.norm(ref[8]) > 0.2


def test_norm_gains_leave_the_weights_of_the_seed():
    a = SyntheticModel(TINY, seed=2)
    b = SyntheticModel(TINY, seed=2, norm_gains=8.0)
    for name in ("token_embedding", "layer01.gate_up", "layer00.qkv"):
        np.testing.assert_array_equal(a.raw(name), b.raw(name))
    final = b.raw_f32("final_norm")
    assert final.min() >= 4.0 and final.max() <= 12.0
    gains = b.raw_f32("layer01.post_attn_norm")
    assert gains.min() >= 0.5 and gains.max() <= 1.5 and np.std(gains) > 0.1
