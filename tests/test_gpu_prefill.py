"""Batched prefill on the GPU: the MFMA GEMM against the oracle's projection
arithmetic, and whole-model prefill against the oracle's per-position prefill
(the reference's own prefill, npu_llm/runtime/generate.py:1110-1125)."""

import numpy as np
import pytest

from _util import announce, check_bf16, check_kv_slot, full_depth_tol, fwd_bound, near_tie, rel_l2
from oracle import bf16
from oracle.cpu_backend import OracleDecoder
from runtime.synthetic import QWEN25_05B, SMOLLM2_135M, SyntheticModel

pytestmark = pytest.mark.gpu


def _dev(array):
    from runtime import hip

    return hip.DeviceBuffer.from_array(np.ascontiguousarray(array))


@pytest.mark.parametrize(
    "m,n,k,epi",
    [(40, 1152, 896, "bias"), (40, 896, 896, "resid"), (100, 4864, 896, "none"),
     (40, 896, 4864, "resid"), (1, 576, 576, "none"), (513, 64, 32, "none"), (70, 960, 576, "bias"),
     # 128-token tiles (M >= 128, K a multiple of 64): ragged M and N, and a
     # case with enough tiles for 128-wide outputs
     (513, 896, 896, "resid"), (300, 1000, 128, "bias"), (1024, 8200, 64, "none"), (128, 64, 4864, "resid"),
     # enough 128-token tiles for the XCD-grouped tile order to span
     # several groups of output tiles: whole and ragged token tiles
     (2048, 1152, 896, "bias"), (1500, 2048, 192, "resid"),
     # 128-wide output tiles: 64-wide ones would take two rounds of workgroups
     (4096, 1152, 128, "bias")],
)
def test_gemm_bf16_matches_oracle(hk_lib, m, n, k, epi):
    from runtime import hip

    announce(f"gemm M={m} N={n} K={k} {epi}")
    rng = np.random.default_rng(m * 7 + n + k)
    a_bits = bf16.to_bits(rng.normal(0, 1, (m, k)).astype(np.float32))
    w_bits = bf16.to_bits(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    bias = rng.normal(0, 0.02, n).astype(np.float32) if epi == "bias" else None
    resid = bf16.to_bits(rng.normal(0, 1, (m, n)).astype(np.float32)) if epi == "resid" else None
    A, W, Y = _dev(a_bits), _dev(w_bits), hip.DeviceBuffer(2 * m * n)
    B = _dev(bias) if bias is not None else None
    R = _dev(resid) if resid is not None else None
    hip.check(hk_lib.hk_gemm_bf16(A.ptr, k, W.ptr, B.ptr if B else None, R.ptr if R else None,
                                  Y.ptr, m, n, k, None), "gemm")
    hip.check(hk_lib.hk_stream_sync(None), "sync")
    y = Y.read(np.uint16, m * n).reshape(m, n)
    a64 = bf16.from_bits(a_bits).astype(np.float64)
    w64 = bf16.from_bits(w_bits).astype(np.float64)
    proj = bf16.round_f32(bf16.from_bits(a_bits) @ bf16.from_bits(w_bits).T)
    bound = fwd_bound(a64, w64.T)  # [m, n]
    # bias and residual epilogues round twice, bf16(bf16(acc) + b): a flip of
    # the inner rounding moves the result by up to one step of proj
    proj_step = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(proj), 2.0**-126))) - 7)
    if epi == "bias":
        ref = bf16.to_bits(proj + bias)
        bound = bound + proj_step
    elif epi == "resid":
        ref = bf16.to_bits(proj + bf16.from_bits(resid))
        bound = bound + proj_step
    else:
        ref = bf16.to_bits(proj)
    check_bf16(y, ref, bound)


def _prefill_case(model, prompt, new_tokens, context, tol, label, w8=False):
    from runtime.qwen_engine import QwenDecoderEngine

    announce(f"prefill parity {label}: prompt {len(prompt)} ctx {context} w8={w8}")
    oracle = OracleDecoder(model, context, w8=w8)
    ref_tokens, ref_logits = oracle.generate_greedy(prompt, new_tokens)
    engine = QwenDecoderEngine(model, context_length=context, w8=w8)
    try:
        tok, logits = engine.prefill(prompt, 0)
        err = rel_l2(logits, ref_logits[0])
        announce(f"  prefill logits rel-L2 {err:.3e}, token {tok} oracle {ref_tokens[0]}")
        assert err <= tol
        assert tok == ref_tokens[0] or near_tie(ref_logits[0])
        # KV slots of the prompt against the oracle's caches: each head
        # within twice the logits bound of the oracle's same head and far
        # from every other head
        worst = 0.0
        for layer in (0, model.metadata["layers"] - 1):
            for slot in sorted({0, len(prompt) // 2, len(prompt) - 1}):
                worst = max(worst, check_kv_slot(engine, oracle.stage, layer, slot, 2 * tol))
        announce(f"  KV slots: worst per-head rel-L2 {worst:.3e}")
        if tok == ref_tokens[0] and new_tokens > 1:
            gen = engine.generate(tok, len(prompt), new_tokens - 1)
            for i, (a, b) in enumerate(zip(gen, ref_tokens[1:])):
                if a != b:
                    assert near_tie(ref_logits[i + 1]), f"token {i + 1}: gpu {a} oracle {b}"
                    break
    finally:
        engine.close()


def _prompt(vocab, n, seed):
    rng = np.random.default_rng(seed)
    return [int(t) for t in rng.integers(0, vocab, n)]


def test_prefill_qwen_4_layer():
    model = SyntheticModel(QWEN25_05B, seed=0, layers=4)
    _prefill_case(model, _prompt(151936, 40, 12), 8, 72, 1e-2, "qwen2.5-0.5b-4L")


def test_prefill_smollm_4_layer():
    model = SyntheticModel(SMOLLM2_135M, seed=0, layers=4)
    _prefill_case(model, _prompt(49152, 35, 11), 8, 64, 1e-2, "smollm2-135m-4L")


def test_prefill_qwen_full_depth():
    model = SyntheticModel(QWEN25_05B, seed=0)
    _prefill_case(model, _prompt(151936, 40, 12), 4, 72,
                  full_depth_tol("qwen2.5-0.5b full depth, last prompt position"), "qwen2.5-0.5b")


# A shape wider than the slab GEMMs' fused RMSNorm takes (hidden > 1024):
# chunks of up to 64 tokens then run the slab GEMMs on row-major
# activations, with separate RMSNorm and RoPE/KV-append launches.
WIDE_1152 = dict(QWEN25_05B, hidden_size=1152, intermediate_size=3072, attention_heads=18, kv_heads=3,
                 layers=2, vocab_size=4096)


@pytest.mark.parametrize("n", [1, 17, 64])
def test_prefill_hidden_1152_short_prompts(n):
    """Hidden 1152 (18 query heads, 3 KV heads, intermediate 3072): prompts of
    1, 17 and 64 tokens against the oracle, logits, greedy continuation and
    KV slots per head."""
    model = SyntheticModel(WIDE_1152, seed=8)
    _prefill_case(model, _prompt(4096, n, 40 + n), 4, 72, 1e-2, f"hidden-1152-2L-{n}")


def test_prefill_long_prompt():
    """600 tokens: causal attention over ten 64-slot KV blocks, the last one
    partly masked."""
    model = SyntheticModel(QWEN25_05B, seed=5, layers=2)
    _prefill_case(model, _prompt(151936, 600, 14), 4, 1024, 1e-2, "qwen-2L-600")


def test_prefill_longer_than_one_chunk():
    """4200 tokens in one call run as a 4096-token chunk and a 104-token chunk
    that attends to it; the same prompt over two calls (1000 + 3200, each a
    single chunk) must agree.  The GEMMs split K only when a chunk has too few
    tiles, so the two runs sum some projections in different orders: they
    are held to the float tolerance of the decode path (rel-L2 <= 1e-2) and
    the same greedy token unless the top two logits nearly tie."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce("prefill over two chunks vs two calls, 4200 tokens")
    model = SyntheticModel(QWEN25_05B, seed=6, layers=2)
    prompt = _prompt(151936, 4200, 16)
    engine = QwenDecoderEngine(model, context_length=8192)
    try:
        t_one, l_one = engine.prefill(prompt, 0)
        engine.reset()
        engine.prefill(prompt[:1000], 0, logits=False)
        t_two, l_two = engine.prefill(prompt[1000:], 1000)
        err = rel_l2(l_two, l_one)
        announce(f"  one call vs two calls: rel-L2 {err:.3e}, tokens {t_one} / {t_two}")
        assert err <= 1e-2
        assert t_one == t_two or near_tie(l_one)
    finally:
        engine.close()


def test_prefill_continues_from_cached_prefix():
    """Prefill at start > 0 after earlier steps equals a prefill from 0."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce("prefill at an offset")
    model = SyntheticModel(QWEN25_05B, seed=2, layers=2)
    prompt = _prompt(151936, 30, 15)
    engine = QwenDecoderEngine(model, context_length=64)
    try:
        t_full, l_full = engine.prefill(prompt, 0)
        engine.reset()
        engine.prefill(prompt[:10], 0, logits=False)
        t_part, l_part = engine.prefill(prompt[10:], 10)
        assert t_part == t_full
        assert rel_l2(l_part, l_full) <= 1e-3
        with pytest.raises(ValueError):
            engine.prefill(prompt, 50)
        with pytest.raises(ValueError):
            engine.prefill([151936], 0)
    finally:
        engine.close()


@pytest.mark.parametrize("n,w8", [(1, False), (16, False), (17, False), (32, False), (33, False), (48, False),
                                  (49, False), (63, False), (64, False), (65, False), (130, False), (1, True),
                                  (17, True), (40, True), (64, True)])
def test_prefill_lengths_around_the_slab_gemm(n, w8):
    """Chunks of up to 64 tokens run the slab GEMMs (one workgroup per 16
    outputs over all of K, RMSNorm applied while loading A, weights from the
    MFMA-native copies, compiled for one to four 16-token blocks: the lengths
    cover each block count's edges); 65 and more take the tiled GEMMs.  Last-token logits
    and KV slots of a 2-layer Qwen2.5-0.5B-shape model with random RMSNorm
    gains against the oracle's prefill at each length, and a second prefill
    of the same prompt bit for bit equal to the first (every sum is added in
    a fixed order)."""
    from runtime.qwen_engine import QwenDecoderEngine
    from test_gpu_engine import _check_kv_slot

    announce(f"prefill length {n} w8={w8}")
    model = SyntheticModel(QWEN25_05B, seed=40 + n, layers=2, norm_gains=1.0)
    prompt = _prompt(151936, n, 60 + n)
    oracle = OracleDecoder(model, 256, w8=w8)
    ref_tok, ref = oracle.prefill(prompt)
    engine = QwenDecoderEngine(model, context_length=256, w8=w8)
    try:
        tok, logits = engine.prefill(prompt, 0)
        err = rel_l2(logits, ref)
        announce(f"  rel-L2 {err:.3e}, token {tok} oracle {ref_tok}")
        assert err <= 1e-2
        assert tok == ref_tok or near_tie(ref)
        for layer in (0, 1):
            for slot in sorted({0, n // 2, n - 1}):
                _check_kv_slot(engine, oracle.stage, layer, slot, 2e-2)
            k, v = engine.read_kv(layer, n)
            assert np.all(k == 0) and np.all(v == 0)
        tok2, logits2 = engine.prefill(prompt, 0)
        assert tok2 == tok and np.array_equal(logits2, logits)
    finally:
        engine.close()


def test_prefill_w8_qwen_4_layer():
    """W8 prefill on the MFMA GEMMs: int8 weight tiles converted exactly to
    bf16 on load, the row scale applied to the finished sums (40 tokens: the
    slab GEMM)."""
    model = SyntheticModel(QWEN25_05B, seed=3, layers=4)
    _prefill_case(model, _prompt(151936, 40, 16), 8, 72, 1e-2, "qwen-4L-w8", w8=True)


def test_prefill_w8_smollm_4_layer():
    model = SyntheticModel(SMOLLM2_135M, seed=3, layers=4)
    _prefill_case(model, _prompt(49152, 35, 17), 8, 64, 1e-2, "smollm-4L-w8", w8=True)


def test_prefill_w8_long_prompt():
    """600 tokens: the 128-token-tile W8 GEMMs (no K split)."""
    model = SyntheticModel(QWEN25_05B, seed=5, layers=2)
    _prefill_case(model, _prompt(151936, 600, 18), 4, 1024, 1e-2, "qwen-2L-600-w8", w8=True)


def test_prefill_split_down_wait_limit(monkeypatch):
    """Short prompts run the down projection with K split four ways inside an
    XCD, part 0 polling the other parts' partial sums with a bounded wait.
    With a spin limit of 0 (set from the host: the first poll that finds a
    part missing gives up) a prefill either completes or raises RuntimeError
    ("prefill abandoned"), every kernel exiting normally; every prefill that
    completes matches the oracle, and after an abandon the engine runs the
    slabs unsplit, so at most one of three prefills is abandoned."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce("prefill: K-split down with a zero wait limit")
    model = SyntheticModel(QWEN25_05B, seed=21, layers=2)
    prompt = _prompt(151936, 40, 22)
    monkeypatch.setenv("HK_PERSISTENT_SPIN", "0")
    engine = QwenDecoderEngine(model, context_length=64)
    monkeypatch.delenv("HK_PERSISTENT_SPIN")
    oracle = OracleDecoder(model, 64)
    ref_tokens, ref_logits = oracle.generate_greedy(prompt, 1)
    abandoned = 0
    try:
        for attempt in range(3):
            try:
                tok, logits = engine.prefill(prompt, 0)
            except RuntimeError as err:
                announce(f"  prefill {attempt}: {err}")
                assert "prefill abandoned" in str(err)
                abandoned += 1
                continue
            err = rel_l2(logits, ref_logits[0])
            announce(f"  prefill {attempt}: rel-L2 {err:.3e}")
            assert err <= 1e-2
            assert tok == ref_tokens[0] or near_tie(ref_logits[0])
        assert abandoned <= 1, "after an abandon the engine runs the slabs unsplit"
    finally:
        engine.close()
