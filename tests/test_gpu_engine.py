"""Whole-model decode parity on the GPU: the hk engine against the oracle
(the reference's NumPy BF16 CPU runtime restated in oracle/).

Protocol (the reference's own gates, npu_llm/tests/validate_qwen_tokens.py and
validate_engine_npu.py):
- teacher-forced: both sides see the oracle's token sequence; per-step logits
  must agree within rel-L2 <= 1e-2 and the argmax must agree unless the
  oracle's top-2 gap is below 2**-7 relative (a bf16 near-tie);
  at full depth (24 / 30 layers) the oracle itself moves by 1.4-1.7% rel-L2
  when only its float32 summation order changes (tests/golden/
  order_sensitivity.json, made by order_sensitivity.py there), so no
  reordered implementation can meet 1e-2 there; each full-depth model is
  held to 1.3 times its own measured floor (SmolLM2 1.84e-2, Qwen 2.06e-2,
  Qwen W8 2.20e-2, and the floors of the 4064-token workload for it) and
  the 1e-2 bound is checked on 4-layer models of the same width (floor
  0.65-0.7%);
- free-running greedy: the engine's own generated ids equal the oracle's up to
  the first near-tie step;
- KV slot indexing: slot p is written at step p only (slots above the last
  position stay zero after a reset) and holds the oracle's values.
"""

import os

import numpy as np
import pytest

from _util import announce, check_kv_slot as _check_kv_slot, full_depth_tol, near_tie, rel_l2
from oracle import bf16
from oracle.cpu_backend import OracleDecoder
from runtime.synthetic import QWEN25_05B, SMOLLM2_135M, SyntheticModel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qwen_model():
    return SyntheticModel(QWEN25_05B, seed=0)


@pytest.fixture(scope="module")
def smol_model():
    return SyntheticModel(SMOLLM2_135M, seed=0)


def _prompt(vocab, n, seed):
    rng = np.random.default_rng(seed)
    return [int(t) for t in rng.integers(0, vocab, n)]


def _check_decode(model, prompt, new_tokens, context, *, w8=False, label="", tol=1e-2):
    from runtime.qwen_engine import QwenDecoderEngine

    announce(f"engine parity {label}: prompt {len(prompt)} new {new_tokens} ctx {context} w8={w8}")
    oracle = OracleDecoder(model, context, w8=w8)
    ref_tokens, ref_logits = oracle.generate_greedy(prompt, new_tokens)
    engine = QwenDecoderEngine(model, context_length=context, w8=w8)
    try:
        # teacher-forced per-step logits
        seq = list(prompt) + ref_tokens[:-1]
        last = len(prompt) - 1
        errors, mismatches = [], []
        for pos, tok in enumerate(seq):
            want = pos >= last
            got_tok, got_logits = engine.step_token(tok, pos, logits=want)
            if not want:
                continue
            i = pos - last
            ref = ref_logits[i]
            errors.append(rel_l2(got_logits, ref))
            if got_tok != int(np.argmax(ref)) and not near_tie(ref):
                mismatches.append((pos, got_tok, int(np.argmax(ref))))
        announce(f"  max rel-L2 {max(errors):.3e}, argmax mismatches {mismatches}")
        assert max(errors) <= tol
        assert not mismatches

        # free-running greedy through the device-driven loop
        engine.reset()
        for pos, tok in enumerate(prompt[:-1]):
            engine.step_token(tok, pos, logits=False)
        gen = engine.generate(prompt[-1], len(prompt) - 1, new_tokens)
        agree = new_tokens
        for i, (a, b) in enumerate(zip(gen, ref_tokens)):
            if a != b:
                assert near_tie(ref_logits[i]), f"token {i}: gpu {a} oracle {b}"
                agree = i
                break
        announce(f"  greedy ids match: {gen == ref_tokens} (first {agree} of {new_tokens})")

        # KV slot indexing after the free run: slots written = positions used;
        # values are compared where both runs saw the same tokens (the slot of
        # generated token i is written by the step that consumes it)
        last_pos = len(prompt) - 1 + new_tokens - 1
        same_until = len(prompt) - 1 + agree  # slots 0..same_until hold shared history
        stage = oracle.stage
        kv_tol = 2 * tol
        for layer in (0, model.metadata["layers"] - 1):
            for slot in sorted({0, len(prompt) - 1, min(last_pos - 1, same_until)}):
                _check_kv_slot(engine, stage, layer, slot, kv_tol)
            if last_pos + 1 < context:
                k, v = engine.read_kv(layer, last_pos + 1)
                assert np.all(k == 0) and np.all(v == 0)
    finally:
        engine.close()


SMOL_TOL = full_depth_tol("smollm2-135m full depth, last prompt position")
QWEN_TOL = full_depth_tol("qwen2.5-0.5b full depth, last prompt position")
QWEN_W8_TOL = full_depth_tol("qwen2.5-0.5b W8 full depth, last prompt position")


def test_smollm_135m_shape_decode(smol_model):
    """SmolLM2-135M shape: 35-token prompt, greedy 16 tokens, 64-slot context."""
    _check_decode(smol_model, _prompt(49152, 35, 11), 16, 64, label="smollm2-135m", tol=SMOL_TOL)


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_hidden_1152_decode_on_the_per_kernel_path(w8):
    """A shape the persistent step is not built for (hidden 1152, 18 query /
    3 KV heads, intermediate 3072) decodes on the per-kernel path: its bf16
    QKV GEMV splits K = 1152 four ways inside the workgroup with the RMSNorm
    prologue (the sum of squares met across the slices in LDS), the W8 down
    projection K = 3072.  Teacher-forced logits and KV slots against the
    oracle."""
    from runtime.qwen_engine import QwenDecoderEngine

    shape = dict(QWEN25_05B, hidden_size=1152, intermediate_size=3072, attention_heads=18, kv_heads=3,
                 layers=2, vocab_size=4096)
    model = SyntheticModel(shape, seed=9)
    engine = QwenDecoderEngine(model, context_length=64, w8=w8)
    try:
        assert engine.step_kind(20) == "kernels"
    finally:
        engine.close()
    _check_decode(model, _prompt(4096, 20, 19), 6, 64, w8=w8, label=f"hidden-1152-2L{' W8' if w8 else ''}")


def test_smollm_4_layer_decode_within_1e2():
    model = SyntheticModel(SMOLLM2_135M, seed=0, layers=4)
    _check_decode(model, _prompt(49152, 35, 11), 16, 64, label="smollm2-135m-4L")


def test_qwen_05b_shape_decode(qwen_model):
    """Qwen2.5-0.5B shape: 40-token prompt, greedy 32 tokens (slots 0..70)."""
    _check_decode(qwen_model, _prompt(151936, 40, 12), 32, 72, label="qwen2.5-0.5b", tol=QWEN_TOL)


def test_qwen_4_layer_decode_within_1e2():
    model = SyntheticModel(QWEN25_05B, seed=0, layers=4)
    _check_decode(model, _prompt(151936, 40, 12), 32, 72, label="qwen2.5-0.5b-4L")


def test_qwen_05b_shape_w8_decode(qwen_model):
    """W8 layer projections (int8 + per-row scale), bf16 LM head."""
    _check_decode(qwen_model, _prompt(151936, 40, 13), 32, 72, w8=True, label="qwen2.5-0.5b-w8",
                  tol=QWEN_W8_TOL)


def test_qwen_4_layer_w8_decode_within_1e2():
    model = SyntheticModel(QWEN25_05B, seed=0, layers=4)
    _check_decode(model, _prompt(151936, 40, 13), 32, 72, w8=True, label="qwen2.5-0.5b-4L-w8")


def test_w8_step_forms():
    """W8 layer weights (int8 rows, float32 row scale applied to the finished
    sum; the split's fused down scales each output after the cross-XCD sum)
    take the same step forms by position as bf16: split by XCD below 4096,
    undivided beyond, and undivided everywhere with HK_XCD_SPLIT=0."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce("W8 step kinds")
    model = SyntheticModel(QWEN25_05B, seed=1, layers=1)
    engine = QwenDecoderEngine(model, context_length=4100, w8=True)
    try:
        kinds = [engine.step_kind(p) for p in (0, 767, 768, 4095, 4096)]
        assert kinds == ["xcd_split"] * 2 + ["xcd_split_long"] * 2 + ["persistent"]
    finally:
        engine.close()
    smol = QwenDecoderEngine(SyntheticModel(SMOLLM2_135M, seed=1, layers=1), context_length=4100, w8=True)
    try:
        # 9 query heads: 153 attention tasks at position 4099, within the long form's 224
        assert [smol.step_kind(p) for p in (0, 4099)] == ["xcd_split", "xcd_split_long"]
    finally:
        smol.close()
    os.environ["HK_XCD_SPLIT"] = "0"
    try:
        flat = QwenDecoderEngine(model, context_length=1100, w8=True)
    finally:
        os.environ.pop("HK_XCD_SPLIT", None)
    try:
        assert [flat.step_kind(p) for p in (0, 1099)] == ["persistent"] * 2
    finally:
        flat.close()


def test_smollm_4_layer_w8_decode_within_1e2():
    model = SyntheticModel(SMOLLM2_135M, seed=0, layers=4)
    _check_decode(model, _prompt(49152, 35, 15), 16, 64, w8=True, label="smollm2-4L-w8")


def test_w8_long_context_split_kv():
    model = SyntheticModel(QWEN25_05B, seed=5, layers=2)
    _check_decode(model, _prompt(151936, 600, 16), 8, 4096, w8=True, label="qwen-2L-ctx4096-w8")


def test_per_kernel_path_w8_decode(monkeypatch):
    monkeypatch.setenv("HK_PERSISTENT", "0")
    model = SyntheticModel(QWEN25_05B, seed=0, layers=4)
    _check_decode(model, _prompt(151936, 40, 13), 32, 72, w8=True, label="qwen-4L-w8-per-kernel")


def test_long_context_split_kv():
    """Positions past 256 take the split-KV attention path (several chunks
    merged by log-sum-exp); 2-layer model keeps the oracle quick."""
    model = SyntheticModel(QWEN25_05B, seed=5, layers=2)
    _check_decode(model, _prompt(151936, 600, 14), 8, 4096, label="qwen2-layer-ctx4096")


def test_xcd_split_is_selected_by_context():
    """On MI355X (8 XCDs, workgroup i on XCD i % 8) the Qwen step runs split
    by XCD: with the attention tasks of a layer (14 query heads x 256-slot
    chunks) on XCD 0 while there are at most 48 (below position 768), on the
    224 MLP workgroups while they fit those (below 4096), and as one
    undivided launch beyond; HK_XCD_SPLIT=0 turns the split off, and
    HK_XCD_SPLIT=1 makes engine creation fail (with the reason) where the
    device cannot run it."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce("step kind by position")
    model = SyntheticModel(QWEN25_05B, seed=1, layers=1)
    for required in ("1", None):
        if required:
            os.environ["HK_XCD_SPLIT"] = required
        try:
            engine = QwenDecoderEngine(model, context_length=4100)
        finally:
            os.environ.pop("HK_XCD_SPLIT", None)
        try:
            kinds = [engine.step_kind(p) for p in (0, 40, 767, 768, 4095, 4096, 4099)]
            announce(f"  kinds {kinds}")
            assert kinds == ["xcd_split"] * 3 + ["xcd_split_long"] * 2 + ["persistent"] * 2
            with pytest.raises(ValueError):
                engine.step_kind(4100)
        finally:
            engine.close()
    os.environ["HK_XCD_SPLIT"] = "0"
    try:
        engine = QwenDecoderEngine(model, context_length=64)
        try:
            assert engine.step_kind(40) == "persistent"
        finally:
            engine.close()
    finally:
        del os.environ["HK_XCD_SPLIT"]



def test_undivided_step_short_context(monkeypatch):
    """The undivided persistent step (HK_XCD_SPLIT=0) at the positions the
    split takes by default holds the same bar."""
    monkeypatch.setenv("HK_XCD_SPLIT", "0")
    model = SyntheticModel(QWEN25_05B, seed=0, layers=4)
    _check_decode(model, _prompt(151936, 40, 12), 32, 72, label="qwen-4L-undivided")


def test_undivided_step_long_context(monkeypatch):
    """The undivided persistent step (HK_XCD_SPLIT=0) at positions past 256,
    where its split-KV attention merges several chunks."""
    monkeypatch.setenv("HK_XCD_SPLIT", "0")
    model = SyntheticModel(QWEN25_05B, seed=5, layers=2)
    _check_decode(model, _prompt(151936, 600, 14), 8, 4096, label="qwen2-layer-ctx4096-undivided")


def test_xcd_split_two_chunk_attention():
    """Positions 256..511 give each head two 256-slot chunks, merged by
    log-sum-exp, all on XCD 0 under the split."""
    model = SyntheticModel(QWEN25_05B, seed=7, layers=2)
    _check_decode(model, _prompt(151936, 300, 16), 8, 512, label="qwen-2L-split-two-chunks")


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_xcd_split_agrees_with_undivided_step(monkeypatch, w8):
    """The split and undivided kernels sum the QKV and O rows over different
    lane groups (split: 16 lanes per pair of bf16 rows, 8 lanes per W8 row;
    undivided: 16 and 64 lanes per row), so they agree to float tolerance;
    the greedy ids agree up to a near-tie.  The second run also
    alternates the two split forms (attention on XCD 0 below 768, on the MLP
    XCDs above), which share tags, epochs and flags with each other and with
    the undivided kernel from launch to launch."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce(f"split vs undivided step, w8={w8}")
    model = SyntheticModel(QWEN25_05B, seed=9, layers=4)
    prompt = _prompt(151936, 24, 17)

    def run(split):
        if split:
            monkeypatch.delenv("HK_XCD_SPLIT", raising=False)
        else:
            monkeypatch.setenv("HK_XCD_SPLIT", "0")
        engine = QwenDecoderEngine(model, context_length=1024, w8=w8)
        try:
            logits = []
            for pos, tok in enumerate(prompt):
                _, lg = engine.step_token(tok, pos, logits=pos >= len(prompt) - 4)
                if pos >= len(prompt) - 4:
                    logits.append(lg.copy())
            first = int(np.argmax(logits[-1]))
            gen = engine.generate(first, len(prompt), 12)
            # cross position 768 within one device-driven run: 760..775
            engine.prefill(_prompt(151936, 760 - len(prompt) - 12, 18), len(prompt) + 12)
            gen2 = engine.generate(gen[-1], 760, 16)
            kinds = (engine.step_kind(760), engine.step_kind(775))
            return logits, gen, gen2, kinds
        finally:
            engine.close()

    l_split, g_split, g2_split, k_split = run(True)
    l_flat, g_flat, g2_flat, k_flat = run(False)
    assert k_split == ("xcd_split", "xcd_split_long") and k_flat == ("persistent", "persistent")
    errs = [rel_l2(a, b) for a, b in zip(l_split, l_flat)]
    announce(f"  rel-L2 split vs undivided {max(errs):.3e}; ids equal {g_split == g_flat}, {g2_split == g2_flat}")
    assert max(errs) <= 1e-2
    for gs, gf in ((g_split, g_flat), (g2_split, g2_flat)):
        if gs != gf:
            i = next(i for i, (x, y) in enumerate(zip(gs, gf)) if x != y)
            announce(f"  first difference at step {i}: {gs[i]} vs {gf[i]}")
            assert i > 0


def test_step_contract_errors(qwen_model):
    from runtime.qwen_engine import QwenDecoderEngine

    announce("engine step contract errors")
    model = SyntheticModel(QWEN25_05B, seed=1, layers=1)
    engine = QwenDecoderEngine(model, context_length=8)
    try:
        with pytest.raises(ValueError):
            engine.step_token(0, 8)
        with pytest.raises(ValueError):
            engine.step_token(0, -1)
        with pytest.raises(ValueError):
            engine.step_token(151936, 0)
        # embedding-row form equals the token form
        row = model.bf16_projection("token_embedding")[123]
        a = engine.step(row, 0)
        _, b = engine.step_token(123, 0)
        np.testing.assert_array_equal(a, b)
    finally:
        engine.close()
        engine.close()  # idempotent


def test_per_kernel_path_bf16_decode(monkeypatch):
    """bf16 models of a shape the persistent step is compiled for run it by
    default; HK_PERSISTENT=0 selects the per-kernel step (one GEMV or
    attention kernel per part, replayed as a hipGraph), which must hold the
    same bar."""
    monkeypatch.setenv("HK_PERSISTENT", "0")
    model = SyntheticModel(QWEN25_05B, seed=0, layers=4)
    _check_decode(model, _prompt(151936, 40, 12), 32, 72, label="qwen-4L-per-kernel")


def test_per_kernel_path_split_kv(monkeypatch):
    monkeypatch.setenv("HK_PERSISTENT", "0")
    model = SyntheticModel(QWEN25_05B, seed=5, layers=2)
    _check_decode(model, _prompt(151936, 600, 14), 8, 4096, label="qwen-2L-ctx4096-per-kernel")


def test_persistent_abandon_is_reported(monkeypatch):
    """A persistent-step wait that runs out of polls abandons the launch: every
    workgroup leaves at its next wait, the host reports RuntimeError and clears
    the step's flags.  A spin limit of 0 forces this from the host -- the first
    poll that is not already satisfied gives up -- with every kernel still
    exiting normally.  A fresh engine then decodes correctly."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce("persistent step: forced abandon")
    model = SyntheticModel(QWEN25_05B, seed=3, layers=4)
    prompt = _prompt(151936, 6, 15)
    monkeypatch.setenv("HK_PERSISTENT_SPIN", "0")
    engine = QwenDecoderEngine(model, context_length=16)
    try:
        with pytest.raises(RuntimeError, match="abandoned"):
            for pos, tok in enumerate(prompt):
                engine.step_token(tok, pos, logits=True)
        with pytest.raises(RuntimeError, match="abandoned"):
            engine.generate(prompt[-1], len(prompt) - 1, 4)
    finally:
        engine.close()
    monkeypatch.delenv("HK_PERSISTENT_SPIN")
    oracle = OracleDecoder(model, 16)
    ref_tokens, ref_logits = oracle.generate_greedy(prompt, 1)
    engine = QwenDecoderEngine(model, context_length=16)
    try:
        for pos, tok in enumerate(prompt[:-1]):
            engine.step_token(tok, pos, logits=False)
        got_tok, got_logits = engine.step_token(prompt[-1], len(prompt) - 1, logits=True)
        announce(f"  after abandon: rel-L2 {rel_l2(got_logits, ref_logits[0]):.3e}")
        assert rel_l2(got_logits, ref_logits[0]) <= 1e-2
        assert got_tok == ref_tokens[0] or near_tie(ref_logits[0])
    finally:
        engine.close()


def _check_prefill_decode(model, prompt, new_tokens, context, *, kinds, w8=False, label="", tol=1e-2):
    """Batched prefill of `prompt`, then greedy decode, against the oracle's
    prefill (rows at once, pinned against its per-position prefill) and its
    decode steps.  Every decode position must run one of the step `kinds`.
    Teacher-forced logits per step, KV slots of the prompt and of the decode
    steps, then a free-running device-driven greedy run."""
    from runtime.qwen_engine import QwenDecoderEngine

    n = len(prompt)
    announce(f"prefill+decode parity {label}: prompt {n} new {new_tokens} ctx {context} w8={w8}")
    oracle = OracleDecoder(model, context, w8=w8)
    layers = model.metadata["layers"]
    # a long prompt at full depth keeps the oracle busy for minutes: a line per layer
    progress = (lambda layer: announce(f"  oracle prefill: layer {layer + 1}/{layers}")) if n * layers > 20000 else None
    first, lg0 = oracle.prefill(prompt, progress=progress)
    ref_tokens, ref_logits = [first], [lg0]
    while len(ref_tokens) < new_tokens:
        tok, lg = oracle.decode_token(ref_tokens[-1], n + len(ref_tokens) - 1)
        ref_tokens.append(tok)
        ref_logits.append(lg)
    engine = QwenDecoderEngine(model, context_length=context, w8=w8)
    try:
        positions = range(n, n + new_tokens - 1)
        seen = [engine.step_kind(p) for p in positions]
        assert set(seen) <= set(kinds) and seen[-1] == kinds[-1], seen
        got_tok, got = engine.prefill(prompt)
        errors, mismatches = [rel_l2(got, lg0)], []
        if got_tok != first and not near_tie(lg0):
            mismatches.append((n - 1, got_tok, first))
        for i, p in enumerate(positions, start=1):
            got_tok, got = engine.step_token(ref_tokens[i - 1], p)
            errors.append(rel_l2(got, ref_logits[i]))
            if got_tok != ref_tokens[i] and not near_tie(ref_logits[i]):
                mismatches.append((p, got_tok, ref_tokens[i]))
        announce(f"  kinds {sorted(set(seen))}; max rel-L2 {max(errors):.3e}; mismatches {mismatches}")
        assert max(errors) <= tol
        assert not mismatches
        last = n + new_tokens - 2
        worst = 0.0
        for layer in (0, model.metadata["layers"] - 1):
            for slot in (0, n // 2, n - 1, n, last):
                worst = max(worst, _check_kv_slot(engine, oracle.stage, layer, slot, 2 * tol))
            if last + 1 < context:
                k, v = engine.read_kv(layer, last + 1)
                assert np.all(k == 0) and np.all(v == 0)
        announce(f"  KV slots: worst per-head rel-L2 {worst:.3e}")
        # free-running greedy in one device-driven run across the positions
        start_tok, _ = engine.prefill(prompt, want_logits_array=False)
        if start_tok != first:
            assert near_tie(lg0)
            return
        gen = engine.generate(first, n, new_tokens - 1)
        for i, (a, b) in enumerate(zip(gen, ref_tokens[1:]), start=1):
            if a != b:
                assert near_tie(ref_logits[i]), f"token {i}: gpu {a} oracle {b}"
                break
        announce(f"  greedy ids match: {gen == ref_tokens[1:]}")
    finally:
        engine.close()


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_long_form_at_context_4096_matches_oracle(w8):
    """The context-4096 workload: a 4064-token prompt in one batched prefill,
    then greedy decode at positions 4064..4071 on the long form of the split
    step (224 attention tasks per layer, the form's maximum, each merging 16
    split-KV chunks), against the oracle."""
    model = SyntheticModel(QWEN25_05B, seed=21, layers=2)
    _check_prefill_decode(model, _prompt(151936, 4064, 31), 9, 4096, kinds=("xcd_split_long",), w8=w8,
                          label="qwen-2L-4064")


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_full_depth_context_4096_matches_oracle(qwen_model, w8):
    """The context-4096 workload at full depth (24 layers): a 4064-token
    prompt in one batched prefill against the oracle's, then four
    teacher-forced decode steps at positions 4064..4067 on the long form of
    the split step, logits within 1.3 times the oracle's own summation-order
    floor for this workload, and KV slots checked per head."""
    label = f"qwen2.5-0.5b{' W8' if w8 else ''} full depth, 4064-token prefill + 4 steps"
    _check_prefill_decode(qwen_model, _prompt(151936, 4064, 31), 5, 4096, kinds=("xcd_split_long",), w8=w8,
                          label="qwen-24L-4064", tol=full_depth_tol(label))


def test_split_forms_across_position_768_match_oracle():
    """Decode positions 760..775 cross from the short split form (attention
    on XCD 0, at most 48 tasks) to the long one within one device-driven run."""
    model = SyntheticModel(QWEN25_05B, seed=22, layers=2)
    _check_prefill_decode(model, _prompt(151936, 760, 32), 17, 1024, kinds=("xcd_split", "xcd_split_long"),
                          label="qwen-2L-760")


@pytest.mark.parametrize("w8", [False, True], ids=["bf16", "w8"])
def test_undivided_step_after_tag_wrap_matches_oracle(w8):
    """Activation tags are 16 bits (epoch % 65535 + 1) and the split step
    never writes act[H..I), so after a split launch those words may still
    hold an old undivided launch's tags; when the epoch has moved on by a
    multiple of 65535 the next undivided launch would accept them.  The
    engine clears act before an undivided launch that follows a split one.
    Here the epoch is advanced so that the undivided step at position 4096,
    after a split step at 4095, expects exactly the tags the earlier
    undivided step left in act; the logits must still match the oracle."""
    from runtime.qwen_engine import QwenDecoderEngine

    announce(f"tag wrap: undivided after split, w8={w8}")
    layers = 2
    model = SyntheticModel(QWEN25_05B, seed=23, layers=layers)
    prompt = _prompt(151936, 4096, 33)
    oracle = OracleDecoder(model, 4200, w8=w8)
    oracle.prefill(prompt, compute_logits=False)
    engine = QwenDecoderEngine(model, context_length=4200, w8=w8)
    try:
        engine.prefill(prompt, logits=False)
        rng = np.random.default_rng(34)
        steps = [(int(rng.integers(0, 151936)), p) for p in (4096, 4095, 4096, 4097)]
        kinds = [engine.step_kind(p) for _, p in steps]
        assert kinds == ["persistent", "xcd_split_long", "persistent", "persistent"]
        # launches end on base + 5 L + 1; the third starts at b1 + 2 (5 L + 1) + skip and
        # its layer-0 act poll expects tag (b1 + 5 (L - 1) + 4), the first launch's last layer
        skip = (65535 - 5 * layers - 7) % 65535
        for i, (tok, pos) in enumerate(steps):
            if i == 2:
                engine.skip_epochs(skip)
            want_tok, want = oracle.decode_token(tok, pos)
            got_tok, got = engine.step_token(tok, pos)
            err = rel_l2(got, want)
            announce(f"  step {i} at {pos} ({kinds[i]}): rel-L2 {err:.3e}")
            assert err <= 1e-2
            assert got_tok == want_tok or near_tie(want)
    finally:
        engine.close()
