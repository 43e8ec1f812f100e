"""The NPUDecoder / DecoderEngine drop-in surface on the GPU, from an on-disk
package in the reference's format (contract of npu_llm/runtime/generate.py:
732-973 and npu_llm/runtime/engine.py:65-82)."""

import numpy as np
import pytest

from _util import announce
from oracle import bf16
from oracle.cpu_backend import OracleDecoder
from runtime.model import XDNA1Model, write_package
from runtime.synthetic import SyntheticModel

pytestmark = pytest.mark.gpu

SMALL = {
    "model_family": "qwen2", "hidden_size": 256, "intermediate_size": 512, "attention_heads": 4,
    "kv_heads": 2, "head_dim": 64, "layers": 2, "vocab_size": 1000, "rope_theta": 1e6,
    "rms_norm_eps": 1e-6, "qkv_bias": True,
}


@pytest.fixture(scope="module")
def package(tmp_path_factory):
    model = SyntheticModel(SMALL, seed=21, std=0.08)
    path = write_package(model, tmp_path_factory.mktemp("pkg") / "small")
    return XDNA1Model(path), path


def test_decode_token_contract(package):
    from runtime.generate import NPUDecoder

    announce("NPUDecoder decode_token contract")
    model, path = package
    dec = NPUDecoder(path, context_length=32)
    oracle = OracleDecoder(model, 32)
    try:
        prompt = [3, 99, 512, 7, 801]
        for pos, tok in enumerate(prompt[:-1]):
            res = dec.decode_token(tok, pos, compute_logits=False)
            assert res[0] is None and res[1] >= 0.0
            oracle.decode_token(tok, pos, compute_logits=False)
        ref_tok, ref_logits = oracle.decode_token(prompt[-1], 4)
        tok, elapsed = dec.decode_token(prompt[-1], 4)
        assert tok == ref_tok and elapsed >= 0.0
        # the same step again with diagnostics and with a custom selector
        tok2, _, diag = dec.decode_token(prompt[-1], 4, diagnostics=True)
        assert tok2 == ref_tok and diag["top_token_ids"][0] == ref_tok
        assert diag["top_logit_margin"] >= 0.0
        picked, _ = dec.decode_token(prompt[-1], 4, select=lambda lg: int(np.argsort(lg)[-2]))
        assert picked == int(np.argsort(ref_logits)[-2])
        with pytest.raises(ValueError):
            dec.decode_token(1, 32)
        with pytest.raises(ValueError):
            dec.decode_token(1, -1)
    finally:
        dec.close()
        dec.close()


def test_generate_ids_and_prefix_reuse(package):
    from runtime.generate import NPUDecoder

    announce("NPUDecoder generate_ids + prefix reuse")
    model, path = package
    dec = NPUDecoder(path, context_length=64)
    try:
        prompt = [11, 22, 33, 44, 55, 66]
        oracle = OracleDecoder(model, 64)
        ref, _ = oracle.generate_greedy(prompt, 10)
        got, stats = dec.generate_ids(prompt, 10)
        assert got == ref
        assert stats["cached_prompt_tokens"] == 0 and stats["decode_steps"] == 9
        again, stats2 = dec.generate_ids(prompt, 10)
        assert again == ref and stats2["cached_prompt_tokens"] == len(prompt) - 1
        dec.reset_prefix_cache()
        _, stats3 = dec.generate_ids(prompt, 3)
        assert stats3["cached_prompt_tokens"] == 0
    finally:
        dec.close()


def test_decoder_engine_returns_final_norm(package):
    from runtime.engine import DecoderEngine

    announce("DecoderEngine final hidden")
    model, _ = package
    eng = DecoderEngine(model, context_length=16)
    oracle = OracleDecoder(model, 16)
    try:
        emb = np.asarray(model.raw("token_embedding")).reshape(1000, 256)
        for pos, tok in enumerate([5, 6, 7]):
            out = eng.step(emb[tok], pos)
            hidden = oracle.hidden_after_layers(tok, pos)
        ref = bf16.to_bits(oracle.stage.norm(hidden, "final_norm"))
        got = bf16.from_bits(out).astype(np.float64)
        want = bf16.from_bits(ref).astype(np.float64)
        assert np.abs(got - want).max() <= 0.02 * np.abs(want).max()
    finally:
        eng.close()


def test_generate_messages_on_the_gpu(tmp_path):
    """The generation stack (ChatML prompt, batched prefill, host sampling,
    stop sequences, log probabilities) over the GPU engine, against the
    oracle's greedy continuation of the same prompt ids."""
    from runtime.generate import NPUDecoder
    from runtime.sampling import SamplingParams
    from runtime.tokenizer import write_chatml_tokenizer

    announce("NPUDecoder generate_messages (synthetic ChatML tokenizer)")
    model = SyntheticModel(SMALL, seed=21, std=0.08)
    path = write_package(model, tmp_path / "chat")
    write_chatml_tokenizer(path, SMALL["vocab_size"])
    dec = NPUDecoder(path, context_length=160)
    try:
        msgs = [{"role": "user", "content": "Hello GPU"}]
        prompt = dec.tokenizer.encode_chat_window(msgs, 160 - 8)[0]
        oracle = OracleDecoder(XDNA1Model(path), 160)
        ref, _ = oracle.generate_greedy(prompt, 8)
        eos = dec.tokenizer.eos_id
        want = ref[:ref.index(eos)] if eos in ref else ref
        chunks = list(dec.generate_messages(msgs, 8))
        stats = chunks[-1][1]
        assert stats["generated_token_ids"] == want
        assert stats["prompt_tokens"] == len(prompt) and stats["cached_prompt_tokens"] == 0
        assert "".join(c[0] for c in chunks) == dec.tokenizer.decode(want)
        # the same request again reuses the prompt; with log probabilities the tokens do not change
        chunks = list(dec.generate_messages(msgs, 8, logprobs=2))
        assert chunks[-1][1]["generated_token_ids"] == want
        assert chunks[-1][1]["cached_prompt_tokens"] == len(prompt) - 1
        entries = [e for c in chunks for e in c[2]]
        assert len(entries) == len(want) and all(len(e["top_logprobs"]) == 2 for e in entries)
        assert all(e["top_logprobs"][0]["logprob"] >= e["top_logprobs"][1]["logprob"] for e in entries)
        # seeded sampling repeats; logit bias forces a token
        p = SamplingParams.build(temperature=0.9, top_k=20, seed=7)
        a = list(dec.generate_messages(msgs, 6, p))[-1][1]["generated_token_ids"]
        b = list(dec.generate_messages(msgs, 6, p))[-1][1]["generated_token_ids"]
        assert a == b
        forced = list(dec.generate_messages(msgs, 4, SamplingParams.build(logit_bias={"65": 100.0})))
        assert forced[-1][1]["generated_token_ids"] == [65] * 4
        text = "".join(c[0] for c in list(dec.generate_messages(msgs, 8, stop=dec.tokenizer.decode([65]))))
        assert dec.tokenizer.decode([65]) not in text
    finally:
        dec.close()
