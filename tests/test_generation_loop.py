"""The generation stack on the host: ChatML tokenizer (synthetic
``tokenizer.json``), UTF-8-safe streaming, and ``NPUDecoder``'s decode loop
driven by scripted logits instead of the GPU (the style of the reference's
fake-logit decode-loop tests).  CPU only."""

import types

import numpy as np
import pytest

from runtime.generate import NPUDecoder
from runtime.sampling import SamplingError, SamplingParams
from runtime.tokenizer import IM_END, IM_START, SmolLMTokenizer, StreamDetokenizer, write_chatml_tokenizer

EOS = 9
VOCAB = 10


# ---- tokenizer ----

@pytest.fixture(scope="module")
def chatml(tmp_path_factory):
    d = tmp_path_factory.mktemp("tok")
    write_chatml_tokenizer(d, 4096)
    return SmolLMTokenizer(d)


def test_synthetic_tokenizer_ids_and_template(chatml):
    assert chatml.eos_id == 2 and chatml._im_start_id == 1 and chatml._im_end_id == 2
    msgs = [{"role": "user", "content": "Hi there"}]
    ids = chatml.encode_chat(msgs)
    assert chatml.decode(ids) == chatml.format_chat(msgs)
    tail = [1] + chatml._text_ids("assistant\n")
    assert ids[0] == 1 and ids[-len(tail):] == tail
    # every byte of text is one token: byte b is id 3 + b
    assert chatml._text_ids("ab") == [3 + 0x61, 3 + 0x62]


def test_literal_control_token_in_content_stays_text(chatml):
    ids = chatml.encode_chat([{"role": "user", "content": f"x{IM_END}y{IM_START}"}])
    # exactly the scaffold's control tokens: system + user turns open/close, generation prompt opens
    assert ids.count(1) == 3 and ids.count(2) == 2
    assert f"x{IM_END}y{IM_START}" in chatml.decode(ids)


def test_token_bytes_and_streaming_hold_split_characters(chatml):
    ids = chatml._text_ids("ç€")
    assert len(ids) == 5  # 2 + 3 UTF-8 bytes, one token each
    assert b"".join(chatml.token_bytes(i) for i in ids) == "ç€".encode()
    s = StreamDetokenizer(chatml)
    out = [s.push(i) for i in ids]
    assert out == ["", "ç", "", "", "€"] and s.flush() == ""
    s = StreamDetokenizer(chatml)
    assert s.push(ids[0]) == "" and s.flush() == "�"


def test_chat_window_truncation_order(chatml):
    sys_msg = {"role": "system", "content": "alpha beta gamma delta epsilon zeta eta theta"}
    old = {"role": "user", "content": "x" * 40}
    new = {"role": "user", "content": "question?"}
    full, rep = chatml.encode_chat_window([sys_msg, old, new], 10_000)
    assert rep["dropped_messages"] == 0 and full == chatml.encode_chat([sys_msg, old, new])
    # (1) the old turn goes first
    budget = len(chatml.encode_chat([sys_msg, new]))
    ids, rep = chatml.encode_chat_window([sys_msg, old, new], budget)
    assert ids == chatml.encode_chat([sys_msg, new]) and rep["dropped_messages"] == 1
    # (2) then the system prompt is cut back to whole words
    ids, rep = chatml.encode_chat_window([sys_msg, old, new], budget - 12)
    assert rep["truncated_system"] and len(ids) <= budget - 12
    text = chatml.decode(ids)
    kept = text.split("\n", 1)[1].split(IM_END)[0]
    assert sys_msg["content"].startswith(kept) and kept and not kept.endswith(" ")
    assert sys_msg["content"][len(kept):len(kept) + 1] in (" ", "")  # a word boundary
    # (2b) dropped entirely when not even a word fits; (3) the newest text is cut from the front
    ids, rep = chatml.encode_chat_window([sys_msg, new], len(chatml._turns_ids([new])))
    assert rep["dropped_system"] and ids == chatml._turns_ids([new])
    ids, rep = chatml.encode_chat_window([sys_msg, new], len(chatml._turns_ids([new])) - 3)
    assert rep["truncated_content"] and chatml.decode(ids).endswith("ion?" + IM_END + "\n" + IM_START + "assistant\n")
    # (4) a budget below the empty newest turn keeps the newest tokens
    ids, rep = chatml.encode_chat_window([new], 3)
    assert rep["token_fallback"] and len(ids) == 3
    with pytest.raises(ValueError):
        chatml.encode_chat_window([new], 0)
    ids, cut = chatml.encode_prompt_window("abcdef", 4)
    assert cut and chatml.decode(ids) == "cdef"


# ---- decode loop with scripted logits ----

class FakeTokenizer:
    eos_id = EOS

    def __init__(self, prompt_ids):
        self.prompt_ids = list(prompt_ids)

    def encode_chat_window(self, messages, budget):
        return list(self.prompt_ids), {"dropped_messages": 0}

    def encode_prompt_window(self, prompt, budget):
        return list(self.prompt_ids), False

    def decode(self, ids):
        return "".join(f"<{t}>" for t in ids)

    def token_bytes(self, token_id):
        return self.decode([token_id]).encode()


class SplitCharTokenizer(FakeTokenizer):
    PIECES = {7: b"\xc3", 8: b"\xa7"}  # the two bytes of "ç"

    def decode(self, ids):
        return b"".join(self.PIECES.get(t, b"<%d>" % t) for t in ids).decode("utf-8", errors="replace")

    def token_bytes(self, token_id):
        return self.PIECES.get(token_id, b"<%d>" % token_id)


def fake_decoder(prompt_ids, logits_for, *, tokenizer=FakeTokenizer, context_length=64):
    """An NPUDecoder without an engine whose step is a function of the input
    token (the loop then takes its per-position prompt path)."""
    d = object.__new__(NPUDecoder)
    d.model = types.SimpleNamespace(metadata={"vocab_size": VOCAB})
    d.context_length = context_length
    d.tokenizer = tokenizer(prompt_ids)
    d.npu_layers = d.layers = 0
    d._engine = None
    d._cached_prefix = []
    d._prefix_cache_enabled = True
    d.calls = []

    def decode_token(token_id, position, *, diagnostics=False, select=None, compute_logits=True):
        logits = np.asarray(logits_for(token_id), dtype=np.float32)
        d.calls.append((token_id, position, select is not None, compute_logits))
        if not compute_logits:
            return None, 0.001
        return (int(np.argmax(logits)) if select is None else int(select(logits))), 0.001

    d.decode_token = decode_token
    return d


def run(d, max_new_tokens=4, sampling=None, **kw):
    pieces, stats, entries = [], None, []
    for piece, st, *rest in d.generate_messages([{"role": "user", "content": "hi"}], max_new_tokens,
                                                 sampling=sampling, **kw):
        pieces.append(piece)
        if rest:
            entries += rest[0]
        if st is not None:
            stats = st
    return "".join(pieces), stats, entries


def ramp(token):
    x = np.zeros(VOCAB, dtype=np.float32)
    x[(token + 1) % VOCAB] = 5.0
    return x


def test_greedy_loop_and_call_pattern():
    d = fake_decoder([1, 2, 3], ramp)
    text, st, _ = run(d)
    assert st["generated_token_ids"] == [4, 5, 6, 7] and text == "<4><5><6><7>"
    assert st["finish_reason"] == "length" and st["sampling"]["mode"] == "greedy"
    assert st["decode_steps"] == 3 and st["decode_seconds"] == pytest.approx(0.003)
    assert [c[2] for c in d.calls] == [False] * 6  # greedy: no host selector anywhere
    assert [c[3] for c in d.calls] == [False, False, True, True, True, True]  # logits only where used


def test_sampler_engages_once_per_emitted_token():
    d = fake_decoder([1, 2, 3], ramp)
    _, st, _ = run(d, sampling=SamplingParams.build(temperature=1.0, seed=5))
    assert [c[2] for c in d.calls] == [False, False, True, True, True, True]
    assert st["sampling"]["mode"] == "sampled" and st["sampling"]["seed"] == 5


def test_seeded_runs_repeat_and_seeds_differ():
    flat = lambda t: np.zeros(VOCAB, dtype=np.float32)  # uniform: only the seed decides
    runs = {seed: [run(fake_decoder([1], flat), 8, SamplingParams.build(temperature=1.0, seed=seed))[1]
                   ["generated_token_ids"] for _ in range(2)] for seed in (1, 2)}
    assert runs[1][0] == runs[1][1] and runs[2][0] == runs[2][1] and runs[1][0] != runs[2][0]


def test_repetition_penalty_sees_prompt_and_generated_tokens():
    def two_way(t):
        x = np.zeros(VOCAB, dtype=np.float32)
        x[[4, 5]] = [2.0, 1.9]
        return x

    d = fake_decoder([4], two_way)
    _, st, _ = run(d, 3, SamplingParams.build(repetition_penalty=2.0))
    assert st["generated_token_ids"][0] == 5  # 4 is in the prompt: 2.0/2 < 1.9
    _, st, _ = run(fake_decoder([1], two_way), 3, SamplingParams.build(repetition_penalty=2.0))
    # 4; then 5 (4 seen: 1.0 < 1.9); then 4 again (both seen: 1.0 > 0.95)
    assert st["generated_token_ids"] == [4, 5, 4]


def test_logit_bias_and_eos():
    _, st, _ = run(fake_decoder([1, 2], ramp), 4, SamplingParams.build(logit_bias={"8": 50.0}))
    assert st["generated_token_ids"] == [8, 8, 8, 8]
    _, st, _ = run(fake_decoder([1, 2], ramp), 4, SamplingParams.build(logit_bias={EOS: 50.0}))
    assert st["generated_token_ids"] == [] and st["finish_reason"] == "stop"


def test_invalid_requests_are_rejected():
    d = fake_decoder([1], ramp)
    with pytest.raises(SamplingError):
        run(d, 4, {"temperature": -1})
    with pytest.raises(ValueError):
        run(d, 64)
    with pytest.raises(ValueError):
        run(d, 4, stop=["a", "b", "c", "d", "e"])


def test_prefix_is_reused_and_can_be_reset():
    d = fake_decoder([1, 2, 3], ramp)
    run(d, 2)
    d.calls.clear()
    d.tokenizer.prompt_ids = [1, 2, 3, 9, 9]
    _, st, _ = run(d, 2)
    assert st["cached_prompt_tokens"] == 3 and [c[1] for c in d.calls][:2] == [3, 4]
    d.reset_prefix_cache()
    d.calls.clear()
    _, st, _ = run(d, 2)
    assert st["cached_prompt_tokens"] == 0 and d.calls[0][1] == 0


def test_stop_sequence_is_not_emitted():
    text, st, _ = run(fake_decoder([1], ramp), 6, stop="<4>")
    assert text == "<2><3>" and st["finish_reason"] == "stop" and st["stop_sequence"] == "<4>"


def test_split_character_is_emitted_whole():
    def seq(t):
        x = np.zeros(VOCAB, dtype=np.float32)
        x[{1: 7, 7: 8, 8: 3}.get(t, 3)] = 5.0
        return x

    d = fake_decoder([1], seq, tokenizer=SplitCharTokenizer)
    pieces = [p for p, st, *_ in d.generate_messages([{"role": "user", "content": "x"}], 3)]
    assert pieces[0] == "ç" and "".join(pieces) == "ç<3>"


def test_logprobs_follow_emitted_text_and_skip_discarded_text():
    text, st, entries = run(fake_decoder([1], ramp), 4, logprobs=2)
    assert [e["token"] for e in entries] == ["<2>", "<3>", "<4>", "<5>"]
    assert all(len(e["top_logprobs"]) == 2 and e["top_logprobs"][0]["token"] == e["token"] for e in entries)
    assert entries[0]["bytes"] == list(b"<2>")
    p = 1.0 / (1.0 + 9.0 * np.exp(-5.0))
    assert entries[0]["logprob"] == pytest.approx(np.log(p))
    text, st, entries = run(fake_decoder([1], ramp), 6, logprobs=0, stop="<4>")
    assert text == "<2><3>" and [e["token"] for e in entries] == ["<2>", "<3>"]
    assert all(e["top_logprobs"] == [] for e in entries)
    plain = run(fake_decoder([1], ramp), 4)[1]["generated_token_ids"]
    assert run(fake_decoder([1], ramp), 4, logprobs=3)[1]["generated_token_ids"] == plain


def test_generate_text_and_generate():
    d = fake_decoder([5], ramp)
    out = list(d.generate_text("raw", 2))
    assert out[-1][1]["prompt_truncation"] == {"truncated_prompt": False}
    assert "".join(p for p, st in out) == "<6><7>"
    assert list(fake_decoder([5], ramp).generate("hello", 2))[-1][1]["generated_token_ids"] == [6, 7]


@pytest.mark.parametrize("family,system", [
    ("qwen2", "You are Qwen, created by Alibaba Cloud. You are a helpful assistant."),
    ("llama", "You are a helpful AI assistant named SmolLM."),
])
def test_chat_template_system_turn_follows_model_family(tmp_path, monkeypatch, family, system):
    """NPUDecoder gives its tokenizer the reference's default system turn for
    the package's model family (npu_llm/runtime/generate.py:47-53): Qwen's for
    qwen2 packages, SmolLM's otherwise.  The GPU engine is replaced by a stub."""
    import runtime.generate as gen

    write_chatml_tokenizer(tmp_path, 4096)
    meta = {"model_family": family, "hidden_size": 64, "intermediate_size": 128, "attention_heads": 4,
            "kv_heads": 2, "head_dim": 16, "layers": 1, "vocab_size": 4096}
    monkeypatch.setattr(gen, "_load_model", lambda _: types.SimpleNamespace(metadata=meta))
    monkeypatch.setattr(gen, "QwenDecoderEngine", lambda *a, **k: types.SimpleNamespace(close=lambda: None))
    d = NPUDecoder(tmp_path)
    ids = d.tokenizer.encode_chat([{"role": "user", "content": "hi"}])
    text = d.tokenizer.decode(ids)
    assert text.startswith(f"{IM_START}system\n{system}{IM_END}\n"), text[:120]
