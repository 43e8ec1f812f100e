"""ChatML tokenizer, UTF-8-safe streaming, and a synthetic ChatML tokenizer
for random-init packages.

Contract of ``npu_llm/runtime/tokenizer.py`` as its callers use it
(``generate.py``, ``api_server.py``, ``chat.py``): ``SmolLMTokenizer(model_dir,
default_system=...)`` with ``eos_token`` / ``eos_id``, ``format_chat``,
``encode_chat``, ``encode_prompt_window``, ``encode_chat_window`` (the
truncation order and report keys of tokenizer.py:119-196), ``decode`` and the
byte-exact ``token_bytes``; ``StreamDetokenizer`` (``push``, ``flush``,
``text``); ``DEFAULT_SYSTEM``, ``IM_START``, ``IM_END``.  Message text is
encoded with special-token parsing off and the control tokens are inserted by
id, so a literal "<|im_end|>" inside a message cannot close its turn.

Design:
- a turn is ``<|im_start|>`` + ids of "role\ncontent" + ``<|im_end|>`` + ids
  of "\n"; the control tokens split the text, so turns encode independently
  and a prompt is the concatenation of its turns' ids plus the generation
  prompt;
- ``encode_chat_window`` walks an ordered list of candidate prompts, from the
  whole conversation to the last-resort token cut, and returns the first that
  fits the budget (candidates are built lazily, so only the ones tried cost
  an encode);
- the streaming detokenizer feeds each token's bytes into an incremental
  UTF-8 decoder, which holds an incomplete character until its last byte
  arrives, so each token costs O(1) instead of a decode of the whole
  sequence.

``write_chatml_tokenizer`` writes a byte-level BPE ``tokenizer.json`` (plus
``tokenizer_config.json``) of any vocabulary size, with <|endoftext|>,
<|im_start|>, <|im_end|> at ids 0-2 and the 256 byte tokens at 3-258, so the
generation stack and the OpenAI-style callers run on synthetic packages
(there are no real checkpoints here).  Text encodes byte by byte; the other
ids decode to fixed 2-3 byte strings.
"""

import codecs
import json
from pathlib import Path

from tokenizers import AddedToken, Tokenizer, decoders, models, pre_tokenizers

__all__ = ["DEFAULT_SYSTEM", "IM_START", "IM_END", "REPLACEMENT_CHARACTER", "SmolLMTokenizer",
           "StreamDetokenizer", "write_chatml_tokenizer"]

DEFAULT_SYSTEM = "You are a helpful AI assistant named SmolLM, trained by Hugging Face"
IM_START = "<|im_start|>"
IM_END = "<|im_end|>"
END_OF_TEXT = "<|endoftext|>"
REPLACEMENT_CHARACTER = "\ufffd"


def _byte_alphabet():
    """The byte-level BPE alphabet: byte b <-> one printable character (the
    GPT-2 convention: printable Latin-1 bytes map to themselves, the rest to
    code points from 256 up, in byte order)."""
    direct = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    chars, extra = {}, 0
    for b in range(256):
        if b in direct:
            chars[b] = chr(b)
        else:
            chars[b] = chr(256 + extra)
            extra += 1
    return chars


_BYTE_TO_CHAR = _byte_alphabet()
_CHAR_TO_BYTE = {c: b for b, c in _BYTE_TO_CHAR.items()}


def _largest_fitting(limit, fits):
    """Largest n in 0..limit with fits(n) for a predicate that holds up to
    some n and not beyond (token counts grow with kept text); None when not
    even fits(0).  Bisection over [known fit, known miss)."""
    if not fits(0):
        return None
    if fits(limit):
        return limit
    good, bad = 0, limit
    while bad - good > 1:
        mid = (good + bad) // 2
        if fits(mid):
            good = mid
        else:
            bad = mid
    return good


def _word_prefix(text, n):
    """The first n characters of text, ended at a word boundary when the cut
    falls inside the text and one exists, without trailing spaces."""
    kept = text[:n]
    if 0 < n < len(text):
        space = kept.rstrip().rfind(" ")
        if space > 0:
            kept = kept[:space]
    return kept.rstrip()


class SmolLMTokenizer:
    """ChatML tokenizer over a package's ``tokenizer.json`` and
    ``tokenizer_config.json``."""

    def __init__(self, model_dir, default_system=DEFAULT_SYSTEM):
        folder = Path(model_dir)
        self._tokenizer = Tokenizer.from_file(str(folder / "tokenizer.json"))
        # message text is untrusted: a second instance encodes it with
        # special-token parsing off
        self._plain = Tokenizer.from_file(str(folder / "tokenizer.json"))
        self._plain.encode_special_tokens = True
        config = json.loads((folder / "tokenizer_config.json").read_text())
        self.eos_token = config.get("eos_token", IM_END)
        self.eos_id = self._tokenizer.token_to_id(self.eos_token)
        self.default_system = default_system
        self._im_start_id = self._tokenizer.token_to_id(IM_START)
        self._im_end_id = self._tokenizer.token_to_id(IM_END)
        if None in (self._im_start_id, self._im_end_id):
            raise ValueError(f"tokenizer does not define the ChatML control tokens {IM_START} and {IM_END}")
        self._turn_end = [self._im_end_id, *self._text_ids("\n")]
        self._reply_start = [self._im_start_id, *self._text_ids("assistant\n")]

    # -- encoding ------------------------------------------------------------
    def _text_ids(self, text):
        return self._plain.encode(text, add_special_tokens=False).ids

    def _conversation(self, messages):
        """The messages with the default system turn in front when they bring none."""
        messages = list(messages)
        if not messages or messages[0]["role"] != "system":
            messages.insert(0, {"role": "system", "content": self.default_system})
        return messages

    def format_chat(self, messages, add_generation_prompt=True):
        turns = (f"{IM_START}{m['role']}\n{m['content']}{IM_END}\n" for m in self._conversation(messages))
        return "".join(turns) + (f"{IM_START}assistant\n" if add_generation_prompt else "")

    def _turn(self, message):
        return [self._im_start_id, *self._text_ids(f"{message['role']}\n{message['content']}"), *self._turn_end]

    def _prompt(self, turn_ids):
        """Concatenated turns plus the generation prompt."""
        out = [t for ids in turn_ids for t in ids]
        out += self._reply_start
        return out

    def _turns_ids(self, messages):
        return self._prompt([self._turn(m) for m in messages])

    def encode_chat(self, messages):
        return self._turns_ids(self._conversation(messages))

    def encode_prompt_window(self, prompt, budget):
        """A raw prompt (no chat turns) in at most ``budget`` tokens, its
        newest ones when it is longer.  Returns ``(ids, truncated)``."""
        if budget <= 0:
            raise ValueError("prompt budget must be positive")
        ids = self._text_ids(prompt)
        truncated = len(ids) > budget
        return (ids[-budget:] if truncated else ids), truncated

    def encode_chat_window(self, messages, budget):
        """A conversation in at most ``budget`` prompt tokens.  The newest
        message stays whole as long as possible; the prompt is shortened at
        turn boundaries, in this order: drop the oldest turns after the
        system prompt; cut the system prompt back to a whole-word prefix, or
        drop it; keep only the newest characters of the newest message; as a
        last resort keep the newest ``budget`` tokens.  Returns ``(ids,
        truncation)`` with the reference's report keys."""
        if budget <= 0:
            raise ValueError("prompt budget must be positive")
        report = {"dropped_messages": 0, "truncated_system": False, "dropped_system": False,
                  "truncated_content": False, "token_fallback": False}
        for ids, changes in self._window_plans(self._conversation(messages), budget):
            if ids is not None and len(ids) <= budget:
                for key, value in changes.items():
                    report[key] = value
                return ids, report
        raise AssertionError("the token cut always fits")  # unreachable

    def _window_plans(self, messages, budget):
        """Candidate prompts in order of preference, each with the report
        entries it implies; None for a plan that has no fitting form."""
        turn_ids = [self._turn(m) for m in messages]
        everything = self._prompt(turn_ids)
        yield everything, {}
        if len(messages) > 1:
            system, system_ids, rest, rest_ids = messages[0], turn_ids[0], messages[1:], turn_ids[1:]
        else:  # a lone system message is the newest message
            system, system_ids, rest, rest_ids = None, [], messages, turn_ids
        for dropped in range(1, len(rest)):
            yield self._prompt([system_ids] + rest_ids[dropped:]), {"dropped_messages": dropped}
        newest = rest[-1]
        dropped = len(rest) - 1
        if system is not None:
            yield self._system_prefix_fit(system, newest, budget), {"dropped_messages": dropped,
                                                                    "truncated_system": True}
            dropped += 1
            yield self._turns_ids([newest]), {"dropped_messages": dropped, "dropped_system": True}
        system_gone = {"dropped_system": True} if system is not None else {}
        yield self._newest_suffix_fit(newest, budget), {"dropped_messages": dropped, **system_gone,
                                                        "truncated_content": True}
        yield everything[-budget:], {"dropped_messages": dropped, **system_gone, "token_fallback": True}

    def _system_prefix_fit(self, system, newest, budget):
        """The longest whole-word beginning (at least one character kept) of
        the system prompt that fits together with the newest turn."""
        text, newest_ids = system["content"], self._turn(newest)

        def prompt(n):
            return self._prompt([self._turn({"role": system["role"], "content": _word_prefix(text, n)}), newest_ids])

        n = _largest_fitting(len(text), lambda n: len(prompt(n)) <= budget)
        return prompt(n) if n else None

    def _newest_suffix_fit(self, turn, budget):
        """The newest turn with the longest tail of its text that fits."""
        text = turn["content"]

        def prompt(n):
            return self._turns_ids([{"role": turn["role"], "content": text[len(text) - n:]}])

        n = _largest_fitting(len(text), lambda n: len(prompt(n)) <= budget)
        return None if n is None else prompt(n)

    # -- decoding ------------------------------------------------------------
    def decode(self, token_ids, skip_special_tokens=False):
        return self._tokenizer.decode(list(token_ids), skip_special_tokens=skip_special_tokens)

    def token_bytes(self, token_id):
        """The exact bytes one token adds to the output (a byte-level piece may
        hold part of a multi-byte UTF-8 character, which ``decode`` alone would
        render as U+FFFD)."""
        piece = self._tokenizer.id_to_token(int(token_id))
        if piece is not None:
            raw = [_CHAR_TO_BYTE.get(ch) for ch in piece]
            if None not in raw:
                return bytes(raw)
        return self.decode([int(token_id)]).encode("utf-8")


class StreamDetokenizer:
    """Text of a growing token sequence, released in whole characters only:
    each token's bytes (``tokenizer.token_bytes``) go through an incremental
    UTF-8 decoder, which keeps an incomplete trailing character until a later
    token completes it or ``flush`` renders it as U+FFFD."""

    def __init__(self, tokenizer):
        self._tokenizer = tokenizer
        self._utf8 = codecs.getincrementaldecoder("utf-8")(errors="replace")
        self._released = []

    @property
    def text(self):
        """Everything decoded so far, a held partial character as U+FFFD."""
        pending, _ = self._utf8.getstate()
        return "".join(self._released) + pending.decode("utf-8", errors="replace")

    def push(self, token_id):
        """Add a token; return the text it completes (possibly empty)."""
        out = self._utf8.decode(self._tokenizer.token_bytes(int(token_id)))
        self._released.append(out)
        return out

    def flush(self):
        """Release whatever is held, an incomplete character as U+FFFD."""
        out = self._utf8.decode(b"", final=True)
        self._released.append(out)
        return out


def write_chatml_tokenizer(directory, vocab_size):
    """Write a synthetic byte-level ChatML ``tokenizer.json`` of exactly
    ``vocab_size`` ids and a ``tokenizer_config.json`` (eos <|im_end|>) into
    ``directory``.  Returns the directory."""
    specials = [END_OF_TEXT, IM_START, IM_END]
    if vocab_size < len(specials) + 256:
        raise ValueError("vocab_size too small for the byte alphabet")
    out = Path(directory)
    out.mkdir(parents=True, exist_ok=True)
    alphabet = [_BYTE_TO_CHAR[b] for b in range(256)]
    vocab = {s: i for i, s in enumerate(specials)}
    for b, ch in enumerate(alphabet):
        vocab[ch] = len(specials) + b

    def filler():
        for a in alphabet:
            for b in alphabet:
                yield a + b
        for a in alphabet:
            for b in alphabet:
                for c in alphabet:
                    yield a + b + c

    pieces = filler()
    while len(vocab) < vocab_size:
        vocab[next(pieces)] = len(vocab)
    tok = Tokenizer(models.BPE(vocab=vocab, merges=[]))
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    tok.add_special_tokens([AddedToken(s, special=True, normalized=False) for s in specials])
    tok.save(str(out / "tokenizer.json"))
    (out / "tokenizer_config.json").write_text(json.dumps(
        {"eos_token": IM_END, "bos_token": None, "pad_token": END_OF_TEXT, "unk_token": None,
         "additional_special_tokens": [IM_START, IM_END]}, indent=1) + "\n")
    return out
