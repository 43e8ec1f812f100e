"""ChatML tokenizer wrapper, UTF-8-safe streaming, and a synthetic ChatML
tokenizer for random-init packages.

Mirrors the reference's ``npu_llm/runtime/tokenizer.py`` interface
(``SmolLMTokenizer``, ``StreamDetokenizer``, ``DEFAULT_SYSTEM``, ``IM_START``,
``IM_END``): the chat template, the control tokens inserted by id (message
text is encoded with special-token parsing off, so a literal "<|im_end|>" in a
message cannot close a turn), the context-window truncation order of
``encode_chat_window`` (tokenizer.py:118-209) and the byte-exact
``token_bytes`` of byte-level BPE pieces.  Built on the ``tokenizers``
library, like the reference.

``write_chatml_tokenizer`` writes a byte-level BPE ``tokenizer.json`` (plus
``tokenizer_config.json``) of any vocabulary size, with <|endoftext|>,
<|im_start|>, <|im_end|> at ids 0-2 and the 256 byte tokens at 3-258, so the
generation stack and the OpenAI-style callers run on synthetic packages
(there are no real checkpoints here).  Text encodes byte by byte; the other
ids decode to fixed 2-3 byte strings.
"""

import json
from pathlib import Path

from tokenizers import AddedToken, Tokenizer, decoders, models, pre_tokenizers

__all__ = ["DEFAULT_SYSTEM", "IM_START", "IM_END", "REPLACEMENT_CHARACTER", "SmolLMTokenizer",
           "StreamDetokenizer", "write_chatml_tokenizer"]

DEFAULT_SYSTEM = "You are a helpful AI assistant named SmolLM, trained by Hugging Face"
IM_START = "<|im_start|>"
IM_END = "<|im_end|>"
END_OF_TEXT = "<|endoftext|>"
REPLACEMENT_CHARACTER = "�"


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


class SmolLMTokenizer:
    """ChatML tokenizer over a package's ``tokenizer.json`` and
    ``tokenizer_config.json``."""

    def __init__(self, model_dir, default_system=DEFAULT_SYSTEM):
        path = str(Path(model_dir) / "tokenizer.json")
        self._tokenizer = Tokenizer.from_file(path)
        self._content_tokenizer = Tokenizer.from_file(path)
        self._content_tokenizer.encode_special_tokens = True
        config = json.loads((Path(model_dir) / "tokenizer_config.json").read_text())
        self.eos_token = config.get("eos_token", IM_END)
        self.eos_id = self._tokenizer.token_to_id(self.eos_token)
        self.default_system = default_system
        self._im_start_id = self._tokenizer.token_to_id(IM_START)
        self._im_end_id = self._tokenizer.token_to_id(IM_END)
        if self._im_start_id is None or self._im_end_id is None:
            raise ValueError(f"tokenizer does not define the ChatML control tokens {IM_START} and {IM_END}")
        self._newline_ids = self._text_ids("\n")

    # -- encoding ------------------------------------------------------------
    def _text_ids(self, text):
        return self._content_tokenizer.encode(text, add_special_tokens=False).ids

    def _with_system(self, messages):
        if messages and messages[0]["role"] == "system":
            return list(messages)
        return [{"role": "system", "content": self.default_system}, *messages]

    def format_chat(self, messages, add_generation_prompt=True):
        text = "".join(f"{IM_START}{m['role']}\n{m['content']}{IM_END}\n" for m in self._with_system(messages))
        return text + (f"{IM_START}assistant\n" if add_generation_prompt else "")

    def _turn_ids(self, role, content):
        # one turn encoded alone gives the same ids as the rendered template:
        # the control tokens split the text and nothing merges across them
        return [self._im_start_id, *self._text_ids(f"{role}\n{content}"), self._im_end_id, *self._newline_ids]

    def _prompt_tail(self):
        return [self._im_start_id, *self._text_ids("assistant\n")]

    def _turns_ids(self, messages):
        out = []
        for m in messages:
            out += self._turn_ids(m["role"], m["content"])
        return out + self._prompt_tail()

    def encode_chat(self, messages):
        return self._turns_ids(self._with_system(messages))

    def encode_prompt_window(self, prompt, budget):
        """A raw prompt in at most ``budget`` tokens (the newest ones).
        Returns ``(ids, truncated)``."""
        if budget <= 0:
            raise ValueError("prompt budget must be positive")
        ids = self._text_ids(prompt)
        return (ids, False) if len(ids) <= budget else (ids[len(ids) - budget:], True)

    def encode_chat_window(self, messages, budget):
        """A conversation in at most ``budget`` prompt tokens, shortened at turn
        boundaries so the newest message stays whole as long as possible:
        (1) drop the oldest turns after the system prompt; (2) cut the system
        prompt back to a whole-word prefix, or drop it; (3) keep only the
        newest characters of the newest message; (4) as a last resort keep the
        newest ``budget`` tokens.  Returns ``(ids, truncation)``."""
        if budget <= 0:
            raise ValueError("prompt budget must be positive")
        messages = self._with_system(messages)
        report = {"dropped_messages": 0, "truncated_system": False, "dropped_system": False,
                  "truncated_content": False, "token_fallback": False}
        per_turn = [self._turn_ids(m["role"], m["content"]) for m in messages]
        tail = self._prompt_tail()
        everything = [t for ids in per_turn for t in ids] + tail
        if len(everything) <= budget:
            return everything, report

        system, turns = messages[0], messages[1:]
        system_ids, turn_ids = per_turn[0], per_turn[1:]
        if not turns:  # the system message is the only, hence newest, message
            system, turns, system_ids, turn_ids = None, [system], [], [system_ids]
        # (1) oldest turns first, the newest always kept
        total = len(everything)
        first = 0
        while len(turns) - first > 1:
            total -= len(turn_ids[first])
            first += 1
            report["dropped_messages"] += 1
            if total <= budget:
                ids = list(system_ids)
                for t in turn_ids[first:]:
                    ids += t
                return ids + tail, report
        newest = turns[-1]
        # (2) a shorter system prompt, else none
        if system is not None:
            ids = self._system_prefix_fit(system, newest, budget)
            if ids is not None:
                report["truncated_system"] = True
                return ids, report
            report["dropped_system"] = True
            report["dropped_messages"] += 1
            ids = self._turns_ids([newest])
            if len(ids) <= budget:
                return ids, report
        # (3) the newest characters of the newest message
        ids = self._newest_suffix_fit(newest, budget)
        if ids is not None:
            report["truncated_content"] = True
            return ids, report
        report["token_fallback"] = True
        return everything[len(everything) - budget:], report

    @staticmethod
    def _largest(n, ok):
        """Largest k in 0..n with ok(k), or None if not even ok(0).  Token
        counts grow only roughly with text length (BPE merges), so the binary
        search result is checked and walked down if needed."""
        if not ok(0):
            return None
        lo, hi = 0, n
        while lo < hi:
            mid = (lo + hi + 1) // 2
            if ok(mid):
                lo = mid
            else:
                hi = mid - 1
        while lo > 0 and not ok(lo):
            lo -= 1
        return lo

    def _system_prefix_fit(self, system, newest, budget):
        text = system["content"]

        def ids_for(k):
            kept = text[:k]
            if 0 < k < len(text):
                cut = kept.rstrip().rfind(" ")  # end on a word boundary when there is one
                if cut > 0:
                    kept = kept[:cut]
            return self._turns_ids([{"role": system["role"], "content": kept.rstrip()}, newest])

        k = self._largest(len(text), lambda k: len(ids_for(k)) <= budget)
        return ids_for(k) if k else None

    def _newest_suffix_fit(self, turn, budget):
        text = turn["content"]

        def ids_for(k):
            return self._turns_ids([{"role": turn["role"], "content": text[len(text) - k:] if k else ""}])

        k = self._largest(len(text), lambda k: len(ids_for(k)) <= budget)
        return None if k is None else ids_for(k)

    # -- decoding ------------------------------------------------------------
    def decode(self, token_ids, skip_special_tokens=False):
        return self._tokenizer.decode(list(token_ids), skip_special_tokens=skip_special_tokens)

    def token_bytes(self, token_id):
        """The exact bytes one token adds to the output (a byte-level piece may
        hold part of a multi-byte UTF-8 character, which ``decode`` alone would
        render as U+FFFD)."""
        piece = self._tokenizer.id_to_token(int(token_id))
        if piece is not None and all(ch in _CHAR_TO_BYTE for ch in piece):
            return bytes(_CHAR_TO_BYTE[ch] for ch in piece)
        return self.decode([int(token_id)]).encode("utf-8")


class StreamDetokenizer:
    """Text of a growing token sequence, released only in whole characters: a
    trailing partial UTF-8 character (decoded as U+FFFD) is held until a later
    token completes it or ``flush``."""

    def __init__(self, tokenizer):
        self._tokenizer = tokenizer
        self._ids = []
        self._text = ""
        self._sent = 0

    @property
    def text(self):
        return self._text

    def push(self, token_id):
        self._ids.append(int(token_id))
        self._text = self._tokenizer.decode(self._ids)
        return "" if self._text.endswith(REPLACEMENT_CHARACTER) else self._release()

    def flush(self):
        return self._release()

    def _release(self):
        out = self._text[self._sent:]
        self._sent = len(self._text)
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
