"""Stop sequences and log-probability options for completions (host side).

Contract of ``npu_llm/runtime/stopping.py`` (used by ``generate.py:1033-1034``,
``1222-1223`` and ``api_server.py:129-140, 700-701``): ``normalize_stop``,
``normalize_logprobs``, ``StopMatcher`` and ``log_softmax``; at most 4 stop
strings of at most 256 characters, at most 20 top log probabilities; the same
``ValueError`` texts.

Design: a matcher compiles its stop strings into one regular expression whose
alternatives are tried in the order given, so ``search`` returns the match
that starts first and, among matches starting at the same character, the
earliest-listed stop (the OpenAI rule: the completion ends before the first
stop).  Text that could still grow into a stop is held back: the matcher
keeps the set of every proper prefix of every stop and holds the longest tail
of the text found in that set.
"""

import re

import numpy as np

__all__ = ["MAX_STOP_SEQUENCES", "MAX_STOP_LENGTH", "MAX_TOP_LOGPROBS", "normalize_stop",
           "normalize_logprobs", "StopMatcher", "log_softmax"]

MAX_STOP_SEQUENCES = 4
MAX_STOP_LENGTH = 256
MAX_TOP_LOGPROBS = 20


def _check_stop_item(item):
    if not isinstance(item, str) or item == "":
        raise ValueError("each stop sequence must be a non-empty string")
    if len(item) > MAX_STOP_LENGTH:
        raise ValueError(f"stop sequences cannot exceed {MAX_STOP_LENGTH} characters")
    return item


def normalize_stop(value):
    """An OpenAI ``stop`` value (None, a string or a list of strings) as a
    tuple of distinct stop strings in their first-seen order."""
    if value is None:
        return ()
    if isinstance(value, str):
        value = (value,)
    elif not isinstance(value, (list, tuple)):
        raise ValueError("stop must be a string or an array of strings")
    if len(value) > MAX_STOP_SEQUENCES:
        raise ValueError(f"stop accepts at most {MAX_STOP_SEQUENCES} sequences")
    # dict keys keep insertion order and drop repeats
    return tuple(dict.fromkeys(_check_stop_item(item) for item in value))


def normalize_logprobs(value):
    """``None`` (no log probabilities) or a count of top alternatives, 0..20."""
    if value is not None:
        if type(value) is bool or not isinstance(value, int):
            raise ValueError("top_logprobs must be an integer")
        if value not in range(MAX_TOP_LOGPROBS + 1):
            raise ValueError(f"top_logprobs must be between 0 and {MAX_TOP_LOGPROBS}")
    return value


class StopMatcher:
    """Streams text through, cutting it before the first stop string; no part
    of a stop string is ever returned.  ``matched`` names the stop that ended
    the text (None until one does)."""

    def __init__(self, stops=()):
        self.stops = tuple(stops)
        self.matched = None
        self._tail = ""  # text withheld because a stop may start in it
        self._finder = re.compile("|".join(map(re.escape, self.stops))) if self.stops else None
        self._prefixes = {stop[:n] for stop in self.stops for n in range(1, len(stop))}
        self._longest_prefix = max((len(stop) - 1 for stop in self.stops), default=0)

    def _withheld(self, text):
        """Length of the longest tail of ``text`` that begins some stop."""
        for n in range(min(self._longest_prefix, len(text)), 0, -1):
            if text[len(text) - n:] in self._prefixes:
                return n
        return 0

    def feed(self, text):
        """Take the next piece of generated text; return the part that is
        certain not to belong to a stop string."""
        if self.matched is not None:
            return ""
        if self._finder is None:
            return text
        window = self._tail + text
        hit = self._finder.search(window)
        if hit is not None:
            self.matched = hit.group(0)
            self._tail = ""
            return window[:hit.start()]
        cut = len(window) - self._withheld(window)
        self._tail = window[cut:]
        return window[:cut]

    def flush(self):
        """End of generation: the withheld text, unless a stop matched."""
        tail, self._tail = self._tail, ""
        return "" if self.matched is not None else tail


def log_softmax(logits):
    """float64 log probabilities of one logit vector; entries that are not
    finite get -inf."""
    x = np.asarray(logits, dtype=np.float64)
    finite = np.isfinite(x)
    if not np.any(finite):
        raise ValueError("logits contain no finite value")
    top = np.max(x, where=finite, initial=-np.inf)
    mass = np.sum(np.exp(x - top, where=finite, out=np.zeros_like(x)))
    return np.where(finite, (x - top) - np.log(mass), -np.inf)
