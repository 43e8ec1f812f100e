"""Stop sequences and log-probability options for completions (host side).

Mirrors the reference's ``npu_llm/runtime/stopping.py`` interface:
``normalize_stop``, ``normalize_logprobs``, ``StopMatcher`` and
``log_softmax``, with the same limits (at most 4 stop strings of at most 256
characters, at most 20 top log probabilities) and error messages.
"""

import numpy as np

__all__ = ["MAX_STOP_SEQUENCES", "MAX_STOP_LENGTH", "MAX_TOP_LOGPROBS", "normalize_stop",
           "normalize_logprobs", "StopMatcher", "log_softmax"]

MAX_STOP_SEQUENCES = 4
MAX_STOP_LENGTH = 256
MAX_TOP_LOGPROBS = 20


def normalize_stop(value):
    """An OpenAI ``stop`` value (string, list or None) as a tuple of distinct
    non-empty strings, in order."""
    if value is None:
        return ()
    items = [value] if isinstance(value, str) else value
    if not isinstance(items, (list, tuple)):
        raise ValueError("stop must be a string or an array of strings")
    if len(items) > MAX_STOP_SEQUENCES:
        raise ValueError(f"stop accepts at most {MAX_STOP_SEQUENCES} sequences")
    out = []
    for item in items:
        if not isinstance(item, str) or item == "":
            raise ValueError("each stop sequence must be a non-empty string")
        if len(item) > MAX_STOP_LENGTH:
            raise ValueError(f"stop sequences cannot exceed {MAX_STOP_LENGTH} characters")
        if item not in out:
            out.append(item)
    return tuple(out)


def normalize_logprobs(value):
    """``None`` (log probabilities off) or a top-alternatives count 0..20."""
    if value is None:
        return None
    if isinstance(value, bool) or not isinstance(value, int):
        raise ValueError("top_logprobs must be an integer")
    if value < 0 or value > MAX_TOP_LOGPROBS:
        raise ValueError(f"top_logprobs must be between 0 and {MAX_TOP_LOGPROBS}")
    return value


class StopMatcher:
    """Cut streamed text at the first stop sequence without ever emitting part
    of one: text that may still begin a stop sequence is held until the next
    piece decides it.  On a match, the sequence and everything after it are
    dropped and ``matched`` names the sequence."""

    def __init__(self, stops=()):
        self.stops = tuple(stops)
        self.matched = None
        self._held = ""

    def _longest_partial(self, text):
        # the longest suffix of text that is a proper prefix of some stop
        best = 0
        for stop in self.stops:
            for n in range(min(len(stop) - 1, len(text)), best, -1):
                if text.endswith(stop[:n]):
                    best = n
                    break
        return best

    def feed(self, text):
        """Take the next piece of text; return what can be emitted now."""
        if self.matched is not None:
            return ""
        if not self.stops:
            return text
        buf = self._held + text
        hit = None
        for stop in self.stops:
            at = buf.find(stop)
            if at >= 0 and (hit is None or at < hit[0]):
                hit = (at, stop)
        if hit is not None:
            self.matched = hit[1]
            self._held = ""
            return buf[:hit[0]]
        keep = self._longest_partial(buf)
        self._held = buf[len(buf) - keep:] if keep else ""
        return buf[:len(buf) - keep]

    def flush(self):
        """Release held text at the end of a generation that did not match."""
        held, self._held = self._held, ""
        return held if self.matched is None else ""


def log_softmax(logits):
    """float64 log probabilities of one logit vector (-inf entries stay -inf)."""
    x = np.asarray(logits, dtype=np.float64)
    finite = np.isfinite(x)
    if not finite.any():
        raise ValueError("logits contain no finite value")
    shifted = np.where(finite, x - x[finite].max(), -np.inf)
    return shifted - np.log(np.exp(shifted).sum())
