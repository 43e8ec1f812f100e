"""Token selection on the host: penalties, logit bias, temperature, top-k,
top-p and a seeded multinomial draw.

Mirrors the reference's ``npu_llm/runtime/sampling.py`` interface
(``SamplingParams``, ``Sampler``, ``GREEDY``, ``SamplingError`` and the
``apply_*`` / ``filter_*`` helpers): the same parameter names, ranges,
validation errors and order of operations (sampling.py:1-19), so a request
behaves the same on either decoder and a seeded request draws the same
tokens for the same logits.  Pure NumPy; it never touches the GPU.

Order for a non-greedy step: penalties over the prompt + generated history,
then ``logit_bias``, then temperature, then top-k, then top-p, then one draw
from ``numpy.random.default_rng(seed).choice`` over the renormalised
distribution.  ``temperature == 0`` (the default) is greedy argmax.
"""

import dataclasses
import math
import secrets

import numpy as np

__all__ = [
    "SamplingError", "SamplingParams", "GREEDY", "Sampler", "apply_penalties", "apply_logit_bias",
    "filter_top_k", "filter_top_p", "TEMPERATURE_RANGE", "TOP_P_RANGE", "REPETITION_PENALTY_RANGE",
    "PENALTY_RANGE", "LOGIT_BIAS_RANGE", "SEED_RANGE", "MAX_LOGIT_BIAS_ENTRIES",
]

# Accepted ranges (sampling.py:26-38).
TEMPERATURE_RANGE = (0.0, 2.0)
TOP_P_RANGE = (0.0, 1.0)            # low end exclusive
REPETITION_PENALTY_RANGE = (0.1, 2.0)
PENALTY_RANGE = (-2.0, 2.0)
LOGIT_BIAS_RANGE = (-100.0, 100.0)
SEED_RANGE = (0, 2**63 - 1)
MAX_LOGIT_BIAS_ENTRIES = 1024


class SamplingError(ValueError):
    """An invalid sampling parameter."""


def _as_float(value, name):
    # bool is an int subclass; a JSON true must not read as 1.0
    if isinstance(value, bool) or not isinstance(value, (int, float)):
        raise SamplingError(f"{name} must be a number")
    try:
        value = float(value)
    except OverflowError:
        raise SamplingError(f"{name} must be finite") from None
    if not math.isfinite(value):
        raise SamplingError(f"{name} must be finite")
    return value


def _in_range(value, name, bounds, low_open=False):
    value = _as_float(value, name)
    low, high = bounds
    if value > high or value < low or (low_open and value == low):
        kind = "exclusive" if low_open else "inclusive"
        raise SamplingError(f"{name} must be between {low} ({kind}) and {high} (inclusive)")
    return value


class _ReadOnlyBias(dict):
    """A validated ``{token_id: bias}`` map that cannot be changed afterwards
    (still a dict, so ``asdict`` and ``json`` handle it)."""

    def _refuse(self, *args, **kwargs):
        raise TypeError("logit_bias is immutable")

    __setitem__ = __delitem__ = clear = pop = popitem = setdefault = update = __ior__ = _refuse

    def __copy__(self):
        return self

    def __deepcopy__(self, memo):
        return self


def _token_key(key):
    if isinstance(key, bool):
        raise SamplingError("logit_bias keys must be token ids")
    if isinstance(key, int):
        token = key
    elif isinstance(key, str):
        if not (key.isascii() and key.isdigit()):
            raise SamplingError(f"logit_bias key {key!r} is not a token id")
        token = int(key, 10)
    else:
        raise SamplingError("logit_bias keys must be token ids")
    if token < 0:
        raise SamplingError("logit_bias token ids cannot be negative")
    return token


def _validated_bias(value):
    """OpenAI ``logit_bias``: string or integer keys; zero entries are dropped
    (a later zero for the same id removes an earlier entry)."""
    if value is None:
        return _ReadOnlyBias()
    if not isinstance(value, dict):
        raise SamplingError("logit_bias must be an object")
    if len(value) > MAX_LOGIT_BIAS_ENTRIES:
        raise SamplingError(f"logit_bias accepts at most {MAX_LOGIT_BIAS_ENTRIES} entries")
    out = {}
    for key, raw in value.items():
        token = _token_key(key)
        bias = _in_range(raw, f"logit_bias[{token}]", LOGIT_BIAS_RANGE)
        if bias == 0.0:
            out.pop(token, None)
        else:
            out[token] = bias
    return _ReadOnlyBias(out)


@dataclasses.dataclass(frozen=True)
class SamplingParams:
    """One request's validated sampling settings (``None`` fields take the
    defaults)."""

    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    logit_bias: dict = dataclasses.field(default_factory=_ReadOnlyBias)
    seed: int = None

    def __post_init__(self):
        def put(name, value):
            object.__setattr__(self, name, value)

        put("temperature", 0.0 if self.temperature is None
            else _in_range(self.temperature, "temperature", TEMPERATURE_RANGE))
        put("top_p", 1.0 if self.top_p is None else _in_range(self.top_p, "top_p", TOP_P_RANGE, low_open=True))
        top_k = 0 if self.top_k is None else self.top_k
        if isinstance(top_k, bool) or not isinstance(top_k, int):
            raise SamplingError("top_k must be an integer")
        if top_k < 0:
            raise SamplingError("top_k cannot be negative")
        put("top_k", top_k)
        put("repetition_penalty", 1.0 if self.repetition_penalty is None
            else _in_range(self.repetition_penalty, "repetition_penalty", REPETITION_PENALTY_RANGE))
        put("presence_penalty", 0.0 if self.presence_penalty is None
            else _in_range(self.presence_penalty, "presence_penalty", PENALTY_RANGE))
        put("frequency_penalty", 0.0 if self.frequency_penalty is None
            else _in_range(self.frequency_penalty, "frequency_penalty", PENALTY_RANGE))
        if self.seed is not None:
            if isinstance(self.seed, bool) or not isinstance(self.seed, int):
                raise SamplingError("seed must be an integer")
            if not SEED_RANGE[0] <= self.seed <= SEED_RANGE[1]:
                raise SamplingError(f"seed must be between {SEED_RANGE[0]} and {SEED_RANGE[1]}")
        put("logit_bias", _validated_bias(self.logit_bias))

    def _order_preserving(self):
        # nothing ahead of top-k / top-p can reorder the logits
        no_penalty = (self.repetition_penalty == 1.0 and self.presence_penalty == 0.0
                      and self.frequency_penalty == 0.0)
        return no_penalty and (self.temperature == 0.0 or self.top_k == 1)

    @property
    def greedy(self):
        """The selection is the argmax whatever the logits."""
        return self._order_preserving() and not self.logit_bias

    def greedy_for(self, vocab_size):
        """``greedy``, ignoring bias entries for ids outside the vocabulary
        (they are never applied)."""
        return self._order_preserving() and not any(0 <= t < vocab_size for t in self.logit_bias)

    @property
    def deterministic(self):
        return self.greedy or self.temperature == 0.0 or self.seed is not None

    def to_dict(self):
        return dataclasses.asdict(self)

    @classmethod
    def build(cls, temperature=None, top_p=None, top_k=None, repetition_penalty=None,
              presence_penalty=None, frequency_penalty=None, logit_bias=None, seed=None):
        return cls(temperature=temperature, top_p=top_p, top_k=top_k,
                   repetition_penalty=repetition_penalty, presence_penalty=presence_penalty,
                   frequency_penalty=frequency_penalty, logit_bias=logit_bias, seed=seed)

    @classmethod
    def from_dict(cls, values):
        """Rebuild (and re-validate) from a transport dict."""
        if values is None:
            return cls()
        if not isinstance(values, dict):
            raise SamplingError("sampling parameters must be an object")
        unknown = sorted(set(values) - {f.name for f in dataclasses.fields(cls)})
        if unknown:
            raise SamplingError("unsupported sampling parameters: " + ", ".join(unknown))
        return cls.build(**values)

    @classmethod
    def from_request(cls, request):
        """From an OpenAI-style request body."""
        names = ("temperature", "top_p", "top_k", "repetition_penalty", "presence_penalty",
                 "frequency_penalty", "logit_bias", "seed")
        return cls.build(**{n: request.get(n) for n in names})


GREEDY = SamplingParams()


def apply_penalties(logits, history, params):
    """Repetition (CTRL: positive scores divided, negative multiplied),
    frequency (count-scaled) and presence penalties over the tokens seen so
    far; ids outside the vocabulary are ignored.  Returns ``logits``."""
    if len(history) == 0 or (params.repetition_penalty == 1.0 and params.presence_penalty == 0.0
                             and params.frequency_penalty == 0.0):
        return logits
    ids, counts = np.unique(np.asarray(history, dtype=np.int64), return_counts=True)
    keep = (ids >= 0) & (ids < logits.shape[0])
    ids, counts = ids[keep], counts[keep].astype(np.float32)
    if ids.size == 0:
        return logits
    seen = logits[ids]
    if params.repetition_penalty != 1.0:
        seen = np.where(seen > 0, seen / params.repetition_penalty, seen * params.repetition_penalty)
    seen = seen - params.frequency_penalty * counts
    seen = seen - params.presence_penalty
    logits[ids] = seen
    return logits


def apply_logit_bias(logits, logit_bias):
    """Add each bias to its token's logit; ids outside the vocabulary are
    skipped.  Returns ``logits``."""
    vocab = logits.shape[0]
    for token, bias in (logit_bias or {}).items():
        token = int(token)
        if 0 <= token < vocab:
            logits[token] += bias
    return logits


def filter_top_k(logits, top_k):
    """Set every score below the k-th highest to -inf (ties at the threshold
    stay).  ``top_k`` 0 or >= the vocabulary is a no-op."""
    if 0 < top_k < logits.shape[0]:
        kth = np.partition(logits, logits.shape[0] - top_k)[logits.shape[0] - top_k]
        logits[logits < kth] = -np.inf
    return logits


def filter_top_p(logits, top_p):
    """Keep the smallest set of highest-probability tokens whose mass reaches
    ``top_p`` (the token that crosses it included; the best token always
    stays)."""
    if top_p >= 1.0:
        return logits
    order = np.argsort(logits)[::-1]
    mass = _softmax(logits[order])
    before = np.cumsum(mass) - mass  # probability mass strictly ahead of each token
    drop = before >= top_p
    drop[0] = False
    logits[order[drop]] = -np.inf
    return logits


def _softmax(scores):
    """Softmax over the finite scores (-inf entries get zero); if everything
    underflows, all the mass goes to the best score."""
    finite = np.isfinite(scores)
    peak = scores[finite].max() if finite.any() else 0.0
    weights = np.zeros_like(scores)
    np.exp(scores - peak, where=finite, out=weights)
    total = weights.sum()
    if not (math.isfinite(float(total)) and total > 0):
        weights = np.zeros_like(scores)
        weights[int(np.argmax(scores))] = 1.0
        return weights
    return weights / total


class Sampler:
    """Selects the tokens of one completion; owns the request's random stream
    (an unseeded sampled request draws a seed and reports it)."""

    def __init__(self, params=GREEDY, vocab_size=None):
        self.params = params
        self.vocab_size = vocab_size
        self.seed = params.seed
        if self.seed is None and not self.greedy:
            self.seed = secrets.randbelow(SEED_RANGE[1] + 1)
        self._rng = None if self.greedy else np.random.default_rng(self.seed)

    @property
    def greedy(self):
        if self.vocab_size is None:
            return self.params.greedy
        return self.params.greedy_for(self.vocab_size)

    def select(self, logits, history=()):
        """The next token id for ``logits`` after ``history``."""
        scores = np.asarray(logits, dtype=np.float32)
        if self.greedy:
            return int(np.argmax(scores))
        p = self.params
        scores = apply_logit_bias(apply_penalties(scores.copy(), history, p), p.logit_bias)
        if p.temperature == 0.0:
            return int(np.argmax(scores))
        scores = filter_top_p(filter_top_k(scores / p.temperature, p.top_k), p.top_p)
        probs = _softmax(scores).astype(np.float64)
        probs /= probs.sum()  # choice() wants the float64 sum within its tolerance
        return int(self._rng.choice(probs.shape[0], p=probs))

    def stats(self):
        return {**self.params.to_dict(), "mode": "greedy" if self.greedy else "sampled", "seed": self.seed}
