"""Token selection on the host: request parameters and the sampling pipeline.

Contract of ``npu_llm/runtime/sampling.py`` (callers: ``generate.py:1050-1200``,
``api_server.py`` request parsing): ``SamplingParams`` (fields, defaults,
``build`` / ``from_dict`` / ``from_request`` / ``to_dict``, ``greedy``,
``greedy_for``, ``deterministic``), ``SamplingError`` with the same messages,
``GREEDY``, the transforms ``apply_penalties``, ``apply_logit_bias``,
``filter_top_k``, ``filter_top_p`` and ``Sampler`` (``select``, ``stats``,
``seed``).  The selection order is the llama.cpp / vLLM one: penalties, logit
bias, temperature, top-k, top-p, then a draw from the renormalised
distribution with ``numpy.random.default_rng(seed).choice`` (so a seeded
request repeats its tokens).  Temperature 0 (the default) is the argmax.

Design: every scalar parameter is described once in ``_FIELDS`` (default and
validator) and ``SamplingParams`` normalises itself by walking that table; a
``Sampler`` turns its parameters into the list of stages that actually change
the scores, once, and ``select`` runs that list.
"""

import math
import secrets
from dataclasses import asdict, dataclass, field

import numpy as np

__all__ = ["TEMPERATURE_RANGE", "TOP_P_RANGE", "REPETITION_PENALTY_RANGE", "PENALTY_RANGE",
           "LOGIT_BIAS_RANGE", "SEED_RANGE", "MAX_LOGIT_BIAS_ENTRIES", "SamplingError",
           "SamplingParams", "GREEDY", "apply_penalties", "apply_logit_bias", "filter_top_k",
           "filter_top_p", "Sampler"]

TEMPERATURE_RANGE = (0.0, 2.0)
TOP_P_RANGE = (0.0, 1.0)            # the low end is excluded
REPETITION_PENALTY_RANGE = (0.1, 2.0)
PENALTY_RANGE = (-2.0, 2.0)
LOGIT_BIAS_RANGE = (-100.0, 100.0)
SEED_RANGE = (0, 2**63 - 1)
MAX_LOGIT_BIAS_ENTRIES = 1024       # bounds the per-step bias work


class SamplingError(ValueError):
    """A sampling parameter outside its documented domain."""


# ---- validators: (name, raw value) -> normalised value ----

def _real(bounds, open_low=False):
    low, high = bounds
    edge = "exclusive" if open_low else "inclusive"

    def check(name, value):
        if type(value) is bool or not isinstance(value, (int, float)):
            raise SamplingError(f"{name} must be a number")
        try:
            x = float(value)
        except OverflowError:
            raise SamplingError(f"{name} must be finite") from None
        if not math.isfinite(x):
            raise SamplingError(f"{name} must be finite")
        above_low = x > low if open_low else x >= low
        if not above_low or x > high:
            raise SamplingError(f"{name} must be between {low} ({edge}) and {high} (inclusive)")
        return x

    return check


def _count(name, value):
    if type(value) is bool or not isinstance(value, int):
        raise SamplingError(f"{name} must be an integer")
    if value < 0:
        raise SamplingError(f"{name} cannot be negative")
    return value


def _seed(name, value):
    if type(value) is bool or not isinstance(value, int):
        raise SamplingError(f"{name} must be an integer")
    if value not in range(SEED_RANGE[0], SEED_RANGE[1] + 1):
        raise SamplingError(f"{name} must be between {SEED_RANGE[0]} and {SEED_RANGE[1]}")
    return value


# scalar fields in validation order: default (also what None means) and validator
_FIELDS = (
    ("temperature", 0.0, _real(TEMPERATURE_RANGE)),
    ("top_p", 1.0, _real(TOP_P_RANGE, open_low=True)),
    ("top_k", 0, _count),
    ("repetition_penalty", 1.0, _real(REPETITION_PENALTY_RANGE)),
    ("presence_penalty", 0.0, _real(PENALTY_RANGE)),
    ("frequency_penalty", 0.0, _real(PENALTY_RANGE)),
    ("seed", None, _seed),
)
_bias_value = _real(LOGIT_BIAS_RANGE)


class _BiasMap(dict):
    """A validated ``{token_id: bias}`` map that cannot be changed afterwards
    (a plain ``dict`` underneath, so ``asdict`` and ``json`` handle it)."""

    def __copy__(self):
        return self

    def __deepcopy__(self, memo):
        return self


def _immutable(*args, **kwargs):
    raise TypeError("logit_bias is immutable")


for _mutator in ("__setitem__", "__delitem__", "__ior__", "clear", "pop", "popitem", "setdefault", "update"):
    setattr(_BiasMap, _mutator, _immutable)


def _bias_token(key):
    """Token id of a ``logit_bias`` key: an int, or a decimal string as JSON
    object keys always are."""
    if isinstance(key, str):
        if not (key.isascii() and key.isdigit()):
            raise SamplingError(f"logit_bias key {key!r} is not a token id")
        key = int(key, 10)
    elif type(key) is bool or not isinstance(key, int):
        raise SamplingError("logit_bias keys must be token ids")
    if key < 0:
        raise SamplingError("logit_bias token ids cannot be negative")
    return key


def _bias_map(value):
    """Normalised ``logit_bias``: int keys, zero biases left out (a later zero
    for a token removes an earlier entry for it)."""
    if value is None:
        return _BiasMap()
    if not isinstance(value, dict):
        raise SamplingError("logit_bias must be an object")
    if len(value) > MAX_LOGIT_BIAS_ENTRIES:
        raise SamplingError(f"logit_bias accepts at most {MAX_LOGIT_BIAS_ENTRIES} entries")
    entries = {}
    for key, raw in value.items():
        token = _bias_token(key)
        bias = _bias_value(f"logit_bias[{token}]", raw)
        entries.pop(token, None)
        if bias != 0.0:
            entries[token] = bias
    return _BiasMap(entries)


@dataclass(frozen=True)
class SamplingParams:
    """One request's sampling parameters, validated on construction (also by
    ``dataclasses.replace``)."""

    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    logit_bias: dict = field(default_factory=_BiasMap)
    seed: int = None

    def __post_init__(self):
        for name, default, check in _FIELDS:
            raw = getattr(self, name)
            object.__setattr__(self, name, default if raw is None else check(name, raw))
        object.__setattr__(self, "logit_bias", _bias_map(self.logit_bias))

    @property
    def _keeps_order(self):
        """No penalty can move a score, and either no draw happens or top-1
        leaves one candidate."""
        penalties = (self.repetition_penalty, self.presence_penalty, self.frequency_penalty) != (1.0, 0.0, 0.0)
        return not penalties and (self.temperature == 0.0 or self.top_k == 1)

    @property
    def greedy(self):
        """Selection is the argmax whatever the logits."""
        return self._keeps_order and not self.logit_bias

    def greedy_for(self, vocab_size):
        """``greedy`` for a vocabulary of ``vocab_size``: bias entries outside
        it are ignored by ``apply_logit_bias`` and so cannot matter."""
        return self._keeps_order and all(not 0 <= token < vocab_size for token in self.logit_bias)

    @property
    def deterministic(self):
        """Repeating the request repeats its tokens."""
        return self.greedy or self.temperature == 0.0 or self.seed is not None

    def to_dict(self):
        return asdict(self)

    @classmethod
    def build(cls, temperature=None, top_p=None, top_k=None, repetition_penalty=None,
              presence_penalty=None, frequency_penalty=None, logit_bias=None, seed=None):
        """From raw request values; None means the default."""
        return cls(temperature, top_p, top_k, repetition_penalty, presence_penalty, frequency_penalty,
                   logit_bias, seed)

    @classmethod
    def from_dict(cls, values):
        """From a transport dict (re-validated: it crossed a process boundary)."""
        if values is None:
            return cls()
        if not isinstance(values, dict):
            raise SamplingError("sampling parameters must be an object")
        extra = sorted(set(values).difference(cls.__dataclass_fields__))
        if extra:
            raise SamplingError("unsupported sampling parameters: " + ", ".join(extra))
        return cls.build(**values)

    @classmethod
    def from_request(cls, request):
        """From an OpenAI chat-completion request body."""
        return cls.build(**{name: request.get(name) for name in cls.__dataclass_fields__})


GREEDY = SamplingParams()


# ---- transforms (each changes `logits` in place and returns it) ----

def apply_penalties(logits, history, params):
    """CTRL repetition penalty (positive scores divided by it, negative ones
    multiplied), then the OpenAI frequency (per occurrence) and presence
    (once) penalties, on tokens of ``history`` inside the vocabulary."""
    rp, fp, pp = params.repetition_penalty, params.frequency_penalty, params.presence_penalty
    if len(history) == 0 or (rp, fp, pp) == (1.0, 0.0, 0.0):
        return logits
    ids = np.asarray(history, dtype=np.int64)
    ids = ids[(ids >= 0) & (ids < logits.shape[0])]  # out-of-range ids must not wrap
    if ids.size == 0:
        return logits
    occurrences = np.bincount(ids, minlength=logits.shape[0])
    seen = np.flatnonzero(occurrences)
    score = logits[seen]
    if rp != 1.0:
        score = np.where(score > 0, score / rp, score * rp)
    score = score - fp * occurrences[seen].astype(np.float32)
    logits[seen] = score - pp
    return logits


def apply_logit_bias(logits, logit_bias):
    """Add each bias to its token's score (OpenAI semantics: -100 bans, +100
    forces); ids outside the vocabulary are skipped."""
    if logit_bias:
        ids = np.fromiter(logit_bias.keys(), dtype=np.int64, count=len(logit_bias))
        bias = np.fromiter(logit_bias.values(), dtype=np.float64, count=len(logit_bias))
        inside = (ids >= 0) & (ids < logits.shape[0])
        logits[ids[inside]] += bias[inside].astype(logits.dtype)
    return logits


def filter_top_k(logits, top_k):
    """Only scores at or above the k-th largest survive (ties at the
    threshold all survive); others become -inf."""
    n = logits.shape[0]
    if 0 < top_k < n:
        kth_largest = np.partition(logits, n - top_k)[n - top_k]
        logits[logits < kth_largest] = -np.inf
    return logits


def filter_top_p(logits, top_p):
    """Nucleus: in descending order of probability a token survives while the
    mass of the tokens before it is below ``top_p``, so the token that crosses
    the threshold stays, and so does the best one always.

    The order and the test are the contract of ``sampling.py:380-394``, so a
    seeded request keeps the reference's tokens also when equal scores sit at
    the nucleus edge: numpy's default (ascending, unstable) argsort read
    backwards -- equal scores come in whatever order that call gives them,
    not by id -- and the mass before token i taken as ``cumsum[i] - p[i]``
    (not ``cumsum[i-1]``, which can round the other way)."""
    if top_p < 1.0:
        order = np.argsort(logits)[::-1]
        p = _softmax(logits[order])
        inside = np.cumsum(p) - p < top_p
        inside[0] = True
        logits[order[~inside]] = -np.inf
    return logits


def _softmax(scores):
    """Probabilities of the finite scores (zero elsewhere); one-hot on the
    best score when everything underflows."""
    finite = np.isfinite(scores)
    top = scores[finite].max() if finite.any() else 0.0
    e = np.exp(scores - top, where=finite, out=np.zeros_like(scores))
    total = e.sum()
    if total > 0 and np.isfinite(total):
        return e / total
    onehot = np.zeros_like(scores)
    onehot[int(np.argmax(scores))] = 1.0
    return onehot


class Sampler:
    """Token selection for one completion; owns its random stream.  An
    unseeded, non-greedy request draws a seed and reports it in ``stats``."""

    def __init__(self, params=GREEDY, vocab_size=None):
        self.params = params
        self.vocab_size = vocab_size
        self.seed = params.seed
        if self.greedy:
            self._rng = None
            self._stages = ()
            return
        if self.seed is None:
            self.seed = secrets.randbelow(SEED_RANGE[1] + 1)
        self._rng = np.random.default_rng(self.seed)
        stages = []
        if (params.repetition_penalty, params.presence_penalty, params.frequency_penalty) != (1.0, 0.0, 0.0):
            stages.append(lambda s, history: apply_penalties(s, history, params))
        if params.logit_bias:
            stages.append(lambda s, history: apply_logit_bias(s, params.logit_bias))
        self._stages = tuple(stages)

    @property
    def greedy(self):
        return self.params.greedy if self.vocab_size is None else self.params.greedy_for(self.vocab_size)

    def select(self, logits, history=()):
        """The next token id for ``logits`` after the tokens in ``history``."""
        scores = np.asarray(logits, dtype=np.float32)
        if self._rng is None:
            return int(np.argmax(scores))
        scores = scores.copy()
        for stage in self._stages:
            scores = stage(scores, history)
        p = self.params
        if p.temperature == 0.0:
            return int(np.argmax(scores))
        scores = filter_top_p(filter_top_k(scores / p.temperature, p.top_k), p.top_p)
        probs = _softmax(scores).astype(np.float64)
        probs /= probs.sum()  # Generator.choice wants a sum of 1 within its tolerance
        return int(self._rng.choice(probs.shape[0], p=probs))

    def stats(self):
        """Parameters, mode and seed, for the generation statistics."""
        return {**self.params.to_dict(), "mode": "greedy" if self.greedy else "sampled", "seed": self.seed}
