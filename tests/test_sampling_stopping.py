"""Host-side sampling and stop-sequence logic (runtime/sampling.py,
runtime/stopping.py): validation, the documented order and conventions, and
closed-form checks of each transform.  CPU only."""

import dataclasses
import math

import numpy as np
import pytest

from runtime.sampling import (GREEDY, SamplingError, SamplingParams, Sampler, apply_logit_bias,
                              apply_penalties, filter_top_k, filter_top_p)
from runtime.stopping import StopMatcher, log_softmax, normalize_logprobs, normalize_stop


# ---- SamplingParams ----

def test_defaults_are_greedy_and_deterministic():
    assert GREEDY.greedy and GREEDY.deterministic
    assert SamplingParams.build() == GREEDY
    assert SamplingParams.build(temperature=0.7, top_k=1).greedy  # top-1 without penalties is argmax
    assert not SamplingParams.build(temperature=0.7, top_k=1, repetition_penalty=1.2).greedy
    assert not SamplingParams.build(temperature=0.7).deterministic
    assert SamplingParams.build(temperature=0.7, seed=3).deterministic


@pytest.mark.parametrize("field,value", [
    ("temperature", -0.1), ("temperature", 2.5), ("temperature", float("nan")), ("temperature", True),
    ("top_p", 0.0), ("top_p", 1.5), ("top_k", -1), ("top_k", 2.0), ("top_k", True),
    ("repetition_penalty", 0.05), ("presence_penalty", 3.0), ("frequency_penalty", -2.5),
    ("seed", -1), ("seed", 2**63), ("seed", 1.0), ("logit_bias", [1, 2]), ("logit_bias", {"x": 1}),
    ("logit_bias", {-1: 1.0}), ("logit_bias", {"1": 101.0}), ("logit_bias", {True: 1.0}),
])
def test_out_of_range_values_are_rejected(field, value):
    with pytest.raises(SamplingError):
        SamplingParams.build(**{field: value})


def test_logit_bias_keys_normalise_and_zero_entries_drop():
    p = SamplingParams.build(logit_bias={"5": 2.0, 7: -1.5, "9": 0.0})
    assert dict(p.logit_bias) == {5: 2.0, 7: -1.5}
    # a later zero for the same id removes the earlier entry
    assert dict(SamplingParams.build(logit_bias={"5": 2.0, 5: 0.0}).logit_bias) == {}
    with pytest.raises(TypeError):
        p.logit_bias[3] = 1.0
    with pytest.raises(SamplingError):
        SamplingParams.build(logit_bias={str(i): 1.0 for i in range(1025)})


def test_bias_outside_vocab_keeps_greedy_for_that_vocab():
    p = SamplingParams.build(logit_bias={100: 5.0})
    assert not p.greedy
    assert p.greedy_for(50) and not p.greedy_for(101)


def test_transport_round_trip_and_unknown_keys():
    p = SamplingParams.build(temperature=0.5, top_p=0.9, top_k=7, seed=11, logit_bias={"3": 1.0})
    q = SamplingParams.from_dict(p.to_dict())
    assert q == p
    with pytest.raises(SamplingError, match="unsupported sampling parameters: bogus"):
        SamplingParams.from_dict({"temperature": 0.5, "bogus": 1})
    assert SamplingParams.from_request({"temperature": None, "top_p": 0.5}) == SamplingParams.build(top_p=0.5)
    with pytest.raises(SamplingError):
        dataclasses.replace(p, temperature=9.0)


# ---- transforms ----

def test_penalties_follow_the_ctrl_and_openai_conventions():
    logits = np.array([2.0, -2.0, 1.0, 0.5], dtype=np.float32)
    p = SamplingParams.build(repetition_penalty=2.0, presence_penalty=0.25, frequency_penalty=0.5)
    out = apply_penalties(logits.copy(), [0, 1, 1, 7, -3], p)  # 7 and -3 are outside the vocabulary
    # positive scores divided, negative multiplied, then count and presence terms
    want = np.array([2.0 / 2 - 0.5 * 1 - 0.25, -2.0 * 2 - 0.5 * 2 - 0.25, 1.0, 0.5], dtype=np.float32)
    np.testing.assert_allclose(out, want, rtol=0, atol=1e-6)
    assert np.array_equal(apply_penalties(logits.copy(), [], p), logits)


def test_logit_bias_adds_and_skips_out_of_range_ids():
    out = apply_logit_bias(np.zeros(4, dtype=np.float32), {1: 3.0, 9: 5.0})
    assert out.tolist() == [0.0, 3.0, 0.0, 0.0]


def test_top_k_keeps_ties_at_the_threshold():
    x = np.array([1.0, 3.0, 2.0, 2.0, 0.0], dtype=np.float32)
    out = filter_top_k(x.copy(), 2)
    assert np.isneginf(out[[0, 4]]).all() and (out[[1, 2, 3]] == x[[1, 2, 3]]).all()
    assert np.array_equal(filter_top_k(x.copy(), 0), x)


def test_top_p_keeps_the_token_that_crosses_the_threshold():
    probs = np.array([0.5, 0.3, 0.15, 0.05])
    x = np.log(probs).astype(np.float32)
    out = filter_top_p(x.copy(), 0.6)  # 0.5 alone is below 0.6; 0.5 + 0.3 crosses it
    assert np.isfinite(out[:2]).all() and np.isneginf(out[2:]).all()
    out = filter_top_p(x.copy(), 1e-9)  # the best token always stays
    assert np.isfinite(out[0]) and np.isneginf(out[1:]).all()


def test_top_p_takes_ties_in_the_order_of_numpys_argsort_reversed():
    # The reference orders by the ascending default argsort read backwards
    # (sampling.py:388), which is not the stable descending order: with three
    # ties of p = e / (3e + 1) = 0.297 each, top_p 0.5 keeps the first two
    # ties of that order, whichever ids they are, and the crossing token too.
    x = np.array([1.0, 1.0, 1.0, 0.0], dtype=np.float32)
    order = np.argsort(x)[::-1]
    out = filter_top_p(x.copy(), 0.5)
    assert sorted(np.flatnonzero(np.isfinite(out)).tolist()) == sorted(order[:2].tolist())
    two = 2 * math.e / (3 * math.e + 1)
    out = filter_top_p(x.copy(), two + 1e-3)  # just above two ties' mass: the third stays
    assert np.flatnonzero(np.isfinite(out)).tolist() == [0, 1, 2]


def test_top_p_on_tied_scores_follows_the_documented_rule():
    # heavily tied scores (rounded to 0.5; up to 200 of them, where numpy's
    # argsort does not keep ties in id order): along numpy's argsort read
    # backwards, a token stays exactly when the probability mass before it is
    # below top_p (the first always)
    rng = np.random.default_rng(3)
    for _ in range(300):
        n = int(rng.integers(2, 200))
        x = (np.round(rng.normal(size=n) * 2) / 2).astype(np.float32)
        top_p = float(rng.uniform(0.05, 0.95))
        out = filter_top_p(x.copy(), top_p)
        order = np.argsort(x)[::-1]
        e = np.exp(x.astype(np.float64) - x.max())
        p = e / e.sum()
        mass = 0.0
        for rank, i in enumerate(order):
            kept = bool(np.isfinite(out[i]))
            if rank == 0:
                assert kept
            elif abs(mass - top_p) > 1e-6:  # away from float32 rounding of the edge
                assert kept == (mass < top_p), (x.tolist(), top_p, i)
            mass += p[i]


def test_seeded_draws_on_tied_scores_repeat_across_samplers():
    # bf16-valued scores tie often; two samplers with one seed draw the same
    # tokens, and every draw lies inside the nucleus the filter keeps
    rng = np.random.default_rng(5)
    x = (np.round(rng.normal(size=12) * 4) / 4).astype(np.float32)
    p = SamplingParams.build(temperature=1.0, top_p=0.7, seed=99)
    a, b = Sampler(p, vocab_size=12), Sampler(p, vocab_size=12)
    keep = np.isfinite(filter_top_p(x.copy(), 0.7))
    for _ in range(200):
        t = a.select(x)
        assert t == b.select(x) and keep[t]


def test_sampler_draws_from_the_filtered_distribution_reproducibly():
    logits = np.log(np.array([0.6, 0.3, 0.1], dtype=np.float32))
    p = SamplingParams.build(temperature=1.0, top_k=2, seed=1234)
    draws = [Sampler(p, vocab_size=3).select(logits) for _ in range(3)]
    assert len(set(draws)) == 1  # a fresh sampler with the same seed repeats
    s = Sampler(p, vocab_size=3)
    seq = [s.select(logits) for _ in range(4000)]
    assert 2 not in seq  # top-k 2 removed it
    frac = seq.count(0) / len(seq)
    assert abs(frac - 0.6 / 0.9) < 0.03
    # the same stream as numpy's generator over the renormalised distribution
    rng = np.random.default_rng(1234)
    want = rng.choice(3, p=np.array([2 / 3, 1 / 3, 0.0]))
    assert Sampler(p, vocab_size=3).select(logits) == want


def test_unseeded_sampler_reports_the_seed_it_drew():
    s = Sampler(SamplingParams.build(temperature=0.8), vocab_size=10)
    assert isinstance(s.seed, int) and s.stats()["mode"] == "sampled" and s.stats()["seed"] == s.seed
    g = Sampler(GREEDY, vocab_size=10)
    assert g.seed is None and g.stats()["mode"] == "greedy"
    assert g.select(np.array([0.0, 2.0, 1.0])) == 1


def test_temperature_zero_with_bias_is_argmax_of_biased_scores():
    s = Sampler(SamplingParams.build(logit_bias={0: 10.0}), vocab_size=3)
    assert not s.greedy
    assert s.select(np.array([0.0, 5.0, 1.0], dtype=np.float32)) == 0


# ---- stopping ----

def test_normalize_stop_limits():
    assert normalize_stop(None) == ()
    assert normalize_stop("END") == ("END",)
    assert normalize_stop(["a", "b", "a"]) == ("a", "b")
    for bad in (["a"] * 5, [""], [3], "x" * 257, 7):
        with pytest.raises(ValueError):
            normalize_stop(bad if not isinstance(bad, str) else [bad])
    assert normalize_logprobs(None) is None and normalize_logprobs(20) == 20
    for bad in (21, -1, True, 1.0):
        with pytest.raises(ValueError):
            normalize_logprobs(bad)


def test_stop_matcher_holds_partial_matches_and_cuts_at_the_earliest_stop():
    m = StopMatcher(("END", "xy"))
    assert m.feed("hello E") == "hello "  # "E" could start END
    assert m.feed("N") == ""
    assert m.feed("Q more") == "ENQ more"  # ruled out, released
    assert m.feed(" fox") == " fo"  # "x" could start "xy"
    assert m.feed("yz") == ""  # "xy" matched: nothing from it onward
    assert m.matched == "xy" and m.feed("later") == "" and m.flush() == ""
    m = StopMatcher(("ab",))
    assert m.feed("ca") == "c" and m.flush() == "a" and m.matched is None
    assert StopMatcher().feed("abc") == "abc"
    # two stops in one piece: the earliest wins
    m = StopMatcher(("zz", "b"))
    assert m.feed("abzz") == "a" and m.matched == "b"


def test_log_softmax_closed_form():
    x = np.array([1.0, 2.0, -np.inf, 0.5])
    lp = log_softmax(x)
    z = math.exp(1.0) + math.exp(2.0) + math.exp(0.5)
    np.testing.assert_allclose(lp[[0, 1, 3]], [1.0 - math.log(z), 2.0 - math.log(z), 0.5 - math.log(z)], rtol=1e-12)
    assert np.isneginf(lp[2])
    with pytest.raises(ValueError):
        log_softmax([-np.inf, -np.inf])


def test_stop_matcher_properties_on_random_streams():
    """Over random texts split into random pieces: the emitted text never
    contains a stop; with a match, the matched stop starts exactly where the
    emitted text ends; without one, everything is emitted.  Same-start ties
    go to the earlier-listed stop."""
    rng = np.random.default_rng(77)
    alphabet = "abc"
    for _ in range(2000):
        stops = tuple(dict.fromkeys("".join(rng.choice(list(alphabet), rng.integers(1, 4)))
                                    for _ in range(rng.integers(1, 4))))
        text = "".join(rng.choice(list(alphabet), rng.integers(0, 14)))
        cuts = sorted(rng.choice(len(text) + 1, rng.integers(0, 4)).tolist()) if text else []
        pieces = [text[a:b] for a, b in zip([0] + cuts, cuts + [len(text)])]
        m = StopMatcher(stops)
        out = "".join(m.feed(p) for p in pieces) + m.flush()
        assert not any(s in out for s in stops), (stops, pieces, out)
        if m.matched is None:
            assert out == text and not any(s in text for s in stops)
        else:
            assert text.startswith(out + m.matched), (stops, pieces, out, m.matched)
    m = StopMatcher(("ab", "a"))
    assert m.feed("xab") == "x" and m.matched == "ab"
    m = StopMatcher(("a", "ab"))
    assert m.feed("xab") == "x" and m.matched == "a"
