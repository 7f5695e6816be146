"""Pins the CPU oracle: the reference's own known-answer tests and exact laws.

Each test re-expresses one of the reference's checks against
oracle/sampling_oracle.py (citations give the reference test it mirrors), or
checks a closed form / exact-rational brute force that a plausible mistake
(a dropped term, wrong sign, inclusive instead of exclusive prefix, unstable
tie order, wrong searchsorted side) would fail.  Planted mistakes at the end
show that these checks catch such errors.
"""
from fractions import Fraction
from itertools import product
import math

import numpy as np
import pytest

from oracle import sampling_oracle as O


def P(**kw):
    return O.Policy(**kw)


class Draws:
    """Interval-midpoint uniforms (tests/test_sampling.py:13-19)."""

    def __init__(self, accept, target=0.5):
        self.accept, self.target = iter(accept), target
        self.calls = []

    def __call__(self, domain):
        self.calls.append(domain)
        return next(self.accept) if domain == "accept" else self.target


def test_temperature_filters_known_answers():
    # tests/test_sampling.py:22-32
    logits = np.log(np.array([.5, .3, .2], np.float64))
    np.testing.assert_allclose(O.probabilities(logits, P()), [.5, .3, .2], rtol=1e-15)
    np.testing.assert_array_equal(O.probabilities(logits, P(temperature=0)), [1, 0, 0])
    np.testing.assert_array_equal(O.probabilities(logits, P(temperature=1e-320)), [1, 0, 0])
    np.testing.assert_allclose(O.probabilities(logits, P(top_k=2)), [.625, .375, 0], rtol=1e-15)
    np.testing.assert_allclose(O.probabilities(logits, P(top_p=.7)), [.625, .375, 0], rtol=1e-15)
    np.testing.assert_array_equal(O.probabilities(logits, P(top_p=0)), [1, 0, 0])
    np.testing.assert_array_equal(O.probabilities(logits, P(min_p=.7)), [1, 0, 0])
    np.testing.assert_array_equal(O.probabilities(logits, P(min_p=.5, top_p=.6)), [1, 0, 0])


def test_penalties_bias_mask_closed_form():
    # tests/test_sampling.py:35-44
    logits = np.array([2., -1., 3., 0.], np.float32)
    counts = np.array([2, 1, 0, 0], np.int32)
    pol = P(repetition_penalty=2, presence_penalty=.25, frequency_penalty=.5)
    got = O.probabilities(logits, pol, counts, logit_bias={3: .2}, allowed=np.array([True, True, False, True]))
    adj = np.array([1 - .25 - 1, -2 - .25 - .5, -np.inf, .2])
    want = np.exp(adj - adj.max())
    np.testing.assert_allclose(got, want / want.sum(), rtol=1e-15)
    with pytest.raises(O.OracleError, match="every"):
        O.probabilities(logits, pol, allowed=np.zeros(4, bool))


def test_categorical_cdf_boundaries():
    # tests/test_sampling.py:49-53
    p = np.array([0., .25, 0., .75, 0.], np.float64)
    assert O.categorical(p, 0.)[0] == 1
    assert O.categorical(p, .25)[0] == 3
    assert O.categorical(p, np.nextafter(1., 0.).item())[0] == 3


def test_categorical_single_support_draws_nothing():
    # sampling.py:120-122
    def never():
        raise AssertionError("uniform requested for a one-point support")
    assert O.categorical(np.array([0., 1., 0.]), never) == (1, False, math.inf)


def test_exact_rejection_marginal():
    # tests/test_sampling.py:56-69
    target, proposal = np.array([.3, .7]), np.array([.8, .2])
    np.testing.assert_array_equal(O.correction(target, proposal), [0, 1])
    mass = [Fraction(0), Fraction(0)]
    q = (Fraction(4, 5), Fraction(1, 5))
    for token in (0, 1):
        for u in (np.arange(8) + .5) / 8:
            _, out, _, _ = O.verify_probs((target, target), (proposal,), (token,), Draws([float(u)]),
                                          greedy=False, output_limit=2)
            mass[out[0]] += q[token] / 8
    assert mass == [Fraction(3, 10), Fraction(7, 10)]


@pytest.mark.parametrize("rejected", range(6))
def test_every_rejection_length(rejected):
    # tests/test_sampling.py:72-84
    proposal = np.array([.5, .5])
    targets = [np.array([.75, .25]) for _ in range(6)]
    if rejected < 5:
        targets[rejected] = np.array([.25, .75])
    acc, out, pending, stop = O.verify_probs(targets, [proposal] * 5, [0] * 5, Draws([.75] * 5),
                                             greedy=False, output_limit=10)
    assert acc == rejected and len(out) == rejected + 1 and pending == out[-1] and stop is None


def test_eos_or_limit_inside_drafts_has_no_bonus():
    # tests/test_sampling.py:87-95
    target, proposal = np.array([.9, .1]), np.array([.5, .5])
    d = Draws([.1])
    assert O.verify_probs([target] * 6, [proposal] * 5, [0] * 5, d, greedy=False, output_limit=10,
                          eos_ids={0}) == (1, (0,), None, "eos")
    assert d.calls == ["accept"]
    assert O.verify_probs([target] * 6, [proposal] * 5, [0] * 5, Draws([.1, .1]), greedy=False,
                          output_limit=2) == (2, (0, 0), None, "length")


def test_greedy_draws_nothing():
    # tests/test_sampling.py:98-107
    d = Draws([])
    out = O.verify_probs([np.array([.2, .8])] * 6, [np.array([.5, .5])] * 5, [0] * 5, d, greedy=True,
                         output_limit=5)
    assert out[1] == (1,) and d.calls == []


def test_two_token_joint_law_exact():
    # tests/test_sampling_reference_law.py:15-42
    q0 = (Fraction(1, 2), Fraction(1, 4), Fraction(1, 4))
    p0 = (Fraction(1, 4), Fraction(3, 8), Fraction(3, 8))
    q1 = [tuple(q0[(t - prev - 1) % 3] for t in range(3)) for prev in range(3)]
    p1 = [tuple(p0[(t - prev - 2) % 3] for t in range(3)) for prev in range(3)]
    seen = [[Fraction(0)] * 3 for _ in range(3)]
    arr = lambda rows: [np.array([float(x) for x in r]) for r in rows]
    for first, second, a, b, c, d in product(range(3), range(3), range(4), range(4), range(8), range(8)):
        _, out, _, _ = O.verify_probs(arr((p0, p1[first], p0)), arr((q0, q1[first])), (first, second),
                                      Draws(((a + .5) / 4, (b + .5) / 4), (c + .5) / 8), greedy=False,
                                      output_limit=2)
        if len(out) == 1:
            out += (O.categorical(np.array([float(x) for x in p1[out[0]]]), (d + .5) / 8)[0],)
        seen[out[0]][out[1]] += q0[first] * q1[first][second] / (16 * 64)
    assert seen == [[p0[f] * p1[f][s] for s in range(3)] for f in range(3)]


def test_equal_coordinates_get_no_correction_mass():
    # tests/test_sampling_reference_law.py:45-50
    np.testing.assert_array_equal(O.correction(np.array([.125, .625, .25]), np.array([.5, .25, .25])), [0., 1., 0.])


def test_cluster_probe_verifier_checks():
    # src/deepseekrpc/cluster_probe.py:22-56 (13 checks)
    point = np.eye(3)
    for rejected in range(6):
        targets = [point[0] if r < rejected else point[1] for r in range(5)] + [point[2]]
        acc, out, _, _ = O.verify_probs(targets, [point[0]] * 5, [0] * 5, Draws([]), greedy=True, output_limit=64)
        assert acc == rejected and out == (0,) * rejected + ((1,) if rejected < 5 else (2,))
    for limit in range(1, 6):
        acc, out, pending, stop = O.verify_probs([point[0]] * 6, [point[0]] * 5, [0] * 5, Draws([.5] * 5),
                                                 greedy=False, output_limit=limit)
        assert out == (0,) * limit and stop == "length" and pending is None
    acc, out, pending, stop = O.verify_probs([point[0]] * 6, [point[0]] * 5, [0] * 5, Draws([.5] * 5),
                                             greedy=False, output_limit=64, eos_ids={0})
    assert (out, acc, stop, pending) == ((0,), 1, "eos", None)
    p, q = np.array([.1, .6, .3]), np.array([.5, .2, .3])
    m = np.minimum(p, q)
    np.testing.assert_allclose(m + (1 - m.sum()) * O.correction(p, q), p, rtol=0, atol=2e-16)


def test_presence_frequency_use_generated_counts_only():
    # tests/test_sampling.py:236-243
    counts, gen = np.array([5, 1, 0], np.int32), np.array([0, 1, 0], np.int32)
    got = O.probabilities(np.array([2., 2., 0.], np.float32),
                          P(repetition_penalty=2, presence_penalty=.5, frequency_penalty=.25), counts, gen)
    want = np.exp(np.array([1., .25, 0.]) - 1)
    np.testing.assert_allclose(got, want / want.sum(), rtol=1e-15, atol=0)


def test_negative_logits_are_multiplied_by_repetition():
    # Keskar et al. (2019) CTRL penalty: positive / rep, negative * rep.
    got = O.adjusted_logits(np.array([-2., 3., -1.]), P(repetition_penalty=4), np.array([1, 1, 0]))
    np.testing.assert_array_equal(got, [-8., .75, -1.])


def test_softmax_temperature_closed_form_and_invariants():
    rng = np.random.default_rng(7)
    x = rng.normal(0, 3, 257)
    for T in (0.3, 1.0, 2.7):
        p = O.probabilities(x, P(temperature=T))
        w = [math.exp((v - x.max()) / T) for v in x]
        s = math.fsum(w)
        np.testing.assert_allclose(p, [v / s for v in w], rtol=1e-13)
        assert abs(p.sum() - 1) < 1e-12


def _rank(values):
    """(value desc, index asc) order by brute force."""
    return sorted(range(len(values)), key=lambda i: (-values[i], i))


@pytest.mark.parametrize("seed", range(6))
def test_topk_keeps_k_largest_with_lower_index_ties(seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(-3, 4, 40).astype(np.float64)   # many exact ties
    k = int(rng.integers(1, 40))
    d = O.Diagnostics()
    O.probabilities(x, P(top_k=k), diagnostics=d)
    want = np.zeros(40, bool)
    want[_rank(list(x))[:k]] = True
    np.testing.assert_array_equal(d.topk_kept, want)


@pytest.mark.parametrize("seed", range(6))
def test_topp_prefix_rule_brute_force(seed):
    # Nucleus rule with the exclusive prefix: element kept iff the exact mass
    # ranked strictly before it is below top_p (rank 0 always), checked with
    # rational arithmetic where no float decision is within 1e-9 of top_p.
    rng = np.random.default_rng(100 + seed)
    x = rng.integers(-4, 3, 30).astype(np.float64)
    top_p = float(rng.uniform(0.05, 0.95))
    base = O.probabilities(x, P())
    order = _rank(list(base))
    before, keep = Fraction(0), np.zeros(30, bool)
    for pos, i in enumerate(order):
        if pos == 0 or before < Fraction(top_p):
            keep[i] = True
        before += Fraction(float(base[i]))
    got = O.probabilities(x, P(top_p=top_p)) > 0
    np.testing.assert_array_equal(got, keep)


def test_minp_threshold_invariant():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, 500)
    base = O.probabilities(x, P())
    got = O.probabilities(x, P(min_p=0.05))
    kept = got > 0
    np.testing.assert_array_equal(kept, base >= 0.05 * base.max())
    np.testing.assert_allclose(got[kept], base[kept] / base[kept].sum(), rtol=1e-14)


def test_categorical_matches_exact_cdf_cells():
    rng = np.random.default_rng(11)
    p = rng.random(50)
    p[rng.random(50) < 0.3] = 0
    p /= p.sum()
    edges = np.cumsum([Fraction(float(v)) for v in p])
    total = edges[-1]
    for u in rng.random(400):
        tok, used, margin = O.categorical(p, float(u))
        if margin < 1e-12:
            continue
        want = next(i for i, e in enumerate(edges) if e / total > Fraction(float(u)))
        assert tok == want and used and p[tok] > 0


def test_error_codes():
    with pytest.raises(O.OracleError) as e:
        O.probabilities(np.array([0., np.nan]), P())
    assert e.value.code == O.E_LOGITS
    with pytest.raises(O.OracleError) as e:
        O.probabilities(np.array([0., 1.]), P(), np.array([1, -1], np.int32))
    assert e.value.code == O.E_COUNTS
    with pytest.raises(O.OracleError) as e:
        O.probabilities(np.array([0., 1.]), P(), np.array([1, 0], np.int32), np.array([2, 0], np.int32))
    assert e.value.code == O.E_GENERATED
    with pytest.raises(O.OracleError) as e:
        O.categorical(np.array([.5, .5]), 1.0)
    assert e.value.code == O.E_UNIFORM
    with pytest.raises(O.OracleError) as e:
        O.correction(np.array([.5, .5]), np.array([.5, .5]))
    assert e.value.code == O.E_CORRECTION


# ---------------------------------------------------------------------------
# Planted mistakes: each mutant of the oracle's source must fail at least one
# of the pinning checks above.

import inspect
import sys
import types

MUTANTS = {
    "inclusive top-p prefix": ("prev = np.cumsum(ordered, dtype=np.float64) - ordered",
                               "prev = np.cumsum(ordered, dtype=np.float64)"),
    "higher index wins top-k ties": ('rank = np.argsort(-v, kind="stable")',
                                     'rank = np.lexsort((-np.arange(len(v)), -v))'),
    "searchsorted left": ('np.searchsorted(c, u, side="right")', 'np.searchsorted(c, u, side="left")'),
    "repetition sign swapped": ("sub / policy.repetition_penalty, sub * policy.repetition_penalty",
                                "sub * policy.repetition_penalty, sub / policy.repetition_penalty"),
    "presence on all counts": ("penalty = policy.presence_penalty * (gen > 0)",
                               "penalty = policy.presence_penalty * (counts > 0)"),
    "temperature multiplies": ("v /= policy.temperature", "v *= policy.temperature"),
    "min-p on unnormalised": ("cut = policy.min_p * np.max(r)", "cut = policy.min_p"),
    "rank 0 removable": ("drop[0] = False", "pass"),
}


def _mutant(src_old, src_new):
    src = inspect.getsource(O)
    assert src.count(src_old) == 1, src_old
    mod = types.ModuleType("oracle_mutant")
    sys.modules["oracle_mutant"] = mod  # dataclasses resolve annotations through sys.modules
    try:
        exec(compile(src.replace(src_old, src_new), "oracle_mutant", "exec"), mod.__dict__)
    finally:
        sys.modules.pop("oracle_mutant", None)
    return mod


def _pinning_checks(mod):
    logits = np.log(np.array([.5, .3, .2]))
    pol = mod.Policy
    np.testing.assert_allclose(mod.probabilities(logits, pol(top_p=.7)), [.625, .375, 0], rtol=1e-15)
    np.testing.assert_array_equal(mod.probabilities(logits, pol(top_p=0)), [1, 0, 0])
    np.testing.assert_array_equal(mod.probabilities(logits, pol(min_p=.7)), [1, 0, 0])
    np.testing.assert_allclose(mod.probabilities(logits, pol(temperature=0.5)),
                               np.array([.25, .09, .04]) / .38, rtol=1e-14)
    p = np.array([0., .25, 0., .75, 0.])
    assert mod.categorical(p, .25)[0] == 3
    counts, gen = np.array([5, 1, 0], np.int32), np.array([0, 1, 0], np.int32)
    got = mod.probabilities(np.array([2., 2., 0.], np.float32),
                            pol(repetition_penalty=2, presence_penalty=.5, frequency_penalty=.25), counts, gen)
    want = np.exp(np.array([1., .25, 0.]) - 1)
    np.testing.assert_allclose(got, want / want.sum(), rtol=1e-15)
    np.testing.assert_array_equal(mod.adjusted_logits(np.array([-2., 3.]), pol(repetition_penalty=4),
                                                      np.array([1, 1])), [-8., .75])
    x = np.array([1., 3., 3., 0., 3.])
    d = mod.Diagnostics()
    mod.probabilities(x, pol(top_k=2), diagnostics=d)
    np.testing.assert_array_equal(d.topk_kept, [False, True, True, False, False])


def test_unmutated_oracle_passes_pinning_checks():
    _pinning_checks(O)


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistake_is_caught(name):
    mod = _mutant(*MUTANTS[name])
    with pytest.raises(Exception):  # a failed assertion, or the mutant's own error
        _pinning_checks(mod)
