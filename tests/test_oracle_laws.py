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


import sampling_law as law


def P(**kw):
    return O.Policy(**kw)


class OracleImpl:
    """The ``sampling_law`` adapter over the oracle."""
    Rejected = O.OracleError

    def probs(self, logits, counts=None, generated=None, bias=None, allowed=None, **policy):
        return O.probabilities(np.asarray(logits), O.Policy(**policy), counts, generated, logit_bias=bias,
                               allowed=allowed)

    def draw(self, p, u):
        return O.categorical(np.asarray(p), u)[0]

    def residual(self, p, q):
        return O.correction(np.asarray(p), np.asarray(q))

    def verify(self, targets, proposals, ids, draws, *, greedy, limit, eos=()):
        return O.verify_probs(targets, proposals, ids, draws.random, greedy=greedy, output_limit=limit, eos_ids=eos)


@pytest.mark.parametrize("name", sorted(law.LAWS))
def test_reference_law(name):
    # The reference's known answers and laws (tests/sampling_law.py cites each source).
    law.LAWS[name](OracleImpl())


def test_two_token_joint_law_at_full_resolution():
    law.check_two_token_joint_law(OracleImpl(), accept_cells=4, target_cells=8)


def test_categorical_reports_no_draw_for_one_point_support():
    # sampling.py:120-122: no uniform, so no margin either.
    assert O.categorical(np.array([0., 1., 0.]), lambda: 0.5) == (1, False, math.inf)


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
