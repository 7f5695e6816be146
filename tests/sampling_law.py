"""The reference's sampling law as data, with checkers written for this repository.

The inputs and expected outputs below are the reference's known answers and
exact laws (its tests/test_sampling.py, tests/test_sampling_reference_law.py
and the verifier checks of src/deepseekrpc/cluster_probe.py:22-56; each case
cites its source).  The checkers are independent of any one implementation:
each takes an ``Impl`` adapter, so the same law runs against the drop-in API
on the GPU (tests/test_sampling.py) and against the CPU oracle
(tests/test_oracle_laws.py).

An ``Impl`` provides:

* ``probs(logits, counts=None, generated=None, bias=None, allowed=None, **policy)``
  -> float64 NumPy probabilities; raises ``impl.Rejected`` on invalid input;
* ``draw(p, u)`` -> token (``u`` a float, or a callable asked only if a draw happens);
* ``residual(p, q)`` -> the normalised positive part of ``p - q``;
* ``verify(targets, proposals, ids, draws, *, greedy, limit, eos=())`` ->
  ``(accepted_drafts, output_ids, pending_token, stop_reason)``, where
  ``draws.random(domain)`` supplies every uniform.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from fractions import Fraction
from itertools import product

import numpy as np

F = np.float64


class Cells:
    """Uniform source of interval midpoints: ``accept`` draws come from a
    fixed list, ``target`` draws are a constant.  It records every request."""

    def __init__(self, accept=(), target=0.5):
        self._accept = list(accept)
        self._target = target
        self.requests = []

    def random(self, domain):
        self.requests.append(domain)
        if domain == "accept":
            return self._accept.pop(0)
        assert domain == "target", domain
        return self._target


# ---------------------------------------------------------------------------
# Probability known answers on the three-token row log([.5, .3, .2])
# (tests/test_sampling.py:22-32): (policy, expected, comparison).

THREE = np.log(np.array([.5, .3, .2], F))
THREE_TOKEN_ANSWERS = [
    ({}, [.5, .3, .2], "rtol"),
    ({"temperature": 0}, [1, 0, 0], "equal"),
    ({"temperature": 1e-320}, [1, 0, 0], "equal"),     # not greedy, yet one survivor
    ({"top_k": 2}, [.625, .375, 0], "rtol"),
    ({"top_p": .7}, [.625, .375, 0], "rtol"),
    ({"top_p": 0}, [1, 0, 0], "equal"),
    ({"min_p": .7}, [1, 0, 0], "equal"),
    ({"min_p": .5, "top_p": .6}, [1, 0, 0], "equal"),
]


def check_three_token_answers(impl):
    for policy, want, how in THREE_TOKEN_ANSWERS:
        got = impl.probs(THREE, **policy)
        if how == "equal":
            np.testing.assert_array_equal(got, want, err_msg=str(policy))
        else:
            np.testing.assert_allclose(got, want, rtol=1e-15, err_msg=str(policy))


# Penalties, bias and mask share one definition (tests/test_sampling.py:35-44):
# the adjusted logits are stated in closed form.
PENALTY_CASE = dict(
    logits=np.array([2., -1., 3., 0.], np.float32), counts=np.array([2, 1, 0, 0], np.int32),
    policy=dict(repetition_penalty=2, presence_penalty=.25, frequency_penalty=.5),
    bias={3: .2}, allowed=np.array([True, True, False, True]),
    adjusted=np.array([2 / 2 - .25 - 2 * .5, -1 * 2 - .25 - 1 * .5, -np.inf, .2]))


def softmax_of(adjusted):
    e = np.exp(adjusted - np.max(adjusted))
    return e / e.sum()


def check_penalty_bias_mask(impl):
    c = PENALTY_CASE
    got = impl.probs(c["logits"], counts=c["counts"], bias=c["bias"], allowed=c["allowed"], **c["policy"])
    np.testing.assert_allclose(got, softmax_of(c["adjusted"]), rtol=1e-15)
    try:
        impl.probs(c["logits"], allowed=np.zeros(4, bool), **c["policy"])
    except impl.Rejected as exc:
        assert "every" in str(exc)
    else:
        raise AssertionError("a fully masked row was accepted")


# Prompt counts drive repetition only; generated counts drive presence and
# frequency (tests/test_sampling.py:236-243).
GENERATED_CASE = dict(
    logits=np.array([2., 2., 0.], np.float32), counts=np.array([5, 1, 0], np.int32),
    generated=np.array([0, 1, 0], np.int32),
    policy=dict(repetition_penalty=2, presence_penalty=.5, frequency_penalty=.25),
    adjusted=np.array([2 / 2, 2 / 2 - .5 - .25, 0.]))


def check_generated_counts(impl):
    c = GENERATED_CASE
    got = impl.probs(c["logits"], counts=c["counts"], generated=c["generated"], **c["policy"])
    np.testing.assert_allclose(got, softmax_of(c["adjusted"]), rtol=1e-15, atol=0)


# CDF cells (tests/test_sampling.py:49-53): a zero-mass index never wins,
# including at the cell edges 0, .25 and the largest double below 1.
CDF_ROW = np.array([0., .25, 0., .75, 0.], F)
CDF_CELLS = [(0.0, 1), (0.25, 3), (float(np.nextafter(1.0, 0.0)), 3)]


def check_cdf_cells(impl):
    for u, want in CDF_CELLS:
        assert impl.draw(CDF_ROW, u) == want, (u, want)


def check_single_support_draws_nothing(impl):
    def refuse():
        raise AssertionError("a one-point support asked for a uniform")
    assert impl.draw(np.array([0., 1., 0.], F), refuse) == 1


# ---------------------------------------------------------------------------
# Verifier laws.


def check_rejection_marginal(impl):
    """One draft against p = (.3, .7), q = (.8, .2): over q's proposals and
    eight equal accept cells, the output law is p exactly, and the residual
    is (0, 1) (tests/test_sampling.py:56-69)."""
    p, q = np.array([.3, .7], F), np.array([.8, .2], F)
    np.testing.assert_array_equal(impl.residual(p, q), [0, 1])
    law = {0: Fraction(0), 1: Fraction(0)}
    q_exact = {0: Fraction(4, 5), 1: Fraction(1, 5)}
    for proposal, cell in product((0, 1), range(8)):
        out = impl.verify([p, p], [q], [proposal], Cells([(cell + .5) / 8]), greedy=False, limit=2)[1]
        law[out[0]] += q_exact[proposal] / 8
    assert law == {0: Fraction(3, 10), 1: Fraction(7, 10)}


def check_rejection_position(impl, position):
    """Five drafts of token 0 under q = (.5, .5).  Every target gives token 0
    p = .75 ≥ q, so it is always accepted, except the target at ``position``
    (p = .25, accepted iff u < .5): an accept uniform of .75 rejects exactly
    there (tests/test_sampling.py:72-84)."""
    accepts, rejects = np.array([.75, .25], F), np.array([.25, .75], F)
    targets = [rejects if j == position else accepts for j in range(6)]
    accepted, out, pending, stop = impl.verify(targets, [np.array([.5, .5], F)] * 5, [0] * 5, Cells([.75] * 5),
                                               greedy=False, limit=10)
    assert accepted == position and len(out) == position + 1
    assert pending == out[-1] and stop is None


def check_stops_inside_drafts(impl):
    """An EOS draft, or the output limit, ends the drafts with no bonus
    draw and no pending token (tests/test_sampling.py:87-95)."""
    p, q = np.array([.9, .1], F), np.array([.5, .5], F)
    cells = Cells([.1])
    assert impl.verify([p] * 6, [q] * 5, [0] * 5, cells, greedy=False, limit=10, eos={0}) == (1, (0,), None, "eos")
    assert cells.requests == ["accept"]
    cells = Cells([.1, .1])
    assert impl.verify([p] * 6, [q] * 5, [0] * 5, cells, greedy=False, limit=2) == (2, (0, 0), None, "length")
    assert cells.requests == ["accept", "accept"]


def check_greedy_draws_nothing(impl):
    """Greedy verification asks for no uniform (tests/test_sampling.py:98-107)."""
    cells = Cells()
    out = impl.verify([np.array([.2, .8], F)] * 6, [np.array([.5, .5], F)] * 5, [0] * 5, cells, greedy=True,
                      limit=5)
    assert out[1] == (1,) and cells.requests == []


def check_equal_coordinates(impl):
    """Coordinates where p == q get no residual mass
    (tests/test_sampling_reference_law.py:45-50)."""
    np.testing.assert_array_equal(impl.residual(np.array([.125, .625, .25], F), np.array([.5, .25, .25], F)),
                                  [0., 1., 0.])


def check_two_token_joint_law(impl, accept_cells=4, target_cells=8):
    """Two drafts with Markov-conditioned rows: enumerating every proposal
    pair, every accept cell and every target cell reproduces the target's
    joint law p0(a)·p1[a](b) exactly (tests/test_sampling_reference_law.py:15-42).
    When the first draft is rejected, the second token is drawn from p1 of
    the replacement over ``target_cells`` cells."""
    third = Fraction(1, 4), Fraction(3, 8), Fraction(3, 8)
    q0 = Fraction(1, 2), Fraction(1, 4), Fraction(1, 4)
    q1 = [tuple(q0[(t - a - 1) % 3] for t in range(3)) for a in range(3)]
    p1 = [tuple(third[(t - a - 2) % 3] for t in range(3)) for a in range(3)]

    def row(values):
        return np.array([float(v) for v in values], F)

    joint = {}
    cell_weight = Fraction(1, accept_cells * accept_cells * target_cells)
    for a, b in product(range(3), range(3)):
        for ca, cb, ct in product(range(accept_cells), range(accept_cells), range(target_cells)):
            cells = Cells([(ca + .5) / accept_cells, (cb + .5) / accept_cells], (ct + .5) / target_cells)
            out = impl.verify([row(third), row(p1[a]), row(third)], [row(q0), row(q1[a])], [a, b], cells,
                              greedy=False, limit=2)[1]
            weight = q0[a] * q1[a][b] * cell_weight
            if len(out) == 2:
                joint[out] = joint.get(out, 0) + weight
                continue
            for cd in range(target_cells):
                second = impl.draw(row(p1[out[0]]), (cd + .5) / target_cells)
                key = (out[0], second)
                joint[key] = joint.get(key, 0) + weight / target_cells
    for a, b in product(range(3), range(3)):
        assert joint.get((a, b), 0) == third[a] * p1[a][b], (a, b)


# ---------------------------------------------------------------------------
# cluster_probe.py:22-56: thirteen verifier checks on one-hot rows.

POINT = np.eye(3, dtype=F)


@dataclass
class ProbeCase:
    name: str
    targets: list
    greedy: bool
    limit: int
    want: tuple                      # (accepted, output_ids, pending, stop); None entries are not checked
    eos: frozenset = field(default_factory=frozenset)


def probe_cases():
    cases = []
    for rejected in range(6):   # greedy rejection at every prefix length, then the bonus
        targets = [POINT[0]] * rejected + [POINT[1]] * (5 - rejected) + [POINT[2]]
        out = (0,) * rejected + ((1,) if rejected < 5 else (2,))
        cases.append(ProbeCase(f"greedy-reject-{rejected}", targets, True, 64, (rejected, out, None, None)))
    for limit in range(1, 6):   # sampled acceptance crossing the output limit
        cases.append(ProbeCase(f"limit-{limit}", [POINT[0]] * 6, False, limit,
                               (None, (0,) * limit, None, "length")))
    cases.append(ProbeCase("eos-inside-drafts", [POINT[0]] * 6, False, 64, (1, (0,), None, "eos"), frozenset({0})))
    return cases


def check_probe_case(impl, case: ProbeCase):
    got = impl.verify(case.targets, [POINT[0]] * 5, [0] * 5, Cells([.5] * 5), greedy=case.greedy, limit=case.limit,
                      eos=case.eos)
    for have, want in zip(got, case.want):
        if want is not None:
            assert have == want, (case.name, got, case.want)


def check_residual_identity(impl):
    """min(p, q) + (1 - Σ min(p, q))·residual(p, q) == p (cluster_probe.py:53-55)."""
    p, q = np.array([.1, .6, .3], F), np.array([.5, .2, .3], F)
    shared = np.minimum(p, q)
    np.testing.assert_allclose(shared + (1 - shared.sum()) * impl.residual(p, q), p, rtol=0, atol=2e-16)


LAWS = {
    "three-token answers": check_three_token_answers,
    "penalties, bias and mask": check_penalty_bias_mask,
    "generated counts": check_generated_counts,
    "cdf cells": check_cdf_cells,
    "single support": check_single_support_draws_nothing,
    "rejection marginal": check_rejection_marginal,
    **{f"rejection at {j}": (lambda impl, j=j: check_rejection_position(impl, j)) for j in range(6)},
    "stops inside drafts": check_stops_inside_drafts,
    "greedy draws nothing": check_greedy_draws_nothing,
    "equal coordinates": check_equal_coordinates,
    "residual identity": check_residual_identity,
    **{f"probe {c.name}": (lambda impl, c=c: check_probe_case(impl, c)) for c in probe_cases()},
}
