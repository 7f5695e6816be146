"""Terminal sampling transactions on the GPU (deepseekrpc_amd.terminal_sampling).

Scenarios follow the behaviour the reference pins for
src/deepseekrpc/terminal_sampling.py: seed and normal-decode commits, Markov
proposals under a grammar that sees each tentative prefix, aborts that
restore the RNG, EOS drafts that end grammar queries, confidence that never
changes a decision (tests/test_sampling.py:149-233,
tests/test_sampling_reference_law.py:53-73), stop strings cut inside the
accepted drafts before commit (tests/test_detokenize.py:103-148), and the RNG
finalising only at the commit of the prepared digest
(tests/test_publication.py:58-90).  The decision digests and final RNG
snapshots were recorded from the reference (tests/golden/).
"""
import json
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from deepseekrpc_amd.jsonutil import ValidationError
from deepseekrpc_amd.sampling import RandomStreams, SamplingPolicy
from deepseekrpc_amd.terminal_sampling import SeedDecision, TerminalSampler

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
V = 129280


class MarkovGraph:
    """A draft graph: ``rows(position, previous)`` gives each proposal row's
    logits; every call is recorded.  ``confidence`` is returned beside the
    logits and must not matter."""

    def __init__(self, rows, confidence=None):
        self.rows, self.confidence, self.calls = rows, confidence, []

    def draft_conditional_logits(self, result, row, previous):
        self.calls.append((row, previous))
        confidence = None if self.confidence is None else self.confidence[row]
        return np.array([self.rows(row, previous)], np.float32), confidence


class Grammar:
    """A grammar mask provider that records the prefixes it is asked about."""

    def __init__(self, mask_for):
        self.mask_for, self.asked = mask_for, []

    def __call__(self, prefix):
        self.asked.append(prefix)
        return np.asarray(self.mask_for(prefix))


def one_hot_logits(tokens, vocabulary=V, low=-80., high=80.):
    rows = np.full((len(tokens), vocabulary), low, np.float32)
    rows[np.arange(len(tokens)), tokens] = high
    return rows


# ---------------------------------------------------------------------------
# Seeds, normal decode, proposals and verification.

def test_seed_commits_only_its_own_digest_then_normal_decode_hits_the_limit():
    sampler = TerminalSampler(1017, vocabulary=3)
    history = np.array([1, 0, 0], np.int32)
    greedy = SamplingPolicy(temperature=0)
    seed = sampler.begin_seed(np.array([[0., 4., 0.]], np.float32), policy=greedy, counts=history, remaining=10)
    assert (seed.decision.output_ids, seed.decision.accepted_target_rows) == ((1,), 0)
    with pytest.raises(ValidationError, match="match"):
        seed.commit("0" * 64)
    assert sampler.active is seed                  # a wrong digest commits nothing
    seed.commit(seed.prepared()["digest"])
    history[1] += 1
    step = sampler.begin_verification(seed_token=1, policy=greedy, counts=history, remaining=1)
    step.use_normal_decode()
    with pytest.raises(ValidationError, match="duplicate"):
        step.use_normal_decode()
    d = step.verify(np.array([[0., 0., 4.]], np.float32))
    assert (d.accepted_target_rows, d.output_ids, d.pending_token, d.stop_reason) == (1, (2,), 2, "length")
    step.commit(step.prepared()["digest"])
    assert sampler.active is None


def test_grammar_and_markov_rows_see_each_tentative_prefix():
    # Flat rows under a greedy policy: the grammar alone decides, alternating
    # between token 2 (even prefix lengths) and token 1 (odd).
    sampler = TerminalSampler(2, vocabulary=3)
    history = np.array([5, 1, 0], np.int32)
    grammar = Grammar(lambda prefix: [False, len(prefix) % 2 == 1, len(prefix) % 2 == 0])
    graph = MarkovGraph(lambda row, previous: [0., 0., 0.])
    work = sampler.begin_verification(seed_token=1, policy=SamplingPolicy(temperature=0), counts=history,
                                      remaining=3, allowed=grammar, grammar_identity="e" * 64)
    assert work.propose(graph, None) == (2, 1, 2)
    assert graph.calls == [(0, 1), (1, 2), (2, 1)]
    assert grammar.asked == [(), (2,), (2, 1)]
    d = work.verify(np.zeros((4, 3), np.float32))
    assert grammar.asked[3:] == [(), (2,), (2, 1)]    # targets: the same prefixes, in order
    assert (d.output_ids, d.pending_token, d.accepted_target_rows) == ((2, 1, 2), None, 4)
    work.commit(work.prepared()["digest"])
    assert history.tolist() == [5, 1, 0]               # the caller's counts are never written


def test_invalid_target_window_aborts_and_restores_the_proposal_draws():
    sampler = TerminalSampler(7, vocabulary=2)
    initial = sampler.random.snapshot()
    work = sampler.begin_verification(seed_token=0, policy=SamplingPolicy(), counts=np.array([1, 0], np.int32),
                                      remaining=10)
    work.propose(MarkovGraph(lambda row, previous: [0., 0.]), None)
    with pytest.raises(ValidationError, match="vocabulary"):
        work.verify(np.zeros((5, 2), np.float32))      # six rows are needed
    assert sampler.active is None
    assert sampler.random.snapshot() == initial


@pytest.mark.parametrize("policy", [SamplingPolicy(), SamplingPolicy(temperature=0.8, top_k=3)])
def test_a_non_finite_cuda_target_window_aborts_the_device_verifier(policy):
    """A NaN, +inf or -inf in CUDA target rows gives the window message on
    both device verifier routes (the window check is read back with the
    decision), and the transaction ends with the RNG as it began."""
    for bad in (float("nan"), float("inf"), -float("inf")):
        sampler = TerminalSampler(17)
        initial = sampler.random.snapshot()
        counts = np.zeros(V, np.int32)
        counts[4] = 1
        work = sampler.begin_verification(seed_token=4, policy=policy, counts=counts, remaining=10)
        ids = work.propose(_DeviceMarkov(lambda row, prev: np.linspace(0, 1, V, dtype=np.float32)), None)
        target = torch.zeros((len(ids) + 1, V), dtype=torch.float32, device="cuda")
        target[len(ids), 5] = bad
        with pytest.raises(ValidationError, match="vocabulary window"):
            work.verify(target)
        assert sampler.active is None and sampler.random.snapshot() == initial


def test_an_accepted_eos_draft_ends_the_grammar_queries():
    def mask(prefix):
        assert prefix == (), "no distribution exists after the grammar's EOS"
        return [False, True]

    sampler = TerminalSampler(7, vocabulary=2)
    work = sampler.begin_verification(seed_token=0, policy=SamplingPolicy(), counts=np.array([1, 0], np.int32),
                                      remaining=10, eos_ids={1}, allowed=Grammar(mask), grammar_identity="f" * 64)
    assert work.propose(MarkovGraph(lambda row, previous: [0., 1.]), None) == (1,)
    d = work.verify(np.array([[0., 1.], [0., 1.]], np.float32))
    assert (d.output_ids, d.stop_reason, d.pending_token) == ((1,), "eos", None)
    work.commit(work.prepared()["digest"])


def test_draft_confidence_never_changes_proposals_decisions_or_rng():
    outcomes = set()
    for confidence in ([0.] * 5, [1.] * 5, [0., 1., .5, .01, .99]):
        sampler = TerminalSampler(41017, vocabulary=3)
        work = sampler.begin_verification(seed_token=0, policy=SamplingPolicy(), remaining=8,
                                          counts=np.array([1, 0, 0], np.int32))
        proposals = work.propose(MarkovGraph(lambda row, previous: [previous * .5, .25, -.5], confidence), None)
        assert len(proposals) == 5
        d = work.verify(np.array([[.1, .5, -.5]] * 6, np.float32))
        work.commit(work.prepared()["digest"])
        outcomes.add((proposals, d, json.dumps(sampler.random.snapshot(), sort_keys=True)))
    assert len(outcomes) == 1


def test_step_guards_follow_the_stage_order():
    sampler = TerminalSampler(5, vocabulary=4)
    seed = sampler.begin_seed(np.array([[0., 1., 2., 3.]], np.float32), policy=SamplingPolicy(temperature=0),
                              counts=np.zeros(4, np.int32), remaining=4)
    for call, match in ((lambda: seed.propose(None, None), "duplicate"), (seed.use_normal_decode, "duplicate"),
                        (lambda: seed.verify(np.zeros((1, 4), np.float32)), "duplicate")):
        with pytest.raises(ValidationError, match=match):
            call()
    with pytest.raises(ValidationError, match="active"):
        sampler.begin_seed(np.zeros((1, 4), np.float32), policy=SamplingPolicy(), counts=np.zeros(4, np.int32),
                           remaining=4)
    seed.abort()
    with pytest.raises(ValidationError, match="closed or stale"):
        seed.prepared()
    with pytest.raises(ValidationError, match="published sampling history"):
        sampler.begin_verification(seed_token=2, policy=SamplingPolicy(), counts=np.zeros(4, np.int32), remaining=4)
    assert sampler.active is None
    step = sampler.begin_verification(seed_token=2, policy=SamplingPolicy(), counts=np.array([0, 0, 1, 0], np.int32),
                                      remaining=4)
    with pytest.raises(ValidationError, match="not been computed"):
        step.prepared()
    with pytest.raises(ValidationError, match="not complete"):
        step.verify(np.zeros((1, 4), np.float32))
    step.abort()


@pytest.mark.parametrize("kw,match", [
    (dict(remaining=0), "remaining"),
    (dict(counts=np.zeros(3, np.int32)), "published token history"),
    (dict(counts=np.full(4, 300_000, np.int64)), "published token history"),
    (dict(eos_ids={4}), "EOS"),
    (dict(allowed=np.ones(4, bool), grammar_identity="a" * 64), "grammar mask provider"),
    (dict(allowed=lambda prefix: np.ones(4, bool)), "frozen grammar"),
    (dict(stop_identity="A" * 64), "detokenizer"),
    (dict(generated_counts=np.array([0, 2, 0, 0], np.int32)), "subset"),
    (dict(policy=dict(temperature=1.0)), "policy is invalid"),
])
def test_controls_are_rejected_with_the_reference_messages(kw, match):
    sampler = TerminalSampler(1, vocabulary=4)
    args = dict(policy=SamplingPolicy(), counts=np.array([0, 1, 0, 0], np.int32), remaining=4)
    args.update(kw)
    with pytest.raises(ValidationError, match=match):
        sampler.begin_seed(np.zeros((1, 4), np.float32), **args)
    assert sampler.active is None and not sampler.random.active


# ---------------------------------------------------------------------------
# The fused draw: one launch per row, the domain advanced by what it consumed.

def test_seed_draw_consumes_a_target_uniform_only_for_a_wider_support():
    sampler = TerminalSampler(1017)
    fresh = RandomStreams(1017)
    # exp(-800) underflows to zero: a support of one token, drawn without a uniform.
    one_point = sampler.begin_seed(one_hot_logits([5], low=-400., high=400.), policy=SamplingPolicy(),
                                   counts=np.zeros(V, np.int32), remaining=3)
    assert one_point.decision.token == 5
    one_point.commit(one_point.prepared()["digest"])
    assert sampler.random.snapshot() == fresh.snapshot()
    logits = np.full((1, V), -80., np.float32)
    logits[0, 7:9] = [1., 0.]
    two_points = sampler.begin_seed(logits, policy=SamplingPolicy(), counts=np.zeros(V, np.int32), remaining=3)
    txn = fresh.begin()
    u = txn.random("target")
    assert two_points.decision.token == (7 if u < 1 / (1 + np.exp(-1.)) else 8)
    two_points.commit(two_points.prepared()["digest"])
    assert sampler.random.snapshot() == txn.commit()


def test_rng_finalises_only_at_the_commit_of_the_prepared_digest():
    sampler = TerminalSampler(1017)
    history = np.zeros(V, np.int32)
    np.add.at(history, [3, 11, 11, 40], 1)
    generated = history.copy()
    generated[3] = 0
    logits = np.full((1, V), -80., np.float32)
    logits[0, 7:9] = [1., 0.]
    work = sampler.begin_seed(logits, policy=SamplingPolicy(), counts=history, generated_counts=generated,
                              remaining=10)
    digest = work.prepared()["digest"]
    assert sampler.random.active
    with pytest.raises(ValidationError, match="idle"):
        sampler.random.snapshot()
    with pytest.raises(ValidationError, match="match"):
        work.commit("f" * 64)
    assert sampler.random.active and sampler.active is work
    work.commit(digest)
    assert not sampler.random.active and sampler.active is None
    reference = RandomStreams(1017).begin()
    reference.random("target")
    assert sampler.random.snapshot() == reference.commit()


def test_device_rows_stay_on_the_device():
    sampler = TerminalSampler(1017)
    logits = torch.full((1, V), -80., dtype=torch.float32, device="cuda")
    logits[0, 7:9] = torch.tensor([1., 0.])
    work = sampler.begin_seed(logits, policy=SamplingPolicy(), counts=np.zeros(V, np.int32), remaining=10)
    assert work.decision.token in (7, 8)
    work.abort()
    work = sampler.begin_seed(logits, policy=SamplingPolicy(temperature=0), counts=np.zeros(V, np.int32), remaining=1)
    assert work.decision.output_ids == (7,) and work.decision.stop_reason == "length"
    work.commit(work.prepared()["digest"])
    with pytest.raises(ValidationError, match="FP32 CUDA"):
        sampler.begin_seed(logits.cpu(), policy=SamplingPolicy(), counts=np.zeros(V, np.int32), remaining=1)


@pytest.mark.parametrize("penalties", [dict(repetition_penalty=1.3, presence_penalty=0.4, frequency_penalty=0.2),
                                       dict()])
def test_seed_rows_read_the_frozen_history(penalties):
    """A seed from CUDA logits with int64 counts and generated counts: its
    draw and float64 distribution are the oracle's (sampling.py:54-66), and
    a one-token prefix counts once more as generated output
    (terminal_sampling.py:127-133).  Without penalties the history changes
    nothing, and the rows are still the oracle's."""
    from oracle import sampling_oracle as O
    rng = np.random.default_rng(29)
    vocab = 3001
    counts = np.zeros(vocab, np.int64)
    np.add.at(counts, rng.integers(0, vocab, 400), 1)
    generated = np.where(np.arange(vocab) % 3 == 0, 0, counts)
    logits = rng.normal(0, 2, (1, vocab)).astype(np.float32)
    kw = dict(temperature=0.8, top_p=0.95, **penalties)
    sampler = TerminalSampler(77, vocabulary=vocab)
    device_logits = torch.from_numpy(logits).cuda()
    work = sampler.begin_seed(device_logits, policy=SamplingPolicy(**kw), counts=counts, generated_counts=generated,
                              remaining=5)
    u = RandomStreams(77).begin().random("target")
    ref = O.sample_row(logits[0], O.Policy(**kw), u, counts, generated)
    assert ref.status == O.OK and work.decision.token == ref.token
    np.testing.assert_allclose(work.distribution(device_logits[0], ()).cpu().numpy(), ref.probs, rtol=1e-12,
                               atol=1e-300)
    token = int(np.flatnonzero(counts == 0)[0])
    grown, grown_generated = counts.copy(), generated.copy()
    grown[token] += 1
    grown_generated[token] += 1
    want = O.probabilities(logits[0], O.Policy(**kw), grown, grown_generated)
    np.testing.assert_allclose(work.distribution(device_logits[0], (token,)).cpu().numpy(), want, rtol=1e-12,
                               atol=1e-300)
    work.abort()
    assert sampler.random.snapshot() == RandomStreams(77).snapshot()


def test_counts_whose_int64_sum_wraps_pass_the_controls_and_fail_the_first_row():
    """Four counts of 2^62 sum to 2^64, which wraps to 0 in int64: the
    controls accept them (terminal_sampling.py:57-60) and the first row's
    distribution rejects the counts (sampling.py:55-58).  The graph is asked
    for that row first, on both graph kinds."""
    counts = np.zeros(8, np.int64)
    counts[:4] = 1 << 62
    sampler = TerminalSampler(5, vocabulary=8)
    with pytest.raises(ValidationError, match="frequency counts"):
        sampler.begin_seed(np.zeros((1, 8), np.float32), policy=SamplingPolicy(), counts=counts, remaining=3)
    assert sampler.active is None and not sampler.random.active

    class DeviceGraph(MarkovGraph):
        def draft_conditional_logits_device(self, result, row, previous):
            raise AssertionError("rows whose counts fail go through the host loop")

    for graph in (MarkovGraph(lambda row, prev: np.zeros(8, np.float32)),
                  DeviceGraph(lambda row, prev: np.zeros(8, np.float32))):
        work = sampler.begin_verification(seed_token=1, policy=SamplingPolicy(), counts=counts, remaining=3)
        with pytest.raises(ValidationError, match="frequency counts"):
            work.propose(graph, None)
        assert graph.calls == [(0, 1)] and sampler.active is None
    assert sampler.random.snapshot() == RandomStreams(5).snapshot()


def test_a_non_finite_cuda_window_is_reported_before_later_errors():
    """NaN, +inf and -inf in a CUDA seed window give the window message
    (terminal_sampling.py:16-27), also when the logit bias is invalid too,
    and the transaction is gone with the RNG untouched."""
    sampler = TerminalSampler(3)
    for bad in (float("nan"), float("inf"), -float("inf")):
        logits = torch.zeros((1, V), dtype=torch.float32, device="cuda")
        logits[0, 9] = bad
        for bias in (None, {V + 5: 1.0}):
            with pytest.raises(ValidationError, match="vocabulary window"):
                sampler.begin_seed(logits, policy=SamplingPolicy(), counts=np.zeros(V, np.int32), remaining=2,
                                   logit_bias=bias)
            assert sampler.active is None and not sampler.random.active
    with pytest.raises(ValidationError, match="biased token"):
        sampler.begin_seed(torch.zeros((1, V), dtype=torch.float32, device="cuda"), policy=SamplingPolicy(),
                           counts=np.zeros(V, np.int32), remaining=2, logit_bias={V + 5: 1.0})
    assert sampler.random.snapshot() == RandomStreams(3).snapshot()


def test_a_seed_launched_ahead_of_its_checks_changes_nothing_when_they_fail():
    """A CUDA seed window with no grammar, bias or penalties is sampled while
    the host checks the controls; a failing check raises its own message and
    leaves the RNG where it was, counts whose int64 sum wraps take the
    ordinary route to the row's error, and the next valid seeds draw the
    oracle's tokens in sequence."""
    from oracle import sampling_oracle as O
    rng = np.random.default_rng(31)
    logits = rng.normal(0, 2, (1, V)).astype(np.float32)
    device_logits = torch.from_numpy(logits).cuda()
    sampler = TerminalSampler(404)
    bad_counts = np.zeros(V, np.int32)
    bad_counts[5] = -1
    with pytest.raises(ValidationError, match="exact published token history"):
        sampler.begin_seed(device_logits, policy=SamplingPolicy(), counts=bad_counts, remaining=3)
    with pytest.raises(ValidationError, match="remaining output capacity"):
        sampler.begin_seed(device_logits, policy=SamplingPolicy(), counts=np.zeros(V, np.int32), remaining=0)
    wrap = np.zeros(V, np.int64)
    wrap[:4] = 1 << 62
    with pytest.raises(ValidationError, match="frequency counts"):
        sampler.begin_seed(device_logits, policy=SamplingPolicy(), counts=wrap, remaining=3)
    assert sampler.active is None and not sampler.random.active
    assert sampler.random.snapshot() == RandomStreams(404).snapshot()
    reference = RandomStreams(404).begin()
    policy = dict(temperature=0.7, top_k=50, top_p=0.9)
    for _ in range(2):
        work = sampler.begin_seed(device_logits, policy=SamplingPolicy(**policy), counts=np.zeros(V, np.int32),
                                  remaining=4)
        with pytest.raises(ValidationError, match="active"):
            sampler.begin_seed(device_logits, policy=SamplingPolicy(**policy), counts=np.zeros(V, np.int32),
                               remaining=4)
        ref = O.sample_row(logits[0], O.Policy(**policy), reference.random("target"))
        assert work.decision.token == ref.token
        work.commit(work.prepared()["digest"])
    assert sampler.random.snapshot() == reference.commit()


def test_proposal_rows_are_kept_on_the_device_for_verification():
    sampler = TerminalSampler(99)
    history = np.zeros(V, np.int32)
    history[0] = 1
    work = sampler.begin_verification(seed_token=0, policy=SamplingPolicy(top_k=2), counts=history, remaining=20)
    graph = MarkovGraph(lambda row, previous: one_hot_logits([(previous + 1) % V], high=2.)[0])
    proposals = work.propose(graph, None)
    assert len(proposals) == 5 and all(isinstance(r, torch.Tensor) and r.is_cuda for r in work.proposal_rows)
    for row, token in zip(work.proposal_rows, proposals):
        assert float(row[token]) > 0 and abs(float(row.sum()) - 1) < 1e-12
    work.abort()


# ---------------------------------------------------------------------------
# Stop strings (tests/test_detokenize.py:103-148), with a tracker stub whose
# preview reports a match after a given number of tokens.

class StopAt:
    def __init__(self, tokens, identity="c" * 64):
        self.tokens, self.identity = tokens, identity
        self.previews = []

    def preview(self, output_ids):
        self.previews.append(tuple(output_ids))
        hit = self.tokens is not None and self.tokens <= len(output_ids)
        return SimpleNamespace(matched="STOP" if hit else None, token_count=self.tokens if hit else len(output_ids))


def _full_acceptance(sampler, tracker, proposals, bonus):
    history = np.zeros(V, np.int32)
    history[0] = 1
    work = sampler.begin_verification(seed_token=0, policy=SamplingPolicy(temperature=0), counts=history,
                                      generated_counts=history, remaining=100, stop_identity=tracker.identity)
    # Proposals supplied by the caller, as complete one-hot distributions.
    work.proposal_ids = list(proposals)
    work.proposal_rows = [np.eye(1, V, t, dtype=np.float64).reshape(-1) for t in proposals]
    work._proposal_ready = True
    decision = work.verify(one_hot_logits([*proposals, bonus]))
    assert (decision.accepted_drafts, decision.pending_token) == (len(proposals), bonus)
    return work


@pytest.mark.parametrize("cut", [1, 2, 5])
def test_stop_inside_the_accepted_drafts_drops_the_pending_token(cut):
    sampler = TerminalSampler(1017)
    tracker = StopAt(cut)
    proposals = [17, 9, 5000, 121, 77]
    work = _full_acceptance(sampler, tracker, proposals, 2)
    with pytest.raises(ValidationError, match="not been computed"):
        work.prepared()                                # the frozen stop policy runs first
    d = work.apply_stop(tracker)
    assert (d.accepted_drafts, d.accepted_target_rows) == (cut, cut + 1)
    assert d.output_ids == tuple(proposals[:cut]) and d.pending_token is None and d.stop_reason == "stop"
    with pytest.raises(ValidationError, match="frozen terminal decision"):
        work.apply_stop(tracker)                       # once only
    work.commit(work.prepared()["digest"])


def test_stop_at_the_bonus_token_keeps_it_pending():
    sampler = TerminalSampler(1017)
    tracker = StopAt(6)
    work = _full_acceptance(sampler, tracker, [4, 5, 6, 7, 8], 2)
    d = work.apply_stop(tracker)
    assert (d.accepted_drafts, d.output_ids, d.pending_token, d.stop_reason) == (5, (4, 5, 6, 7, 8, 2), 2, "stop")
    work.abort()


def test_no_stop_match_leaves_the_decision():
    sampler = TerminalSampler(1017)
    tracker = StopAt(None)
    work = _full_acceptance(sampler, tracker, [4, 5], 9)
    before = work.decision
    assert work.apply_stop(tracker) == before and tracker.previews == [(4, 5, 9)]
    work.commit(work.prepared()["digest"])


def test_stop_on_a_seed_keeps_its_token_pending():
    sampler = TerminalSampler(1017)
    tracker = StopAt(1)
    work = sampler.begin_seed(one_hot_logits([321]), policy=SamplingPolicy(temperature=0),
                              counts=np.zeros(V, np.int32), remaining=8, stop_identity=tracker.identity)
    d = work.apply_stop(tracker)
    assert isinstance(d, SeedDecision)
    assert (d.token, d.pending_token, d.accepted_target_rows, d.stop_reason) == (321, 321, 0, "stop")
    work.abort()


def test_stop_needs_the_frozen_tracker_identity():
    sampler = TerminalSampler(1017)
    work = sampler.begin_seed(one_hot_logits([3]), policy=SamplingPolicy(temperature=0),
                              counts=np.zeros(V, np.int32), remaining=8, stop_identity="c" * 64)
    with pytest.raises(ValidationError, match="frozen terminal decision"):
        work.apply_stop(StopAt(1, identity="d" * 64))
    work.abort()
    plain = sampler.begin_seed(one_hot_logits([3]), policy=SamplingPolicy(temperature=0),
                               counts=np.zeros(V, np.int32), remaining=8)
    with pytest.raises(ValidationError, match="frozen terminal decision"):
        plain.apply_stop(StopAt(1))                   # no stop identity was frozen
    plain.commit(plain.prepared()["digest"])


# ---------------------------------------------------------------------------
# Digests and RNG snapshots recorded from the reference.

def test_digests_match_the_reference_recording():
    meta = json.load(open(os.path.join(HERE, "golden", "sampling_golden.json")))
    gold = {d["name"]: d for d in meta["digests"]}
    sampler = TerminalSampler(1017, vocabulary=8)
    counts = np.array([1, 0, 2, 0, 0, 1, 0, 0], np.int32)
    seed_logits = np.array([[0.5, 1.0, -0.25, 2.0, 0.0, 1.5, -1.0, 0.75]], np.float32)
    work = sampler.begin_seed(seed_logits, policy=SamplingPolicy(temperature=0.9, top_k=5), counts=counts,
                              remaining=6, eos_ids={7})
    assert list(work.decision.output_ids) == gold["seed"]["decision"]
    assert work.prepared()["digest"] == gold["seed"]["digest"]
    work.commit(work.prepared()["digest"])
    counts[work.decision.token] += 1

    def draft_row(row, previous):
        base = np.array([0.1, 0.4, -0.3, 0.9, 0.2, 0.0, -0.6, 0.3], np.float32)
        base[previous] += 0.5
        return base

    work = sampler.begin_verification(seed_token=work.decision.token, policy=SamplingPolicy(top_p=0.95),
                                      counts=counts, remaining=6, eos_ids={7}, logit_bias={2: 1.25, 5: -0.5})
    proposals = work.propose(MarkovGraph(draft_row), None)
    assert list(proposals) == gold["verify"]["proposals"]
    d = work.verify(np.array(gold["verify"]["target"], np.float32))
    assert [d.accepted_drafts, list(d.output_ids), d.pending_token, d.stop_reason] == gold["verify"]["decision"]
    assert work.prepared()["digest"] == gold["verify"]["digest"]
    work.commit(work.prepared()["digest"])
    assert sampler.random.snapshot() == gold["final_rng"]["snapshot"]


class _DeviceMarkov(MarkovGraph):
    """A graph that also makes its rows on the device (the proposal chain's
    device route); the previous token arrives as a device int32 tensor."""

    def draft_conditional_logits_device(self, result, row, previous):
        base = torch.as_tensor(self.rows(row, 0), device="cuda").reshape(1, -1).clone()
        base[0].index_add_(0, previous.long(), torch.full((1,), 2.5, device="cuda"))
        return base, None


@pytest.mark.parametrize("device_graph", [False, True])
def test_batched_device_draws_decide_as_the_host_verifier(device_graph, monkeypatch):
    """The speculative step with every draw on the device (the seed, the
    proposals, the accept tests and the replacement or bonus draw: one
    ``dsr_verify_drafts`` call on the logits for unfiltered requests, one
    ``dsr_verify_probs`` call on the float64 rows for the others) against
    the same steps through the host verifier loop: equal decisions, digests
    and RNG snapshots, over penalties, bias, filters, EOS ids and output
    limits."""
    import deepseekrpc_amd.terminal_sampling as TS
    rng = np.random.default_rng(4242 + device_graph)
    base = rng.normal(0, 2, (6, V)).astype(np.float32)
    batched = []
    real_logits, real_rows = TS.SamplingWork._verify_logits, TS.SamplingWork._verify_rows

    def spy_logits(self, rows, ids, deferred):
        batched.append("logits")
        return real_logits(self, rows, ids, deferred)

    def spy_rows(self, rows, targets, status, ids, deferred):
        batched.append("rows")
        return real_rows(self, rows, targets, status, ids, deferred)

    def run(force_host, seed, policy, remaining, eos, bias):
        if force_host:
            monkeypatch.setattr(TS.SamplingWork, "_draws_fit", lambda self, K: False)
        else:
            monkeypatch.setattr(TS.SamplingWork, "_verify_logits", spy_logits)
            monkeypatch.setattr(TS.SamplingWork, "_verify_rows", spy_rows)
        sampler = TerminalSampler(seed)
        counts = np.zeros(V, np.int32)
        counts[rng_hist] = 1
        work = sampler.begin_seed(base[:1], policy=policy, counts=counts, remaining=remaining, eos_ids=eos,
                                  logit_bias=bias)
        out = [work.prepared()]
        work.commit(work.prepared()["digest"])
        counts[work.decision.token] += 1
        draft = (lambda row, prev: base[1 + row % 4] * 0.9) if device_graph else \
            (lambda row, prev: base[1 + row % 4] * 0.9 + (prev % 7) * 0.01)
        graph = _DeviceMarkov(draft) if device_graph else MarkovGraph(draft)
        work = sampler.begin_verification(seed_token=work.decision.token, policy=policy, counts=counts,
                                          remaining=remaining, eos_ids=eos, logit_bias=bias)
        ids = work.propose(graph, None)
        targets = base[:len(ids) + 1] + rng_noise[:len(ids) + 1]
        work.verify(targets)
        out.append(work.prepared())
        work.commit(work.prepared()["digest"])
        out.append(sampler.random.snapshot())
        monkeypatch.undo()
        return out

    cases = [
        (SamplingPolicy(), 20, frozenset(), None),
        (SamplingPolicy(temperature=0.8, top_k=40, top_p=0.9), 20, frozenset(), {3: 2.0, 11: -1.5}),
        (SamplingPolicy(temperature=1.1, repetition_penalty=1.3, presence_penalty=0.4, frequency_penalty=0.2),
         3, frozenset(), None),
        (SamplingPolicy(temperature=0.0), 20, frozenset(), None),
        (SamplingPolicy(temperature=0.6, min_p=0.02), 20, frozenset(range(0, V, 3)), None),
    ]
    for i, (policy, remaining, eos, bias) in enumerate(cases):
        rng_hist = rng.choice(V, 200, replace=False)
        rng_noise = rng.normal(0, 0.3, (6, V)).astype(np.float32)
        n_before = len(batched)
        dev = run(False, 700 + i, policy, remaining, eos, bias)
        host = run(True, 700 + i, policy, remaining, eos, bias)
        assert len(batched) == n_before + 1, "the device route was not taken"
        assert dev == host, (i, dev[1]["decision"], host[1]["decision"])
    assert batched == ["logits", "rows", "rows", "logits", "rows"], batched
