"""The reference's finite probability laws (tests/test_sampling_reference_law.py
of Protonburn35/DeepSeekRPC) on the drop-in API, plus the reference-recorded
digests and the full-vocabulary terminal flows."""
from fractions import Fraction
from itertools import product
import json
import os

import numpy as np
import pytest
import torch

from deepseekrpc_amd.sampling import SamplingPolicy, categorical, correction_distribution, verify_drafts
from deepseekrpc_amd.terminal_sampling import TerminalSampler

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_conditional_two_token_verification_has_the_exact_target_joint_law():
    # Every proposal and every equal-width RNG cell is enumerated.
    q0 = (Fraction(1, 2), Fraction(1, 4), Fraction(1, 4))
    p0 = (Fraction(1, 4), Fraction(3, 8), Fraction(3, 8))
    q1 = [tuple(q0[(t - prev - 1) % 3] for t in range(3)) for prev in range(3)]
    p1 = [tuple(p0[(t - prev - 2) % 3] for t in range(3)) for prev in range(3)]
    observed = [[Fraction(0) for _ in range(3)] for _ in range(3)]

    class Draws:
        def __init__(self, accept, target):
            self.accept, self.target = iter(accept), target

        def random(self, domain):
            assert domain in {"accept", "target"}
            return next(self.accept) if domain == "accept" else self.target

    arrays = lambda rows: [np.array(row, np.float64) for row in rows]
    # The device path is exact but slow per call; the laws are checked on every
    # proposal pair with one accept cell per position and all target cells.
    for first, second, a, b, c in product(range(3), range(3), range(4), range(4), range(8)):
        result = verify_drafts(arrays((p0, p1[first], p0)), arrays((q0, q1[first])), (first, second),
                               Draws(((a + .5) / 4, (b + .5) / 4), (c + .5) / 8), greedy=False, output_limit=2)
        output = result.output_ids
        weight = q0[first] * q1[first][second] / (16 * 8)
        if len(output) == 1:
            for d in range(8):
                tail = categorical(np.array(p1[output[0]], np.float64), lambda: (d + .5) / 8)
                observed[output[0]][tail] += weight / 8
        else:
            observed[output[0]][output[1]] += weight
    assert observed == [[p0[f] * p1[f][s] for s in range(3)] for f in range(3)]


def test_equal_probability_coordinates_receive_no_rejection_correction_mass():
    target = np.array([.125, .625, .25], np.float64)
    proposal = np.array([.5, .25, .25], np.float64)
    np.testing.assert_array_equal(correction_distribution(target, proposal), [0., 1., 0.])


def test_future_confidence_values_cannot_change_actual_sampling_or_rng_commit():
    class LogitFixture:
        def __init__(self, confidence):
            self.confidence = confidence

        def draft_conditional_logits(self, result, row, previous):
            return np.array([[previous * .5, .25, -.5]], np.float32), self.confidence[row]

    receipts = []
    for confidence in ([0.] * 5, [1.] * 5, [0., 1., .5, .01, .99]):
        sampler = TerminalSampler(41017, vocabulary=3)
        work = sampler.begin_verification(seed_token=0, policy=SamplingPolicy(), counts=np.array([1, 0, 0], np.int32),
                                          remaining=8)
        proposals = work.propose(LogitFixture(confidence), None)
        assert len(proposals) == 5
        decision = work.verify(np.array([[.1, .5, -.5]] * 6, np.float32))
        work.commit(work.prepared()["digest"])
        receipts.append((proposals, decision, sampler.random.snapshot()))
    assert receipts[0] == receipts[1] == receipts[2]


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

    class Graph:
        def draft_conditional_logits(self, result, row, previous):
            base = np.array([[0.1, 0.4, -0.3, 0.9, 0.2, 0.0, -0.6, 0.3]], np.float32)
            base[0, previous] += 0.5
            return base, None

    work = sampler.begin_verification(seed_token=work.decision.token, policy=SamplingPolicy(top_p=0.95),
                                      counts=counts, remaining=6, eos_ids={7}, logit_bias={2: 1.25, 5: -0.5})
    proposals = work.propose(Graph(), None)
    assert list(proposals) == gold["verify"]["proposals"]
    target = np.array(gold["verify"]["target"], np.float32)
    d = work.verify(target)
    assert [d.accepted_drafts, list(d.output_ids), d.pending_token, d.stop_reason] == gold["verify"]["decision"]
    assert work.prepared()["digest"] == gold["verify"]["digest"]
    work.commit(work.prepared()["digest"])
    assert sampler.random.snapshot() == gold["final_rng"]["snapshot"]


def test_full_vocabulary_device_logits_stay_on_device():
    # Full 129,280-token rows arriving as FP32 CUDA tensors (the vocabulary
    # head's output) are sampled without a host copy of the row.
    sampler = TerminalSampler(1017)
    logits = torch.full((1, 129280), -80., dtype=torch.float32, device="cuda")
    logits[0, 7:9] = torch.tensor([1., 0.])
    counts = np.zeros(129280, np.int32)
    work = sampler.begin_seed(logits, policy=SamplingPolicy(), counts=counts, remaining=10)
    assert work.decision.token in (7, 8)
    work.abort()
    work = sampler.begin_seed(logits, policy=SamplingPolicy(temperature=0), counts=counts, remaining=1)
    assert work.decision.output_ids == (7,) and work.decision.stop_reason == "length"
    work.commit(work.prepared()["digest"])
