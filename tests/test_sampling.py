"""The reference's sampling law on the drop-in API, computed by the HIP library.

The law's cases live in tests/sampling_law.py (data from the reference's
tests, checkers written here); this file runs them through
``deepseekrpc_amd.sampling`` and adds the RNG-domain behaviour the reference
pins: transactional draws, commit / abort, snapshot and restore
(src/deepseekrpc/sampling.py:142-231, tests/test_sampling.py:98-146).
"""
from copy import deepcopy

import numpy as np
import pytest

import sampling_law as law
from deepseekrpc_amd.jsonutil import ValidationError
from deepseekrpc_amd.sampling import (DOMAINS, RandomStreams, SamplingPolicy, categorical, correction_distribution,
                                      verify_drafts)

pytestmark = pytest.mark.gpu


class DropIn:
    """The ``sampling_law`` adapter over the drop-in API."""
    Rejected = ValidationError

    def probs(self, logits, counts=None, generated=None, bias=None, allowed=None, **policy):
        return SamplingPolicy(**policy).probabilities(logits, counts=counts, generated_counts=generated,
                                                      logit_bias=bias, allowed=allowed)

    def draw(self, p, u):
        return categorical(p, u if callable(u) else (lambda: u))

    def residual(self, p, q):
        return correction_distribution(p, q)

    def verify(self, targets, proposals, ids, draws, *, greedy, limit, eos=frozenset()):
        d = verify_drafts(targets, proposals, ids, draws, greedy=greedy, output_limit=limit, eos_ids=eos)
        assert d.accepted_target_rows == 1 + d.accepted_drafts
        return d.accepted_drafts, d.output_ids, d.pending_token, d.stop_reason


@pytest.mark.parametrize("name", sorted(law.LAWS))
def test_reference_law(name):
    law.LAWS[name](DropIn())


def test_two_token_joint_law():
    law.check_two_token_joint_law(DropIn())


def test_bool_temperature_is_rejected():
    with pytest.raises(ValidationError):
        SamplingPolicy(temperature=True)


def _draw_all(transaction, per_domain):
    return {domain: [transaction.random(domain) for _ in range(per_domain)] for domain in DOMAINS}


def test_committed_draws_persist_and_abort_restores_every_domain():
    streams = RandomStreams(42)
    initial = streams.snapshot()
    txn = streams.begin()
    for _ in range(5):
        txn.random("draft")
    after_proposals = txn.prepared_state()["domains"]["draft"]
    # A sampled rejection at the first draft takes one accept draw; its
    # residual (0, 1) has one positive entry and takes no target draw.
    d = verify_drafts([np.array([0., 1.])] * 6, [np.array([.5, .5])] * 5, [0] * 5, txn, greedy=False,
                      output_limit=10)
    assert (d.accepted_drafts, d.output_ids) == (0, (1,))
    txn.commit()
    committed = streams.snapshot()
    assert committed["domains"]["draft"] == after_proposals
    assert committed != initial
    txn = streams.begin()
    _draw_all(txn, 1)
    with pytest.raises(ValidationError, match="idle"):
        streams.snapshot()
    txn.abort()
    assert streams.snapshot() == committed


def test_greedy_verification_leaves_the_streams_untouched():
    streams = RandomStreams(1017)
    initial = streams.snapshot()
    txn = streams.begin()
    d = verify_drafts([np.array([.2, .8])] * 6, [np.array([.5, .5])] * 5, [0] * 5, txn, greedy=True, output_limit=5)
    assert d.output_ids == (1,)
    txn.commit()
    assert streams.snapshot() == initial


def test_restore_validates_every_domain_before_replacing_any():
    source, target = RandomStreams(9), RandomStreams(0)
    saved = source.snapshot()
    broken = deepcopy(saved)
    broken["domains"]["accept"]["increment"] = "0" * 32        # an even PCG64 increment
    untouched = target.snapshot()
    with pytest.raises(ValidationError, match="odd"):
        target.restore(broken)
    assert target.snapshot() == untouched
    target.restore(saved)
    a, b = source.begin(), target.begin()
    assert _draw_all(a, 5) == _draw_all(b, 5)
    assert a.commit() == b.commit()


def test_transaction_window_and_closed_guards():
    txn = RandomStreams(3).begin()
    for _ in range(64):
        txn.random("target")
    with pytest.raises(ValidationError, match="window"):
        txn.random("target")
    with pytest.raises(ValidationError):
        txn.random("nonsense")
    txn.abort()
    with pytest.raises(ValidationError, match="closed"):
        txn.commit()


def test_preview_reads_the_next_draw_without_advancing():
    streams = RandomStreams(77)
    txn = streams.begin()
    for domain in DOMAINS:
        upcoming = txn._preview(domain)
        assert txn._preview(domain) == upcoming
        assert txn.random(domain) == upcoming
    txn.abort()
