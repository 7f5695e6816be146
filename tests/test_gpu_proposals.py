"""Draft proposals drawn on the device without a host round trip per row.

A graph that offers ``draft_conditional_logits_device`` gets the previous
token as a device tensor, and each proposal row is one launch that draws from
the ``draft`` domain's PCG64 state on the device (batch.propose_rows).  The
chain must equal the host loop (one row per round trip, the uniform taken on
the host) and the oracle: the same proposals, float64 distributions within
1e-12 relative, the same RNG snapshot, the same cut at an EOS
(terminal_sampling.py:138-161).
"""
import numpy as np
import pytest
import torch

from deepseekrpc_amd import batch
from deepseekrpc_amd.jsonutil import ValidationError
from deepseekrpc_amd.sampling import SamplingPolicy
from deepseekrpc_amd.terminal_sampling import TerminalSampler
from oracle import sampling_oracle as O

pytestmark = pytest.mark.gpu
V = 129280
DEV = "cuda"


class MarkovRows:
    """Five base rows; the previous token's logit is raised by ``bump``.
    Host and device variants compute the same float32 values."""

    def __init__(self, seed, bump=4.0, poison=None):
        rng = np.random.default_rng(seed)
        self.base = rng.normal(0, 2, (5, V)).astype(np.float32)
        self.base_dev = torch.from_numpy(self.base).to(DEV)
        self.bump = np.float32(bump)
        self.poison = poison   # a position whose row is made non-finite
        self.host_calls, self.device_calls = [], []

    def host_row(self, position, previous):
        row = self.base[position].copy()
        row[previous] += self.bump
        if position == self.poison:
            row[7] = np.nan
        return row

    def draft_conditional_logits(self, result, row, previous):
        self.host_calls.append((row, previous))
        return self.host_row(row, previous)[None], None


class DeviceMarkovRows(MarkovRows):
    def draft_conditional_logits_device(self, result, row, previous):
        self.device_calls.append(row)
        out = self.base_dev[row].clone()
        out.index_add_(0, previous.long(), torch.full((1,), float(self.bump), device=DEV))
        if row == self.poison:
            out[7] = float("nan")
        return out.reshape(1, V), None


POLICIES = [dict(temperature=0.7, top_k=50, top_p=0.9), dict(temperature=1.0), dict(temperature=0.0, top_k=5),
            dict(temperature=1.2, top_p=0.8, repetition_penalty=1.3, presence_penalty=0.4)]


def history():
    counts = np.zeros(V, np.int32)
    counts[[3, 77, 5000, 129279]] = [2, 1, 1, 3]
    return counts


def run(graph_cls, seed, policy, eos=frozenset(), poison=None):
    sampler = TerminalSampler(900 + seed)
    graph = graph_cls(seed, poison=poison)
    work = sampler.begin_verification(seed_token=77, policy=SamplingPolicy(**policy), counts=history(),
                                      remaining=9, eos_ids=eos)
    proposals = work.propose(graph, None)
    rows = [r.cpu().numpy() for r in work.proposal_rows]
    state = work.transaction.prepared_state()
    work.abort()
    return proposals, rows, state, graph, sampler


def oracle_chain(seed, policy, eos=frozenset()):
    """The reference's loop on the CPU: each row conditioned on the previous
    token and on the prefix counts, the draft uniform drawn only if needed."""
    sampler = TerminalSampler(900 + seed)
    txn = sampler.random.begin()
    graph = MarkovRows(seed)
    counts = history()
    previous, out, rows = 77, [], []
    for position in range(5):
        c = counts.copy()
        for t in out:
            c[t] += 1
        row = graph.host_row(position, previous)
        upcoming = txn._preview("draft")
        ref = O.sample_row(row, O.Policy(**policy), upcoming, c, c)
        assert ref.status == 0
        if ref.consumed:
            assert txn.random("draft") == upcoming
        out.append(ref.token)
        rows.append(ref.probs)
        previous = ref.token
        if ref.token in eos:
            break
    state = txn.prepared_state()
    txn.abort()
    return tuple(out), state, rows


@pytest.mark.parametrize("k", range(len(POLICIES)))
def test_device_chain_equals_host_loop_and_oracle(k):
    policy = POLICIES[k]
    dev_ids, dev_rows, dev_state, graph, _ = run(DeviceMarkovRows, k, policy)
    host_ids, host_rows, host_state, _, _ = run(MarkovRows, k, policy)
    assert graph.device_calls == [0, 1, 2, 3, 4] and graph.host_calls == []
    assert dev_ids == host_ids and dev_state == host_state
    # Without penalties the host loop's first row carries no history table
    # and may run on another kernel, so the float64 rows agree to 1e-12.
    for a, b in zip(dev_rows, host_rows):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-300)
    want_ids, want_state, want_rows = oracle_chain(k, policy)
    assert dev_ids == want_ids and dev_state == want_state
    for a, b in zip(dev_rows, want_rows):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-300)


def test_an_eos_proposal_cuts_the_chain_and_its_draws():
    policy = POLICIES[0]
    full, _, _, _, _ = run(DeviceMarkovRows, 11, policy)
    eos = frozenset({full[1]}) if full[1] not in full[:1] else frozenset({full[2]})
    dev_ids, _, dev_state, graph, _ = run(DeviceMarkovRows, 11, policy, eos)
    host_ids, _, host_state, _, _ = run(MarkovRows, 11, policy, eos)
    assert len(dev_ids) < 5 and dev_ids[-1] in eos
    assert graph.device_calls == [0, 1, 2, 3, 4]     # later rows were computed speculatively
    assert (dev_ids, dev_state) == (host_ids, host_state) == oracle_chain(11, policy, eos)[:2]


def test_non_finite_row_aborts_and_restores_the_domains():
    for cls in (DeviceMarkovRows, MarkovRows):
        sampler = TerminalSampler(5)
        initial = sampler.random.snapshot()
        work = sampler.begin_verification(seed_token=77, policy=SamplingPolicy(), counts=history(), remaining=9)
        with pytest.raises(ValidationError, match="vocabulary window"):
            work.propose(cls(5, poison=2), None)
        assert sampler.active is None and sampler.random.snapshot() == initial


def test_chain_primitive_keeps_speculative_rows_and_states():
    graph = DeviceMarkovRows(3)
    gen = np.random.default_rng(44)
    state = batch.pcg64_states([gen], DEV)
    start = state.clone()
    seed = torch.tensor([9], dtype=torch.int32, device=DEV)
    chain = batch.propose_rows(lambda j, prev: graph.draft_conditional_logits_device(None, j, prev)[0], seed, 5,
                               dict(temperature=0.8, top_k=20), state)
    ids, rows, draws, final, failed = batch.finish_proposals(chain, eos_ids=())
    assert failed is None and len(ids) == 5 and rows.shape == (5, V) and draws == 5
    assert torch.equal(chain.states[0], start[0]) and torch.equal(final, state)
    # Each row's state advanced by exactly its one draw.
    s0 = start.cpu().numpy().view(np.uint64)[0]
    host = np.random.Generator(np.random.PCG64(0))
    st = host.bit_generator.state
    st["state"] = {"state": int(s0[0]) | (int(s0[1]) << 64), "inc": int(s0[2]) | (int(s0[3]) << 64)}
    host.bit_generator.state = st
    words = chain.states.cpu().numpy().view(np.uint64)
    for j in range(5):
        host.random()
        assert int(words[j + 1, 0]) | (int(words[j + 1, 1]) << 64) == host.bit_generator.state["state"]["state"]


@pytest.mark.parametrize("cls", [DeviceMarkovRows, MarkovRows])
def test_a_history_the_prefix_pushes_past_the_limit_fails_at_that_row(cls):
    """Without penalties the rows carry no history table until the prefix
    could push the counts past 2^20 (sampling.py:55-58): counts summing to
    2^20 - 2 let rows 0-2 through, and row 3 fails with the counts message."""
    limit = 1048576
    counts = np.zeros(V, np.int32)
    counts[77] = limit - 2
    sampler = TerminalSampler(31)
    initial = sampler.random.snapshot()
    work = sampler.begin_verification(seed_token=77, policy=SamplingPolicy(**POLICIES[0]), counts=counts,
                                      remaining=9)
    graph = cls(31)
    with pytest.raises(ValidationError, match="frequency counts"):
        work.propose(graph, None)
    assert sampler.active is None and sampler.random.snapshot() == initial
    if cls is MarkovRows:
        assert [row for row, _ in graph.host_calls] == [0, 1, 2, 3]


def test_rows_below_the_limit_match_the_oracle_without_a_table():
    """The same chain one count lower stays within 2^20 at every row: its
    proposals and RNG state are the oracle's."""
    limit = 1048576
    counts = np.zeros(V, np.int32)
    counts[77] = limit - 4
    sampler = TerminalSampler(32)
    work = sampler.begin_verification(seed_token=77, policy=SamplingPolicy(**POLICIES[0]), counts=counts,
                                      remaining=9)
    graph = DeviceMarkovRows(32)
    proposals = work.propose(graph, None)
    state = work.transaction.prepared_state()
    work.abort()
    txn = TerminalSampler(32).random.begin()
    host = MarkovRows(32)
    previous, want = 77, []
    for position in range(5):
        c = counts.copy()
        for t in want:
            c[t] += 1
        upcoming = txn._preview("draft")
        ref = O.sample_row(host.host_row(position, previous), O.Policy(**POLICIES[0]), upcoming, c, c)
        assert ref.status == 0
        if ref.consumed:
            txn.random("draft")
        want.append(ref.token)
        previous = ref.token
    assert proposals == tuple(want) and state == txn.prepared_state()
    txn.abort()


class FailingPastRows(DeviceMarkovRows):
    """Raises for every row from ``fail_from`` on, as a graph that cannot
    make rows past a stop token might."""

    def __init__(self, seed, fail_from, poison=None):
        super().__init__(seed, poison=poison)
        self.fail_from = fail_from

    def draft_conditional_logits_device(self, result, row, previous):
        if row >= self.fail_from:
            self.device_calls.append(row)
            raise RuntimeError(f"no draft row {row}")
        return super().draft_conditional_logits_device(result, row, previous)


def test_a_row_the_graph_cannot_make_past_an_eos_is_not_needed():
    """The reference never asks the graph for a row after an EOS proposal
    (terminal_sampling.py:146-158): the device chain asks speculatively, so
    an error there is dropped when an earlier row is a stop token, and
    raised (aborting the transaction) when that row is kept."""
    policy = POLICIES[0]
    full, _, _, _, _ = run(DeviceMarkovRows, 11, policy)
    eos = frozenset({full[1]}) if full[1] not in full[:1] else frozenset({full[2]})
    cut = len(run(DeviceMarkovRows, 11, policy, eos)[0])
    sampler = TerminalSampler(900 + 11)
    work = sampler.begin_verification(seed_token=77, policy=SamplingPolicy(**policy), counts=history(),
                                      remaining=9, eos_ids=eos)
    graph = FailingPastRows(11, fail_from=cut)
    proposals = work.propose(graph, None)
    state = work.transaction.prepared_state()
    work.abort()
    assert graph.device_calls == list(range(cut + 1))   # the chain stopped at the failing row
    assert (proposals, state) == oracle_chain(11, policy, eos)[:2]
    # The same failure on a row the chain keeps: raised, and the domains restored.
    sampler = TerminalSampler(900 + 11)
    initial = sampler.random.snapshot()
    work = sampler.begin_verification(seed_token=77, policy=SamplingPolicy(**policy), counts=history(),
                                      remaining=9)
    with pytest.raises(RuntimeError, match=f"no draft row {cut}"):
        work.propose(FailingPastRows(11, fail_from=cut), None)
    assert sampler.active is None and sampler.random.snapshot() == initial
