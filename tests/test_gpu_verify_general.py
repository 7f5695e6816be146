"""The batched verifier's general path against the oracle on conditioned requests.

Every request carries a token history (repetition, presence and frequency
penalties away from neutral), a logit bias and a different allow mask per
position, and row j of its targets and proposals is conditioned on the
accepted prefix draft_ids[:j] (each prefix token adds one to both count
vectors, terminal_sampling.py:127-136,234-244).  The decision of every
request -- status, accepted drafts, output ids, pending token, stop reason
and the draws it consumed -- must equal the oracle's
(sampling.py:247-294).  No request is waived.

Special requests: a history whose total the prefix pushes past 2^20 only at
the bonus row (reached by a greedy chain that accepts every draft: the lazy
target fails; sampling.py:264-270), the same history under a sampled policy,
a token whose own count the prefix pushes past 2^20, generated counts above
the counts, a proposal masked at its position, EOS ids among the drafts and
output limits down to one.
"""
import numpy as np
import pytest
import torch

from deepseekrpc_amd import batch
from oracle import sampling_oracle as O

pytestmark = pytest.mark.gpu

MAX = 1 << 20
STOP = {0: None, 1: "eos", 2: "length"}

POLICIES = [
    dict(temperature=0.9, repetition_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.2),
    dict(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.15, presence_penalty=-0.4,
         frequency_penalty=0.6),
    dict(temperature=1.2, top_p=0.8, min_p=0.02, repetition_penalty=0.8, frequency_penalty=-0.3),
    dict(temperature=0.0, repetition_penalty=1.5, presence_penalty=1.0, frequency_penalty=0.25),
    dict(temperature=1.0, top_k=2000, repetition_penalty=2.0, presence_penalty=2.0, frequency_penalty=-2.0),
    dict(temperature=0.5, min_p=0.05, repetition_penalty=1.05, presence_penalty=0.3),
]


def _history(rng, V, n, gen_from):
    h = rng.integers(0, V, n)
    counts = np.bincount(h, minlength=V).astype(np.int32)
    gen = np.bincount(h[gen_from:], minlength=V).astype(np.int32)
    return counts, gen


def _conditioned(counts, gen, prefix):
    c, g = counts.copy(), gen.copy()
    for t in prefix:
        c[t] += 1
        g[t] += 1
    return c, g


def _case(V, R, K, seed):
    rng = np.random.default_rng(seed)
    tgt = rng.normal(0, 2, (R, K + 1, V)).astype(np.float32)
    drf = (tgt[:, :K] + rng.normal(0, 0.5, (R, K, V))).astype(np.float32)
    pols = [dict(POLICIES[r % len(POLICIES)]) for r in range(R)]
    counts = np.zeros((R, V), np.int32)
    gens = np.zeros((R, V), np.int32)
    biases, eos, limits = [], [], []
    allowed = rng.random((R, K + 1, V)) < 0.9
    for r in range(R):
        n = int(rng.integers(8, 600))
        counts[r], gens[r] = _history(rng, V, n, int(rng.integers(0, n)))
        ids = rng.choice(V, 6, replace=False)
        biases.append({int(t): float(b) for t, b in zip(ids, (5.0, -100.0, 3.5, -7.25, 0.5, 2.0))})
        limits.append(int((10, 1, 2, 3)[r % 4]))
        eos.append([])
    # Special requests (see the module docstring).
    big = int(rng.integers(0, V))
    counts[1] = 0
    gens[1] = 0
    counts[1, big] = MAX - K + 1 - 5      # total MAX - K + 1: draft rows fit, the bonus row does not
    counts[1, (big + 1) % V] = 5
    gens[1] = counts[1]
    pols[1] = dict(temperature=0.0, repetition_penalty=1.1, presence_penalty=0.2)
    limits[1] = 10
    counts[2], gens[2] = counts[1], gens[1]
    pols[2] = dict(temperature=1.0, repetition_penalty=1.1, frequency_penalty=0.1)
    limits[2] = 10
    counts[3] = 0
    gens[3] = 0
    counts[3, big] = MAX - 1              # one token's own count: the prefix repeats it
    gens[3, big] = 3
    pols[3] = dict(temperature=0.0, presence_penalty=0.5)
    limits[3] = 10
    gens[4] = counts[4]
    hot = int(np.flatnonzero(counts[4])[0])
    gens[4, hot] = counts[4, hot] + 1     # generated above counts
    limits[5] = 10
    # A greedy proposal row is one-hot at its own argmax: greedy requests
    # draft from their target rows, so their proposals keep positive mass.
    for r in range(R):
        if pols[r]["temperature"] == 0.0:
            drf[r] = tgt[r, :K]
    return dict(tgt=tgt, drf=drf, pols=pols, counts=counts, gens=gens, biases=biases, eos=eos, limits=limits,
                allowed=allowed, big=big, rng=rng)


def _draft_ids(c, seen_tgt, seen_drf, K):
    """Draft ids drawn from each request's own conditioned proposal rows;
    greedy requests propose the argmax of their conditioned target rows (a
    chain that accepts every draft).  Request 3 repeats its heavy token, and
    request 5 proposes, at position 1, a token its mask there removes."""
    rng, R, V = c["rng"], seen_tgt.shape[0], seen_tgt.shape[2]
    ids = np.zeros((R, K), np.int32)
    for r in range(R):
        pol = O.Policy(**c["pols"][r])
        prefix = []
        for j in range(K):
            cc, gg = _conditioned(c["counts"][r], c["gens"][r], prefix)
            rows = seen_tgt[r, j] if pol.temperature == 0 else seen_drf[r, j]
            try:
                p = O.probabilities(rows, pol, cc, gg, c["biases"][r], c["allowed"][r, j])
                x = int(np.argmax(p)) if pol.temperature == 0 else O.categorical(p, float(rng.random()))[0]
            except O.OracleError:
                x = int(rng.integers(0, V))
            if r == 3:
                x = c["big"]
            prefix.append(x)
            ids[r, j] = x
    masked = np.flatnonzero(~c["allowed"][5, 1])
    ids[5, 1] = int(masked[0])
    # EOS: request 6 stops at its second draft, request 7 names an id no draft uses.
    c["eos"][6] = [int(ids[6, 1]), 0]
    c["eos"][7] = [int((ids[7].max() + 1) % V)]
    c["eos"][8] = [int(ids[8, 0])]
    return ids


def _run(V, R, K, dtype, seed):
    c = _case(V, R, K, seed)
    dev = "cuda"
    tgt = torch.from_numpy(c["tgt"]).to(dev).to(dtype)
    drf = torch.from_numpy(c["drf"]).to(dev).to(dtype)
    seen_tgt, seen_drf = tgt.float().cpu().numpy(), drf.float().cpu().numpy()
    ids = _draft_ids(c, seen_tgt, seen_drf, K)
    rng = c["rng"]
    ua, ut = rng.random((R, K)), rng.random(R)
    hist = batch.HistoryTable.from_dense(c["counts"], c["gens"], device=dev)
    bias = batch.BiasTable.from_dicts(c["biases"], device=dev)
    allow = torch.from_numpy(batch.pack_allow(c["allowed"]).view(np.int32)).to(dev)
    eos_off = torch.tensor(np.cumsum([0] + [len(e) for e in c["eos"]]), dtype=torch.int64, device=dev)
    eos_ids = torch.tensor([t for e in c["eos"] for t in e], dtype=torch.int32, device=dev)
    res = batch.verify_drafts(tgt, drf, torch.from_numpy(ids).to(dev), c["pols"], torch.from_numpy(ua).to(dev),
                              torch.from_numpy(ut).to(dev),
                              torch.tensor(c["limits"], dtype=torch.int32, device=dev),
                              history=hist, bias=bias, allow_bits=allow, eos_offsets=eos_off, eos_ids=eos_ids)
    torch.cuda.synchronize()
    assert res.args.hints == 0
    outcome = {}
    for r in range(R):
        ref = O.verify(seen_tgt[r], seen_drf[r], list(ids[r]), O.Policy(**c["pols"][r]), ua[r], float(ut[r]),
                       counts=c["counts"][r], generated_counts=c["gens"][r], logit_bias=c["biases"][r],
                       allowed=c["allowed"][r], eos_ids=tuple(c["eos"][r]), output_limit=c["limits"][r])
        n = int(res.count[r])
        got = (int(res.status[r]), int(res.accepted[r]), tuple(res.ids[r, :n].tolist()),
               None if int(res.pending[r]) < 0 else int(res.pending[r]), STOP[int(res.stop[r])],
               int(res.used_accept[r]), int(res.used_target[r]))
        if ref.status:
            want = (ref.status, 0, (), None, None, 0, 0)
        else:
            want = (0, ref.accepted, ref.output_ids, ref.pending, ref.stop, ref.used_accept, ref.used_target)
        assert got == want, (r, got, want, ref.margin)
        outcome[r] = want
    print({r: o[:3] for r, o in outcome.items()}, flush=True)
    # The special requests reached the cases they were built for.
    assert outcome[1][0] == O.E_COUNTS          # the bonus row of an all-accepting chain
    assert outcome[3][0] == O.E_COUNTS          # one token's count past the limit
    assert outcome[4][0] == O.E_GENERATED
    return outcome


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_general_conditioned_small_vocab(dtype):
    outcome = _run(5003, 24, 4, dtype, seed=301)
    assert sum(o[0] == 0 for o in outcome.values()) >= 15


def test_verify_general_conditioned_full_vocab():
    outcome = _run(129280, 12, 4, torch.float32, seed=302)
    assert sum(o[0] == 0 for o in outcome.values()) >= 7


def test_verify_general_five_drafts():
    outcome = _run(2053, 18, 5, torch.float32, seed=303)
    assert sum(o[0] == 0 for o in outcome.values()) >= 10
