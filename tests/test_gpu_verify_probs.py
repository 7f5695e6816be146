"""dsr_verify_probs (verify_drafts, src/deepseekrpc/sampling.py:247-294, over
float64 rows already on the device) against the oracle's verify_probs on
the same rows and uniforms.

Every comparison is exact: the rows are the oracle's own inputs, the accept
ratio is one IEEE division as in NumPy, the sums checked against 1 +- 1e-10
follow NumPy's order, and the categorical draws settle any rounding-band
case with the sequential cumulative sum.  The checks cover the reference's
order of rejections (proposals, first target, tokens, then targets as the
chain reaches them), target rows whose builder failed, single-support
corrections and bonus rows (no draw), greedy requests, EOS and length
stops, and device PCG64 draws with the states written back.
"""
import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch
from oracle import pcg64_oracle as P
from oracle import sampling_oracle as O

pytestmark = pytest.mark.gpu
M64 = (1 << 64) - 1
STOPS = {None: N.STOP_NONE, "eos": N.STOP_EOS, "length": N.STOP_LENGTH}


def dist(rng, V, keep=None, scale=2.0):
    """A normalised float64 row; ``keep`` positives (the rest zero) when given."""
    x = rng.normal(0, scale, V)
    if keep is not None and keep < V:
        x[np.argsort(-x)[keep:]] = -np.inf
    e = np.exp(x - x.max())
    return e / e.sum()


class Lazy:
    """Target rows for the oracle: a failed row raises its status when read."""

    def __init__(self, rows, status):
        self.rows, self.status = rows, status

    def __len__(self):
        return len(self.rows)

    def __getitem__(self, j):
        if self.status[j] != O.OK:
            raise O.OracleError(self.status[j], "target row failed")
        return self.rows[j]


def oracle_request(tgt, drf, ids, ua, ut, greedy, limit, eos, status):
    used = {"accept": 0, "target": 0}

    def draw(domain):
        used[domain] += 1
        return float(ua[used["accept"] - 1]) if domain == "accept" else float(ut)

    try:
        acc, out, pend, stop = O.verify_probs(Lazy(tgt, status), drf, [int(t) for t in ids], draw, greedy=greedy,
                                              output_limit=limit, eos_ids=eos)
    except O.OracleError as exc:
        return dict(status=exc.code)
    return dict(status=O.OK, accepted=acc, ids=list(out), pending=-1 if pend is None else pend, stop=STOPS[stop],
                used_accept=used["accept"], used_target=used["target"])


def run(reqs, V, K, states=None):
    """One dsr_verify_probs call over ``reqs`` (dicts of numpy rows and
    controls); returns the per-request results as dicts."""
    R = len(reqs)
    cuda = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    trows = [cuda(t) if s == O.OK else None for q in reqs for t, s in zip(q["tgt"], q["status"])]
    drows = [cuda(d) for q in reqs for d in q["drf"]]
    ids = cuda(np.array([q["ids"] for q in reqs], np.int32).reshape(-1))
    eos = [q["eos"] for q in reqs]
    off = np.cumsum([0] + [len(e) for e in eos]).astype(np.int64)
    flat_eos = np.array([t for e in eos for t in e] or [0], np.int32)
    kw = dict(greedy=cuda(np.array([q["greedy"] for q in reqs], np.uint8)),
              target_status=cuda(np.array([s for q in reqs for s in q["status"]], np.int32)),
              eos_offsets=cuda(off), eos_ids=cuda(flat_eos) if off[-1] else None)
    if states is None:
        kw.update(u_accept=cuda(np.array([q["ua"] for q in reqs], np.float64).reshape(-1)),
                  u_target=cuda(np.array([q["ut"] for q in reqs], np.float64)))
    else:
        kw.update(rng_accept=states[0], rng_target=states[1])
    res = batch.verify_probs(trows, drows, ids, cuda(np.array([q["limit"] for q in reqs], np.int32)), vocab=V,
                             requests=R, **kw)
    host = {f: getattr(res, f).cpu().numpy() for f in ("status", "accepted", "ids", "count", "pending", "stop",
                                                       "used_accept", "used_target")}
    out = []
    for r in range(R):
        got = dict(status=int(host["status"][r]))
        if got["status"] == N.OK:
            got.update(accepted=int(host["accepted"][r]), ids=host["ids"][r][:host["count"][r]].tolist(),
                       pending=int(host["pending"][r]), stop=int(host["stop"][r]),
                       used_accept=int(host["used_accept"][r]), used_target=int(host["used_target"][r]))
        out.append(got)
    return out


def request(rng, V, K, *, greedy=False, limit=1 << 20, eos=(), alike=0.9, keep=None):
    """Drafts drawn from their own rows; targets close to the drafts (``alike``
    of their mass shared) so that chains accept some drafts and reject
    others."""
    drf = [dist(rng, V, keep) for _ in range(K)]
    tgt = []
    for j in range(K + 1):
        t = dist(rng, V, keep)
        if j < K:
            t = alike * drf[j] + (1 - alike) * t
            t = t / t.sum()
        tgt.append(t)
    ids = [int(rng.choice(V, p=d)) for d in drf]
    return dict(tgt=tgt, drf=drf, ids=ids, ua=rng.random(K).tolist(), ut=float(rng.random()), greedy=greedy,
                limit=limit, eos=list(eos), status=[O.OK] * (K + 1))


def check(reqs, V, K):
    got = run(reqs, V, K)
    for r, q in enumerate(reqs):
        want = oracle_request(q["tgt"], q["drf"], q["ids"], q["ua"], q["ut"], q["greedy"], q["limit"], q["eos"],
                              q["status"])
        assert got[r] == want, (r, got[r], want)
    return got


# Vocabularies whose last 8,192-entry buffer is full (8192), a pairwise tree
# (129280: 6,400 entries), a plain running sum (8193: 1 entry; 16390: 6).
@pytest.mark.parametrize("K,V", [(0, 129280), (1, 129280), (3, 129280), (5, 129280), (5, 1000), (2, 7), (4, 8192),
                                 (3, 8193), (2, 16390)])
def test_random_requests_match_the_oracle(K, V):
    rng = np.random.default_rng(900 + 10 * K + V % 97)
    reqs = []
    for r in range(12):
        q = request(rng, V, K, greedy=r % 5 == 4, alike=[0.0, 0.5, 0.9, 0.99][r % 4],
                    keep=[None, 50, 1, None][r % 4] if V > 50 else None)
        if r % 6 == 1 and K:
            q["eos"] = [q["ids"][min(1, K - 1)], V - 1]         # EOS inside the drafts
        if r % 6 == 3:
            q["limit"] = 1 + r % 3                             # length stops
        reqs.append(q)
    got = check(reqs, V, K)
    if K and V > 50:
        acc = [g["accepted"] for g in got if g["status"] == N.OK]
        assert min(acc) < K and max(acc) > 0, acc          # both rejections and acceptances


def test_single_support_draws_nothing():
    """A one-hot bonus row and a correction with one positive entry decide
    without a target draw (sampling.py:120-122)."""
    rng = np.random.default_rng(31)
    V, K = 4096, 2
    a = request(rng, V, K, alike=1.0)              # targets equal the drafts: every draft accepted
    a["tgt"][K] = np.eye(V)[17]                    # one-hot bonus row
    b = request(rng, V, K)
    t = b["drf"][0].copy()                         # target 0 = draft 0 with mass moved onto token 5 only
    x = b["ids"][0]
    shift = t[x] * 0.5
    t[x] -= shift
    t[5 if x != 5 else 6] += shift
    b["tgt"][0] = t
    b["ua"][0] = 0.999                             # rejects (ratio 0.5)
    got = check([a, b], V, K)
    assert got[0]["ids"][-1] == 17 and got[0]["used_target"] == 0
    assert got[1]["accepted"] == 0 and got[1]["used_target"] == 0


def test_errors_in_the_reference_order():
    rng = np.random.default_rng(41)
    V, K = 2048, 3
    reqs = []
    q = request(rng, V, K)                          # 0: draft 1 off by 2e-10 and target 0 negative: draft first
    q["drf"][1] = q["drf"][1] * (1 + 2e-10)
    q["tgt"][0] = q["tgt"][0].copy()
    q["tgt"][0][3] = -1e-300
    reqs.append(q)
    q = request(rng, V, K)                          # 1: target 0 negative
    q["tgt"][0] = q["tgt"][0].copy()
    q["tgt"][0][3] = -1e-300
    reqs.append(q)
    q = request(rng, V, K, alike=1.0)               # 2: target 2 off-sum, reached (every draft accepted)
    q["tgt"][2] = q["tgt"][2] * (1 + 1e-9)
    reqs.append(q)
    q = request(rng, V, K, alike=0.0)               # 3: target 2 off-sum, never reached (draft 0 rejected)
    q["ua"][0] = 0.9999999
    q["tgt"][0][q["ids"][0]] = 0.0
    q["tgt"][0] /= q["tgt"][0].sum()
    q["tgt"][2] = q["tgt"][2] * (1 + 1e-9)
    reqs.append(q)
    q = request(rng, V, K, alike=1.0)               # 4: target 1's builder failed, reached
    q["status"][1] = O.E_NO_MASS
    reqs.append(q)
    q = request(rng, V, K, alike=1.0)               # 5: the bonus row's builder failed
    q["status"][K] = O.E_MASKED
    reqs.append(q)
    q = request(rng, V, K)                          # 6: a draft id with zero draft probability
    q["drf"][0] = q["drf"][0].copy()
    z = int(np.argmin(q["drf"][0]))
    q["drf"][0][z] = 0.0
    q["drf"][0] /= q["drf"][0].sum()
    q["ids"][0] = z
    reqs.append(q)
    q = request(rng, V, K, eos=[V])                 # 7: an EOS id out of range
    reqs.append(q)
    q = request(rng, V, K, alike=1.0)               # 8: a bonus draw with an invalid uniform
    q["ut"] = 1.0
    reqs.append(q)
    q = request(rng, V, K, alike=1.0, greedy=True)  # 9: greedy, target 1 failed and reached
    q["status"][1] = O.E_LOGITS
    reqs.append(q)
    got = check(reqs, V, K)
    codes = [g["status"] for g in got]
    assert codes[:3] == [N.E_DISTRIBUTION] * 3 and codes[3] == N.OK
    assert codes[4] == N.E_NO_MASS and codes[5] == N.E_MASKED
    assert codes[6] == N.E_PROPOSAL_ZERO and codes[7] == N.E_TOKEN and codes[8] == N.E_UNIFORM
    assert codes[9] in (N.OK, N.E_LOGITS)            # greedy: reached only if target 0's argmax is draft 0


def test_device_draws_advance_the_states():
    rng = np.random.default_rng(51)
    V, K, R = 129280, 4, 10
    reqs = [request(rng, V, K, alike=[0.3, 0.9, 0.99][r % 3], greedy=r == 7) for r in range(R)]
    gens = [(np.random.default_rng(600 + 2 * r), np.random.default_rng(601 + 2 * r)) for r in range(R)]
    acc = batch.pcg64_states([g[0] for g in gens])
    tgt = batch.pcg64_states([g[1] for g in gens])
    before = (acc.cpu().numpy().view(np.uint64).copy(), tgt.cpu().numpy().view(np.uint64).copy())
    got = run(reqs, V, K, states=(acc, tgt))
    after = (acc.cpu().numpy().view(np.uint64), tgt.cpu().numpy().view(np.uint64))
    for r, q in enumerate(reqs):
        words = [[int(w) for w in b[r]] for b in before]
        seeds = [(w[0] | (w[1] << 64), w[2] | (w[3] << 64)) for w in words]
        _, ua = P.draws(*seeds[0], K)
        _, (ut,) = P.draws(*seeds[1], 1)
        want = oracle_request(q["tgt"], q["drf"], q["ids"], ua, ut, q["greedy"], q["limit"], q["eos"], q["status"])
        assert got[r] == want, (r, got[r], want)
        for d, n in ((0, want["used_accept"]), (1, want["used_target"])):
            s, _ = P.draws(*seeds[d], n)
            assert (int(after[d][r, 0]), int(after[d][r, 1])) == (s & M64, s >> 64), (r, d)
    assert sum(g["used_accept"] for g in got) > R and sum(g["used_target"] for g in got) > 0
    assert got[7]["used_accept"] == 0 and got[7]["used_target"] == 0


@pytest.mark.parametrize("V", [129280, 8192, 8193, 16390, 300])
def test_uniforms_on_cell_edges(V):
    """Target uniforms placed on the oracle's CDF cell edges (and one ulp to
    either side) of a bonus row and of a correction: the decision sits inside
    the rounding band of the chunk sums, and the sequential cumulative sum
    (np.cumsum, then searchsorted right) must settle it exactly."""
    rng = np.random.default_rng(61 + V)
    K = 1
    reqs = []
    for trial in range(6):
        bonus = trial % 2 == 0
        q = request(rng, V, K, alike=1.0 if bonus else 0.0)
        if not bonus:                               # draft 0 rejected: ratio 0
            t = q["tgt"][0].copy()
            t[q["ids"][0]] = 0.0
            q["tgt"][0] = t / t.sum()
            q["ua"][0] = 0.5
            row = O.correction(q["tgt"][0], q["drf"][0])
        else:
            row = q["tgt"][K]
        c = np.cumsum(row, dtype=np.float64)
        c /= c[-1]
        i = int(rng.integers(V // 4, V - 1))
        edge = float(c[i])
        q["ut"] = [edge, float(np.nextafter(edge, 0.0)), float(np.nextafter(edge, 1.0))][trial // 2]
        if not 0.0 <= q["ut"] < 1.0:
            q["ut"] = 0.5
        reqs.append(q)
    check(reqs, V, K)
