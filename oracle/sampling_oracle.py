"""CPU float64 oracle for the token-sampling hot path.

TEST INFRASTRUCTURE ONLY.  This module is the oracle that the HIP path is
compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package never
does, and it is never the thing that is measured or shipped.

It restates, step for step, the NumPy float64 arithmetic of the reference
sampler (Protonburn35/DeepSeekRPC):

* ``probabilities``   -> src/deepseekrpc/sampling.py:48-106
* ``validate_distribution`` -> src/deepseekrpc/sampling.py:109-115
* ``categorical``     -> src/deepseekrpc/sampling.py:118-128
* ``correction``      -> src/deepseekrpc/sampling.py:131-139
* ``verify``          -> src/deepseekrpc/sampling.py:247-294 together with the
  conditional target / proposal construction of
  src/deepseekrpc/terminal_sampling.py:127-136,138-161,170-183,234-244

The operation order is the reference's own, because the exact float64 result
depends on it: the float64 copy, repetition (divide non-negative, multiply
negative), ``presence*(g>0) + frequency*g`` built as one vector and then
subtracted, bias, mask, greedy argmax, ``-max``, ``/T``, stable top-k,
``exp``, ``/sum`` (NumPy pairwise sum), min-p, stable top-p with the exclusive
prefix ``cumsum - r``, and the final ``/sum``.  ``categorical`` uses the
sequential float64 ``cumsum`` divided by its last element and the first entry
strictly greater than ``u``.

Besides the reference's outputs each function returns the *decision margins*
(how far a threshold decision was from flipping).  The GPU path computes the
same decisions with a different exp implementation and summation order, so a
decision is only comparable bit-for-bit when its margin exceeds the rounding
bound; the margins let the parity tests say which rows are in that regime.

Pinning (see tests/test_oracle_*.py): the reference's known-answer tests
(tests/test_sampling.py:22-53,56-107, tests/test_sampling_reference_law.py,
src/deepseekrpc/cluster_probe.py:22-56) re-expressed against this module,
closed forms (softmax, nucleus, rejection-sampling identity), exact-rational
brute force on tiny vocabularies, and golden vectors written by importing the
reference's own sampling module (tests/golden/).
"""
from __future__ import annotations

from dataclasses import dataclass, field
import math

import numpy as np

VOCAB = 129280
MAX_COUNT = 1048576

# Error codes shared with the native library's per-row status (the messages
# are those of the reference's ValidationError raises).
OK = 0
E_LOGITS = 1          # sampling.py:50-52
E_MASKED = 2          # sampling.py:80-81
E_NO_MASS = 3         # sampling.py:104-105
E_UNIFORM = 4         # sampling.py:124-125
E_COUNTS = 5          # sampling.py:56-58,63-65
E_BIAS = 6            # sampling.py:70-74
E_PROPOSAL_ZERO = 7   # sampling.py:276-277
E_CORRECTION = 8      # sampling.py:137-138
E_TOKEN = 9           # sampling.py:271-272
E_DISTRIBUTION = 10   # sampling.py:111-114
E_POLICY = 11         # sampling.py:38-43
E_GENERATED = 12      # sampling.py:62-65,67-68


class OracleError(ValueError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


@dataclass(frozen=True)
class Policy:
    """The seven sampling controls (sampling.py:29-36)."""
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0


@dataclass
class Diagnostics:
    """Side information for parity: the surviving set and decision margins."""
    greedy: bool = False
    topk_kept: np.ndarray | None = None     # bool [V]: finite after the top-k step
    margin_minp: float = math.inf
    margin_topp: float = math.inf
    extras: dict = field(default_factory=dict)


def _check_logits(values):
    # sampling.py:49-52
    if (values.ndim != 1 or not 1 <= len(values) <= VOCAB or values.dtype not in (np.float32, np.float64)
            or np.isnan(values).any() or np.isposinf(values).any()):
        raise OracleError(E_LOGITS, "sampling needs one bounded finite-or-masked floating logit vector")


def _check_counts(counts, shape):
    # sampling.py:55-58
    counts = np.asarray(counts)
    if (counts.shape != shape or counts.dtype not in (np.int32, np.int64) or (counts < 0).any()
            or (counts > MAX_COUNT).any() or int(counts.sum(dtype=np.int64)) > MAX_COUNT):
        raise OracleError(E_COUNTS, "sampling frequency counts do not match the vocabulary")
    return counts


def adjusted_logits(logits, policy, counts=None, generated_counts=None, logit_bias=None, allowed=None):
    """Steps 1-6 of sampling.py:48-81: float64 copy, penalties, bias, mask."""
    values = np.asarray(logits)
    _check_logits(values)
    v = np.array(values, dtype=np.float64, copy=True)                       # :53
    if counts is not None:
        counts = _check_counts(counts, v.shape)
        hit = counts > 0                                                     # :59
        sub = v[hit]
        v[hit] = np.where(sub >= 0, sub / policy.repetition_penalty, sub * policy.repetition_penalty)  # :60-61
        gen = counts if generated_counts is None else np.asarray(generated_counts)   # :62
        if (gen.shape != v.shape or gen.dtype not in (np.int32, np.int64) or (gen < 0).any()
                or (gen > counts).any()):
            raise OracleError(E_GENERATED, "generated token counts must be a subset of complete sampling history")
        # One float64 penalty vector, then one subtraction (:66).
        penalty = policy.presence_penalty * (gen > 0) + policy.frequency_penalty * gen
        v -= penalty
    elif generated_counts is not None:                                       # :67-68
        raise OracleError(E_GENERATED, "generated counts require complete repetition-penalty history")
    if logit_bias is not None:                                               # :69-74
        if not isinstance(logit_bias, dict) or len(logit_bias) > len(v):
            raise OracleError(E_BIAS, "invalid logit bias mapping")
        for token, bias in logit_bias.items():
            if type(token) is not int or not 0 <= token < len(v):
                raise OracleError(E_BIAS, "biased token out of range")
            if isinstance(bias, bool) or not isinstance(bias, (int, float)) or not math.isfinite(bias) \
                    or not -100 <= bias <= 100:
                raise OracleError(E_BIAS, "invalid logit bias")
            v[token] += float(bias)
    if allowed is not None:                                                  # :75-79
        allowed = np.asarray(allowed)
        if allowed.shape != v.shape or allowed.dtype != np.bool_:
            raise OracleError(E_MASKED, "sampling grammar/token mask does not match the vocabulary")
        v[~allowed] = -np.inf
    if not np.isfinite(v).any():                                             # :80-81
        raise OracleError(E_MASKED, "sampling controls masked every vocabulary token")
    return v


def probabilities(logits, policy, counts=None, generated_counts=None, logit_bias=None, allowed=None,
                  diagnostics=None):
    """Full restatement of SamplingPolicy.probabilities (sampling.py:48-106)."""
    diag = diagnostics if diagnostics is not None else Diagnostics()
    v = adjusted_logits(logits, policy, counts, generated_counts, logit_bias, allowed)
    n = len(v)
    if policy.temperature == 0:                                              # :82-85
        out = np.zeros(n, dtype=np.float64)
        out[int(np.argmax(v))] = 1.0
        diag.greedy = True
        diag.topk_kept = out > 0
        return out
    v -= np.max(v)                                                           # :86
    with np.errstate(over="ignore", under="ignore"):
        v /= policy.temperature                                              # :87-88
    if policy.top_k and policy.top_k < n:                                    # :89-91
        rank = np.argsort(-v, kind="stable")
        v[rank[policy.top_k:]] = -np.inf
    diag.topk_kept = np.isfinite(v)
    r = np.exp(v)                                                            # :92
    r /= r.sum(dtype=np.float64)                                             # :93
    if policy.min_p:                                                         # :94-96
        cut = policy.min_p * np.max(r)
        live = r > 0
        if live.any():
            diag.margin_minp = float(np.min(np.abs(r[live] - cut)) / max(cut, 1e-300))
        r[r < cut] = 0.0
        r /= r.sum(dtype=np.float64)
    if policy.top_p < 1:                                                     # :97-102
        rank = np.argsort(-r, kind="stable")
        ordered = r[rank]
        prev = np.cumsum(ordered, dtype=np.float64) - ordered
        drop = prev >= policy.top_p
        drop[0] = False
        if n > 1:
            diag.margin_topp = float(np.min(np.abs(prev[1:] - policy.top_p)))
        r[rank[drop]] = 0.0
    total = r.sum(dtype=np.float64)                                          # :103-105
    if not np.isfinite(total) or total <= 0:
        raise OracleError(E_NO_MASS, "sampling controls produced no positive probability")
    return r / total                                                         # :106


def validate_distribution(p):
    """sampling.py:109-115."""
    p = np.asarray(p)
    if (p.ndim != 1 or not 1 <= len(p) <= VOCAB or p.dtype != np.float64 or not np.isfinite(p).all()
            or (p < 0).any() or not math.isclose(float(p.sum(dtype=np.float64)), 1.0, rel_tol=0, abs_tol=1e-10)):
        raise OracleError(E_DISTRIBUTION, "verifier requires a normalized complete FP64 probability vector")
    return p


def categorical(p, u):
    """sampling.py:118-128.  ``u`` is a pre-drawn uniform or a zero-argument
    callable that is only called when a draw is needed.

    Returns ``(token, consumed, margin)``.  ``consumed`` is False when the
    support has exactly one entry: the reference never calls its uniform then.
    ``margin`` is the distance of ``u`` from the nearer edge of the chosen
    CDF cell (``inf`` when no draw happened).
    """
    p = validate_distribution(p)
    support = np.flatnonzero(p)
    if len(support) == 1:
        return int(support[0]), False, math.inf
    if callable(u):
        u = u()
    if not isinstance(u, float) or not 0 <= u < 1:
        raise OracleError(E_UNIFORM, "sampling uniform must lie in [0,1)")
    c = np.cumsum(p, dtype=np.float64)
    c /= c[-1]
    token = int(np.searchsorted(c, u, side="right"))
    upper = c[token] - u
    lower = u - c[token - 1] if token > 0 else u
    return token, True, float(min(upper, lower))


def correction(target, proposal):
    """sampling.py:131-139: normalised positive part of ``p - q``."""
    target, proposal = validate_distribution(target), validate_distribution(proposal)
    if target.shape != proposal.shape:
        raise OracleError(E_CORRECTION, "target and proposal vocabulary sizes differ")
    residual = np.maximum(target - proposal, 0.0)
    total = residual.sum(dtype=np.float64)
    if total <= 0 or not np.isfinite(total):
        raise OracleError(E_CORRECTION, "a rejected proposal has no positive correction distribution")
    return residual / total


# ---------------------------------------------------------------------------
# Row-level drivers used by the parity tests and the CPU baseline.


@dataclass
class RowResult:
    token: int = -1
    consumed: bool = False
    status: int = OK
    probs: np.ndarray | None = None
    topk_kept: np.ndarray | None = None
    margin: float = math.inf      # smallest decision margin on this row


def dense_counts(table, vocab):
    """Expand a sparse ``(ids, counts, generated)`` table to dense int32 vectors."""
    ids, cnt, gen = table
    counts = np.zeros(vocab, np.int32)
    generated = np.zeros(vocab, np.int32)
    counts[np.asarray(ids, np.int64)] = cnt
    generated[np.asarray(ids, np.int64)] = gen
    return counts, generated


def sample_row(logits, policy, uniform, counts=None, generated_counts=None, logit_bias=None, allowed=None,
               keep_probs=True):
    """One terminal draw: ``categorical(probabilities(...), u)`` (terminal_sampling.py:83-95)."""
    res = RowResult()
    diag = Diagnostics()
    try:
        p = probabilities(logits, policy, counts, generated_counts, logit_bias, allowed, diag)
        res.token, res.consumed, m_draw = categorical(p, uniform)
    except OracleError as exc:
        res.status = exc.code
        return res
    res.topk_kept = diag.topk_kept
    res.margin = min(m_draw, diag.margin_topp, diag.margin_minp)
    if keep_probs:
        res.probs = p
    return res


@dataclass
class VerifyResult:
    accepted: int = 0
    output_ids: tuple = ()
    pending: int | None = None
    stop: str | None = None
    used_accept: int = 0
    used_target: int = 0
    status: int = OK
    margin: float = math.inf


def verify_probs(target_rows, proposal_rows, proposal_ids, draw, *, greedy, output_limit, eos_ids=(), margins=None):
    """sampling.py:247-294 on probability rows.

    ``target_rows`` may be lazy (indexing evaluates a row); ``draw(domain)``
    returns the next uniform of ``"accept"`` or ``"target"`` and is called
    exactly when the reference calls ``transaction.random``.  Returns
    ``(accepted_drafts, output_ids, pending, stop)``; decision margins are
    appended to ``margins`` when given.
    """
    margins = [] if margins is None else margins
    if not 0 <= len(proposal_ids) <= 5 or not 1 <= output_limit <= MAX_COUNT:
        raise OracleError(E_TOKEN, "proposal length or output limit out of range")
    if len(proposal_rows) != len(proposal_ids) or len(target_rows) != len(proposal_ids) + 1:
        raise OracleError(E_TOKEN, "target/proposal verification row counts differ")
    proposals = [validate_distribution(row) for row in proposal_rows]
    first = validate_distribution(target_rows[0])
    vocab = len(first)
    eos = set(int(t) for t in eos_ids)
    for t in (*proposal_ids, *eos):
        if not 0 <= int(t) < vocab:
            raise OracleError(E_TOKEN, "verification token out of range")
    output = []
    for j, x in enumerate(proposal_ids):
        p = first if j == 0 else validate_distribution(target_rows[j])
        q = proposals[j]
        if q[x] <= 0:
            raise OracleError(E_PROPOSAL_ZERO, "a proposed token has zero probability")
        if greedy:
            ok = x == int(np.argmax(p))
        else:
            u, ratio = draw("accept"), min(1.0, float(p[x] / q[x]))
            margins.append(abs(u - ratio))
            ok = u < ratio
        if not ok:
            if greedy:
                rep = int(np.argmax(p))
            else:
                rep, _, m = categorical(correction(p, q), lambda: draw("target"))
                margins.append(m)
            stop = "eos" if rep in eos else "length" if len(output) + 1 >= output_limit else None
            return j, tuple(output) + (rep,), rep, stop
        output.append(int(x))
        if x in eos or len(output) >= output_limit:
            return j + 1, tuple(output), None, "eos" if x in eos else "length"
    p = first if not proposal_ids else validate_distribution(target_rows[len(proposal_ids)])
    if greedy:
        bonus = int(np.argmax(p))
    else:
        bonus, _, m = categorical(p, lambda: draw("target"))
        margins.append(m)
    stop = "eos" if bonus in eos else "length" if len(output) + 1 >= output_limit else None
    return len(proposal_ids), tuple(output) + (bonus,), bonus, stop


def verify(target_logits, draft_logits, draft_ids, policy, u_accept, u_target, *, counts=None,
           generated_counts=None, logit_bias=None, allowed=None, eos_ids=(), output_limit=1048576):
    """Batched-row restatement of SamplingWork.verify -> verify_drafts.

    ``target_logits`` is ``[K+1, V]`` and ``draft_logits`` ``[K, V]``; row ``j``
    of both is conditioned on the accepted prefix ``draft_ids[:j]``: each
    prefix token adds one to both count vectors (terminal_sampling.py:127-136,
    234-244).  ``allowed`` is ``None`` or a ``[K+1, V]`` bool array (one mask
    per prefix).  Uniforms are pre-drawn: ``u_accept[j]`` for the j-th accept
    test and one ``u_target``; ``used_*`` count the draws the reference makes.
    """
    K = len(draft_ids)
    ids = [int(x) for x in draft_ids]
    res = VerifyResult()

    def dist(values, prefix, j):
        c = g = None
        if counts is not None:
            c = np.array(counts, copy=True)
            g = np.array(counts if generated_counts is None else generated_counts, copy=True)
            for t in prefix:
                c[t] += 1
                g[t] += 1
        mask = None if allowed is None else allowed[j]
        return probabilities(values, policy, c, g, logit_bias, mask)

    class LazyTargets:
        def __init__(self):
            self.cache = {}

        def __len__(self):
            return K + 1

        def __getitem__(self, j):
            if j not in self.cache:
                self.cache[j] = dist(target_logits[j], ids[:j], j)
            return self.cache[j]

    def draw(domain):
        if domain == "accept":
            res.used_accept += 1
            return float(u_accept[res.used_accept - 1])
        res.used_target += 1
        return float(u_target)

    try:
        proposals = [dist(draft_logits[j], ids[:j], j) for j in range(K)]
        margins = []
        res.accepted, res.output_ids, res.pending, res.stop = verify_probs(
            LazyTargets(), proposals, ids, draw, greedy=policy.temperature == 0, output_limit=output_limit,
            eos_ids=eos_ids, margins=margins)
        res.margin = min(margins, default=math.inf)
        return res
    except OracleError as exc:
        res.status = exc.code
        return res
