"""Drop-in replacement of the reference's sampling API, computed on the GPU.

Same names, signatures, validation and error messages as the reference's
src/deepseekrpc/sampling.py:

* ``SamplingPolicy`` (:28-46) and ``probabilities`` (:48-106): validated on the
  host exactly as the reference does, then computed by ``dsr_sample_rows``;
* ``categorical`` (:118-128), ``correction_distribution`` (:131-139) and
  ``verify_drafts`` (:247-294): control flow on the host (lazy targets, one
  uniform per tested position, drawn only when needed), arithmetic by the
  ``dsr_prob_*`` kernels;
* ``RandomStreams`` / ``RandomTransaction`` (:142-231): three NumPy PCG64
  domains on the host with transactional begin/commit/abort and the same
  snapshot format.

Arrays may be NumPy arrays (uploaded; results come back as NumPy) or CUDA
tensors (kept on the device; results stay device tensors).  There is no CPU
arithmetic path: without the HIP library every computing call raises.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, field
import hashlib
import math

import numpy as np
import torch

from . import _native as N
from . import batch
from .jsonutil import ValidationError, hex_id, integer

DOMAINS = ("target", "draft", "accept")
VOCAB = 129280
MAX_COUNT = 1048576

_MESSAGES = {
    N.E_LOGITS: "sampling needs one bounded finite-or-masked floating logit vector",
    N.E_MASKED: "sampling controls masked every vocabulary token",
    N.E_NO_MASS: "sampling controls produced no positive probability",
    N.E_COUNTS: "sampling frequency counts do not match the vocabulary",
    N.E_GENERATED: "generated token counts must be a subset of complete sampling history",
    N.E_HISTORY: "history needs bounded exact integer token IDs",
    N.E_BIAS: "invalid logit bias mapping",
    N.E_UNIFORM: "sampling uniform must lie in [0,1)",
    N.E_CORRECTION: "a rejected proposal has no positive correction distribution",
    N.E_POLICY: "invalid sampling policy",
}


def _real(value, name, low, high):
    if isinstance(value, bool) or not isinstance(value, (int, float)) or not math.isfinite(value) \
            or not low <= value <= high:
        raise ValidationError(f"invalid {name}")
    return float(value)


def _device():
    return torch.device("cuda", torch.cuda.current_device())


def _on_device(values, dtype=None):
    """(device tensor, was_numpy) for a NumPy array or a CUDA tensor."""
    if isinstance(values, torch.Tensor):
        if not values.is_cuda:
            raise ValidationError("sampling tensors must live on the GPU")
        t = values.detach()
        return (t if dtype is None else t.to(dtype)).contiguous(), False
    arr = np.ascontiguousarray(values)
    return torch.from_numpy(arr).to(_device(), non_blocking=False), True


def _raise_status(code):
    raise ValidationError(_MESSAGES.get(int(code), N.status_message(int(code))))


@dataclass(frozen=True)
class SamplingPolicy:
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    def __post_init__(self):
        for name, low, high in (("temperature", 0, 100), ("top_p", 0, 1), ("min_p", 0, 1),
                                ("repetition_penalty", 0.01, 100), ("presence_penalty", -2, 2),
                                ("frequency_penalty", -2, 2)):
            object.__setattr__(self, name, _real(getattr(self, name), name, low, high))
        integer(self.top_k, "top-k", 0, VOCAB)

    def as_dict(self):
        return asdict(self)

    def _device_tensor(self, device, rows=1):
        """The policy packed for the kernels on ``device`` (``rows`` copies,
        one per row of a launch), made once per device and row count: the
        policy is immutable.  Copies and pickles leave it out."""
        cache = self.__dict__.get("_packed")
        if cache is None:
            cache = {}
            object.__setattr__(self, "_packed", cache)
        packed = cache.get((device.index, rows))
        if packed is None:
            packed = cache[(device.index, rows)] = batch.policy_tensor([self] * rows, device)
        return packed

    def __getstate__(self):
        return {k: v for k, v in self.__dict__.items() if k != "_packed"}

    def probabilities(self, logits, *, counts=None, generated_counts=None, logit_bias=None, allowed=None):
        """Adjusted, filtered and normalised float64 probabilities (sampling.py:48-106)."""
        n, device_input = _logit_vector(logits)
        table = None
        if counts is not None:
            table = _history_table(counts, generated_counts, n)
        elif generated_counts is not None:
            raise ValidationError("generated counts require complete repetition-penalty history")
        res = self._launch_row(logits, n, table, _bias_table(logit_bias, n), _allow_row(allowed, n))
        status = int(res.status.item())
        if status != N.OK:
            _raise_status(status)
        out = res.probs[0]
        return out if device_input else out.cpu().numpy()

    def _launch_row(self, logits, n, table, bias, allow, uniform=None, rng_state=None, out=None, probs="f64"):
        """One ``dsr_sample_rows`` launch over a single validated row: its
        float64 probabilities (unless ``probs`` is None; ``out`` may hold the
        per-row outputs, as ``sample_rows`` takes them), and with a pre-drawn
        ``uniform`` (a float64 device tensor of one element) or a PCG64
        ``rng_state`` (int64 ``[1, 4]``, advanced on the device only if the
        draw is needed) also its
        categorical draw and whether the draw consumed a uniform.  Nothing is
        synchronised."""
        x, _ = _on_device(logits)
        return batch.sample_rows(x.reshape(1, n), self._device_tensor(x.device), history=table, bias=bias,
                                 allow_bits=allow, uniforms=uniform, rng_state=rng_state, probs=probs, out=out)


def _bias_table(logit_bias, n, rows=1):
    """A validated logit-bias mapping as a device table, the same for each of
    ``rows`` rows (sampling.py:69-74)."""
    if logit_bias is None:
        return None
    if not isinstance(logit_bias, dict) or len(logit_bias) > n:
        raise ValidationError("invalid logit bias mapping")
    checked = {}
    for token, value in logit_bias.items():
        integer(token, "biased token", 0, n - 1)
        checked[token] = _real(value, "logit bias", -100, 100)
    return batch.BiasTable.from_dicts([checked] * rows, device=_device())


def _allow_row(allowed, n):
    """A validated boolean token mask as one packed device row of allow bits (sampling.py:75-79)."""
    if allowed is None:
        return None
    mask = np.asarray(allowed.cpu() if isinstance(allowed, torch.Tensor) else allowed)
    if mask.shape != (n,) or mask.dtype != np.bool_:
        raise ValidationError("sampling grammar/token mask does not match the vocabulary")
    return torch.from_numpy(batch.pack_allow(mask[None]).astype(np.int32)).to(_device())


def _logit_vector(logits):
    """(length, is a device tensor) of a logit vector the reference accepts
    (sampling.py:50-52); NaN / +inf in device tensors are reported by the
    kernel, in the same order."""
    if isinstance(logits, torch.Tensor):
        if logits.dim() != 1 or not 1 <= logits.numel() <= VOCAB or \
                logits.dtype not in (torch.float32, torch.float64, torch.bfloat16):
            raise ValidationError("sampling needs one bounded finite-or-masked floating logit vector")
        return logits.numel(), True
    values = np.asarray(logits)
    if (values.ndim != 1 or not 1 <= len(values) <= VOCAB or values.dtype not in (np.float32, np.float64)
            or np.isnan(values).any() or np.isposinf(values).any()):
        raise ValidationError("sampling needs one bounded finite-or-masked floating logit vector")
    return len(values), False


_COUNTS_MSG = "sampling frequency counts do not match the vocabulary"
_GENERATED_MSG = "generated token counts must be a subset of complete sampling history"


def _count_vector(x, n):
    """A count vector as a device int32 [1, n] tensor, or None if its shape or
    dtype is wrong.  Values are clamped to [-1, MAX_COUNT + 1] first, so an
    out-of-range int64 count stays out of range after the int32 cast."""
    if isinstance(x, torch.Tensor):
        t = x.detach()
        ok = t.shape == (n,) and t.dtype in (torch.int32, torch.int64)
        t = t if t.is_cuda else t.to(_device())
    else:
        arr = np.asarray(x)
        ok = arr.shape == (n,) and arr.dtype in (np.int32, np.int64)
        t = torch.from_numpy(np.ascontiguousarray(arr)).to(_device()) if ok else None
    if not ok:
        return None
    return t.clamp(-1, MAX_COUNT + 1).to(torch.int32).reshape(1, n).contiguous()


def _history_table(counts, generated_counts, n):
    """Dense counts / generated counts -> a device history table, validated in
    the reference's order (sampling.py:54-58, then :62-65) by the device
    builder."""
    c = _count_vector(counts, n)
    if c is None:
        raise ValidationError(_COUNTS_MSG)
    g = None
    if generated_counts is not None:
        g = _count_vector(generated_counts, n)
        if g is None:
            # The counts are fully validated before the generated counts are looked at.
            _, st = batch.HistoryTable.from_dense_device(c)
            if int(st.item()) != N.OK:
                _raise_status(int(st.item()))
            raise ValidationError(_GENERATED_MSG)
    table, st = batch.HistoryTable.from_dense_device(c, g)
    if int(st.item()) != N.OK:
        _raise_status(int(st.item()))
    return table


_DIST_MSG = "verifier requires a normalized complete FP64 probability vector"


def _dist_input(values):
    """A probability vector of the shape and dtype the reference accepts
    (sampling.py:109-111), as a device tensor."""
    if isinstance(values, torch.Tensor):
        ok = values.dim() == 1 and 1 <= values.numel() <= VOCAB and values.dtype == torch.float64
    else:
        values = np.asarray(values)
        ok = values.ndim == 1 and 1 <= len(values) <= VOCAB and values.dtype == np.float64
    if not ok:
        raise ValidationError(_DIST_MSG)
    return _on_device(values)[0].contiguous()


def _dist_checked(t, stats):
    """The vector's statistics checked as sampling.py:112-115 checks them."""
    total, valid, npos, first, argmax = stats
    if not valid or not math.isclose(total, 1.0, rel_tol=0, abs_tol=1e-10):
        raise ValidationError(_DIST_MSG)
    return _Dist(t, npos, first, argmax)


def _distribution(values):
    """Validated float64 probability vector on the device (sampling.py:109-115)."""
    t = _dist_input(values)
    return _dist_checked(t, batch.prob_stats(t))


def _token_index(token, n):
    """``token`` as an index into a vector of ``n``, or None where it is not one
    (the verifier's own range check reports such tokens later)."""
    return token if type(token) is int and 0 <= token < n else None


def _distributions(rows, tokens=None):
    """``_as_dist`` of every row, with one synchronisation for all the rows
    that still need their statistics; with ``tokens`` (one per row), each
    such row's probability at its token comes back in the same copy.  Every
    rejection carries the same message, so checking the shapes first and the
    values after reports what checking row by row would."""
    items = [row if isinstance(row, _Dist) else _dist_input(row) for row in rows]
    pending = [i for i, item in enumerate(items) if not isinstance(item, _Dist)]
    if pending:
        m = len(pending)
        buf = torch.empty(4 * m, dtype=torch.float64, device=items[pending[0]].device)  # [m, 3] stats, m values
        stats = buf[:3 * m].view(m, 3)
        index = {i: None if tokens is None else _token_index(tokens[i], items[i].numel()) for i in pending}
        if len({items[i].numel() for i in pending}) == 1:
            batch.prob_stats_rows_launch([items[i] for i in pending], stats)
        else:
            for n, i in enumerate(pending):
                batch.prob_stats_launch(items[i], stats[n])
        for n, i in enumerate(pending):
            if index[i] is not None:
                buf[3 * m + n:3 * m + n + 1].copy_(items[i][index[i]:index[i] + 1])
        host = buf.cpu()
        for n, i in enumerate(pending):
            d = _dist_checked(items[i], batch.prob_stats_read(host[3 * n:3 * n + 3]))
            if index[i] is not None:
                d.at[index[i]] = float(host[3 * m + n])
            items[i] = d
    return tuple(items)


def _residual(target, proposal):
    """The validated normalised residual of two distributions (sampling.py:131-139,
    then :109-115) behind one synchronisation: the correction's status and the
    residual's statistics come back together."""
    if len(target) != len(proposal):
        raise ValidationError("target and proposal vocabulary sizes differ")
    buf = torch.empty(4, dtype=torch.float64, device=target.tensor.device)  # stats slot, then the status
    out = batch.prob_correction_launch(target.tensor, proposal.tensor, buf[3:4].view(torch.int32)[0:1])
    batch.prob_stats_launch(out, buf[0:3])
    host = buf.cpu()
    if int(host[3:4].view(torch.int32)[0]) != N.OK:
        raise ValidationError("a rejected proposal has no positive correction distribution")
    return _dist_checked(out, batch.prob_stats_read(host[0:3]))


@dataclass
class _Dist:
    tensor: torch.Tensor
    positive: int
    first: int
    argmax: int
    at: dict = field(default_factory=dict)  # {token: probability} read back with the statistics

    def __len__(self):
        return self.tensor.numel()


def _as_dist(values):
    return values if isinstance(values, _Dist) else _distribution(values)


def categorical(probabilities, uniform):
    """Index drawn from ``probabilities``; the uniform is requested only if needed (sampling.py:118-128)."""
    d = _as_dist(probabilities)
    if d.positive == 1:
        return d.first
    value = uniform()
    if not isinstance(value, float) or not 0 <= value < 1:
        raise ValidationError("sampling uniform must lie in [0,1)")
    token, _flags = batch.prob_categorical(d.tensor, value)
    return token


def _correction(target, proposal):
    if len(target) != len(proposal):
        raise ValidationError("target and proposal vocabulary sizes differ")
    out, status = batch.prob_correction(target.tensor, proposal.tensor)
    if status != N.OK:
        raise ValidationError("a rejected proposal has no positive correction distribution")
    return out


def correction_distribution(target, proposal):
    """Normalised positive part of ``target - proposal`` (sampling.py:131-139)."""
    numpy_out = not isinstance(target, torch.Tensor)
    out = _correction(_as_dist(target), _as_dist(proposal))
    return out.cpu().numpy() if numpy_out else out


def _export(generator):
    return _export_state(generator.bit_generator.state)


def _export_state(state):
    return {"state": f"{state['state']['state']:032x}", "increment": f"{state['state']['inc']:032x}",
            "has_uint32": state["has_uint32"], "uinteger": state["uinteger"]}


def _import(state):
    if not isinstance(state, dict) or set(state) != {"state", "increment", "has_uint32", "uinteger"}:
        raise ValidationError("invalid PCG64 snapshot fields")
    for key in ("state", "increment"):
        hex_id(state[key], 32, f"PCG64 {key}")
    integer(state["has_uint32"], "PCG64 cached half-word flag", 0, 1)
    integer(state["uinteger"], "PCG64 cached word", 0, (1 << 32) - 1)
    increment = int(state["increment"], 16)
    if increment % 2 != 1:
        raise ValidationError("PCG64 increment must be odd")
    generator = np.random.Generator(np.random.PCG64(0))
    generator.bit_generator.state = {"bit_generator": "PCG64",
                                     "state": {"state": int(state["state"], 16), "inc": increment},
                                     "has_uint32": state["has_uint32"], "uinteger": state["uinteger"]}
    return generator


class RandomStreams:
    """Three independent PCG64 domains seeded from SHA-256 (sampling.py:166-202)."""

    def __init__(self, seed: int):
        integer(seed, "sampling seed", 0, (1 << 64) - 1)
        self._streams = {}
        for domain in DOMAINS:
            digest = hashlib.sha256(b"DeepSeekRPC/PCG64/v1/" + seed.to_bytes(8, "little") + domain.encode()).digest()
            self._streams[domain] = np.random.Generator(np.random.PCG64(int.from_bytes(digest[:16], "little")))
        self.active = False

    def snapshot(self):
        if self.active:
            raise ValidationError("terminal RNG snapshot requires a committed idle boundary")
        return self._snapshot()

    def _snapshot(self):
        return {"algorithm": "PCG64-domains-v1", "domains": {name: _export(g) for name, g in self._streams.items()}}

    def restore(self, state):
        if self.active:
            raise ValidationError("RNG restore requires an idle terminal sampler")
        self._restore(state)

    def _restore(self, state):
        if (not isinstance(state, dict) or set(state) != {"algorithm", "domains"}
                or state["algorithm"] != "PCG64-domains-v1" or not isinstance(state["domains"], dict)
                or set(state["domains"]) != set(DOMAINS)):
            raise ValidationError("incompatible terminal RNG snapshot")
        # Every domain is validated before any live state is replaced.
        self._streams = {name: _import(state["domains"][name]) for name in DOMAINS}

    def begin(self):
        if self.active:
            raise ValidationError("terminal RNG transaction is already active")
        # The domains' raw bit-generator states: an abort puts them back in
        # place, with no snapshot text to format or parse.
        before = {name: g.bit_generator.state for name, g in self._streams.items()}
        self.active = True
        return RandomTransaction(self, before)


class RandomTransaction:
    """One bounded window of draws, committed or fully rolled back (sampling.py:205-231)."""

    def __init__(self, owner, before):
        self.owner, self._before, self.closed = owner, before, False
        self.draws = dict.fromkeys(DOMAINS, 0)

    @property
    def before(self):
        """The snapshot taken when the transaction began."""
        return {"algorithm": "PCG64-domains-v1", "domains": {name: _export_state(st) for name, st in self._before.items()}}

    def random(self, domain):
        if self.closed or domain not in DOMAINS or self.draws[domain] >= 64:
            raise ValidationError("terminal RNG domain is closed, invalid or exceeds its bounded window")
        self.draws[domain] += 1
        return float(self.owner._streams[domain].random())

    def _preview(self, domain):
        """The value the next ``random(domain)`` will return, read from a copy
        of the domain's generator: the live stream does not move.  A kernel
        takes it pre-drawn and ``random(domain)`` is called only if the kernel
        reports the draw consumed, so the stream advances exactly as a lazy
        ``uniform()`` callback would advance it."""
        copy = np.random.Generator(np.random.PCG64(0))
        copy.bit_generator.state = self.owner._streams[domain].bit_generator.state
        return float(copy.random())

    def commit(self):
        if self.closed:
            raise ValidationError("terminal RNG transaction is already closed")
        self.closed, self.owner.active = True, False
        return self.owner.snapshot()

    def prepared_state(self):
        if self.closed:
            raise ValidationError("terminal RNG transaction is already closed")
        return self.owner._snapshot()

    def abort(self):
        if self.closed:
            raise ValidationError("terminal RNG transaction is already closed")
        for name, state in self._before.items():
            self.owner._streams[name].bit_generator.state = state
        self.closed, self.owner.active = True, False


@dataclass(frozen=True)
class VerificationDecision:
    accepted_drafts: int
    output_ids: tuple[int, ...]
    pending_token: int | None
    stop_reason: str | None

    @property
    def accepted_target_rows(self):
        # Rows checked: the seed's own target row, then one per draft kept.
        return 1 + self.accepted_drafts


def verify_drafts(target_rows, proposal_rows, proposal_ids, transaction, *, greedy: bool, output_limit: int,
                  eos_ids=frozenset()):
    """Exact speculative verification: accept with min(1, p/q), else resample
    from the normalised residual; one target bonus draw when all accept
    (sampling.py:247-294).  Targets are evaluated lazily, in order."""
    integer(len(proposal_ids), "proposal length", 0, 5)
    integer(output_limit, "remaining output limit", 1, MAX_COUNT)
    if type(greedy) is not bool or len(proposal_rows) != len(proposal_ids) or len(target_rows) != len(proposal_ids) + 1:
        raise ValidationError("target/proposal verification row counts differ")
    proposals = _distributions(proposal_rows, proposal_ids)
    first_target = _as_dist(target_rows[0])
    vocabulary = len(first_target)
    if any(len(row) != vocabulary for row in proposals):
        raise ValidationError("verification probability vocabularies differ")

    def target_at(index):
        # A finished grammar never builds a later distribution: only used prefixes are evaluated.
        result = first_target if index == 0 else _as_dist(target_rows[index])
        if len(result) != vocabulary:
            raise ValidationError("verification probability vocabularies differ")
        return result

    for token in (*proposal_ids, *eos_ids):
        integer(token, "verification token", 0, vocabulary - 1)
    output = []
    for index, token in enumerate(proposal_ids):
        target, proposal = target_at(index), proposals[index]
        p, q = target.at.get(token), proposal.at.get(token)
        if p is not None and q is not None:
            # Both probabilities came back with the rows' statistics: the
            # reference's own host arithmetic (sampling.py:276-281).
            if not q > 0.0:
                raise ValidationError("a proposed token has zero probability under its claimed conditional proposal")
            if greedy:
                accepted = token == target.argmax
            else:
                accepted = transaction.random("accept") < min(1.0, p / q)
        elif greedy:
            positive, _ = batch.prob_accept(target.tensor, proposal.tensor, token, 0.0)
            if not positive:
                raise ValidationError("a proposed token has zero probability under its claimed conditional proposal")
            accepted = token == target.argmax
        else:
            preview = getattr(transaction, "_preview", None)
            # One launch tests q(x) > 0 and the draw together when the draw can
            # be read ahead; the domain still advances only after the test.
            u = preview("accept") if preview is not None else 0.0
            positive, accepted = batch.prob_accept(target.tensor, proposal.tensor, token, u)
            if not positive:
                raise ValidationError("a proposed token has zero probability under its claimed conditional proposal")
            if preview is None:
                u = transaction.random("accept")
                _, accepted = batch.prob_accept(target.tensor, proposal.tensor, token, u)
            elif transaction.random("accept") != u:
                raise RuntimeError("RNG domain moved between the preview and the draw")
        if not accepted:
            if greedy:
                replacement = target.argmax
            else:
                residual = _residual(target, proposal)
                replacement = categorical(residual, lambda: transaction.random("target"))
            stop = "eos" if replacement in eos_ids else "length" if len(output) + 1 >= output_limit else None
            return VerificationDecision(index, tuple(output) + (replacement,), replacement, stop)
        output.append(token)
        if token in eos_ids or len(output) >= output_limit:
            return VerificationDecision(index + 1, tuple(output), None, "eos" if token in eos_ids else "length")
    bonus_target = target_at(len(proposal_ids))
    bonus = bonus_target.argmax if greedy else categorical(bonus_target, lambda: transaction.random("target"))
    stop = "eos" if bonus in eos_ids else "length" if len(output) + 1 >= output_limit else None
    return VerificationDecision(len(proposal_ids), tuple(output) + (bonus,), bonus, stop)
