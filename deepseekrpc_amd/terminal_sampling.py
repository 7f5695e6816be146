"""Terminal sampling transactions whose rows never leave the GPU.

Public surface of the reference's src/deepseekrpc/terminal_sampling.py:
``TerminalSampler`` (begin_seed / begin_verification, :48-106),
``SamplingWork`` (distribution / propose / use_normal_decode / verify /
prepared / apply_stop / commit / abort, :109-231) and ``SeedDecision``
(:30-45), with the same validation order, messages, RNG consumption and
decision digest.

How it is built here:

* ``_Controls`` is the transaction's frozen input record.  ``_check_controls``
  validates it once, in the reference's order, and the counts become one
  device history table when the first row needs them.
* A ``SamplingWork`` walks a small stage machine (``_Stage``): seeded, awaiting
  proposals, proposed, decided.  Every guard reads the stage, and the
  reference's error messages name the guard that fails.
* Every draw (the seed, each proposal) is one fused ``dsr_sample_rows`` launch
  on the current stream: the row's float64 distribution and its categorical
  draw together.  The uniform is the domain's next value, read from a copy of
  the generator (``RandomTransaction._preview``); the live domain advances
  only when the kernel reports the draw consumed.  That is the draw sequence
  of the reference's lazy ``uniform()`` callback, with one host round trip
  per row in place of a device-to-host copy of the row and three passes over
  it.
* Proposal distributions stay on the device for the verifier, and target
  rows are conditioned on the accepted prefix when the verifier first asks
  for them (``_LazyRows``).
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from contextlib import contextmanager
from dataclasses import asdict, dataclass, replace
import enum
import hashlib
import os

import numpy as np
import torch

from . import _native as N
from . import batch
from .jsonutil import ValidationError, fingerprint, hex_id, integer
from .sampling import (_COUNTS_MSG, RandomStreams, SamplingPolicy, VerificationDecision, _allow_row, _bias_table,
                       _device, _dist_checked, _logit_vector, _on_device, _raise_status, _token_index, verify_drafts)

_HISTORY_LIMIT = 1048576
_MAX_PROPOSALS = 5

_MSG_WINDOW = "terminal logits do not match the complete bounded vocabulary window"
_MSG_HEAD = "terminal logits must come from the actual FP32 CUDA vocabulary head"


_M64 = (1 << 64) - 1


def _state_words(generators):
    """uint64 ``[n, 4]``: each PCG64 generator's state lo, hi, increment lo, hi."""
    out = np.zeros((len(generators), 4), np.uint64)
    for i, g in enumerate(generators):
        st = g.bit_generator.state["state"]
        out[i] = (st["state"] & _M64, st["state"] >> 64, st["inc"] & _M64, st["inc"] >> 64)
    return out


def _states_on_device(generators, device):
    """The generators' PCG64 states as an int64 ``[n, 4]`` device tensor,
    uploaded from pinned memory without a synchronisation."""
    host = torch.from_numpy(_state_words(generators).view(np.int64)).pin_memory()
    return host.to(device, non_blocking=True)


def _set_state(generator, lo, hi):
    """Give a PCG64 generator the state a kernel advanced (two int64 words)."""
    bg = generator.bit_generator
    st = bg.state
    st["state"]["state"] = (lo & _M64) | ((hi & _M64) << 64)
    bg.state = st


def _logits_device(logits, rows, vocabulary):
    """``[rows, vocabulary]`` FP32 finite logits as a device tensor.

    The reference copies CUDA rows to the host here (terminal_sampling.py:16-27);
    they stay on the device instead, and NumPy windows are uploaded.  The
    same inputs are rejected with the same messages."""
    if isinstance(logits, np.ndarray):
        if logits.dtype != np.float32 or logits.shape != (rows, vocabulary) or not np.isfinite(logits).all():
            raise ValidationError(_MSG_WINDOW)
        return _on_device(logits)[0]
    if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32):
        raise ValidationError(_MSG_HEAD)
    if tuple(logits.shape) != (rows, vocabulary):
        raise ValidationError(_MSG_WINDOW)
    window = logits.detach().contiguous()
    _require_finite(batch.rows_finite(window))
    return window


def _logits_deferred(logits, rows, vocabulary):
    """``_logits_device`` with the finiteness test of a CUDA window left to
    the caller: ``(window, deferred)``, ``deferred`` True when the caller
    must still run ``dsr_rows_finite`` on the window (into flags it has set
    to 1) and read the flags with its next synchronisation.  Every other
    check runs at once, as in ``_logits_device``."""
    if (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32
            and tuple(logits.shape) == (rows, vocabulary)):
        return logits.detach().contiguous(), True
    return _logits_device(logits, rows, vocabulary), False


def _require_finite(finite):
    """Reports a deferred non-finite window, ahead of any later error."""
    if finite is not None and int(finite.min()) == 0:
        raise ValidationError(_MSG_WINDOW)


class _DrawIO:
    """A sampler's device buffer for single-row draws on one device: the
    domain's PCG64 state (advanced in place by the kernel), the row's token,
    status, consumed and flags outputs and the window's finite flag, all in
    64 bytes read back with one copy."""

    def __init__(self, device):
        self.dev = torch.zeros(8, dtype=torch.int64, device=device)
        b32, b8 = self.dev.view(torch.int32), self.dev.view(torch.uint8)
        self.state = self.dev[0:4].view(1, 4)
        self.out = {"tokens": b32[8:9], "status": b32[9:10], "consumed": b8[40:41], "flags": b8[41:42]}
        self.finite = b32[12:13]

    def upload(self, generator, finite=False):
        """The generator's state into the buffer (and with ``finite`` the
        window's flag set to 1 for ``dsr_rows_finite``), from pinned memory,
        without a synchronisation (the caching host allocator keeps the
        pinned block until the copy has run)."""
        host = torch.zeros(8 if finite else 4, dtype=torch.int64, pin_memory=True)
        words = host.numpy()
        words[:4] = _state_words([generator]).view(np.int64)[0]
        if finite:
            words.view(np.int32)[12] = 1
        self.dev[:host.numel()].copy_(host, non_blocking=True)

    def read(self):
        w = self.dev.cpu().numpy()
        i32, u8 = w.view(np.int32), w.view(np.uint8)
        return int(w[0]), int(w[1]), int(i32[8]), int(i32[9]), int(u8[40]), int(i32[12])


@dataclass(frozen=True)
class SeedDecision:
    token: int
    stop_reason: str | None

    @property
    def output_ids(self):
        return (self.token,)

    @property
    def pending_token(self):
        return self.token

    @property
    def accepted_target_rows(self):
        # A seed decision consumed no verification row.
        return 0


class _Counts:
    """A frozen count vector kept as its positive entries: ``support`` (the
    increasing token ids), their ``values``, and the vector's length and
    dtype.  The dense read-only vector is built on first use only (a draw
    that reads no history table and a transaction without a digest never
    need it)."""

    __slots__ = ("support", "values", "length", "dtype", "_dense")

    def __init__(self, support, values, length, dtype):
        self.support, self.values, self.length, self.dtype = support, values, length, dtype
        self._dense = None

    def dense(self):
        if self._dense is None:
            out = np.zeros(self.length, self.dtype)
            out[self.support] = self.values
            out.setflags(write=False)
            self._dense = out
        return self._dense

    def at(self, token):
        i = int(np.searchsorted(self.support, token))
        return int(self.values[i]) if i < self.support.size and self.support[i] == token else 0

    def int64(self):
        """A fresh dense int64 copy (for the digest hashes, on any thread)."""
        out = np.zeros(self.length, np.int64)
        out[self.support] = self.values
        return out


@dataclass(frozen=True)
class _Controls:
    """The frozen inputs of one transaction (copies: callers cannot mutate them)."""
    policy: SamplingPolicy
    counts: _Counts
    generated: _Counts              # the same object when no separate generated counts were given
    remaining: int
    eos_ids: frozenset
    logit_bias: dict | None
    allowed: object
    grammar_identity: str | None
    stop_identity: str | None
    support: np.ndarray           # the token ids with a positive count, increasing
    total: int | None             # the sum of the counts; None when a count exceeds 2^20


def _sha256_i8(values):
    """SHA-256 hex digest of a count vector's little-endian int64 bytes."""
    return hashlib.sha256(np.ascontiguousarray(values, dtype="<i8")).hexdigest()


def _count_hashes(counts, generated):
    """The digest's two count hashes of two ``_Counts``; equal vectors (no
    separate generated counts) share one."""
    sha = _sha256_i8(counts.int64())
    same = generated is counts or np.array_equal(counts.values, generated.values)  # one support
    return sha, sha if same else _sha256_i8(generated.int64())


# The count hashes (about 0.4 ms per megabyte vector) of a verification run on
# a worker thread from the moment its transaction opens, while its rows are on
# the device (hashlib and NumPy release the GIL), so that prepared() finds
# them done.
# One worker per process: a forked child makes its own (an executor
# inherited over fork has no thread to run its work).
_hasher = None
_hasher_pid = None


def _hash_worker():
    global _hasher, _hasher_pid
    if _hasher is None or _hasher_pid != os.getpid():
        _hasher = ThreadPoolExecutor(max_workers=1, thread_name_prefix="dsr-count-sha")
        _hasher_pid = os.getpid()
    return _hasher


def _valid_count_vector(values, vocabulary):
    return values.shape == (vocabulary,) and values.dtype in (np.int32, np.int64) and values.min() >= 0


def _check_controls(sampler, policy, counts, remaining, eos_ids, generated_counts, logit_bias, allowed,
                    grammar_identity, stop_identity) -> _Controls:
    """Validation of terminal_sampling.py:54-81, in its order and with its messages."""
    integer(remaining, "remaining output capacity", 1, _HISTORY_LIMIT)
    if sampler.active is not None or not isinstance(policy, SamplingPolicy):
        raise ValidationError("terminal sampling is active or its policy is invalid")
    counts = np.asarray(counts)
    # One native pass: no negative entry, the positive entries and their
    # int64 total (zero entries add nothing; the sum wraps as NumPy's does).
    scan = (batch.count_scan(counts) if counts.shape == (sampler.vocabulary,)
            and counts.dtype in (np.int32, np.int64) else None)
    support, total, largest = (None, None, None) if scan is None else scan
    if total is None or total > _HISTORY_LIMIT:
        raise ValidationError("terminal counts differ from the exact published token history")
    if support.size and largest > _HISTORY_LIMIT:
        total = None   # the int64 sum wrapped: every row's distribution rejects these counts
    for token in eos_ids:
        integer(token, "terminal EOS token", 0, sampler.vocabulary - 1)
    if allowed is not None and not callable(allowed):
        raise ValidationError("grammar mask provider must evaluate a bounded tentative token prefix")
    if (allowed is None) != (grammar_identity is None):
        raise ValidationError("a grammar mask requires its frozen grammar/prefix identity")
    for identity, what in ((grammar_identity, "frozen grammar and committed-prefix identity"),
                           (stop_identity, "frozen original detokenizer and stop-prefix identity")):
        if identity is not None:
            hex_id(identity, 64, what)
    generated = counts if generated_counts is None else np.asarray(generated_counts)
    if generated is not counts and (generated.shape != counts.shape or not _valid_count_vector(
            generated, sampler.vocabulary) or (generated > counts).any()):
        raise ValidationError("generated sampling counts must be a subset of the complete history")
    # Frozen copies of the positive entries; generated counts lie within the
    # support (0 <= generated <= counts), and without separate generated
    # counts both names hold one copy.
    frozen = _Counts(support, counts[support], counts.size, counts.dtype)
    if generated is counts:
        generated = frozen
    else:
        generated = _Counts(support, generated[support], generated.size, generated.dtype)
    return _Controls(policy, frozen, generated, remaining, frozenset(eos_ids),
                     None if logit_bias is None else dict(logit_bias), allowed, grammar_identity, stop_identity,
                     support, total)


class TerminalSampler:
    """Owns the three RNG domains and at most one open ``SamplingWork``."""

    def __init__(self, seed, *, vocabulary=129280):
        self.random = RandomStreams(seed)
        self.vocabulary = integer(vocabulary, "sampling vocabulary", 1, 129280)
        self.active = None

    def _io(self, device):
        """The ``_DrawIO`` of ``device`` (made on first use)."""
        ios = self.__dict__.setdefault("_ios", {})
        io = ios.get(device.index)
        if io is None:
            io = ios[device.index] = _DrawIO(device)
        return io

    def _open_work(self, stage, *controls):
        checked = _check_controls(self, *controls)   # nothing starts unless every control is valid
        work = SamplingWork(self, self.random.begin(), checked, stage)
        self.active = work
        if stage is _Stage.AWAITING_PROPOSALS:
            # The digest's count hashes, on the worker thread while the
            # proposals and the verification run (a seed's digest follows its
            # one launch at once, so its hashes wait for prepared()).
            work._counts_sha = _hash_worker().submit(_count_hashes, work._controls.counts, work._controls.generated)
        return work

    def begin_seed(self, logits, *, policy, counts, remaining, eos_ids=frozenset(), generated_counts=None,
                   logit_bias=None, allowed=None, grammar_identity=None, stop_identity=None):
        """Sample the first token of a request from one row of target logits."""
        early = self._seed_launch(logits, policy, logit_bias, allowed)
        work = self._open_work(_Stage.SEEDING, policy, counts, remaining, eos_ids, generated_counts, logit_bias,
                               allowed, grammar_identity, stop_identity)
        with work._aborting_on_error():
            if early is not None and not work._needs_history(0):
                token = work._take_draw(early, "target")
                stop = "eos" if token in work.eos_ids else "length" if remaining == 1 else None
                work._decide(SeedDecision(token, stop))
                return work
            # Without a grammar provider nothing the caller sees happens
            # between the window check and the draw, so the window's
            # finiteness is read with the draw's result.
            if work.allowed is None:
                window, deferred = _logits_deferred(logits, 1, self.vocabulary)
            else:
                window, deferred = _logits_device(logits, 1, self.vocabulary), False
            # The seed's row is not kept.
            token, _ = work._draw(window[0], (), "target", window if deferred else None, probs=None)
            stop = "eos" if token in work.eos_ids else "length" if remaining == 1 else None
            work._decide(SeedDecision(token, stop))
        return work

    def _seed_launch(self, logits, policy, logit_bias, allowed):
        """The seed's draw, launched ahead of the control checks when the call
        hands a CUDA FP32 window and has no grammar, bias or penalties: the
        host checks then run while the row is sampled.  Nothing the caller
        sees changes until the result is read, which happens only once every
        check has passed and the row needs no history table; otherwise the
        launch is dropped and the call takes the ordinary route (which
        raises what it would have raised).  Returns the sampler's ``_DrawIO``
        holding the launch, or None."""
        if (self.active is not None or allowed is not None or logit_bias is not None
                or not isinstance(policy, SamplingPolicy) or policy.repetition_penalty != 1
                or policy.presence_penalty != 0 or policy.frequency_penalty != 0):
            return None
        if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32
                and tuple(logits.shape) == (1, self.vocabulary)):
            return None
        window = logits.detach().contiguous()
        io = self._io(window.device)
        try:
            io.upload(self.random._streams["target"], True)
            batch.rows_finite(window, io.finite)
            policy._launch_row(window[0], self.vocabulary, None, None, None, rng_state=io.state, out=io.out,
                               probs=None)
        except Exception:
            return None
        return io

    def begin_verification(self, *, seed_token, policy, counts, remaining, eos_ids=frozenset(), generated_counts=None,
                           logit_bias=None, allowed=None, grammar_identity=None, stop_identity=None):
        """Open a speculative step after ``seed_token``, which must already be in the history."""
        integer(seed_token, "pending verification seed", 0, self.vocabulary - 1)
        work = self._open_work(_Stage.AWAITING_PROPOSALS, policy, counts, remaining, eos_ids, generated_counts,
                               logit_bias, allowed, grammar_identity, stop_identity)
        if min(work._controls.counts.at(seed_token), work._controls.generated.at(seed_token)) < 1:
            work.abort()
            raise ValidationError("pending seed must already belong to published sampling history")
        work.seed_token = seed_token
        return work


class _Stage(enum.Enum):
    SEEDING = "seeding"                        # begin_seed: decided when the seed is drawn
    AWAITING_PROPOSALS = "awaiting proposals"  # begin_verification: propose or use_normal_decode next
    PROPOSED = "proposed"                      # verify next
    DECIDED = "decided"                        # apply_stop (if a stop identity is frozen), prepared, commit


class _LazyRows:
    """A sequence whose items are built on first access and kept."""

    def __init__(self, count, build):
        self._slots = [None] * count
        self._build = build

    def __len__(self):
        return len(self._slots)

    def __getitem__(self, index):
        item = self._slots[index]
        if item is None:
            item = self._slots[index] = self._build(index)
        return item


class _TargetRows:
    """The verifier's target rows, all launched at once: row j conditioned on
    the proposals ``ids[:j]`` (terminal_sampling.py:234-244).  A row's
    failure, at launch or on the device, is raised when the verifier reaches
    that row, as the lazily built rows of the reference raise it.

    ``device()`` hands the rows and their statuses to ``dsr_verify_probs``
    when every row launched.  Otherwise (or with ``host=True``) the rows'
    statistics are launched together, and each row's status and its
    probability at proposal j come back with one synchronisation when the
    host verifier first asks for a row."""

    def __init__(self, work, rows, ids, host=True):
        n = len(rows)
        self._rows, self._ids, self._host, self._status, self._stats = [], ids, None, [], None
        if not work._needs_history(len(ids)):
            self._launch_together(work, rows)
        else:
            self._launch_each(work, rows, ids)
        if host:
            self._host_inputs()

    def _launch_together(self, work, rows):
        """No row reads a history table, so the rows are independent: one
        launch over all of them (a launch-time failure is the same for every
        row, and the first row reports it)."""
        n = len(rows)
        try:
            result = work._rows_launch(rows)
        except Exception as exc:
            self._rows = [exc] * n
            return
        self._rows = [result.probs[j] for j in range(n)]
        self._status = [result.status]

    def _launch_each(self, work, rows, ids):
        for j in range(len(rows)):
            try:
                result, _ = work._row_launch(rows[j], ids[:j])
            except Exception as exc:
                self._rows.append(exc)
                continue
            self._rows.append(result.probs[0])
            self._status.append(result.status)

    def device(self):
        """(rows, int32 statuses) for ``dsr_verify_probs``, or None if a row
        failed at launch."""
        if any(isinstance(r, Exception) for r in self._rows):
            return None
        return self._rows, self._status[0] if len(self._status) == 1 else torch.cat(self._status)

    def _host_inputs(self):
        """The host verifier's inputs: [n, 3] statistics, then n statuses
        (int32 in a double each), then n probabilities at the proposals, in
        one buffer read back when the first row is asked for."""
        n = len(self._rows)
        launched = [j for j in range(n) if not isinstance(self._rows[j], Exception)]
        if not launched:
            return
        self._buf = torch.empty(5 * n, dtype=torch.float64, device=self._rows[launched[0]].device)
        if len(launched) == n and len(self._status) == 1 and self._status[0].numel() == n:
            self._buf[3 * n:4 * n].view(torch.int32)[0::2].copy_(self._status[0])
        else:  # one status per launched row
            for status, j in zip(self._status, launched):
                self._buf[3 * n + j:3 * n + j + 1].view(torch.int32)[0:1].copy_(status)
        for j in launched:
            x = _token_index(self._ids[j], self._rows[j].numel()) if j < len(self._ids) else None
            if x is not None:
                self._buf[4 * n + j:4 * n + j + 1].copy_(self._rows[j][x:x + 1])
        self._stats = self._buf[:3 * n].view(n, 3)
        # The rows that launched fill their own slots (a failed row's slot stays unread).
        lo = launched[0]
        if launched == list(range(lo, lo + len(launched))):
            batch.prob_stats_rows_launch([self._rows[j] for j in launched], self._stats[lo:lo + len(launched)])
        else:
            for j in launched:
                batch.prob_stats_launch(self._rows[j], self._stats[j])

    def __len__(self):
        return len(self._rows)

    def __getitem__(self, j):
        n = len(self._rows)
        row = self._rows[j]
        if isinstance(row, Exception):
            raise row
        if self._host is None:
            self._host = self._buf.cpu()
        code = int(self._host[3 * n + j:3 * n + j + 1].view(torch.int32)[0])
        if code != N.OK:
            _raise_status(code)
        dist = _dist_checked(row, batch.prob_stats_read(self._host[3 * j:3 * j + 3]))
        x = _token_index(self._ids[j], row.numel()) if j < len(self._ids) else None
        if x is not None:
            dist.at[x] = float(self._host[4 * n + j])
        return dist


class SamplingWork:
    """One open sampling transaction of a ``TerminalSampler``."""

    def __init__(self, owner, transaction, controls: _Controls, stage: _Stage):
        self.owner, self.transaction, self._controls = owner, transaction, controls
        self._stage = stage
        self._stop_pending = controls.stop_identity is not None
        self.closed = False
        self.seed_token = None
        self.decision = None
        self.proposal_ids, self.proposal_rows = [], []
        # Each proposal row's FP32 logits (None once a row came without them):
        # with them the verifier runs as one batched launch that draws on the device.
        self._draft_logits = []
        self._device_history = None   # the counts as a device table, built for the first row
        # SHA-256 of the frozen count vectors, for the digest (a future while a
        # worker thread computes it).
        self._counts_sha = None

    # -- the frozen controls, under the reference's attribute names --------
    policy = property(lambda self: self._controls.policy)
    counts = property(lambda self: self._controls.counts.dense())
    generated_counts = property(lambda self: self._controls.generated.dense())
    remaining = property(lambda self: self._controls.remaining)
    eos_ids = property(lambda self: self._controls.eos_ids)
    logit_bias = property(lambda self: self._controls.logit_bias)
    allowed = property(lambda self: self._controls.allowed)
    grammar_identity = property(lambda self: self._controls.grammar_identity)
    stop_identity = property(lambda self: self._controls.stop_identity)

    @property
    def _proposal_ready(self):
        return self._stage in (_Stage.PROPOSED, _Stage.DECIDED)

    @_proposal_ready.setter
    def _proposal_ready(self, ready):
        # Callers that supply proposals themselves mark them complete this way.
        if ready and self._stage is _Stage.AWAITING_PROPOSALS:
            self._stage = _Stage.PROPOSED

    # -- guards -------------------------------------------------------------
    def _require_open(self):
        if self.closed or self.owner.active is not self:
            raise ValidationError("terminal sampling transaction is closed or stale")

    def _require_stage(self, stage, message):
        self._require_open()
        if self._stage is not stage:
            raise ValidationError(message)

    @contextmanager
    def _aborting_on_error(self):
        """A failing step ends the transaction and restores every RNG domain."""
        try:
            yield
        except BaseException:
            self.abort()
            raise

    def _decide(self, decision):
        self.decision = decision
        self._stage = _Stage.DECIDED

    # -- rows -----------------------------------------------------------------
    def _history(self, prefix):
        """The device history table with each prefix token counted once more,
        as generated output (terminal_sampling.py:127-133)."""
        if self._controls.total is None:
            raise ValidationError(_COUNTS_MSG)   # sampling.py:55-58 rejects a count above 2^20
        if self._device_history is None:
            # The controls were checked on entry (no negative count, 2^20 in
            # total, generated <= counts), so nothing here can be rejected and
            # the table is built on the host from the positive entries.
            c = self._controls
            self._device_history = batch.HistoryTable.from_support(
                c.support, c.counts.values, c.generated.values, device=_device())
        if not prefix:
            return self._device_history
        dev = self._device_history.offsets.device
        tokens = torch.tensor(list(prefix), dtype=torch.int32, device=dev)
        bounds = torch.tensor([0, len(prefix)], dtype=torch.int64, device=dev)
        table, status = self._device_history.append(tokens, bounds, vocab=self._controls.counts.length)
        code = int(status.item())
        if code != N.OK:
            _raise_status(code)
        return table

    def _needs_history(self, grown):
        """Whether rows whose prefix holds up to ``grown`` tokens carry the
        history table.  Penalties read it; repetition 1 and presence and
        frequency 0 leave every logit as it is, and then only a history that
        the prefix could push past the count limit needs the table, whose
        append reports the overflow at the row where it happens
        (sampling.py:55-58)."""
        p, total = self.policy, self._controls.total
        return (p.repetition_penalty != 1 or p.presence_penalty != 0 or p.frequency_penalty != 0
                or total is None or total + grown > _HISTORY_LIMIT)

    def _rows_launch(self, rows):
        """All the verifier's target rows in one launch, for rows that read no
        history table and no grammar mask (``_row_launch``'s checks, which
        are the same for every row)."""
        size, _ = _logit_vector(rows[0])
        if size != self._controls.counts.length:
            raise ValidationError(_COUNTS_MSG)
        n = len(rows)
        bias = _bias_table(self.logit_bias, size, rows=n)
        return batch.sample_rows(rows, self.policy._device_tensor(rows.device, rows=n), bias=bias, probs="f64")

    def _row_launch(self, logits, prefix, uniform=None, rng_state=None, out=None, probs="f64"):
        """Validate one row and launch its distribution (and draw, given a
        uniform).  The grammar is asked for its mask first, then the row and
        controls are checked in the order of sampling.py:50-79."""
        mask = None if self.allowed is None else self.allowed(tuple(prefix))
        size, device_input = _logit_vector(logits)
        if size != self._controls.counts.length:
            raise ValidationError(_COUNTS_MSG)
        table = self._history(prefix) if self._needs_history(len(prefix)) else None
        bias = _bias_table(self.logit_bias, size)
        allow = _allow_row(mask, size)
        return self.policy._launch_row(logits, size, table, bias, allow, uniform, rng_state, out, probs), device_input

    def distribution(self, logits, prefix):
        """Float64 distribution of one row given a tentative accepted prefix
        (terminal_sampling.py:127-136); device rows in, device rows out."""
        self._require_open()
        result, device_input = self._row_launch(logits, prefix)
        code = int(result.status.item())
        if code != N.OK:
            _raise_status(code)
        row = result.probs[0]
        return row if device_input else row.cpu().numpy()

    def _target(self, logits, prefix):
        """A verifier target row: ``distribution`` of the row and the
        verifier's check of it (sampling.py:109-115), with the kernel's status
        and the row's statistics read back together."""
        self._require_open()
        result, _ = self._row_launch(logits, prefix)
        row = result.probs[0]
        buf = torch.empty(4, dtype=torch.float64, device=row.device)  # stats slot, then the status
        batch.prob_stats_launch(row, buf[0:3])
        buf[3:4].view(torch.int32)[0:1].copy_(result.status)
        host = buf.cpu()
        code = int(host[3:4].view(torch.int32)[0])
        if code != N.OK:
            _raise_status(code)
        return _dist_checked(row, batch.prob_stats_read(host[0:3]))

    def _draw(self, logits, prefix, domain, window=None, probs="f64"):
        """(token, distribution): one fused launch draws from the row's
        distribution with the domain's next ``Generator.random()``, taken on
        the device from the domain's PCG64 state; the domain takes the state
        the kernel wrote back (advanced only when the draw was needed) and the
        draw counts in the transaction's window.  ``window`` is a CUDA window
        whose finiteness is still to be checked: ``dsr_rows_finite`` runs on
        it into the sampler's ``_DrawIO``, and a non-finite window is reported
        ahead of any later error.  The token, status, state and window flag
        come back with one copy.  With ``probs=None`` the distribution is not
        kept.  A window already full takes the uniform from a preview of the
        generator instead, so that ``RandomTransaction.random`` raises
        exactly when the draw is needed."""
        self._require_open()
        tr = self.transaction
        if tr.draws[domain] >= 64:
            if window is not None:
                _require_finite(batch.rows_finite(window))
            return self._draw_previewed(logits, prefix, domain)
        generator = tr.owner._streams[domain]
        io = self.owner._io(logits.device)
        io.upload(generator, window is not None)
        if window is not None:
            batch.rows_finite(window, io.finite)
        try:
            result, _ = self._row_launch(logits, prefix, rng_state=io.state, out=io.out, probs=probs)
        except Exception:
            if window is not None:
                _require_finite(io.finite)
            raise
        token = self._take_draw(io, domain, window is not None)
        return token, None if result.probs is None else result.probs[0]

    def _take_draw(self, io, domain, window=True):
        """The token of a launched single-row draw, read back with its status,
        the domain's advanced state and (with ``window``) the window's finite
        flag; the domain takes the state when the draw consumed its uniform."""
        lo, hi, token, code, consumed, ok = io.read()
        if window and not ok:
            raise ValidationError(_MSG_WINDOW)
        if code != N.OK:
            _raise_status(code)
        if consumed:
            _set_state(self.transaction.owner._streams[domain], lo, hi)
            self.transaction.draws[domain] += 1
        return token

    def _draw_previewed(self, logits, prefix, domain):
        """``_draw`` with the uniform read from a copy of the generator; the
        domain advances (and may raise) only if the kernel consumed it."""
        upcoming = self.transaction._preview(domain)
        # A fill kernel, not a host-to-device copy: nothing waits for it.
        uniform = torch.full((1,), upcoming, dtype=torch.float64, device=logits.device)
        result, _ = self._row_launch(logits, prefix, uniform)
        parts = [result.tokens.long(), result.consumed.long(), result.status.long()]
        token, consumed, code = torch.stack(parts).view(-1).tolist()
        if code != N.OK:
            _raise_status(code)
        if consumed and self.transaction.random(domain) != upcoming:
            raise RuntimeError("RNG domain moved between the preview and the draw")
        return token, result.probs[0]

    # -- the transaction's steps ------------------------------------------------
    def propose(self, graph, result):
        """Up to five draft tokens, each row conditioned on the previous token
        by the graph (terminal_sampling.py:138-161); an EOS ends the chain."""
        self._require_stage(_Stage.AWAITING_PROPOSALS,
                            "proposal generation is duplicate or lacks a committed pending seed")
        with self._aborting_on_error():
            steps = min(_MAX_PROPOSALS, self.remaining)
            device_step = getattr(graph, "draft_conditional_logits_device", None)
            # Counts the first row rejects keep the host loop, which asks the
            # graph for that row before rejecting it, as the reference does.
            if device_step is not None and self.allowed is None and self._controls.total is not None:
                self._propose_on_device(device_step, result, steps)
            else:
                previous = self.seed_token
                for position in range(steps):
                    # The graph's confidence output is diagnostic only.
                    logits, _ = graph.draft_conditional_logits(result, position, previous)
                    row = _logits_device(logits, 1, self.owner.vocabulary)[0]
                    previous, dist = self._draw(row, tuple(self.proposal_ids), "draft")
                    self.proposal_ids.append(previous)
                    self.proposal_rows.append(dist)
                    self._draft_logits.append(row.clone())  # the caller may reuse its buffer
                    if previous in self.eos_ids:
                        break
            self._stage = _Stage.PROPOSED
        return tuple(self.proposal_ids)

    def _propose_on_device(self, device_step, result, steps):
        """The proposal chain without a host round trip per row.  A graph that
        offers ``draft_conditional_logits_device(result, row, previous)``
        takes the previous token as a device int32 tensor of one element and
        returns the row's ``(1, V)`` FP32 logits on the device; each row is one
        launch that draws from the ``draft`` domain's PCG64 state on the
        device.  Rows after a stop token are computed speculatively and
        dropped at the one synchronisation, where the domain takes the state
        saved after the last kept row and the draws it consumed are counted
        in the transaction's window, exactly as the host loop draws them.
        The device method may therefore be called for rows past a stop
        token: an error it raises there (or a row of the wrong type or
        shape) stops the chain and is raised only if the row is kept."""
        vocab = self.owner.vocabulary
        device = torch.device("cuda", torch.cuda.current_device())
        generator = self.transaction.owner._streams["draft"]
        state = batch.pcg64_states([generator], device)
        seed = torch.tensor([self.seed_token], dtype=torch.int32, device=device)

        def row_logits(position, previous):
            logits, _confidence = device_step(result, position, previous)
            if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32):
                raise ValidationError(_MSG_HEAD)
            if tuple(logits.shape) != (1, vocab):
                raise ValidationError(_MSG_WINDOW)
            return logits

        grow = self._needs_history(max(steps - 1, 0))   # row j's prefix holds j proposals
        chain = batch.propose_rows(row_logits, seed, steps, self.policy._device_tensor(device), state,
                                   history=self._history(()) if grow else None, grow=grow,
                                   bias=_bias_table(self.logit_bias, vocab), vocab=vocab)
        ids, rows, draws, final, failed = batch.finish_proposals(chain, self.eos_ids)
        if failed is not None:
            if isinstance(failed[1], BaseException):
                raise failed[1]
            if failed[1] == -1:
                raise ValidationError(_MSG_WINDOW)
            _raise_status(failed[1])
        if self.transaction.draws["draft"] + draws > 64:
            raise ValidationError("terminal RNG domain is closed, invalid or exceeds its bounded window")
        batch.pcg64_restore([generator], final)
        self.transaction.draws["draft"] += draws
        self.proposal_ids.extend(ids)
        self.proposal_rows.extend(rows[j] for j in range(len(ids)))
        self._draft_logits.extend(chain.logits[j] for j in range(len(ids)))

    def use_normal_decode(self):
        """Verify with no proposals: the target row's draw is the bonus token."""
        self._require_stage(_Stage.AWAITING_PROPOSALS, "normal decode is duplicate or lacks its pending seed")
        self._stage = _Stage.PROPOSED

    def verify(self, target_logits):
        """Exact sampled verification of the proposals against ``K + 1`` target rows."""
        self._require_stage(_Stage.PROPOSED, "target verification is duplicate or proposals are not complete")
        with self._aborting_on_error():
            ids = list(self.proposal_ids)
            K = len(ids)
            if self.allowed is not None:
                rows = _logits_device(target_logits, K + 1, self.owner.vocabulary)
                # A grammar is asked for the masks of the prefixes the verifier reaches only.
                targets = _LazyRows(len(rows), lambda j: self._target(rows[j], ids[:j]))
            else:
                # Without a grammar nothing the caller sees happens before the
                # decision is read back, so the window's finiteness is read with it.
                rows, deferred = _logits_deferred(target_logits, K + 1, self.owner.vocabulary)
                if self._draws_fit(K) and self._unfiltered(K):
                    self._decide(self._device_decision(lambda: self._verify_logits(rows, ids, deferred), K))
                    return self.decision
                device = self._draws_fit(K) and self._rows_at_hand(K, rows.device)
                targets = _TargetRows(self, rows, ids, host=not device)
                ready = targets.device() if device else None
                if ready is not None:
                    self._decide(self._device_decision(lambda: self._verify_rows(rows, *ready, ids, deferred), K))
                    return self.decision
                if deferred:
                    _require_finite(batch.rows_finite(rows))
                if device:
                    targets._host_inputs()
            self._decide(verify_drafts(targets, self.proposal_rows, ids, self.transaction,
                                       greedy=self.policy.temperature == 0, output_limit=self.remaining,
                                       eos_ids=self.eos_ids))
        return self.decision

    def _draws_fit(self, K):
        """Whether the accept and target windows hold every draw the verifier
        may take (else the host verifier draws, and the window raises at the
        draw that overflows it)."""
        tr = self.transaction
        return self.policy.temperature == 0 or (tr.draws["accept"] + K <= 64 and tr.draws["target"] + 1 <= 64)

    def _rows_at_hand(self, K, device):
        """Whether the K proposal rows are contiguous float64 vocabulary rows
        on ``device`` (the proposal steps leave them there; rows a caller
        supplies in another form go to the host verifier)."""
        V = self.owner.vocabulary
        return len(self.proposal_rows) == K and all(
            isinstance(r, torch.Tensor) and r.device == device and r.dtype == torch.float64 and r.numel() == V
            and r.is_contiguous() for r in self.proposal_rows)

    def _unfiltered(self, K):
        """Whether ``dsr_verify_drafts`` takes the request on its fast path:
        the proposal logits at hand, no history table, no bias and a policy
        with no top-k, top-p or min-p."""
        return (len(self._draft_logits) == K == len(self.proposal_rows)
                and all(t is not None for t in self._draft_logits)
                and not self._needs_history(K) and not self.logit_bias
                and batch.verify_hints(batch.policy_array([self.policy]), self.owner.vocabulary, True) != 0)

    def _upload(self, ids, dev, rows, deferred):
        """One pinned upload: the accept and target PCG64 states, then (int32)
        the proposal ids, the output limit, the EOS ids and, for a window
        whose finiteness is ``deferred``, one flag per target row set to 1,
        on which ``dsr_rows_finite`` then runs.  Returns the generators, the
        device states, ids, limit, EOS arguments and flags (or None)."""
        tr, K, eos = self.transaction, len(ids), sorted(self.eos_ids)
        gens = [tr.owner._streams["accept"], tr.owner._streams["target"]]
        nflag = K + 1 if deferred else 0
        n32 = K + 1 + len(eos) + nflag
        host = torch.zeros(8 + (n32 + 1) // 2, dtype=torch.int64, pin_memory=True)
        words = host.numpy()
        words[:8] = _state_words(gens).view(np.int64).reshape(-1)
        small = words[8:].view(np.int32)
        small[:K] = ids
        small[K] = self.remaining
        small[K + 1:K + 1 + len(eos)] = eos
        small[K + 1 + len(eos):n32] = 1
        up = host.to(dev, non_blocking=True)
        states, small_d = up[:8].view(2, 4), up[8:].view(torch.int32)
        eos_kw = {}
        if eos:
            eos_kw = dict(eos_offsets=torch.tensor([0, len(eos)], dtype=torch.int64).pin_memory().to(dev, non_blocking=True),
                          eos_ids=small_d[K + 1:K + 1 + len(eos)])
        finite = None
        if deferred:
            finite = small_d[K + 1 + len(eos):n32]
            batch.rows_finite(rows, finite)
        return gens, states, small_d[:K], small_d[K:K + 1], eos_kw, finite

    def _device_decision(self, launch, K):
        """The decision of a device verifier ``launch()`` (returning its result,
        the two generators, their device states and the window's deferred
        finite flags or None), read back with the status, the draws used, the
        advanced states and the flags in one synchronisation; a non-finite
        window is reported first.  Each domain then takes its state and counts
        its draws."""
        res, gens, states, finite = launch()
        parts = [res.status.long(), res.accepted.long(), res.count.long(), res.pending.long(), res.stop.long(),
                 res.used_accept.long(), res.used_target.long(), res.ids.long().view(-1), states.view(-1)]
        if finite is not None:
            parts.append(finite.long().view(-1))
        out = torch.cat(parts).tolist()
        if finite is not None and not all(out[len(out) - finite.numel():]):
            raise ValidationError(_MSG_WINDOW)
        code, accepted, count, pending, stop, used_a, used_t = out[:7]
        out_ids, words = out[7:7 + K + 1], out[8 + K:16 + K]
        if code != N.OK:
            _raise_status(code)
        tr = self.transaction
        for g, used, domain, w in ((gens[0], used_a, "accept", words[0:2]), (gens[1], used_t, "target", words[4:6])):
            if used:
                _set_state(g, w[0], w[1])
                tr.draws[domain] += used
        return VerificationDecision(accepted, tuple(out_ids[:count]), None if pending < 0 else pending,
                                    {N.STOP_NONE: None, N.STOP_EOS: "eos", N.STOP_LENGTH: "length"}[stop])

    def _verify_logits(self, rows, ids, deferred):
        """verify_drafts (sampling.py:247-294) as one ``dsr_verify_drafts``
        call on the target and proposal logits (its fast path: no filter,
        history or bias), the accept test with the accept domain's next draws
        and the replacement or bonus draw with the target domain's, all taken
        on the device from the domains' PCG64 states.  Returns the launch's
        result, the two generators and their device states."""
        K, V = len(ids), self.owner.vocabulary
        dev = rows.device
        gens, states, ids_d, limit, eos_kw, finite = self._upload(ids, dev, rows, deferred)
        draft = torch.stack(self._draft_logits).reshape(1, K, V) if K else None
        try:
            res = batch.verify_drafts(rows.contiguous().reshape(1, K + 1, V), draft, ids_d,
                                      self.policy._device_tensor(dev), None, None, limit,
                                      rng_accept=states[0:1], rng_target=states[1:2], **eos_kw)
        except Exception:
            _require_finite(finite)
            raise
        return res, gens, states, finite

    def _verify_rows(self, rows, targets, status, ids, deferred):
        """verify_drafts (sampling.py:247-294) as one ``dsr_verify_probs`` call
        on the float64 target rows (row j conditioned on ``ids[:j]``,
        terminal_sampling.py:127-136) and the proposal rows the proposals
        were drawn from, with the accept and target draws taken on the device
        from the domains' PCG64 states; a target row whose launch failed on
        the device fails when the chain reaches it.  Returns what
        ``_verify_logits`` returns."""
        K, dev = len(ids), targets[0].device
        gens, states, ids_d, limit, eos_kw, finite = self._upload(ids, dev, rows, deferred)
        greedy = torch.ones(1, dtype=torch.uint8, device=dev) if self.policy.temperature == 0 else None
        try:
            res = batch.verify_probs(targets, self.proposal_rows, ids_d, limit, vocab=self.owner.vocabulary,
                                     greedy=greedy, rng_accept=states[0:1], rng_target=states[1:2],
                                     target_status=status, **eos_kw)
        except Exception:
            _require_finite(finite)
            raise
        return res, gens, states, finite

    def _digest_record(self):
        """The fields the decision digest covers (terminal_sampling.py:189-196).
        The two count hashes cover the transaction's frozen copies, so they
        are computed once per transaction (prepared() runs at prepare and
        again at commit)."""
        if self._counts_sha is None:
            self._counts_sha = _count_hashes(self._controls.counts, self._controls.generated)
        elif not isinstance(self._counts_sha, tuple):
            self._counts_sha = self._counts_sha.result()
        decision = asdict(self.decision)
        return {
            "decision": decision, "accepted_target_rows": self.decision.accepted_target_rows,
            "policy": self.policy.as_dict(), "RNG": self.transaction.prepared_state(),
            "seed": self.seed_token, "proposals": self.proposal_ids,
            "counts_sha256": self._counts_sha[0], "generated_counts_sha256": self._counts_sha[1],
            "logit_bias": self.logit_bias, "grammar_identity": self.grammar_identity,
            "stop_identity": self.stop_identity, "remaining": self.remaining, "eos_ids": sorted(self.eos_ids),
        }

    def prepared(self):
        """The decision and the SHA-256 digest every stage must commit against."""
        self._require_open()
        if self._stage is not _Stage.DECIDED or self._stop_pending:
            raise ValidationError("terminal decision has not been computed")
        return {"decision": asdict(self.decision), "accepted_target_rows": self.decision.accepted_target_rows,
                "digest": fingerprint(self._digest_record())}

    def apply_stop(self, tracker):
        """Cut the decision at a stop string the frozen tracker finds in its output."""
        self._require_open()
        if self._stage is not _Stage.DECIDED or not self._stop_pending or self.stop_identity != tracker.identity:
            raise ValidationError("stop processing lacks the exact frozen terminal decision/prefix")
        found = tracker.preview(self.decision.output_ids)
        if found.matched is not None:
            self.decision = _cut_at_stop(self.decision, found.token_count)
        self._stop_pending = False
        return self.decision

    def commit(self, expected_digest):
        self._require_open()
        if self.prepared()["digest"] != expected_digest:
            raise ValidationError("all-stage commit does not match the prepared terminal decision/RNG")
        self.transaction.commit()
        self._close()
        return self.decision

    def abort(self):
        self._require_open()
        self.transaction.abort()
        self._close()

    def _close(self):
        self.closed = True
        self.owner.active = None
        if self._counts_sha is not None and not isinstance(self._counts_sha, tuple):
            self._counts_sha.cancel()   # a hash not yet started is dropped


def _cut_at_stop(decision, kept):
    """The decision with its output cut to ``kept`` tokens by a stop string
    (terminal_sampling.py:200-216).  A seed keeps its token as the pending
    one; a cut inside the accepted drafts drops the pending token and the
    later drafts; a cut at the replacement or bonus token keeps it pending."""
    if isinstance(decision, SeedDecision):
        return replace(decision, stop_reason="stop")
    cut = {"output_ids": decision.output_ids[:kept], "stop_reason": "stop"}
    if kept <= decision.accepted_drafts:
        cut.update(accepted_drafts=kept, pending_token=None)
    return replace(decision, **cut)
