"""Drop-in replacement of the reference's terminal sampling transaction.

Same classes and behaviour as src/deepseekrpc/terminal_sampling.py:
``TerminalSampler`` (:48-106), ``SamplingWork`` (:109-231), ``SeedDecision``
(:30-45) and the lazy ``_ConditionalTargets`` (:234-244).  The difference is
where the rows live: the reference copies every FP32 logit row to the host
(``_logits_cpu``, :16-27); here logits stay on the GPU and every
distribution, draw and verification runs through the HIP library.  Host
logic (counts bookkeeping, the RNG transaction, grammar callbacks, digests)
is unchanged.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, replace
import hashlib

import numpy as np
import torch

from .jsonutil import ValidationError, fingerprint, hex_id, integer
from .sampling import (_COUNTS_MSG, RandomStreams, SamplingPolicy, _history_table, _logit_vector, _on_device,
                       _raise_status, categorical, verify_drafts)


def _logits_device(logits, rows, vocabulary):
    """A bounded logit window on the GPU: ``[rows, vocabulary]`` FP32, all finite."""
    if isinstance(logits, np.ndarray):
        if logits.dtype != np.float32 or logits.shape != (rows, vocabulary) or not np.isfinite(logits).all():
            raise ValidationError("terminal logits do not match the complete bounded vocabulary window")
        result, _ = _on_device(logits)
        return result
    if not isinstance(logits, torch.Tensor) or not logits.is_cuda or logits.dtype != torch.float32:
        raise ValidationError("terminal logits must come from the actual FP32 CUDA vocabulary head")
    if tuple(logits.shape) != (rows, vocabulary) or not bool(torch.isfinite(logits).all()):
        raise ValidationError("terminal logits do not match the complete bounded vocabulary window")
    return logits.detach().contiguous()


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
        return 0


class TerminalSampler:
    def __init__(self, seed, *, vocabulary=129280):
        self.random = RandomStreams(seed)
        self.vocabulary = integer(vocabulary, "sampling vocabulary", 1, 129280)
        self.active = None

    def _begin(self, policy, counts, remaining, eos_ids, *, generated_counts, logit_bias, allowed, grammar_identity,
               stop_identity):
        integer(remaining, "remaining output capacity", 1, 1048576)
        if self.active is not None or not isinstance(policy, SamplingPolicy):
            raise ValidationError("terminal sampling is active or its policy is invalid")
        counts = np.asarray(counts)
        if (counts.shape != (self.vocabulary,) or counts.dtype not in (np.int32, np.int64) or (counts < 0).any()
                or counts.sum(dtype=np.int64) > 1048576):
            raise ValidationError("terminal counts differ from the exact published token history")
        for token in eos_ids:
            integer(token, "terminal EOS token", 0, self.vocabulary - 1)
        if allowed is not None and not callable(allowed):
            raise ValidationError("grammar mask provider must evaluate a bounded tentative token prefix")
        if (allowed is None) != (grammar_identity is None):
            raise ValidationError("a grammar mask requires its frozen grammar/prefix identity")
        if grammar_identity is not None:
            hex_id(grammar_identity, 64, "frozen grammar and committed-prefix identity")
        if stop_identity is not None:
            hex_id(stop_identity, 64, "frozen original detokenizer and stop-prefix identity")
        generated = counts if generated_counts is None else np.asarray(generated_counts)
        if (generated.shape != counts.shape or generated.dtype not in (np.int32, np.int64) or (generated < 0).any()
                or (generated > counts).any()):
            raise ValidationError("generated sampling counts must be a subset of the complete history")
        # The caller cannot mutate the controls of a running transaction.
        bias = None if logit_bias is None else dict(logit_bias)
        work = SamplingWork(self, self.random.begin(), policy, counts.copy(), generated.copy(), remaining,
                            frozenset(eos_ids), bias, allowed, grammar_identity, stop_identity)
        self.active = work
        return work

    def begin_seed(self, logits, *, policy, counts, remaining, eos_ids=frozenset(), generated_counts=None,
                   logit_bias=None, allowed=None, grammar_identity=None, stop_identity=None):
        work = self._begin(policy, counts, remaining, eos_ids, generated_counts=generated_counts, logit_bias=logit_bias,
                           allowed=allowed, grammar_identity=grammar_identity, stop_identity=stop_identity)
        try:
            values = _logits_device(logits, 1, self.vocabulary)[0]
            distribution = work.distribution(values, ())
            token = categorical(distribution, lambda: work.transaction.random("target"))
            work.decision = SeedDecision(token, "eos" if token in work.eos_ids else "length" if remaining == 1 else None)
            return work
        except BaseException:
            work.abort()
            raise

    def begin_verification(self, *, seed_token, policy, counts, remaining, eos_ids=frozenset(), generated_counts=None,
                           logit_bias=None, allowed=None, grammar_identity=None, stop_identity=None):
        integer(seed_token, "pending verification seed", 0, self.vocabulary - 1)
        work = self._begin(policy, counts, remaining, eos_ids, generated_counts=generated_counts, logit_bias=logit_bias,
                           allowed=allowed, grammar_identity=grammar_identity, stop_identity=stop_identity)
        if work.counts[seed_token] < 1 or work.generated_counts[seed_token] < 1:
            work.abort()
            raise ValidationError("pending seed must already belong to published sampling history")
        work.seed_token = seed_token
        return work


class SamplingWork:
    def __init__(self, owner, transaction, policy, counts, generated_counts, remaining, eos_ids, logit_bias, allowed,
                 grammar_identity, stop_identity):
        self.owner, self.transaction, self.policy = owner, transaction, policy
        self.counts, self.remaining, self.eos_ids = counts, remaining, eos_ids
        self.generated_counts = generated_counts
        self.logit_bias, self.allowed = logit_bias, allowed
        self.grammar_identity = grammar_identity
        self.stop_identity = stop_identity
        self._stop_checked = stop_identity is None
        self.seed_token = None
        self.proposal_ids, self.proposal_rows = [], []
        self.decision, self.closed = None, False
        self._proposal_ready = False
        self._table = None  # device history table of counts / generated_counts, built on first use

    def _open(self):
        if self.closed or self.owner.active is not self:
            raise ValidationError("terminal sampling transaction is closed or stale")

    def distribution(self, logits, prefix):
        """Device distribution of one row conditioned on a tentative prefix
        (terminal_sampling.py:127-136): the transaction's counts live in one
        device history table, and each prefix token is appended to it on the
        device (one more count and generated count each) instead of copying
        and updating the dense vectors on the host."""
        self._open()
        n, device_input = _logit_vector(logits)
        if n != len(self.counts):
            raise ValidationError(_COUNTS_MSG)
        table = self._history(prefix)
        mask = None if self.allowed is None else self.allowed(tuple(prefix))
        return self.policy._probabilities_with(logits, n, device_input, table, self.logit_bias, mask)

    def _history(self, prefix):
        if self._table is None:
            self._table = _history_table(self.counts, self.generated_counts, len(self.counts))
        if not prefix:
            return self._table
        dev = self._table.offsets.device
        tokens = torch.tensor([int(t) for t in prefix], dtype=torch.int32, device=dev)
        off = torch.tensor([0, len(prefix)], dtype=torch.int64, device=dev)
        table, status = self._table.append(tokens, off, vocab=len(self.counts))
        if int(status.item()) != 0:
            _raise_status(int(status.item()))
        return table

    def propose(self, graph, result):
        """Sequential Markov-conditioned proposals over the five-row draft graph."""
        self._open()
        if self.seed_token is None or self._proposal_ready or self.decision is not None:
            raise ValidationError("proposal generation is duplicate or lacks a committed pending seed")
        try:
            previous = self.seed_token
            for row in range(min(5, self.remaining)):
                # The graph applies the conditional Markov bias; its confidence never prunes.
                logits, _confidence = graph.draft_conditional_logits(result, row, previous)
                values = _logits_device(logits, 1, self.owner.vocabulary)[0]
                distribution = self.distribution(values, self.proposal_ids)
                token = categorical(distribution, lambda: self.transaction.random("draft"))
                self.proposal_rows.append(distribution)
                self.proposal_ids.append(token)
                previous = token
                if token in self.eos_ids:
                    break
            self._proposal_ready = True
            return tuple(self.proposal_ids)
        except BaseException:
            self.abort()
            raise

    def use_normal_decode(self):
        """Explicit no-proposal path, including the end of context."""
        self._open()
        if self.seed_token is None or self._proposal_ready:
            raise ValidationError("normal decode is duplicate or lacks its pending seed")
        self._proposal_ready = True

    def verify(self, target_logits):
        self._open()
        if self.seed_token is None or not self._proposal_ready or self.decision is not None:
            raise ValidationError("target verification is duplicate or proposals are not complete")
        try:
            values = _logits_device(target_logits, len(self.proposal_ids) + 1, self.owner.vocabulary)
            targets = _ConditionalTargets(self, values)
            self.decision = verify_drafts(targets, self.proposal_rows, self.proposal_ids, self.transaction,
                                          greedy=self.policy.temperature == 0, output_limit=self.remaining,
                                          eos_ids=self.eos_ids)
            return self.decision
        except BaseException:
            self.abort()
            raise

    def prepared(self):
        self._open()
        if self.decision is None or not self._stop_checked:
            raise ValidationError("terminal decision has not been computed")
        data = {"decision": asdict(self.decision), "accepted_target_rows": self.decision.accepted_target_rows,
                "policy": self.policy.as_dict(), "RNG": self.transaction.prepared_state(),
                "seed": self.seed_token, "proposals": self.proposal_ids,
                "counts_sha256": hashlib.sha256(self.counts.astype("<i8").tobytes()).hexdigest(),
                "generated_counts_sha256": hashlib.sha256(self.generated_counts.astype("<i8").tobytes()).hexdigest(),
                "logit_bias": self.logit_bias, "grammar_identity": self.grammar_identity,
                "stop_identity": self.stop_identity, "remaining": self.remaining, "eos_ids": sorted(self.eos_ids)}
        return {"decision": asdict(self.decision), "accepted_target_rows": self.decision.accepted_target_rows,
                "digest": fingerprint(data)}

    def apply_stop(self, tracker):
        """Trim a stop string inside accepted proposals before any target GPU finish."""
        self._open()
        if self.decision is None or self._stop_checked or self.stop_identity != tracker.identity:
            raise ValidationError("stop processing lacks the exact frozen terminal decision/prefix")
        preview = tracker.preview(self.decision.output_ids)
        if preview.matched is not None:
            count = preview.token_count
            if isinstance(self.decision, SeedDecision):
                self.decision = replace(self.decision, stop_reason="stop")
            elif count <= self.decision.accepted_drafts:
                self.decision = replace(self.decision, accepted_drafts=count, output_ids=self.decision.output_ids[:count],
                                        pending_token=None, stop_reason="stop")
            else:
                self.decision = replace(self.decision, output_ids=self.decision.output_ids[:count], stop_reason="stop")
        self._stop_checked = True
        return self.decision

    def commit(self, expected_digest):
        self._open()
        if self.prepared()["digest"] != expected_digest:
            raise ValidationError("all-stage commit does not match the prepared terminal decision/RNG")
        self.transaction.commit()
        self.closed, self.owner.active = True, None
        return self.decision

    def abort(self):
        self._open()
        self.transaction.abort()
        self.closed, self.owner.active = True, None


class _ConditionalTargets:
    """Lazy, cached target distributions; row j sees the accepted prefix proposal_ids[:j]."""

    def __init__(self, work, values):
        self.work, self.values, self.cache = work, values, {}

    def __len__(self):
        return len(self.values)

    def __getitem__(self, index):
        if index not in self.cache:
            self.cache[index] = self.work.distribution(self.values[index], self.work.proposal_ids[:index])
        return self.cache[index]
