"""Throughput of the fused sampling kernels on one MI355X.

Default workload (c3, the headline): 256 rows x 129,280-token bf16 logits
with a heavy tail (N(0,1) plus 32 spikes of +U[8,15] per row), per-row
temperature U[0.2,1.5], top-k U{1..1024}, top-p U[0.5,1], a packed allow
bitmask disallowing 10% of tokens, one pre-drawn uniform per row.  Inputs are
resident in HBM before the timed region; one step is one ``dsr_sample_rows``
launch over the batch.

``--workload`` selects one of the other seeded row families instead (see
deepseekrpc_amd/workloads.py): c1 (1 fp32 row with probabilities out), c2 (64
bf16 rows with 4,096-token histories), c4 (32 verifier requests x 4 fp32
drafts; one step is one ``dsr_verify_drafts`` call), c5 (1,024 bf16 rows,
mixed greedy, 16,384-token histories), whole (256 bf16 rows whose policies
set no top-k: the reference's default, top-p only, min-p only), hist (1,024
rows x 16,384 token ids built into device history tables; one step is one
``dsr_history_append`` call), and three drop-in workloads that time the
reference's API as its callers use it (host dense counts, FP32 CUDA rows):
propose (one 5-row proposal step drawn on the device), seed (one
``TerminalSampler.begin_seed`` call) and step (one speculative decode step:
proposals, verification against six target rows, the prepared digest).

Distinct input batches rotate through the timed region: the workload's rows
with their vocabulary positions rolled by a different shift each
(``workloads.rolled``), enough of them to exceed 256 MB together, so no step
reads its inputs from the 256 MB Infinity Cache a previous step filled.

Prints one JSON line: the throughput, the roofline of the step (algorithmic
HBM bytes / HIP-event time of the launches on their stream, against 8 TB/s)
and the CPU baseline: the float64 oracle (a restatement of the reference's
NumPy sampler) timed on the host over a bounded sample of the same workload,
on 16 worker processes (the host's CPU share for one GPU) and on one process
alone.
"""
from __future__ import annotations

import argparse
import json
import multiprocessing as mp
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PEAK_HBM_GBS = 8000.0

# name -> (metric, unit, CPU sample passes over the workload's rows, kernels of one step)
WORKLOADS = {
    "c3": ("sampled rows/sec at B=256×V=129,280 bf16; % of HBM roofline", "rows/s", 5,
           "k_sample_bf16_fast"),
    "c3f32": ("sampled rows/sec at B=256×V=129,280 fp32; % of HBM roofline", "rows/s", 5,
              "k_sample_f32"),
    "c1": ("sampled rows/sec at B=1×V=129,280 fp32 with fp32 probabilities out", "rows/s", 1000,
           "k_zero_probs + k_sample_f32"),
    "c2": ("sampled rows/sec at B=64×V=129,280 bf16 with 4,096-token histories", "rows/s", 20,
           "k_sample_bf16_full"),
    "c4": ("verify-rows/sec at B=32 requests × K=4 drafts × V=129,280 fp32", "verify-rows/s", 60,
           "k_verify_stats + k_verify_chain + k_verify_draw + k_verify_finish"),
    "c5": ("sampled rows/sec at B=1024×V=129,280 bf16, mixed greedy, 16,384-token histories", "rows/s", 2,
           "k_sample_bf16_full"),
    "hist": ("history rows/sec: 1,024 rows x 16,384 token ids -> sparse count tables over V=129,280", "rows/s", 10,
             "k_history_append (count) + k_history_offsets + k_history_append (write)"),
    "whole": ("sampled rows/sec at B=256×V=129,280 bf16 with no top-k (default / top-p / min-p policies)", "rows/s",
              5, "k_sample_bf16_full"),
    "step": ("drop-in speculative steps/sec: propose 5 rows on the device, verify against 6 fp32 rows, digest",
             "steps/s", 30, "k_zero_probs + k_sample_f32 (each proposal; the six targets in one launch) + "
             "k_rows_finite + k_vprobs_stats + k_vprobs_chain + k_vprobs_draw + k_vprobs_finish"),
    "seed": ("drop-in TerminalSampler.begin_seed calls/sec (1 fp32 row, V=129,280, dense counts)", "calls/s",
             300, "k_rows_finite + k_zero_probs + k_sample_f32 (a policy without penalties carries no history "
             "table)"),
    "head": ("verify-rows/sec with the vocabulary projection: B=32 requests × K=4 drafts, 160 target rows × "
             "dim 5,120 → V=129,280 fp32 logits", "verify-rows/s", 30,
             "k_vocab_head + k_head_shares + k_verify_chain + k_verify_draw + k_verify_finish"),
    "headk": ("sampled rows/sec with the vocabulary projection: 8 rows × dim 5,120 → V=129,280 fp32 logits, top-k "
              "50 sampled from the projection's per-tile records", "rows/s", 32,
              "k_vocab_head + k_sample_f32 (from the records)"),
    "propose": ("drop-in 5-row draft proposal steps/sec at V=129,280 fp32, one host synchronisation per step",
                "chains/s", 100, "k_zero_probs + k_sample_f32 (5x; a policy without penalties carries no "
                "history table)"),
}

# Name prefix of a workload's committed profile summaries when it is not its first kernel's.
PROFILE_PREFIX = {"c4": "k_verify", "c1": "k_sample_f32", "propose": "k_sample_f32", "seed": "k_sample_f32",
                  "step": "k_sample_f32",
                  "head": "k_vocab_head", "headk": "k_vocab_head"}

DESCRIPTIONS = {
    "c1": "c1: 1 row x 129280 fp32 N(0,2^2), T 0.7, top-k 50, top-p 0.9, fp32 probabilities out",
    "c2": "c2: 64 rows x 129280 bf16 N(0,3^2), 4096-token generated histories, rep 1.1 / pres 0.5 / freq 0.3, "
          "T 1, top-p 0.95",
    "c3": "c3: 256 rows x 129280 bf16 heavy-tail logits, per-row T/top-k/top-p, 10% allow mask",
    "c3f32": "c3f32: c3's rows as fp32 logits (before bf16 rounding), per-row T/top-k/top-p, 10% allow mask",
    "c4": "c4: 32 requests x 4 drafts, fp32 target [32,5,129280] and draft [32,4,129280], default policy, limit 10",
    "c5": "c5: 1024 rows x 129280 bf16 (N(0,1) / near-flat with 8-way max ties), even rows greedy, odd rows T 1 "
          "top-p 0.9, rep 1.1 / pres 0.5 / freq 0.3 over 16384-token histories",
    "hist": "hist: 1024 rows x 16384 token ids U{0..129279}, all generated, appended into an empty history table "
            "(one dsr_history_append call)",
    "whole": "whole: 256 rows x 129280 bf16 heavy-tail logits, 10% allow mask, no top-k: default policy, "
             "top-p ~ U[0.8,0.99], min-p 0.05, top-p 0.95 + min-p 0.01 (by row mod 4)",
    "step": "step: TerminalSampler.begin_verification, SamplingWork.propose over a device graph (5 fp32 rows x "
            "129280 N(0,2^2), previous token +4), verify against 6 fp32 target rows (base + N(0,0.25^2)), prepared "
            "digest, then abort; T 0.7 / top-k 50 / top-p 0.9, dense int32 counts of a 64-token history",
    "seed": "seed: TerminalSampler.begin_seed then abort on 1 fp32 row x 129280 N(0,2^2), T 0.7 / top-k 50 / "
            "top-p 0.9, dense int32 counts of a 64-token history (the reference's calling pattern)",
    "head": "head: the terminal stage's vocabulary projection of 32 requests x 5 target rows (bf16 hidden "
            "[160, 5120] x bf16 weight [129280, 5120] -> fp32 logits with per-tile verifier records), then "
            "verification of 4 drafts per request whose rows and records came from the same projection; default "
            "policy, limit 10",
    "headk": "headk: the terminal stage's vocabulary projection of 8 rows (bf16 hidden [8, 5120] x bf16 weight "
             "[129280, 5120] -> fp32 logits with per-tile records), then top-k sampling of every row from the "
             "records (T 0.7, top-k 50, top-p 0.9, pre-drawn uniforms)",
    "propose": "propose: TerminalSampler.begin_verification, SamplingWork.propose over a device graph, then abort; "
               "5 fp32 rows x 129280 N(0,2^2), row j = base j with the previous token raised by 4 on the device, "
               "T 0.7 / top-k 50 / top-p 0.9, dense int32 counts of a 64-token history, draft PCG64 draws on the "
               "device",
}

_CPU = {}


def _units(name, w):
    """Rows of a sampling or history workload; requests of the verifier workloads."""
    if name == "c4":
        return w.extra["target"].shape[0]
    if name == "head":
        return w.extra["requests"]
    if name == "headk":
        return w.extra["rows"]
    if name in ("propose", "seed", "step"):
        return 1
    return w.extra["tokens"].shape[0] if name == "hist" else w.rows


def _draft_ids_cpu(e, r):
    """Draft ids of request r drawn from its draft rows by the oracle (the
    proposal step the GPU run performs with the sampling kernel)."""
    from oracle import sampling_oracle as O
    ids = []
    for j in range(e["K"]):
        ids.append(O.sample_row(e["draft"][r][j], O.Policy(), float(e["u_draft"][r][j]), keep_probs=False).token)
    return ids


def _cpu_rows(span):
    from oracle import history_oracle as H
    from oracle import sampling_oracle as O
    w, name = _CPU["w"], _CPU["name"]
    lo, hi = span
    V = w.logits.shape[1]
    if name == "hist":
        toks = w.extra["tokens"]
        rows = [toks[r % toks.shape[0]] for r in range(lo, hi)]
        t0 = time.perf_counter()
        for row in rows:
            H.append(None, None, None, None, [row], V)
        return hi - lo, time.perf_counter() - t0
    if name == "propose":
        return hi - lo, _cpu_chains(w, hi - lo)
    if name == "step":
        return hi - lo, _cpu_steps(w, hi - lo)
    if name == "headk":
        e = w.extra
        t0 = time.perf_counter()
        for r in range(lo, hi):
            r %= e["rows"]
            O.sample_row(e["cpu_logits"][r], O.Policy(**w.policies[r]), float(w.uniforms[r]), keep_probs=False)
        return hi - lo, time.perf_counter() - t0
    if name == "head":
        e = w.extra
        t0 = time.perf_counter()
        for r in range(lo, hi):
            r %= e["requests"]
            O.verify(e["cpu_target"][r], e["cpu_draft"][r], e["cpu_ids"][r], O.Policy(), e["u_accept"][r],
                     float(e["u_target"][r]), output_limit=int(e["limit"][r]))
        return hi - lo, time.perf_counter() - t0
    if name == "seed":
        counts = np.bincount(np.asarray(w.histories[0]), minlength=V).astype(np.int32)
        gen = np.random.default_rng(w.extra["rng_seed"])
        t0 = time.perf_counter()
        for _ in range(hi - lo):
            probe = np.random.Generator(np.random.PCG64(0))
            probe.bit_generator.state = gen.bit_generator.state
            O.sample_row(w.logits[0], O.Policy(**w.policies[0]), float(probe.random()), counts, counts)
        return hi - lo, time.perf_counter() - t0
    jobs = []
    for r in range(lo, hi):
        r = r % _units(name, w)
        if name == "c4":
            jobs.append((r, _draft_ids_cpu(w.extra, r)))
        else:
            counts = None
            if w.histories is not None:
                counts = np.bincount(np.asarray(w.histories[r]), minlength=V).astype(np.int32)
            jobs.append((r, counts))
    t0 = time.perf_counter()  # input preparation above is not timed
    for r, x in jobs:
        if name == "c4":
            e = w.extra
            O.verify(e["target"][r], e["draft"][r], x, O.Policy(), e["u_accept"][r], float(e["u_target"][r]),
                     output_limit=int(e["limit"][r]))
        else:
            allowed = None if w.allowed is None else w.allowed[r]
            O.sample_row(w.logits[r], O.Policy(**w.policies[r]), float(w.uniforms[r]), x, x, None, allowed,
                         keep_probs=name == "c1")
    return hi - lo, time.perf_counter() - t0


def _cpu_chains(w, n):
    """n proposal chains by the oracle: each row conditioned on the previous
    token (the +4 bias) and on the prefix counts, the draft uniform drawn only
    when needed (terminal_sampling.py:138-161)."""
    from oracle import sampling_oracle as O
    V = w.logits.shape[1]
    counts0 = np.bincount(np.asarray(w.histories[0]), minlength=V).astype(np.int32)
    gen = np.random.default_rng(w.extra["rng_seed"])
    t0 = time.perf_counter()
    for _ in range(n):
        counts, previous = counts0.copy(), w.extra["seed_token"]
        for j in range(w.extra["steps"]):
            row = w.logits[j].copy()
            row[previous] += np.float32(w.extra["bump"])
            probe = np.random.Generator(np.random.PCG64(0))
            probe.bit_generator.state = gen.bit_generator.state
            ref = O.sample_row(row, O.Policy(**w.policies[0]), float(probe.random()), counts, counts, keep_probs=True)
            if ref.consumed:
                gen.random()
            counts[ref.token] += 1
            previous = ref.token
    return time.perf_counter() - t0


def _cpu_steps(w, n):
    """n speculative steps by the oracle, as the reference runs them: the
    proposal chain (each row conditioned on the previous token and the prefix
    counts, its distribution kept), then verification with each target row's
    distribution computed when the step first reaches it
    (terminal_sampling.py:138-183, sampling.py:247-294)."""
    from oracle import sampling_oracle as O
    V = w.logits.shape[1]
    pol = O.Policy(**w.policies[0])
    counts0 = np.bincount(np.asarray(w.histories[0]), minlength=V).astype(np.int32)
    gen = np.random.default_rng(w.extra["rng_seed"])
    t0 = time.perf_counter()
    for _ in range(n):
        counts, previous, ids, rows = counts0.copy(), w.extra["seed_token"], [], []
        for j in range(w.extra["steps"]):
            row = w.logits[j].copy()
            row[previous] += np.float32(w.extra["bump"])
            ref = O.sample_row(row, pol, float(gen.random()), counts, counts, keep_probs=True)
            counts[ref.token] += 1
            ids.append(ref.token)
            rows.append(ref.probs)
            previous = ref.token

        class Targets:
            def __len__(self):
                return len(ids) + 1

            def __getitem__(self, j):
                c = counts0.copy()
                for t in ids[:j]:
                    c[t] += 1
                return O.probabilities(w.extra["target"][j], pol, c, c)

        O.verify_probs(Targets(), rows, ids, lambda domain: float(gen.random()), greedy=False,
                       output_limit=1048576)
    return time.perf_counter() - t0


def _head_cpu_rows(w):
    """The head workload's logits for the CPU sample, by NumPy's float32
    product of the same bf16 values, and draft ids drawn from the draft rows
    by the oracle (both untimed: the reference projects on its GPU and
    samples the copied rows on the host, so only the verification is timed)."""
    from deepseekrpc_amd import workloads
    from oracle import sampling_oracle as O
    e = w.extra
    R, K, V = e["requests"], e["K"], e["weight_q"].shape[0]
    wt = e["weight_q"].astype(np.float32)
    wt *= np.float32(workloads.head_weight_scale())
    e["cpu_target"] = (e["hidden_target"] @ wt.T).reshape(R, K + 1, V)
    e["cpu_draft"] = (e["hidden_draft"] @ wt.T).reshape(R, K, V)
    del wt
    e["cpu_ids"] = [[O.sample_row(e["cpu_draft"][r][j], O.Policy(), float(e["u_draft"][r][j]),
                                  keep_probs=False).token for j in range(K)] for r in range(R)]


def _headk_cpu_rows(w):
    """The headk workload's logits for the CPU sample, by NumPy's float32
    product of the same bf16 values (untimed: the reference projects on its
    GPU and samples the copied rows on the host, so only the sampling is
    timed)."""
    from deepseekrpc_amd import workloads
    e = w.extra
    wt = e["weight_q"].astype(np.float32)
    wt *= np.float32(workloads.head_weight_scale())
    e["cpu_logits"] = e["hidden"] @ wt.T
    del wt


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# Worker processes of the CPU baseline: the host's CPU share for one GPU
# (pools are sized by that share, not by os.cpu_count(), which counts every
# CPU of the machine).
CPU_WORKERS = 16


def cpu_baseline(name, w, passes):
    """Oracle throughput on the host: CPU_WORKERS forked workers with the
    sample split evenly, then one worker alone on an eighth of the sample
    (the single-core figure); run before the GPU is initialised."""
    if name == "head":
        _head_cpu_rows(w)
    if name == "headk":
        _headk_cpu_rows(w)
    _CPU.update(w=w, name=name)
    os.environ["OMP_NUM_THREADS"] = "1"
    cores = max(1, min(CPU_WORKERS, os.cpu_count() or 1))
    total = _units(name, w) * passes
    edges = np.linspace(0, total, cores + 1).astype(int)
    spans = [(int(a), int(b)) for a, b in zip(edges[:-1], edges[1:]) if b > a]
    with mp.get_context("fork").Pool(cores) as pool:
        pool.map(_cpu_rows, [(0, 1)] * cores)            # warm the workers
        t0 = time.perf_counter()
        done = pool.map(_cpu_rows, spans, chunksize=1)
        wall = time.perf_counter() - t0
    with mp.get_context("fork").Pool(1) as pool:   # one process alone: the single-core figure
        pool.map(_cpu_rows, [(0, 1)])
        one_n, one_wall = pool.map(_cpu_rows, [(0, max(1, total // 8))])[0]
    n = sum(d[0] for d in done)
    busy = sum(d[1] for d in done)
    unit = WORKLOADS[name][1]
    what = {"c4": "requests", "head": "requests", "propose": "chains", "seed": "calls", "step": "steps"}.get(name, "rows")
    oracle = "NumPy history oracle (np.add.at on dense counts)" if name == "hist" else "float64 NumPy oracle"
    if name in ("head", "headk"):
        oracle += (f" ({'verification' if name == 'head' else 'sampling'} only: the reference projects on its "
                   "GPU; the rows' logits were computed beforehand by NumPy's float32 product, untimed)")
    return {"value": n / wall, "unit": unit, "cores": cores, "kind": "port",
            "value_1core": one_n / one_wall, "host_cpus": os.cpu_count(), "cpu_model": _cpu_model(),
            "sample": f"{n} {what} ({passes} pass(es) over the {_units(name, w)} of the same workload, "
                      f"{busy:.1f} s of CPU work) with the {oracle} on {cores} worker processes; "
                      f"{one_n} {what} on one process alone: {one_n / one_wall:.2f} {unit}"}


class _HistResult:
    """Status and (empty) flags of a history build, shaped like a sampling result."""

    def __init__(self, status):
        import torch
        self.status = status
        self.flags = torch.zeros_like(status)


_DONE = []


def _done_result():
    """A status-OK result for the drop-in legs (which raise on any error),
    made once so that the timed calls allocate nothing for it."""
    if not _DONE:
        import torch
        _DONE.append(_HistResult(torch.zeros(1, dtype=torch.int32, device="cuda")))
    return _DONE[0]


# Inputs rotated through the timed region exceed this many bytes together.
ROTATION_BYTES = 300 * 2**20


def _batch_bytes(name, w):
    if name in ("head", "headk"):
        return w.extra["weight_q"].nbytes * 2   # the bf16 weight
    if name == "hist":
        return w.extra["tokens"].nbytes
    if name in ("propose", "seed"):
        return w.logits.nbytes
    if name == "step":
        return w.logits.nbytes + w.extra["target"].nbytes
    if name == "c4":
        return w.extra["target"].nbytes + w.extra["draft"].nbytes
    return w.logits.shape[0] * w.logits.shape[1] * (2 if w.dtype == "bf16" else 4)


def variants(name, w):
    """Distinct input batches of the workload (vocabulary layouts rolled by
    different shifts), at least 4 and together above ROTATION_BYTES."""
    from deepseekrpc_amd import workloads
    if name in ("head", "headk"):
        return [w]   # its weight stream (1.3 GB per step) is read from HBM on every step
    count = max(4, -(-ROTATION_BYTES // max(1, _batch_bytes(name, w))))
    V = w.logits.shape[1]
    return [w] + [workloads.rolled(w, (i * 7919) % V) for i in range(1, count)]


class _Chain:
    """One drop-in proposal step per launch, as the reference's callers make
    it: TerminalSampler.begin_verification with dense counts, then
    SamplingWork.propose over a graph that makes each row on the device (the
    Markov bias step reads the previous token the sampling kernel wrote), so
    the five rows take one host synchronisation; then abort, which restores
    the RNG domains, so every step is the same."""

    def __init__(self, w):
        import torch

        from deepseekrpc_amd.sampling import SamplingPolicy
        from deepseekrpc_amd.terminal_sampling import TerminalSampler
        self.w = w
        self.base = torch.from_numpy(w.logits).cuda()
        self.bump = torch.full((1,), float(w.extra["bump"]), device="cuda")
        self.sampler = TerminalSampler(w.extra["rng_seed"])
        self.policy = SamplingPolicy(**w.policies[0])
        self.counts = np.bincount(np.asarray(w.histories[0]), minlength=w.logits.shape[1]).astype(np.int32)
        self.inputs = (self.base,)
        self.launch()

    def draft_conditional_logits_device(self, result, row, previous):
        out = self.base[row].clone()
        out.index_add_(0, previous.long(), self.bump)
        return out.reshape(1, -1), None

    def launch(self):
        import torch
        work = self.sampler.begin_verification(seed_token=self.w.extra["seed_token"], policy=self.policy,
                                               counts=self.counts, remaining=9)
        ids = work.propose(self, None)
        if len(ids) != self.w.extra["steps"]:
            raise SystemExit(f"the proposal chain stopped after {len(ids)} rows")
        work.abort()
        self.result = _done_result()
        return self


class _Step(_Chain):
    """One drop-in speculative decode step per launch: begin_verification,
    propose over the device graph, verify against the target rows, the
    prepared digest, then abort (which restores the RNG domains)."""

    def __init__(self, w):
        import torch
        self.target = torch.from_numpy(w.extra["target"]).cuda()
        super().__init__(w)

    def launch(self):
        import torch
        work = self.sampler.begin_verification(seed_token=self.w.extra["seed_token"], policy=self.policy,
                                               counts=self.counts, remaining=9)
        ids = work.propose(self, None)
        work.verify(self.target[: len(ids) + 1])
        work.prepared()
        work.abort()
        self.result = _done_result()
        return self


class _Seed:
    """One drop-in call per launch: TerminalSampler.begin_seed on one FP32
    CUDA row with dense count vectors, as the reference's callers make it,
    then abort (which restores the RNG domains, so every call is the same)."""

    def __init__(self, w):
        import torch

        from deepseekrpc_amd.sampling import SamplingPolicy
        from deepseekrpc_amd.terminal_sampling import TerminalSampler
        self.sampler = TerminalSampler(w.extra["rng_seed"])
        self.policy = SamplingPolicy(**w.policies[0])
        self.logits = torch.from_numpy(w.logits).cuda()
        self.counts = np.bincount(np.asarray(w.histories[0]), minlength=w.logits.shape[1]).astype(np.int32)
        self.inputs = (self.logits,)
        self.launch()

    def launch(self):
        import torch
        work = self.sampler.begin_seed(self.logits, policy=self.policy, counts=self.counts, remaining=9)
        work.abort()
        self.result = _done_result()
        return self


class _Head:
    """One verification step at the terminal stage: the vocabulary projection
    of the 160 target rows with its records, then dsr_verify_drafts_head
    against the draft rows and records projected at proposal time (setup).
    ``fused=False`` is the same step without records: the projection alone,
    then the verifier's statistics pass over the logits."""

    def __init__(self, w, fused=True):
        import torch

        from deepseekrpc_amd import batch, workloads
        e = w.extra
        R, K = e["requests"], e["K"]
        dev = "cuda"
        self.weight = (torch.from_numpy(e["weight_q"]).to(dev).to(torch.bfloat16)
                       * workloads.head_weight_scale()).contiguous()
        xt = torch.from_numpy(e["hidden_target"]).to(dev).to(torch.bfloat16)
        xd = torch.from_numpy(e["hidden_draft"]).to(dev).to(torch.bfloat16)
        self.policies = batch.policy_tensor(w.policies, dev)
        self.th = batch.vocab_head(xt, self.weight, policies=self.policies, rows_per_policy=K + 1, records=fused)
        self.dh = batch.vocab_head(xd, self.weight, policies=self.policies, rows_per_policy=K, records=fused)
        V = self.weight.shape[0]
        draw = batch.sample_rows(self.dh.logits, [dict()] * (R * K),
                                 uniforms=torch.from_numpy(e["u_draft"].reshape(-1)).to(dev))
        ids = draw.tokens.reshape(R, K).contiguous()
        self.verify = batch.PreparedVerify(
            self.th.logits.view(R, K + 1, V), self.dh.logits.view(R, K, V), ids, self.policies,
            torch.from_numpy(e["u_accept"]).to(dev), torch.from_numpy(e["u_target"]).to(dev),
            torch.from_numpy(e["limit"]).to(dev), head=(self.th, self.dh) if fused else None)
        self.result = self.verify.result
        self.inputs = (self.weight,)
        self._launch_head = batch.vocab_head_launch

    def launch(self):
        self._launch_head(self.th)
        self.verify.launch()
        return self


class _HeadK:
    """The vocabulary projection of the workload's rows with its records, then
    dsr_sample_rows_head over the logits and records.  ``records=False`` is
    the same step without records: the projection alone, then
    dsr_sample_rows over the logits."""

    def __init__(self, w, records=True):
        import torch

        from deepseekrpc_amd import batch, workloads
        e = w.extra
        dev = "cuda"
        self.weight = (torch.from_numpy(e["weight_q"]).to(dev).to(torch.bfloat16)
                       * workloads.head_weight_scale()).contiguous()
        x = torch.from_numpy(e["hidden"]).to(dev).to(torch.bfloat16)
        self.policies = batch.policy_tensor(w.policies, dev)
        self.uniforms = torch.from_numpy(np.asarray(w.uniforms, np.float64)).to(dev)
        self.hr = batch.vocab_head(x, self.weight, records=records)
        self.records = records
        self.inputs = (self.weight,)
        self.launch()

    def launch(self):
        from deepseekrpc_amd import batch
        batch.vocab_head_launch(self.hr)
        self.result = batch.sample_rows(self.hr.logits, self.policies, uniforms=self.uniforms,
                                        head_parts=self.hr.parts if self.records else None)
        return self


def _prepare(name, w, device_rng=False):
    """Device inputs and a launch closure for one step of the workload."""
    import torch

    from deepseekrpc_amd import batch, workloads
    if name == "head":
        e = w.extra
        R, K, V, D = e["requests"], e["K"], e["weight_q"].shape[0], e["dim"]
        # The weight stream, the hidden rows, the target logits and records
        # written, the draft records read, and the verifier's scalar inputs
        # and decision (as c4).
        tiles = V // batch.HEAD_TILE
        alg = V * D * 2 + R * (K + 1) * (D * 2 + V * 4 + tiles * 16) + R * K * tiles * 16 + R * 120
        return _Head(w), alg, R
    if name == "headk":
        e = w.extra
        R, V, D = e["rows"], e["weight_q"].shape[0], e["dim"]
        # The weight stream, the hidden rows, the logits and records written,
        # the records read again and each row's k = 50 kept tokens' logits,
        # and the policy, uniform and outputs.
        tiles = V // batch.HEAD_TILE
        alg = V * D * 2 + R * (D * 2 + V * 4 + 2 * tiles * 16 + 50 * 4 + 68)
        return _HeadK(w), alg, R
    if name == "propose":
        per_row = w.logits.shape[1] * (4 + 8) + 64 + 4   # logits in, float64 distribution out, controls, token
        return _Chain(w), w.extra["steps"] * per_row + 4 * len(w.histories[0]), 1
    if name == "step":
        # Proposal rows as in propose; each of the six target rows read and its distribution written.
        per_row = w.logits.shape[1] * (4 + 8) + 64 + 4
        return _Step(w), (w.extra["steps"] + w.extra["target"].shape[0]) * per_row + 4 * len(w.histories[0]), 1
    if name == "seed":
        # The row's logits and its dense counts and generated counts in, the decision out.
        return _Seed(w), w.logits.shape[1] * (4 + 4 + 4) + 64 + 4, 1
    if name == "hist":
        toks = w.extra["tokens"]
        off = np.arange(toks.shape[0] + 1, dtype=np.int64) * toks.shape[1]
        prep = batch.PreparedHistoryAppend(torch.from_numpy(toks.reshape(-1)).cuda(), torch.from_numpy(off).cuda(),
                                           vocab=w.logits.shape[1])
        prep.launch()
        prep.result = _HistResult(prep.status)
        return prep, workloads.algorithmic_bytes_history(w), toks.shape[0]
    if name == "c4":
        e = w.extra
        R, K, V = e["target"].shape[0], e["K"], e["target"].shape[2]
        tgt = torch.from_numpy(e["target"]).cuda()
        drf = torch.from_numpy(e["draft"]).cuda()
        draw = batch.sample_rows(drf.reshape(R * K, V), [dict()] * (R * K),
                                 uniforms=torch.from_numpy(e["u_draft"].reshape(-1)).cuda())
        ids = draw.tokens.reshape(R, K).contiguous()
        prep = batch.PreparedVerify(tgt, drf, ids, [dict()] * R, torch.from_numpy(e["u_accept"]).cuda(),
                                    torch.from_numpy(e["u_target"]).cuda(), torch.from_numpy(e["limit"]).cuda())
        return prep, workloads.algorithmic_bytes_verify(w), R
    d = workloads.to_device(w)
    draws = dict(uniforms=d.uniforms)
    if device_rng:  # one PCG64 stream per row, drawn and advanced on the device
        draws = dict(rng_state=batch.pcg64_states([np.random.default_rng(41117 + r) for r in range(w.rows)]))
    prep = batch.PreparedSample(d.logits, d.policies, history=d.history, allow_bits=d.allow_bits,
                                probs="f32" if name == "c1" else None, **draws)
    probs_bytes = 4 * w.logits.shape[1] if name == "c1" else 0
    return prep, workloads.algorithmic_bytes(w, probs_bytes), w.rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--device-rng", action="store_true",
                    help="sampling workloads: draw each row's uniform on the device from a PCG64 state")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain copy kernel over the batch's logit bytes (for HBM counter scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: rows are independent, so each "
              "GPU would run these kernels on its own share of the rows, and only one GPU's share is measured",
              file=sys.stderr)
        sys.exit(2)

    from deepseekrpc_amd import workloads
    name = args.workload
    metric, unit, passes, kernels = WORKLOADS[name]
    w = getattr(workloads, name)()
    cpu = None if args.no_cpu_baseline else cpu_baseline(name, w, passes)

    import torch
    from deepseekrpc_amd import _native as N

    N.load()
    if args.device_rng and name in ("c4", "head", "headk", "hist", "propose", "seed", "step"):
        raise SystemExit("--device-rng applies to the sampling workloads (c1, c2, c3, c5)")
    batches = variants(name, w)
    preps = []
    for v in batches:
        prep, alg_bytes, units = _prepare(name, v, args.device_rng)
        preps.append(prep)
    torch.cuda.synchronize()
    for prep in preps:
        status = prep.result.status.cpu().numpy()
        if (status != 0).any():
            raise SystemExit(f"kernel reported row errors: {np.unique(status)}")

    for i in range(args.warmup):
        preps[i % len(preps)].launch()
    torch.cuda.synchronize()
    # The timed region: K back-to-back steps on the launch stream, each on the
    # next of the rotated input batches, bracketed by synchronisation (host
    # wall clock) and by HIP events on that stream (average duration of one
    # step's launches).
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        preps[i % len(preps)].launch()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = ev0.elapsed_time(ev1) / args.steps
    general = 0
    for prep in preps:
        res = prep.result
        if (res.status.cpu().numpy() != 0).any():
            raise SystemExit("kernel reported row errors in the timed region")
        general = max(general, int(((res.flags.cpu().numpy() & N.FLAG_GENERAL) != 0).sum()))
    prep = preps[0]
    calibration_bytes = None
    if args.copy_calibration:
        # A plain read-N/write-N kernel over the batch's logit bytes, for
        # scaling the FETCH_SIZE / WRITE_SIZE counters.
        src = prep.inputs[0] if name == "hist" else prep.inputs[0][0] if name == "c4" else prep.inputs[0]
        src = src.reshape(-1).view(torch.int32)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        calibration_bytes = src.numel() * 4

    head_extra = {}
    if name == "head":
        # The same step without the projection's records: the projection
        # alone, then the verifier's statistics pass over the logits.
        plain = _Head(w, fused=False)
        for _ in range(args.warmup):
            plain.launch()
        ev2, ev3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev2.record(stream)
        for _ in range(args.steps):
            plain.launch()
        ev3.record(stream)
        torch.cuda.synchronize()
        same = all(torch.equal(getattr(plain.result, f), getattr(prep.result, f))
                   for f in ("accepted", "ids", "count", "pending", "stop", "used_accept", "used_target", "status"))
        if not same:
            raise SystemExit("the fused and unfused steps decided differently")
        head_extra = {"unfused_step_ms": ev2.elapsed_time(ev3) / args.steps,
                      "unfused_kernels": "k_vocab_head (no records) + k_verify_stats + k_verify_chain + "
                                         "k_verify_draw + k_verify_finish", "decisions_equal": same}
        del plain
    if name == "headk" and not args.copy_calibration:
        # The same step without records: the projection alone, then
        # dsr_sample_rows over the logits (left out of the counter runs, whose
        # per-kernel averages would mix the two steps).
        plain = _HeadK(w, records=False)
        for _ in range(args.warmup):
            plain.launch()
        ev2, ev3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev2.record(stream)
        for _ in range(args.steps):
            plain.launch()
        ev3.record(stream)
        torch.cuda.synchronize()
        same = all(torch.equal(getattr(plain.result, f), getattr(prep.result, f))
                   for f in ("tokens", "consumed", "status", "flags"))
        if not same:
            raise SystemExit("the steps with and without records decided differently")
        head_extra = {"unrecorded_step_ms": ev2.elapsed_time(ev3) / args.steps,
                      "unrecorded_kernels": "k_vocab_head (no records) + k_sample_f32 (a pass over each row)",
                      "decisions_equal": same}
        del plain
    ms_per_step = wall * 1e3 / args.steps
    achieved = alg_bytes / (kern_ms * 1e-3) / 1e9
    # HBM traffic per launch is not measurable from inside the run (counters
    # need their own rocprofv3 pass); it is read from the committed counter
    # summary of the same command and labelled as such.
    traffic, traffic_source = None, None
    tf = os.path.join(ROOT, "profiles", f"{PROFILE_PREFIX.get(name, kernels.split(' ')[0])}_{name}_traffic.json")
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("bytes_per_launch")
        traffic_source = os.path.relpath(tf, ROOT) + " (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; calibrated)"
    cfg = {"workload": DESCRIPTIONS[name], "rows": units, "vocab": int(w.logits.shape[1]), "input_dtype": w.dtype,
           "general_path_rows": general, "kernels": kernels,
           "input_batches": len(batches), "input_bytes_rotated": sum(_batch_bytes(name, v) for v in batches)}
    if name not in ("c4", "head", "hist", "propose", "seed", "step"):
        cfg["draws"] = "device PCG64 state per row" if args.device_rng else "pre-drawn uniforms"
    if name in ("head", "headk"):
        cfg.update(head_extra)
    if calibration_bytes is not None:
        cfg["calibration_bytes"] = calibration_bytes  # bytes the copy kernel reads, and writes, per launch
    line = {
        "metric": metric, "value": units / (ms_per_step * 1e-3), "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak",
        # Every decision is taken in float64 (the reference's arithmetic) and
        # fixed-point integers; the input type is reported in the config.
        "vs_baseline": None, "dtype": "int32" if name == "hist" else "f64", "data": "synthetic",
        "config": cfg,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic, "traffic_source": traffic_source,
                     "kernel_ms": kern_ms, "algorithmic_bytes": alg_bytes},
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
