"""CPU oracle for the vocabulary projection and its per-tile records.

TEST INFRASTRUCTURE ONLY.  This module is the oracle that ``dsr_vocab_head``
and ``dsr_verify_drafts_head`` are compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package never does.

The terminal stage computes FP32 logits as ``logits_processor(lm_head,
norm(hidden))`` and checks ``torch.isfinite(logits).all()``
(src/deepseekrpc/stage_graph.py:356-362; the draft rows, :396).  The head
itself is vLLM's ``ParallelLMHead``, outside the reference tree, so the
projection is restated from its definition:

* ``project`` -> logits[r, v] = sum_k hidden[r, k] * weight[v, k] over the
  bf16 values, every product exact and the sum in float64, together with
  sum_k |hidden[r, k] * weight[v, k]|, the scale of the FP32 accumulation
  bound the tests state;
* ``records`` -> per (row, tile of ``tile`` columns) of FP32 logits: the
  largest logit (NaN ignored, -inf if none), the first column holding it,
  flags (1: a NaN or +inf, 2: a finite logit, 4: a -inf) and
  sum exp((v - max) / T) in float64 at the row's temperature (0 for T == 0,
  T outside (0, 100] or a non-finite maximum), as ``dsr_head_part_t`` holds
  them;
* ``combine`` -> a row's (maximum, first column of the maximum, flags,
  sum exp((v - M) / T)) from its records: the verifier fast path's per-row
  statistics (the quantities ``k_verify_stats`` takes from the logits,
  sampling.py:86-106 with no filter: exp((v - M) / T) / sum).

Pinning (tests/test_oracle_head.py): ``project`` on integer-valued inputs
against NumPy's exact int64 product; ``records`` against element-by-element
Python loops (``math.exp``, explicit first-index search) on small rows,
including NaN, +inf, -inf, ties and all-masked tiles; ``combine`` against the
statistics of the whole row computed directly; and a planted mistake (the
last column of the maximum instead of the first) that the loop check fails.
"""
from __future__ import annotations

import math

import numpy as np


def project(hidden, weight):
    """(logits, scale): float64 product of bf16-valued ``hidden [R, D]`` and
    ``weight [V, D]`` (float32 arrays holding bf16 values), and
    sum_k |x_k w_k| per output."""
    x = np.asarray(hidden, np.float64)
    w = np.asarray(weight, np.float64)
    return x @ w.T, np.abs(x) @ np.abs(w).T


def records(logits, temperatures, tile=128):
    """(sums [R, T], maxima [R, T] float32, first [R, T], flags [R, T]) of
    FP32 logits ``[R, V]`` with V a multiple of ``tile``; ``first`` is -1
    where no column holds the maximum."""
    v = np.asarray(logits, np.float32)
    rows, vocab = v.shape
    tiles = vocab // tile
    t = v.reshape(rows, tiles, tile)
    nan = np.isnan(t)
    mx = np.where(nan, -np.inf, t).max(axis=2).astype(np.float32)
    flags = (np.any(nan | (t == np.inf), axis=2) * 1 | np.any(np.isfinite(t), axis=2) * 2
             | np.any(t == -np.inf, axis=2) * 4)
    hit = t == mx[..., None]
    first = np.where(hit.any(axis=2), hit.argmax(axis=2), -1)
    sums = np.zeros((rows, tiles))
    for r in range(rows):
        T = float(temperatures[r])
        if not 0.0 < T <= 100.0:
            continue
        for k in range(tiles):
            m = float(mx[r, k])
            if not math.isfinite(m):
                continue
            with np.errstate(invalid="ignore", over="ignore"):
                e = np.exp((t[r, k].astype(np.float64) - m) / T)
            sums[r, k] = float(np.sum(np.where(np.isnan(e), 0.0, e)))
    return sums, mx, first, flags.astype(np.int64)


def combine(sums, maxima, first, flags, T, tile=128):
    """(M, first column of M, flags, sum exp((v - M) / T)) of one row from its
    records; tiles without a finite logit take no part in M and the sum."""
    finite = (flags & 2) != 0
    fl = int(np.bitwise_or.reduce(flags)) if len(flags) else 0
    if not finite.any():
        return -math.inf, -1, fl, 0.0
    M = float(np.max(maxima[finite]))
    col = -1
    for k in np.flatnonzero(finite):
        if float(maxima[k]) == M and first[k] >= 0:
            col = int(k) * tile + int(first[k])
            break
    s = 0.0
    if T > 0.0:
        for k in np.flatnonzero(finite):
            s += float(sums[k]) * math.exp((float(maxima[k]) - M) / T)
    return M, col, fl, s


def row_statistics(row, T):
    """The same four quantities straight from one row of FP32 logits."""
    v = np.asarray(row, np.float64)
    nan = np.isnan(v)
    fl = (1 if (nan | (v == np.inf)).any() else 0) | (2 if np.isfinite(v).any() else 0) | \
        (4 if (v == -np.inf).any() else 0)
    if not np.isfinite(v).any():
        return -math.inf, -1, fl, 0.0
    M = float(np.max(np.where(nan, -np.inf, v)))
    col = int(np.flatnonzero(v == M)[0])
    s = 0.0
    if T > 0.0:
        with np.errstate(invalid="ignore", over="ignore"):
            e = np.exp((v - M) / T)
        s = float(np.sum(np.where(np.isnan(e), 0.0, e)))
    return M, col, fl, s
