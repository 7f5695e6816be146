"""CPU oracle for the device history tables.

TEST INFRASTRUCTURE ONLY.  This module is the oracle that the HIP history
builders are compared against.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product
package never does.

The reference keeps a request's history as two dense int32 vectors over the
vocabulary (src/deepseekrpc/history.py:46-47): ``counts`` (every history
token) and ``generated_counts`` (output tokens only).  ``set_prompt`` fills
``counts`` with ``np.bincount`` of the prompt and clears the generated
counts (history.py:92-94); ``append`` adds each output token to both with
``np.add.at`` (history.py:136-137); ``SamplingWork.distribution`` copies both
and adds one per tentative prefix token (terminal_sampling.py:127-133);
``SamplingPolicy.probabilities`` validates them (sampling.py:54-58, 62-65).
The GPU path keeps the same information as a sparse table per row: the ids
with ``counts > 0`` in increasing order, with both counts.  This module
restates those dense operations and compacts the result:

* ``from_dense`` -> validation of sampling.py:54-58 then :62-65, then
  ``np.flatnonzero(counts > 0)``;
* ``append``     -> the row densified, ``np.add.at`` of the new tokens into
  the counts and of the generated ones (positions >= ``gen_from``) into the
  generated counts, compacted again.

Statuses are the library's per-row codes (include/dsr_sampling.h).

Pinning (tests/test_oracle_history.py): token-by-token counting with
``collections.Counter`` over the full token history (a different
computation from ``np.add.at``), the reference's own count-history laws
(the prompt counts only toward repetition; tests/test_sampling.py:236-243
and terminal_sampling.py:127-133), round trips through the dense form, the
equality of appending in pieces and at once, and each validation rule on a
vector built to break exactly that rule.
"""
from __future__ import annotations

import numpy as np

MAX_COUNT = 1048576   # sampling.py:57
MAX_APPEND = 16384    # new tokens per row in one append call (a library limit)

OK, E_COUNTS, E_GENERATED, E_HISTORY, E_APPEND = 0, 5, 12, 13, 14


def _pack(rows):
    """Per-row (ids, counts, generated) -> CSR arrays."""
    off = np.zeros(len(rows) + 1, np.int64)
    for r, (i, _, _) in enumerate(rows):
        off[r + 1] = off[r] + len(i)
    cat = lambda k: (np.concatenate([x[k] for x in rows]).astype(np.int32) if rows and off[-1]
                     else np.zeros(0, np.int32))
    return off, cat(0), cat(1), cat(2)


def from_dense(counts, generated=None):
    """Dense [rows, V] counts (and generated counts) -> (off, ids, count, gen, status).

    A row is rejected as SamplingPolicy.probabilities rejects it: counts
    outside [0, MAX_COUNT] or a total above MAX_COUNT (sampling.py:55-58)
    first, then generated counts outside [0, counts] (:62-65).  A rejected
    row has no entries."""
    counts = np.atleast_2d(np.asarray(counts, np.int64))
    generated = counts if generated is None else np.atleast_2d(np.asarray(generated, np.int64))
    rows, status = [], np.zeros(counts.shape[0], np.int32)
    for r in range(counts.shape[0]):
        c, g = counts[r], generated[r]
        if (c < 0).any() or (c > MAX_COUNT).any() or int(c.sum()) > MAX_COUNT:
            status[r] = E_COUNTS
        elif (g < 0).any() or (g > c).any():
            status[r] = E_GENERATED
        if status[r]:
            rows.append((np.zeros(0, np.int64),) * 3)
            continue
        nz = np.flatnonzero(c > 0)
        rows.append((nz, c[nz], g[nz]))
    return (*_pack(rows), status)


def row_valid(ids, cnt, gen, vocab):
    """A table row the library accepts: ids strictly increasing in [0, vocab),
    1 <= count <= MAX_COUNT, 0 <= gen <= count."""
    ids, cnt, gen = (np.asarray(x, np.int64) for x in (ids, cnt, gen))
    return (len(ids) <= vocab and ((ids >= 0) & (ids < vocab)).all() and (np.diff(ids) > 0).all()
            and ((cnt >= 1) & (cnt <= MAX_COUNT)).all() and ((gen >= 0) & (gen <= cnt)).all())


def append(off, ids, cnt, gen, token_rows, vocab, gen_from=None):
    """Table (off None: every row empty) plus new tokens per row -> (off, ids,
    count, gen, status).  Token ``t`` at position ``i`` of its row adds one to
    count[t] and, when ``i >= gen_from[r]`` (every position without gen_from),
    one to gen[t]: np.add.at on both dense vectors (history.py:136-137)."""
    out, status = [], np.zeros(len(token_rows), np.int32)
    for r, toks in enumerate(token_rows):
        toks = np.asarray(toks, np.int64)
        if off is None:
            oi = oc = og = np.zeros(0, np.int64)
        else:
            a, b = int(off[r]), int(off[r + 1])
            oi, oc, og = (np.asarray(x[a:b], np.int64) for x in (ids, cnt, gen))
        if len(toks) > MAX_APPEND:
            status[r] = E_APPEND
        elif not row_valid(oi, oc, og, vocab) or ((toks < 0) | (toks >= vocab)).any():
            status[r] = E_HISTORY
        if status[r]:
            out.append((np.zeros(0, np.int64),) * 3)
            continue
        c = np.zeros(vocab, np.int64)
        g = np.zeros(vocab, np.int64)
        c[oi], g[oi] = oc, og
        np.add.at(c, toks, 1)
        gf = 0 if gen_from is None else max(0, int(gen_from[r]))
        np.add.at(g, toks[gf:], 1)
        nz = np.flatnonzero(c > 0)
        out.append((nz, c[nz], g[nz]))
    return (*_pack(out), status)


def densify(off, ids, cnt, gen, vocab):
    """CSR table -> dense [rows, vocab] (counts, generated)."""
    rows = len(off) - 1
    c = np.zeros((rows, vocab), np.int64)
    g = np.zeros((rows, vocab), np.int64)
    for r in range(rows):
        a, b = int(off[r]), int(off[r + 1])
        c[r, ids[a:b]] = cnt[a:b]
        g[r, ids[a:b]] = gen[a:b]
    return c, g
