"""Pins the history-table oracle (oracle/history_oracle.py).

The oracle restates the reference's dense count bookkeeping with np.add.at
and np.flatnonzero.  These checks reach the same numbers another way:
token-by-token counting with collections.Counter, the reference's own
count-history law (the prompt counts toward repetition only), dense round
trips, appending in pieces against appending at once, and one vector per
validation rule.  Planted mistakes at the end show that the checks catch the
plausible ones (prompt tokens counted as generated, a dropped token, an
off-by-one in the generated split).
"""
from collections import Counter

import numpy as np
import pytest

from oracle import history_oracle as H

V = 97


def rows_of(off, ids, cnt, gen):
    return [(ids[off[r]:off[r + 1]].tolist(), cnt[off[r]:off[r + 1]].tolist(), gen[off[r]:off[r + 1]].tolist())
            for r in range(len(off) - 1)]


def counter_row(tokens, gen_from):
    """Token-by-token counts of one history: every token counts; those at
    positions >= gen_from are also generated."""
    c, g = Counter(), Counter()
    for i, t in enumerate(tokens):
        c[t] += 1
        if i >= gen_from:
            g[t] += 1
    ids = sorted(c)
    return ids, [c[t] for t in ids], [g[t] for t in ids]


def random_rows(rng, n_rows, max_len, vocab=V):
    return [rng.integers(0, vocab, rng.integers(0, max_len + 1)).tolist() for _ in range(n_rows)]


def test_append_to_empty_matches_token_by_token_counting():
    rng = np.random.default_rng(1)
    toks = random_rows(rng, 40, 300)
    gf = [int(rng.integers(0, len(t) + 2)) for t in toks]
    off, ids, cnt, gen, st = H.append(None, None, None, None, toks, V, gen_from=gf)
    assert (st == 0).all()
    assert rows_of(off, ids, cnt, gen) == [counter_row(t, f) for t, f in zip(toks, gf)]


def test_prompt_counts_toward_repetition_only():
    # tests/test_sampling.py:236-243 uses counts [5, 1, 0] with generated
    # [0, 1, 0]: a prompt of five 0s (history.py:92-94 fills counts only)
    # followed by the output token 1 (history.py:136-137 fills both).
    off, ids, cnt, gen, st = H.append(None, None, None, None, [[0, 0, 0, 0, 0]], 3, gen_from=[5])
    off, ids, cnt, gen, st2 = H.append(off, ids, cnt, gen, [[1]], 3)
    c, g = H.densify(off, ids, cnt, gen, 3)
    assert st[0] == 0 and st2[0] == 0
    assert c[0].tolist() == [5, 1, 0] and g[0].tolist() == [0, 1, 0]


def test_tentative_prefix_adds_one_to_both_counts():
    # terminal_sampling.py:127-133: counts[token] += 1; generated[token] += 1.
    rng = np.random.default_rng(2)
    counts = rng.integers(0, 4, V)
    generated = np.minimum(counts, rng.integers(0, 3, V))
    prefix = [5, 9, 5, 96]
    c, g = counts.copy(), generated.copy()
    for t in prefix:
        c[t] += 1
        g[t] += 1
    off, ids, cnt, gen, st = H.from_dense(counts, generated)
    off, ids, cnt, gen, st2 = H.append(off, ids, cnt, gen, [prefix], V)
    dc, dg = H.densify(off, ids, cnt, gen, V)
    assert st[0] == 0 and st2[0] == 0
    assert (dc[0] == c).all() and (dg[0] == g).all()


def test_dense_round_trip_and_id_order():
    rng = np.random.default_rng(3)
    counts = rng.integers(0, 3, (6, V)) * (rng.random((6, V)) < 0.3)
    generated = counts - rng.integers(0, 2, (6, V)).clip(0, counts)
    off, ids, cnt, gen, st = H.from_dense(counts, generated)
    assert (st == 0).all()
    for r in range(6):
        seg = ids[off[r]:off[r + 1]]
        assert (np.diff(seg) > 0).all() and (cnt[off[r]:off[r + 1]] > 0).all()
    c, g = H.densify(off, ids, cnt, gen, V)
    assert (c == counts).all() and (g == generated).all()


def test_appending_in_pieces_equals_appending_at_once():
    rng = np.random.default_rng(4)
    a, b = random_rows(rng, 10, 50), random_rows(rng, 10, 50)
    t1 = H.append(None, None, None, None, a, V)
    t2 = H.append(*t1[:4], b, V)
    t3 = H.append(None, None, None, None, [x + y for x, y in zip(a, b)], V)
    assert rows_of(*t2[:4]) == rows_of(*t3[:4])


@pytest.mark.parametrize("counts,generated,status", [
    ([0, -1, 0], None, H.E_COUNTS),                         # sampling.py:56 negative count
    ([0, H.MAX_COUNT + 1, 0], [0, 0, 0], H.E_COUNTS),       # :56 count above the bound
    ([H.MAX_COUNT, 1, 0], [0, 0, 0], H.E_COUNTS),           # :57 total above the bound
    ([H.MAX_COUNT, 0, 0], [0, 0, 0], H.OK),                 # the bound itself is allowed
    ([2, 1, 0], [3, 0, 0], H.E_GENERATED),                  # :64 generated above count
    ([2, 1, 0], [0, -1, 0], H.E_GENERATED),                 # :64 negative generated
    ([-1, 1, 0], [3, 0, 0], H.E_COUNTS),                    # counts are checked first
])
def test_dense_validation_rules(counts, generated, status):
    off, ids, cnt, gen, st = H.from_dense(np.array(counts), None if generated is None else np.array(generated))
    assert st[0] == status
    if status != H.OK:
        assert off[1] == 0  # a rejected row has no entries


@pytest.mark.parametrize("table,tokens,status", [
    (([3], [1], [0]), [V], H.E_HISTORY),            # token beyond the vocabulary
    (([3], [1], [0]), [-1], H.E_HISTORY),           # negative token
    (([3, 3], [1, 1], [0, 0]), [1], H.E_HISTORY),   # ids not strictly increasing
    (([3], [0], [0]), [1], H.E_HISTORY),            # count below one
    (([3], [2], [3]), [1], H.E_HISTORY),            # generated above count
    (([3], [1], [0]), [1] * (H.MAX_APPEND + 1), H.E_APPEND),
    (([3], [1], [0]), [1] * H.MAX_APPEND, H.OK),
])
def test_append_validation_rules(table, tokens, status):
    ids, cnt, gen = (np.array(x, np.int32) for x in table)
    off = np.array([0, len(ids)], np.int64)
    st = H.append(off, ids, cnt, gen, [tokens], V)[4]
    assert st[0] == status


# Planted mistakes: each variant must fail at least one of the checks above.
_good_append = H.append


def _prompt_as_generated(off, ids, cnt, gen, rows, vocab, gen_from=None):
    return _good_append(off, ids, cnt, gen, rows, vocab, gen_from=None)


def _drops_last_token(off, ids, cnt, gen, rows, vocab, gen_from=None):
    return _good_append(off, ids, cnt, gen, [list(r)[:-1] for r in rows], vocab, gen_from)


def _generated_off_by_one(off, ids, cnt, gen, rows, vocab, gen_from=None):
    gf = [1] * len(rows) if gen_from is None else [g + 1 for g in gen_from]
    return _good_append(off, ids, cnt, gen, rows, vocab, gf)


@pytest.mark.parametrize("bad", [_prompt_as_generated, _drops_last_token, _generated_off_by_one])
def test_planted_mistakes_are_caught(bad, monkeypatch):
    monkeypatch.setattr(H, "append", bad)
    failures = 0
    for check in (test_append_to_empty_matches_token_by_token_counting, test_prompt_counts_toward_repetition_only,
                  test_tentative_prefix_adds_one_to_both_counts):
        try:
            check()
        except AssertionError:
            failures += 1
    assert failures >= 1
