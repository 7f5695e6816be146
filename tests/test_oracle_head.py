"""Pins oracle/head_oracle.py: the float64 projection, the per-tile records
and their combination into the verifier's row statistics, each against a
different computation (CPU only)."""
import math

import numpy as np
import pytest

from oracle import head_oracle as H


def test_projection_is_exact_on_integer_values():
    rng = np.random.default_rng(1)
    xi = rng.integers(-64, 64, (7, 256))
    wi = rng.integers(-64, 64, (384, 256))
    logits, scale = H.project(xi.astype(np.float32), wi.astype(np.float32))
    assert np.array_equal(logits, (xi @ wi.T).astype(np.float64))
    assert np.array_equal(scale, (np.abs(xi) @ np.abs(wi).T).astype(np.float64))


def loop_records(row, T, tile):
    """Element by element: the maximum, its first column, the flags and the exp sum of each tile."""
    out = []
    for k in range(len(row) // tile):
        vals = [float(x) for x in row[k * tile:(k + 1) * tile]]
        m, first, fl = -math.inf, -1, 0
        for c, x in enumerate(vals):
            if math.isnan(x) or x == math.inf:
                fl |= 1
            if math.isfinite(x):
                fl |= 2
            if x == -math.inf:
                fl |= 4
            if not math.isnan(x) and x > m:
                m = x
        for c, x in enumerate(vals):
            if x == m:
                first = c
                break
        s = 0.0
        if 0 < T <= 100 and math.isfinite(m):
            for x in vals:
                if not math.isnan(x) and x != math.inf:
                    s += math.exp((x - m) / T)
        out.append((s, m, first, fl))
    return out


def sample_rows(rng, rows=6, tile=16, tiles=5):
    v = rng.normal(0, 3, (rows, tile * tiles)).astype(np.float32)
    v[1, 3] = np.nan                       # NaN in tile 0
    v[1, 20] = np.inf                      # +inf in tile 1
    v[2, :tile] = -np.inf                  # an all-masked tile
    v[2, 40] = -np.inf
    v[3, [5, 9]] = 20.0                    # a tie for the maximum inside one tile
    v[3, 70] = 20.0                        # and in a later tile
    v[4, :] = 0.0                          # constant row
    v[5, :] = np.nan                       # nothing but NaN
    return v


@pytest.mark.parametrize("T", [1.0, 0.35, 0.0, 2.5])
def test_records_equal_element_loops(T):
    rng = np.random.default_rng(2)
    tile = 16
    v = sample_rows(rng, tile=tile)
    sums, mx, first, flags = H.records(v, [T] * len(v), tile=tile)
    for r in range(len(v)):
        for k, (s, m, f, fl) in enumerate(loop_records(v[r], T, tile)):
            assert float(mx[r, k]) == m or (math.isinf(m) and float(mx[r, k]) == m)
            assert first[r, k] == f and flags[r, k] == fl, (r, k)
            assert math.isclose(sums[r, k], s, rel_tol=1e-13, abs_tol=0.0), (r, k, sums[r, k], s)


def test_a_planted_last_column_is_caught():
    """The loops tell the first column of a tied maximum from the last."""
    rng = np.random.default_rng(3)
    tile = 16
    v = sample_rows(rng, tile=tile)
    _, mx, first, _ = H.records(v, [1.0] * len(v), tile=tile)
    t = v.reshape(len(v), -1, tile)
    last = np.where(first >= 0, tile - 1 - np.argmax((t == mx[..., None])[..., ::-1], axis=2), -1)
    want = np.array([[f for (_, _, f, _) in loop_records(v[r], 1.0, tile)] for r in range(len(v))])
    assert np.array_equal(first, want) and not np.array_equal(last, want)


@pytest.mark.parametrize("T", [1.0, 0.7, 0.0])
def test_combined_records_equal_the_row_statistics(T):
    rng = np.random.default_rng(4)
    tile = 128
    v = rng.normal(0, 2.6, (5, tile * 40)).astype(np.float32)
    v[1, 1000] = v[1, 3000] = np.float32(30.0)      # tied maximum in two tiles: the first wins
    v[2, :tile * 3] = -np.inf                       # masked tiles take no part
    v[3, 77] = -np.inf
    sums, mx, first, flags = H.records(v, [T] * len(v), tile=tile)
    for r in range(len(v)):
        M, col, fl, s = H.combine(sums[r], mx[r], first[r], flags[r], T, tile=tile)
        M2, col2, fl2, s2 = H.row_statistics(v[r], T)
        assert M == M2 and col == col2 and fl == fl2
        assert math.isclose(s, s2, rel_tol=1e-13, abs_tol=0.0), (r, s, s2)
    assert H.combine(sums[1], mx[1], first[1], flags[1], T, tile=tile)[1] == 1000
