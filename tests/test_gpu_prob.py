"""Probability-vector kernels at V = 129,280 against the oracle.

``dsr_prob_stats`` / ``_categorical`` / ``_correction`` / ``_accept`` carry the
drop-in's ``_distribution``, ``categorical``, ``correction_distribution`` and
accept test (src/deepseekrpc/sampling.py:109-139,276-281).  Their sums follow
NumPy's own order, so the checks here are bit for bit: the sum tested against
1 +- 1e-10, the normalised residual, and the categorical draw with the uniform
placed exactly on the oracle's CDF cell edges and one ulp either side.
"""
import math

import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch
from deepseekrpc_amd.jsonutil import ValidationError
from deepseekrpc_amd.sampling import _distribution, categorical, correction_distribution
from oracle import sampling_oracle as O

pytestmark = pytest.mark.gpu
V = 129280
DEV = "cuda"


def softmax_row(rng, scale=2.0, zeros=0.0, n=V):
    x = rng.normal(0, scale, n)
    if zeros:
        x[rng.random(n) < zeros] = -np.inf
    e = np.exp(x - x.max())
    return e / e.sum()


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


@pytest.mark.parametrize("n", [1, 5, 7, 8, 9, 127, 128, 129, 1000, 8191, 8192, 8193, 16384, 100_003, V])
def test_stats_sum_is_numpy_sum_bit_for_bit(n):
    rng = np.random.default_rng(n)
    for trial in range(3):
        p = rng.random(n) * np.exp(rng.normal(0, 6, n))     # wide magnitudes: every rounding shows
        if trial == 2:
            p[rng.random(n) < 0.5] = 0.0
        total, valid, npos, first, argmax = batch.prob_stats(dev(p))
        assert total == float(p.sum(dtype=np.float64)), (n, trial)
        pos = np.flatnonzero(p > 0)
        assert valid and npos == len(pos)
        assert first == (int(pos[0]) if len(pos) else -1) and argmax == int(np.argmax(p))


def test_batched_stats_equal_the_one_row_kernel():
    """dsr_prob_stats_rows (one launch for the verifier's rows) gives every
    row what dsr_prob_stats gives it: 20 rows (two launches) with valid,
    off-sum, negative, NaN, sparse and single-positive rows."""
    rng = np.random.default_rng(21)
    rows = []
    for k in range(20):
        p = softmax_row(rng, zeros=0.3 if k % 3 == 0 else 0.0)
        if k == 4:
            p *= 1.0 + 2e-10
        if k == 7:
            p[99] = -1e-3
        if k == 11:
            p[5] = np.nan
        if k == 13:
            p[:] = 0.0
            p[1234] = 1.0
        rows.append(dev(p))
    out = torch.empty(len(rows), 3, dtype=torch.float64, device=DEV)
    batch.prob_stats_rows_launch(rows, out)
    host = out.cpu()
    for k, r in enumerate(rows):
        got = batch.prob_stats_read(host[k])
        want = batch.prob_stats(r)
        assert (got[0] == want[0] or (math.isnan(got[0]) and math.isnan(want[0]))) and got[1:] == want[1:], k
    assert not batch.prob_stats_read(host[7])[1] and not batch.prob_stats_read(host[11])[1]
    assert batch.prob_stats_read(host[13])[2:4] == (1, 1234)


@pytest.mark.parametrize("offset", [0.9e-10, -0.9e-10, 1.1e-10, -1.1e-10, 0.0])
def test_sum_tolerance_decides_as_the_oracle(offset):
    rng = np.random.default_rng(abs(hash(offset)) % 1000)
    p = softmax_row(rng, zeros=0.1) * (1.0 + offset)
    want_ok = True
    try:
        O.validate_distribution(p)
    except O.OracleError:
        want_ok = False
    assert want_ok == (abs(offset) < 1e-10)
    try:
        _distribution(dev(p))
        got_ok = True
    except ValidationError:
        got_ok = False
    assert got_ok == want_ok


@pytest.mark.parametrize("bad", ["negative", "nan", "inf", "tiny-negative"])
def test_invalid_entries_are_rejected(bad):
    rng = np.random.default_rng(3)
    p = softmax_row(rng)
    p[777] = {"negative": -1e-3, "nan": np.nan, "inf": np.inf, "tiny-negative": -5e-324}[bad]
    with pytest.raises(O.OracleError):
        O.validate_distribution(p)
    _, valid, *_ = batch.prob_stats(dev(p))
    assert not valid
    with pytest.raises(ValidationError):
        categorical(dev(p), lambda: 0.5)


def edge_uniforms(p, rng, cells=24):
    """Uniforms on the oracle's normalised CDF cell edges, and one ulp either side."""
    c = np.cumsum(p, dtype=np.float64)
    c /= c[-1]
    edges = c[rng.choice(np.flatnonzero(c < 1.0), cells, replace=False)]
    us = []
    for e in edges:
        us += [float(e), float(np.nextafter(e, 0.0)), float(np.nextafter(e, 1.0))]
    us += [0.0, float(np.nextafter(1.0, 0.0))]
    return [u for u in us if 0.0 <= u < 1.0]


@pytest.mark.parametrize("zeros", [0.0, 0.4, 0.999])
def test_categorical_matches_the_oracle_on_cell_edges(zeros):
    rng = np.random.default_rng(int(zeros * 1000) + 17)
    p = softmax_row(rng, zeros=zeros)
    t = dev(p)
    checked = 0
    for u in edge_uniforms(p, rng) + list(rng.random(20)):
        want = O.categorical(p, float(u))[0]
        tok, _flags = batch.prob_categorical(t, float(u))
        assert tok == want, (u, tok, want)
        assert categorical(t, lambda u=u: float(u)) == want
        checked += 1
    assert checked >= 60


def test_residual_is_numpy_residual_bit_for_bit_and_draws_on_its_edges():
    rng = np.random.default_rng(44)
    x = rng.normal(0, 2, V)
    p = np.exp(x - x.max())
    p /= p.sum()
    y = x + rng.normal(0, 0.5, V)
    q = np.exp(y - y.max())
    q /= q.sum()
    want = O.correction(p, q)
    got = correction_distribution(dev(p), dev(q)).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    t = dev(got)
    for u in edge_uniforms(want, rng, cells=12):
        assert categorical(t, lambda u=u: u) == O.categorical(want, u)[0], u


def test_residual_with_equal_rows_has_no_mass():
    rng = np.random.default_rng(5)
    p = softmax_row(rng)
    with pytest.raises(O.OracleError):
        O.correction(p, p)
    _, status = batch.prob_correction(dev(p), dev(p))
    assert status == N.E_CORRECTION
    with pytest.raises(ValidationError, match="correction"):
        correction_distribution(dev(p), dev(p))


def test_accept_test_on_the_ratio_edge():
    rng = np.random.default_rng(6)
    p, q = softmax_row(rng), softmax_row(rng)
    tp, tq = dev(p), dev(q)
    for x in rng.choice(V, 10, replace=False):
        ratio = min(1.0, float(p[x] / q[x]))
        for u in (ratio, float(np.nextafter(ratio, 0.0)), 0.0, float(np.nextafter(1.0, 0.0))):
            if not 0.0 <= u < 1.0:
                continue
            positive, accepted = batch.prob_accept(tp, tq, int(x), u)
            assert positive and accepted == (u < ratio), (x, u, ratio)
    q[123] = 0.0
    positive, accepted = batch.prob_accept(tp, dev(q), 123, 0.5)
    assert not positive and not accepted


@pytest.mark.parametrize("n,offset", [(129280, 0), (129281, 1), (7, 0), (1, 3), (4096, 2)])
def test_rows_finite_is_numpy_isfinite_all(n, offset):
    """dsr_rows_finite against np.isfinite(row).all() (terminal_sampling.py:25):
    NaN, +inf and -inf anywhere (first, last, middle), FLT_MAX and
    subnormals (finite), rows that start off a 16-byte boundary and lengths
    that are not a multiple of 4."""
    rng = np.random.default_rng(n + offset)
    R = 9
    x = rng.normal(0, 3, (R, n + offset + 5)).astype(np.float32)
    x[1, offset + n - 1] = np.nan
    x[2, offset] = np.inf
    x[3, offset + n // 2] = -np.inf
    x[4, offset:offset + n] = np.finfo(np.float32).max
    x[5, offset:offset + n:2] = np.float32(1e-45)
    x[6, offset + n:] = np.nan                              # past the row: not read
    x[7, offset:offset + n] = -np.finfo(np.float32).max
    x[8, offset + (n - 1) // 3] = np.nan
    t = torch.from_numpy(x).cuda()[:, offset:offset + n]
    got = batch.rows_finite(t).cpu().numpy()
    want = np.isfinite(x[:, offset:offset + n]).all(axis=1).astype(np.int32)
    np.testing.assert_array_equal(got, want)
