"""The streamed bf16 top-k kernel (k_sample_bf16_fast) on rows built to sit on
its decision boundaries, against the oracle on identical inputs and uniforms:
token ids, consumption flags and top-k index sets bit-exact, fp32
probabilities within 1e-5 relative, and no row excused by the oracle's
rounding band.  Rows the kernel must hand to the general path (a top-k
reaching zero or below, too many candidates, NaN) still have to match, and
the tests check which rows stayed on the register path."""
import numpy as np
import pytest

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import workloads
from parity_util import compare, run_gpu

pytestmark = pytest.mark.gpu


def check(w, probs="f32"):
    gpu = run_gpu(w, probs=probs, kept=True)
    rep = compare(w, gpu)
    print(f"{w.name}: rows={rep.rows} exact={rep.exact} margin={rep.margin_rows} flagged={rep.flagged}", flush=True)
    assert not rep.mismatches, rep.mismatches[:10]
    assert not rep.margin_rows, rep.margin_rows
    return gpu


def general(gpu):
    return (gpu["flags"] & N.FLAG_GENERAL) != 0


def tied_rows(V, rng):
    """bf16 values on a coarse grid, so the k-th value and the top-p boundary
    fall inside groups of equal values (ties resolved by lowest index)."""
    R = 12
    x = np.round(rng.normal(0, 1, (R, V)) * 4) / 4          # steps of 0.25: exact in bf16
    x[:, rng.choice(V, 6, replace=False)] = 3.0              # six equal maxima
    pols = []
    for r in range(R):
        pols.append(dict(temperature=[0.3, 0.7, 1.0, 1.5][r % 4], top_k=[1, 2, 6, 7, 50, 333, 1000, 1024][r % 8],
                         top_p=[1.0, 0.5, 0.9, 0.999][r % 4]))
    pols[0] = dict(temperature=0.0, top_k=5)                   # greedy: first of the six maxima
    pols[1] = dict(temperature=1.0, top_k=6, top_p=0.4)        # top-p inside the tie group of the maximum
    return workloads.Workload(f"tied{V}", "bf16", workloads.bf16_round(x), pols, rng.random(R))


@pytest.mark.parametrize("V", [129280, 50000, 16384, 4096, 1000, 64])
def test_ties_at_the_top_k_and_top_p_boundaries(V):
    rng = np.random.default_rng(7100 + V)
    w = tied_rows(V, rng)
    gpu = check(w)
    # With V >= 50,000 the first half holds thousands of positive pair maxima,
    # so every row here stays on the register path.  Smaller vocabularies may
    # have fewer pair maxima than k and hand rows over.
    if V >= 50000:
        assert not general(gpu).any(), np.flatnonzero(general(gpu))


def test_heavy_tail_rows_with_min_p_and_masks():
    """C3-like rows (N(0,1) plus spikes) with min-p, top-p extremes and masks
    from 1% to 99.9% disallowed."""
    rng = np.random.default_rng(7201)
    R, V = 16, workloads.VOCAB
    x = rng.normal(0, 1, (R, V))
    for r in range(R):
        x[r, rng.choice(V, 32, replace=False)] += rng.uniform(8, 15, 32)
    keep_frac = [0.99, 0.9, 0.5, 0.1, 0.01, 0.002] + [0.9] * 10
    allowed = np.stack([rng.random(V) < keep_frac[r] for r in range(R)])
    allowed[5, :] = False
    allowed[5, rng.choice(V, 40, replace=False)] = True         # 40 allowed tokens, k = 64: fewer than k
    pols = [dict(temperature=float(rng.uniform(0.2, 1.5)), top_k=int(rng.integers(1, 1025)),
                 top_p=float(rng.uniform(0.5, 1.0))) for _ in range(R)]
    pols[5]["top_k"] = 64
    pols[6].update(min_p=0.05)
    pols[7].update(min_p=0.5, top_p=1.0)
    pols[8].update(top_p=0.0)
    pols[9].update(top_p=1e-9, top_k=1024)
    pols[10].update(temperature=0.05, top_k=1024)
    pols[11].update(temperature=50.0, top_k=1024, top_p=0.999)
    pols[12].update(top_k=1)
    pols[13].update(temperature=0.0, top_k=1024)
    w = workloads.Workload("tail", "bf16", workloads.bf16_round(x), pols, rng.random(R), allowed=allowed)
    gpu = check(w)
    assert not general(gpu)[[0, 1, 2, 6, 7, 8, 9, 10, 11, 12, 13]].any()


def test_rows_handed_to_the_general_path_still_match():
    """A top-k reaching zero or below (all-negative logits), a first half far
    below the second (the lower bound admits too many candidates), sorted
    logits, and a row with a NaN or +inf."""
    rng = np.random.default_rng(7302)
    R, V = 6, workloads.VOCAB
    x = rng.normal(0, 1, (R, V))
    x[0] = -np.abs(x[0]) - 1.0                                 # every value negative
    # Slots 12..15 of every wave far above slots 0..11: the lower bound taken
    # from the earlier slots admits most of the last ones as candidates.  Wave w
    # holds chunks [1010 w, 1010 (w + 1)), slot j its chunks 64 j .. 64 j + 63.
    for wv in range(16):
        x[1, 8 * (1010 * wv + 768):8 * 1010 * (wv + 1)] += 6.0
    x[2] = np.sort(x[2])                                       # increasing
    x[3, 17] = np.nan
    x[4, 99] = np.inf
    pols = [dict(temperature=1.0, top_k=100, top_p=0.9), dict(temperature=0.8, top_k=1024),
            dict(temperature=0.8, top_k=1000, top_p=0.95), dict(top_k=10), dict(top_k=10),
            dict(temperature=1.2, top_k=700)]
    w = workloads.Workload("handed", "bf16", workloads.bf16_round(x), pols, rng.random(R))
    gpu = check(w)
    assert general(gpu)[[0, 1, 2]].all()
    assert int(gpu["status"][3]) == N.E_LOGITS and int(gpu["status"][4]) == N.E_LOGITS
    assert not general(gpu)[5]


def test_odd_vocabulary_sizes_and_f64_probabilities():
    """Vocabularies whose chunk count is not a multiple of 16 (the last wave's
    range is short) and float64 probability outputs."""
    rng = np.random.default_rng(7403)
    for V in (129272, 8008, 520, 8):
        R = 4
        x = rng.normal(0, 2, (R, V))
        pols = [dict(temperature=0.9, top_k=min(40, V - 1), top_p=0.95), dict(temperature=0.0, top_k=3),
                dict(temperature=1.3, top_k=min(1024, V - 1), min_p=0.01), dict(temperature=0.5, top_k=1)]
        w = workloads.Workload(f"odd{V}", "bf16", workloads.bf16_round(x), pols, rng.random(R))
        check(w, probs="f64")
