"""The one-workgroup FP32 top-k kernel (k_sample_f32) against the oracle on
identical inputs and uniforms: token ids, consumption flags, statuses and
top-k index sets bit-exact, probabilities within 1e-5 relative, and no row
excused by the oracle's rounding band.  The rows sit on the kernel's
decision points: ties at the k-th value and the top-p boundary (values on a
coarse grid), greedy rows with tied maxima, all-negative rows, rows whose
top-k reaches past zero, masks from 1% to 99.9% disallowed, -inf, +-0, and
rows it must hand to the general path (NaN / +inf, fewer allowed tokens
than k).  Each test also checks which kernel decided each row."""
import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch, workloads
from oracle import pcg64_oracle as P
from oracle import sampling_oracle as O
from parity_util import compare, run_gpu

pytestmark = pytest.mark.gpu


def check(w, probs="f32"):
    gpu = run_gpu(w, probs=probs, kept=True)
    rep = compare(w, gpu)
    print(f"{w.name}: rows={rep.rows} exact={rep.exact} margin={rep.margin_rows} flagged={rep.flagged}", flush=True)
    assert not rep.mismatches, rep.mismatches[:10]
    assert not rep.margin_rows, rep.margin_rows
    return gpu


def f32_path(gpu):
    return (gpu["flags"] & N.FLAG_F32_TOPK) != 0


def test_c3_rows_as_fp32():
    w = workloads.c3f32()
    gpu = check(w)
    assert f32_path(gpu).all(), np.flatnonzero(~f32_path(gpu))


def tied_rows(V, rng, R=12, sign=1.0):
    """Values on a grid of 0.25 (exact in FP32), so that the k-th value and the
    top-p boundary fall inside groups of equal values (ties cut by index)."""
    x = np.round(rng.normal(0, 1, (R, V)) * 4) / 4
    if sign > 0:
        x[:, rng.choice(V, 6, replace=False)] = 3.0
    else:
        # Every value negative (continuous, so no tie group at the top holds
        # thousands of tokens), six maxima tied at -0.25.
        x = -np.abs(rng.normal(0, 1, (R, V))) - 0.5
        x[:, rng.choice(V, 6, replace=False)] = -0.25
    pols = []
    for r in range(R):
        pols.append(dict(temperature=[0.3, 0.7, 1.0, 1.5][r % 4],
                         top_k=min([1, 2, 6, 7, 50, 333, 1000, 1024][r % 8], V - 1),
                         top_p=[1.0, 0.5, 0.9, 0.999][r % 4]))
    pols[0] = dict(temperature=0.0, top_k=5)                   # greedy: first of the tied maxima
    pols[1] = dict(temperature=1.0, top_k=min(6, V - 1), top_p=0.4)
    pols[2] = dict(temperature=0.8, top_k=min(50, V - 1), min_p=0.3)
    return workloads.Workload(f"tied{V}", "f32", x.astype(np.float32), pols, rng.random(R))


@pytest.mark.parametrize("V", [129280, 50000, 4096, 1000, 64, 8])
def test_ties_at_the_top_k_and_top_p_boundaries(V):
    rng = np.random.default_rng(8100 + V)
    w = tied_rows(V, rng)
    gpu = check(w, probs="f64")
    # The lower bound comes from the row's V / 4 quad maxima: a top-k above
    # that count hands the row over (small vocabularies only).
    fits = np.array([p["temperature"] == 0.0 or p["top_k"] <= V // 4 for p in w.policies])
    assert (f32_path(gpu) == fits).all(), (np.flatnonzero(~f32_path(gpu)), np.flatnonzero(~fits))


def test_all_negative_rows_and_top_k_past_zero():
    rng = np.random.default_rng(8201)
    V = 129280
    w = tied_rows(V, rng, R=8, sign=-1.0)              # every value <= 0: top-k among negatives
    gpu = check(w)
    assert f32_path(gpu).all()
    x = rng.normal(0, 1, (6, V)).astype(np.float32)
    x[:, :V // 2] -= 20.0                             # half the row far below zero
    pols = [dict(temperature=1.0, top_k=k) for k in (1024, 700, 64, 1, 1000, 333)]
    w = workloads.Workload("past0", "f32", x, pols, rng.random(6))
    gpu = check(w)
    assert f32_path(gpu).all()


def test_masks_infinities_and_signed_zeros():
    rng = np.random.default_rng(8302)
    R, V = 10, 129280
    x = rng.normal(0, 2, (R, V)).astype(np.float32)
    keep = [0.99, 0.9, 0.5, 0.1, 0.01, 0.001, 0.9, 0.9, 0.9, 0.9]
    allowed = np.stack([rng.random(V) < keep[r] for r in range(R)])
    x[6, rng.choice(V, 5000, replace=False)] = -np.inf   # -inf tokens are never kept
    x[7] -= 10.0
    zeros = rng.choice(V, 40, replace=False)
    x[7, zeros] = np.where(np.arange(40) % 2 == 0, 0.0, -0.0)   # +-0: one tie group of 40
    x[7, rng.choice(np.setdiff1d(np.arange(V), zeros), 3, replace=False)] = 1.0
    x[8, :] = -np.inf
    x[8, rng.choice(V, 30, replace=False)] = rng.normal(0, 1, 30)   # 30 finite tokens, k = 64: too few
    pols = [dict(temperature=float(rng.uniform(0.3, 1.5)), top_k=int(rng.integers(1, 1025)),
                 top_p=float(rng.uniform(0.5, 1.0))) for _ in range(R)]
    pols[5]["top_k"] = 64                                # 0.1% allowed: about 129 tokens
    pols[7].update(top_k=8, temperature=1.0)
    pols[8].update(top_k=64)
    pols[9] = dict(temperature=0.0, top_k=10)
    w = workloads.Workload("masks", "f32", x, pols, rng.random(R), allowed=allowed)
    gpu = check(w, probs="f64")
    on = f32_path(gpu)
    assert on[[0, 1, 2, 3, 4, 5, 6, 7, 9]].all(), np.flatnonzero(~on)
    assert not on[8] and gpu["flags"][8] & N.FLAG_GENERAL   # fewer finite tokens than k: handed over


def test_invalid_rows_take_the_general_path():
    rng = np.random.default_rng(8403)
    R, V = 4, 4096
    x = rng.normal(0, 1, (R, V)).astype(np.float32)
    x[0, 17] = np.nan
    x[1, 4095] = np.inf
    x[2, :] = -np.inf
    pols = [dict(top_k=10)] * R
    w = workloads.Workload("invalid", "f32", x, pols, rng.random(R))
    gpu = check(w)
    assert int(gpu["status"][0]) == N.E_LOGITS and int(gpu["status"][1]) == N.E_LOGITS
    assert int(gpu["status"][2]) == N.E_MASKED
    assert f32_path(gpu)[3] and not f32_path(gpu)[:3].any()


def test_vocabularies_off_the_kernel_take_other_paths():
    """A vocabulary that is not a multiple of 4, or rows that do not start on a
    16-byte boundary, leave the FP32 kernel; the results are the same."""
    rng = np.random.default_rng(8504)
    for V in (1002, 16385):
        x = rng.normal(0, 2, (3, V)).astype(np.float32)
        pols = [dict(temperature=0.9, top_k=40), dict(temperature=0.0, top_k=3), dict(top_k=7, min_p=0.05)]
        w = workloads.Workload(f"odd{V}", "f32", x, pols, rng.random(3))
        gpu = check(w)
        assert not f32_path(gpu).any()
    # Strided rows (ld = V + 1): not 16-byte aligned past the first row.
    V = 4096
    base = rng.normal(0, 1, (4, V + 1)).astype(np.float32)
    t = torch.from_numpy(base).cuda()[:, :V]
    pols = [dict(temperature=0.8, top_k=30)] * 4
    u = rng.random(4)
    res = batch.sample_rows(t, pols, uniforms=torch.from_numpy(u).cuda())
    for r in range(4):
        ref = O.sample_row(base[r, :V], O.Policy(**pols[r]), float(u[r]))
        assert int(res.tokens[r]) == ref.token
    assert not (res.flags.cpu().numpy() & N.FLAG_F32_TOPK).any()


def test_device_draws_and_repeated_rows():
    rng = np.random.default_rng(8605)
    B, V = 6, 129280
    logits = rng.normal(0, 2, (B, V)).astype(np.float32)
    pols = [dict(top_k=50, top_p=0.9, temperature=0.7), dict(top_k=1), dict(temperature=0.0, top_k=3),
            dict(top_k=300, min_p=0.02), dict(top_k=1024, temperature=2.0), dict(top_k=2, top_p=0.1)]
    gens = [np.random.default_rng(300 + r) for r in range(B)]
    st0 = [g.bit_generator.state["state"] for g in gens]
    states = batch.pcg64_states(gens, "cuda")
    res = batch.sample_rows(torch.from_numpy(logits).cuda(), pols, rng_state=states)
    words = states.cpu().numpy().view(np.uint64)
    flags = res.flags.cpu().numpy()
    for r in range(B):
        s_next, u = P.random(st0[r]["state"], st0[r]["inc"])
        ref = O.sample_row(logits[r], O.Policy(**pols[r]), u)
        assert int(res.tokens[r]) == ref.token and bool(res.consumed[r]) == ref.consumed, r
        now = int(words[r, 0]) | (int(words[r, 1]) << 64)
        assert now == (s_next if ref.consumed else st0[r]["state"]), r
    assert (flags & N.FLAG_F32_TOPK).all(), flags


def test_sorted_tail_edge_rows():
    """Rows whose float64 steps collapse distinct values: logits near 1e-30
    (every exp rounds to 1, so the top-p tie group holds tokens of different
    z, cut by index), a denormal temperature (every z but the maximum's is
    -inf), and an exact two-way tie at the maximum under a tiny top-p; both
    tails (lists of at most 64 candidates finish in one wave, longer ones
    in the workgroup's sorted tail)."""
    rng = np.random.default_rng(8706)
    V = 4096
    x = rng.normal(0, 1, (8, V)).astype(np.float32)
    x[0] *= np.float32(1e-30)
    x[1] *= np.float32(1e-30)
    x[6] *= np.float32(1e-30)
    x[7] *= np.float32(1e-30)
    x[3, rng.choice(V, 2, replace=False)] = 9.0
    pols = [dict(temperature=1.0, top_k=100, top_p=0.37),
            dict(temperature=0.5, top_k=1000, top_p=0.999, min_p=0.5),
            dict(temperature=1e-320, top_k=50, top_p=0.9),
            dict(temperature=1.0, top_k=20, top_p=1e-9),
            dict(temperature=0.05, top_k=7, min_p=1e-3),
            dict(temperature=2.0, top_k=1024, top_p=0.6),
            dict(temperature=1.0, top_k=40, top_p=0.37),                 # short lists: one wave's tail
            dict(temperature=0.9, top_k=60, top_p=0.8, min_p=0.5)]
    w = workloads.Workload("edges", "f32", x, pols, rng.random(8))
    gpu = check(w, probs="f64")
    assert f32_path(gpu).all(), np.flatnonzero(~f32_path(gpu))
