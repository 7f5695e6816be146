"""Split-row top-k path: float32 / float64 rows with a top-k filter (k <= 1024)
or a greedy policy, no history or bias, V >= 16,384.  The row's slices keep
their k largest values in several workgroups and one workgroup per row
finishes from those candidates; rows the candidates cannot decide go to the
general path (flags bits 4-7 = 7, or 6 for invalid logits).

Every row is checked against the oracle on the same uniforms: statuses, the
top-k kept set, consumption and tokens bit-exact, probabilities within
1e-12 relative.  No row is waived: a token that differs fails its test even
where the oracle's own decision sits within 1e-11 of its threshold (the
kernel's rounding-band flag excuses nothing).
"""
import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch, workloads
from oracle import sampling_oracle as O
from parity_util import compare, run_gpu

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run(logits, pols, u, allowed=None, dtype=torch.float32, probs="f64", **kw):
    # No TOPK_ALL hint: fp32 top-k batches would otherwise take the one-workgroup
    # FP32 kernel (tests/test_gpu_f32.py), and these tests are the split path's.
    kw.setdefault("hints", 0)
    x = torch.from_numpy(np.ascontiguousarray(logits)).to(DEV).to(dtype)
    allow = None if allowed is None else torch.from_numpy(batch.pack_allow(allowed).view(np.int32)).to(DEV)
    res = batch.sample_rows(x, pols, allow_bits=allow, uniforms=torch.from_numpy(np.asarray(u, np.float64)).to(DEV),
                            probs=probs, kept=True, **kw)
    torch.cuda.synchronize()
    return res


def check(logits, pols, u, res, allowed=None, rtol=1e-12, skip=()):
    V = logits.shape[1]
    kept = batch.unpack_bits(res.kept_bits.cpu().numpy().view(np.uint32), V)
    probs = res.probs.cpu().numpy().astype(np.float64)
    flags = res.flags.cpu().numpy()
    for r in range(len(pols)):
        if r in skip:
            continue
        ref = O.sample_row(logits[r], O.Policy(**pols[r]), float(u[r]),
                           allowed=None if allowed is None else allowed[r])
        assert int(res.status[r]) == ref.status, (r, int(res.status[r]), ref.status)
        if ref.status:
            continue
        got = (int(res.tokens[r]), bool(res.consumed[r]))
        assert got == (ref.token, ref.consumed), (r, got, ref.token, ref.margin, pols[r])
        np.testing.assert_array_equal(kept[r], ref.topk_kept, err_msg=f"row {r}")
        np.testing.assert_allclose(probs[r], ref.probs, rtol=rtol, atol=1e-300, err_msg=f"row {r}")
    return flags


def reason(flags):
    return (flags >> 4) & 15


def policies(rng, rows, ks=(1, 2, 7, 50, 333, 1024)):
    out = []
    for r in range(rows):
        k = int(ks[r % len(ks)])
        out.append(dict(temperature=float(rng.choice([0.3, 0.7, 1.0, 1.6])), top_k=k,
                        top_p=float(rng.choice([1.0, 0.9, 0.5])), min_p=float(rng.choice([0.0, 0.0, 0.05]))))
    return out


def test_c1_takes_the_split_path():
    w = workloads.c1()
    gpu = run_gpu(w, hints=0)
    rep = compare(w, gpu)
    assert not rep.mismatches, rep.mismatches
    assert gpu["flags"][0] & N.FLAG_SPLIT and not gpu["flags"][0] & N.FLAG_GENERAL


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("V", [129280, 20000, 16384])
def test_random_rows_match_oracle(dtype, V):
    rng = np.random.default_rng(V + (7 if dtype == torch.float64 else 0))
    B = 12
    logits = rng.normal(0, 2, (B, V))
    if dtype == torch.float32:
        logits = logits.astype(np.float32)
    pols = policies(rng, B)
    pols[5] = dict(temperature=0.0, top_k=0)   # greedy rows take the path whatever their top-k
    pols[11] = dict(temperature=0.0, top_k=40)
    allowed = rng.random((B, V)) < 0.9
    u = rng.random(B)
    res = run(logits, pols, u, allowed, dtype=dtype)
    flags = check(logits, pols, u, res, allowed)
    assert (flags & N.FLAG_SPLIT).all(), flags


@pytest.mark.parametrize("B,V", [(1, 129280), (3, 129280), (64, 32768), (300, 16384)])
def test_batch_sizes_and_slice_counts(B, V):
    rng = np.random.default_rng(B)
    logits = rng.normal(0, 1.5, (B, V)).astype(np.float32)
    pols = policies(rng, B, ks=(1, 16, 100, 700, 1024, 3))
    u = rng.random(B)
    res = run(logits, pols, u, probs="f32")
    V_ = logits.shape[1]
    kept = batch.unpack_bits(res.kept_bits.cpu().numpy().view(np.uint32), V_)
    probs = res.probs.cpu().numpy().astype(np.float64)
    flags = res.flags.cpu().numpy()
    assert (flags & N.FLAG_SPLIT).all()
    for r in range(B):
        ref = O.sample_row(logits[r], O.Policy(**pols[r]), float(u[r]))
        assert int(res.status[r]) == 0
        np.testing.assert_array_equal(kept[r], ref.topk_kept)
        pos = ref.probs > 0
        assert np.all(probs[r][~pos] == 0)
        assert np.max(np.abs(probs[r][pos] - ref.probs[pos]) / ref.probs[pos]) < 1e-6
        assert int(res.tokens[r]) == ref.token, (r, int(res.tokens[r]), ref.token, ref.margin)


def test_exact_ties_at_the_kth_value_are_cut_by_index():
    """bf16-valued fp32 logits and integer logits put many equal values at the
    k-th place, spread over slices; the kept ties are the lowest indices."""
    rng = np.random.default_rng(3)
    V = 129280
    rows = [workloads.bf16_round(rng.normal(0, 2, V)), np.round(rng.normal(0, 2, V)).astype(np.float32),
            np.zeros(V, np.float32), np.round(rng.normal(0, 0.5, V)).astype(np.float32)]
    logits = np.stack(rows)
    pols = [dict(top_k=50, temperature=0.8), dict(top_k=1000, top_p=0.95), dict(top_k=50),
            dict(top_k=700, temperature=2.0, min_p=0.1)]
    u = rng.random(len(pols))
    res = run(logits, pols, u)
    flags = check(logits, pols, u, res)
    assert flags[2] & N.FLAG_SPLIT  # all-equal row: every slice's kept ties precede the cut or end it


def test_values_merged_by_rounding_go_to_the_general_path():
    """A huge maximum makes (v - max) / T equal for many distinct v: the k-th
    tie group then mixes values, which the candidates cannot order."""
    rng = np.random.default_rng(4)
    V = 65536
    x = rng.normal(0, 1, V).astype(np.float32)
    x[12345] = 1e30
    logits = np.stack([x])
    pols = [dict(top_k=20, temperature=1.0)]
    u = np.array([0.3])
    res = run(logits, pols, u)
    flags = check(logits, pols, u, res)
    assert flags[0] & N.FLAG_GENERAL and reason(flags[0]) == 7


def test_invalid_masked_and_ineligible_rows():
    rng = np.random.default_rng(6)
    V = 40000
    logits = rng.normal(0, 1, (7, V)).astype(np.float32)
    logits[0, 777] = np.nan
    logits[1, 39999] = np.inf
    allowed = np.ones((7, V), bool)
    allowed[2] = False
    pols = [dict(top_k=5), dict(top_k=5), dict(top_k=5), dict(top_k=0, top_p=0.8), dict(top_k=2000),
            dict(top_k=5, temperature=-1.0), dict(top_k=V - 1)]
    u = rng.random(7)
    res = run(logits, pols, u, allowed)
    # Row 5's policy is out of bounds: the reference rejects it when the policy
    # is built (sampling.py:38-43), so the oracle has no row result for it.
    flags = check(logits, pols, u, res, allowed, skip=(5,))
    st = res.status.cpu().numpy()
    assert list(st[:3]) == [N.E_LOGITS, N.E_LOGITS, N.E_MASKED] and st[5] == N.E_POLICY
    assert not (flags & N.FLAG_SPLIT).any()
    assert reason(flags[0]) == 6 and reason(flags[2]) == 6


def test_slices_with_few_finite_values():
    """Whole slices masked, and fewer than k finite tokens in the row."""
    rng = np.random.default_rng(8)
    V = 131072 - 1792  # 129,280
    logits = rng.normal(0, 1, (3, V)).astype(np.float32)
    allowed = np.ones((3, V), bool)
    allowed[0, :100000] = False
    allowed[1] = rng.random(V) < 0.002  # about 260 finite tokens
    allowed[2, :] = False
    allowed[2, [5, 70000, 129279]] = True
    pols = [dict(top_k=64, top_p=0.9), dict(top_k=1000), dict(top_k=10, temperature=0.5)]
    u = rng.random(3)
    res = run(logits, pols, u, allowed)
    check(logits, pols, u, res, allowed)


def test_strided_rows_and_f32_probabilities():
    rng = np.random.default_rng(12)
    V, ld = 30001, 30080
    base = rng.normal(0, 1, (5, ld)).astype(np.float32)
    x = torch.from_numpy(base).to(DEV)[:, :V]
    pols = [dict(top_k=k, top_p=0.8, temperature=0.9) for k in (1, 9, 64, 512, 1024)]
    u = rng.random(5)
    res = batch.sample_rows(x, pols, uniforms=torch.from_numpy(u).to(DEV), probs="f32", hints=0)
    torch.cuda.synchronize()
    for r in range(5):
        ref = O.sample_row(base[r, :V], O.Policy(**pols[r]), float(u[r]))
        assert int(res.tokens[r]) == ref.token, (r, int(res.tokens[r]), ref.token, ref.margin)
        assert int(res.flags[r]) & N.FLAG_SPLIT


def test_device_draws_on_the_split_path():
    from oracle import pcg64_oracle as P
    rng = np.random.default_rng(21)
    B, V = 4, 129280
    logits = rng.normal(0, 2, (B, V)).astype(np.float32)
    pols = [dict(top_k=50, top_p=0.9, temperature=0.7), dict(top_k=1), dict(temperature=0.0, top_k=3),
            dict(top_k=300, min_p=0.02)]
    gens = [np.random.default_rng(100 + r) for r in range(B)]
    st0 = [g.bit_generator.state["state"] for g in gens]
    states = batch.pcg64_states(gens, DEV)
    x = torch.from_numpy(logits).to(DEV)
    res = batch.sample_rows(x, pols, rng_state=states, hints=0)
    torch.cuda.synchronize()
    words = states.cpu().numpy().view(np.uint64)
    for r in range(B):
        s_next, u = P.random(st0[r]["state"], st0[r]["inc"])
        ref = O.sample_row(logits[r], O.Policy(**pols[r]), u)
        assert int(res.tokens[r]) == ref.token, (r, int(res.tokens[r]), ref.token, ref.margin)
        assert bool(res.consumed[r]) == ref.consumed
        now = int(words[r, 0]) | (int(words[r, 1]) << 64)
        assert now == (s_next if ref.consumed else st0[r]["state"])
        assert int(res.flags[r]) & N.FLAG_SPLIT


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_rows_with_histories_match_oracle(dtype):
    """Penalised and biased rows: each slice applies the history and bias
    entries that fall in it."""
    rng = np.random.default_rng(31 if dtype == torch.float32 else 32)
    B, V = 6, 129280
    logits = rng.normal(0, 2, (B, V))
    if dtype == torch.float32:
        logits = logits.astype(np.float32)
    counts = np.zeros((B, V), np.int32)
    gens = np.zeros((B, V), np.int32)
    for r, n in enumerate((0, 10, 300, 4096, 16384, 60000)):
        h = rng.integers(0, V, n)
        counts[r] = np.bincount(h, minlength=V)
        gens[r] = np.minimum(counts[r], np.bincount(h[n // 3:], minlength=V))
    ks = (1, 50, 1024, 7, 300, 0)
    pols = []
    for r in range(B):
        pol = dict(temperature=float(rng.choice([0.5, 1.0, 1.4])), top_k=ks[r], top_p=float(rng.choice([1.0, 0.9])),
                   repetition_penalty=float(rng.uniform(0.5, 2)), presence_penalty=float(rng.uniform(-2, 2)),
                   frequency_penalty=float(rng.uniform(-2, 2)))
        if ks[r] == 0:
            pol["temperature"] = 0.0  # greedy over the penalised logits
        pols.append(pol)
    allowed = rng.random((B, V)) < 0.9
    biases = [{int(t): float(rng.uniform(-100, 100)) for t in rng.choice(V, int(rng.integers(1, 40)), replace=False)}
              for _ in range(B)]
    biases[0] = {}
    biases[1][int(np.argmin(logits[1]))] = 100.0  # lifts the row's smallest logit into its top-k
    u = rng.random(B)
    x = torch.from_numpy(np.ascontiguousarray(logits)).to(DEV).to(dtype)
    res = batch.sample_rows(x, pols, history=batch.HistoryTable.from_dense(counts, gens, device=DEV),
                            bias=batch.BiasTable.from_dicts(biases, device=DEV),
                            allow_bits=torch.from_numpy(batch.pack_allow(allowed).view(np.int32)).to(DEV),
                            uniforms=torch.from_numpy(u).to(DEV), probs="f64", kept=True)
    torch.cuda.synchronize()
    kept = batch.unpack_bits(res.kept_bits.cpu().numpy().view(np.uint32), V)
    probs = res.probs.cpu().numpy()
    flags = res.flags.cpu().numpy()
    for r in range(B):
        ref = O.sample_row(logits[r], O.Policy(**pols[r]), float(u[r]), counts[r], gens[r], biases[r], allowed[r])
        assert int(res.status[r]) == ref.status == 0
        assert (int(res.tokens[r]), bool(res.consumed[r])) == (ref.token, ref.consumed), (r, ref.margin)
        np.testing.assert_array_equal(kept[r], ref.topk_kept)
        np.testing.assert_allclose(probs[r], ref.probs, rtol=1e-12, atol=1e-300)
    assert (flags & N.FLAG_SPLIT).all(), flags


def test_invalid_history_tables_take_the_general_path():
    V = 20000
    rng = np.random.default_rng(33)
    logits = rng.normal(0, 1, (3, V)).astype(np.float32)
    d = DEV
    # Row 0: generated above counts; row 1: counts summing past the limit; row 2: valid.
    off = torch.tensor([0, 1, 3, 4], device=d)
    ids = torch.tensor([5, 7, 9, 11], dtype=torch.int32, device=d)
    cnt = torch.tensor([1, 600_000, 600_000, 2], dtype=torch.int32, device=d)
    gen = torch.tensor([2, 0, 0, 1], dtype=torch.int32, device=d)
    h = batch.HistoryTable(off, ids, cnt, gen)
    pols = [dict(top_k=5)] * 3
    res = batch.sample_rows(torch.from_numpy(logits).to(d), pols, history=h,
                            uniforms=torch.tensor([0.5] * 3, dtype=torch.float64, device=d))
    torch.cuda.synchronize()
    st = res.status.cpu().numpy()
    flags = res.flags.cpu().numpy()
    assert list(st) == [N.E_GENERATED, N.E_COUNTS, 0]
    assert reason(flags[0]) == 6 and reason(flags[1]) == 6 and flags[2] & N.FLAG_SPLIT
    c2 = np.zeros(V, np.int32)
    c2[11] = 2
    g2 = np.zeros(V, np.int32)
    g2[11] = 1
    ref = O.sample_row(logits[2], O.Policy(top_k=5), 0.5, c2, g2)
    assert int(res.tokens[2]) == ref.token


def test_invalid_bias_lists_take_the_general_path():
    V = 20000
    rng = np.random.default_rng(34)
    logits = rng.normal(0, 1, (3, V)).astype(np.float32)
    d = DEV
    # Row 0: ids out of order; row 1: a bias above 100; row 2: valid.
    b = batch.BiasTable(torch.tensor([0, 2, 3, 4], device=d), torch.tensor([9, 3, 5, 17], dtype=torch.int32, device=d),
                        torch.tensor([1.0, 2.0, 150.0, -3.5], dtype=torch.float64, device=d))
    pols = [dict(top_k=5, temperature=0.8)] * 3
    res = batch.sample_rows(torch.from_numpy(logits).to(d), pols, bias=b,
                            uniforms=torch.tensor([0.25] * 3, dtype=torch.float64, device=d))
    torch.cuda.synchronize()
    st = res.status.cpu().numpy()
    flags = res.flags.cpu().numpy()
    assert list(st) == [N.E_BIAS, N.E_BIAS, 0]
    assert reason(flags[0]) == 6 and reason(flags[1]) == 6 and flags[2] & N.FLAG_SPLIT
    ref = O.sample_row(logits[2], O.Policy(**pols[2]), 0.25, None, None, {17: -3.5})
    assert int(res.tokens[2]) == ref.token


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_rows_without_top_k(dtype):
    """Top-p / min-p rows with no top-k: decided from the row's 512 largest
    values when the kept tokens lie among them (peaked rows), otherwise by the
    general path (flat rows, reason 8)."""
    rng = np.random.default_rng(41 if dtype == torch.float32 else 42)
    B, V = 10, 129280
    x = rng.normal(0, 1, (B, V))
    for r in range(B - 2):
        pos = rng.choice(V, 24, replace=False)
        x[r, pos] += rng.uniform(8, 15, 24)
    x[B - 2] = rng.normal(0, 0.1, V)   # flat: top-p keeps most of the row
    x[B - 1] = rng.normal(0, 0.1, V)
    logits = x.astype(np.float32) if dtype == torch.float32 else x
    pols = [dict(temperature=0.7, top_p=0.9), dict(top_p=0.5), dict(temperature=1.3, top_p=0.95, min_p=0.02),
            dict(min_p=0.05), dict(temperature=0.5, min_p=0.2, top_p=0.99), dict(top_p=0.8, top_k=V),
            dict(temperature=0.9, top_p=0.0), dict(top_p=0.9, min_p=1.0),
            dict(top_p=0.95), dict(min_p=0.5)]
    allowed = rng.random((B, V)) < 0.9
    u = rng.random(B)
    res = run(logits, pols, u, allowed, dtype=dtype)
    flags = check(logits, pols, u, res, allowed)
    assert (flags[:B - 2] & N.FLAG_SPLIT).all(), flags
    assert reason(flags[B - 2]) == 8


def test_rows_without_top_k_with_history_and_bias():
    rng = np.random.default_rng(43)
    B, V = 4, 65536
    x = rng.normal(0, 1, (B, V))
    for r in range(B):
        pos = rng.choice(V, 16, replace=False)
        x[r, pos] += rng.uniform(14, 18, 16)  # peaked: the 0.9 top-p set lies among the spikes
    logits = x.astype(np.float32)
    counts = np.zeros((B, V), np.int32)
    for r in range(B):
        counts[r] = np.bincount(rng.integers(0, V, 3000), minlength=V)
    biases = [{int(t): float(rng.uniform(-5, 5)) for t in rng.choice(V, 20, replace=False)} for _ in range(B)]
    pols = [dict(top_p=0.9, repetition_penalty=1.2, presence_penalty=0.4, frequency_penalty=0.2)] * B
    u = rng.random(B)
    xt = torch.from_numpy(logits).to(DEV)
    res = batch.sample_rows(xt, pols, history=batch.HistoryTable.from_dense(counts, counts, device=DEV),
                            bias=batch.BiasTable.from_dicts(biases, device=DEV),
                            uniforms=torch.from_numpy(u).to(DEV), probs="f64", kept=True)
    torch.cuda.synchronize()
    kept = batch.unpack_bits(res.kept_bits.cpu().numpy().view(np.uint32), V)
    probs = res.probs.cpu().numpy()
    flags = res.flags.cpu().numpy()
    for r in range(B):
        ref = O.sample_row(logits[r], O.Policy(**pols[r]), float(u[r]), counts[r], counts[r], biases[r])
        assert int(res.status[r]) == ref.status == 0
        assert int(res.tokens[r]) == ref.token, (r, int(res.tokens[r]), ref.token, ref.margin)
        np.testing.assert_array_equal(kept[r], ref.topk_kept)
        np.testing.assert_allclose(probs[r], ref.probs, rtol=1e-12, atol=1e-300)
    assert (flags & N.FLAG_SPLIT).all(), flags


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("V", [129280, 20000])
def test_rows_without_any_filter(dtype, V):
    """The default policy (T 1, no top-k / top-p / min-p) and temperature-only
    rows: the slices' sums and one pass over the row decide them."""
    rng = np.random.default_rng(V + (51 if dtype == torch.float32 else 52))
    B = 6
    logits = rng.normal(0, 2, (B, V))
    logits[3] = rng.normal(0, 0.01, V)  # nearly flat
    if dtype == torch.float32:
        logits = logits.astype(np.float32)
    pols = [dict(), dict(temperature=0.5), dict(temperature=2.0), dict(), dict(temperature=1e-3), dict(top_k=V)]
    allowed = rng.random((B, V)) < 0.9
    allowed[4] = False
    allowed[4, [17, 18]] = True  # two tokens left
    u = rng.random(B)
    res = run(logits, pols, u, allowed, dtype=dtype)
    flags = check(logits, pols, u, res, allowed)
    assert (flags & N.FLAG_SPLIT).all(), flags


def test_rows_without_any_filter_draw_on_device_and_skip_history_rows():
    from oracle import pcg64_oracle as P
    rng = np.random.default_rng(53)
    B, V = 3, 129280
    logits = rng.normal(0, 2, (B, V)).astype(np.float32)
    gens = [np.random.default_rng(200 + r) for r in range(B)]
    st0 = [g.bit_generator.state["state"] for g in gens]
    states = batch.pcg64_states(gens, DEV)
    counts = np.zeros((B, V), np.int32)
    counts[2, :50] = 1  # row 2 has a history: the general path decides it
    res = batch.sample_rows(torch.from_numpy(logits).to(DEV), [dict()] * B,
                            history=batch.HistoryTable.from_dense(counts, counts, device=DEV), rng_state=states)
    torch.cuda.synchronize()
    words = states.cpu().numpy().view(np.uint64)
    flags = res.flags.cpu().numpy()
    for r in range(B):
        s_next, u = P.random(st0[r]["state"], st0[r]["inc"])
        ref = O.sample_row(logits[r], O.Policy(), u, counts[r], counts[r])
        assert int(res.tokens[r]) == ref.token, (r, int(res.tokens[r]), ref.token, ref.margin)
        assert int(words[r, 0]) | (int(words[r, 1]) << 64) == s_next
    assert flags[0] & N.FLAG_SPLIT and flags[1] & N.FLAG_SPLIT
    assert flags[2] & N.FLAG_GENERAL and not flags[2] & N.FLAG_SPLIT
