"""HIP path against the oracle on identical inputs and pre-drawn uniforms.

Token ids, consumption flags, top-k index sets and statuses must be bit-exact;
fp32 probabilities within 1e-5 relative (exactly zero where the oracle is
zero).  The only tolerated token difference is a decision that the oracle
itself places inside the float64 rounding band (its margin below 1e-11, where
a different exp or summation order may legitimately pick the neighbour); the
kernel's own rounding-band flag excuses nothing.  The benchmark
configurations assert the observed count of such rows: zero.
"""
import json
import os

import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch, workloads
from oracle import sampling_oracle as O
from parity_util import MARGIN, compare, oracle_row, run_gpu

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def check(rep, margin_rows=0):
    """No mismatch, and at most ``margin_rows`` rows whose token differs
    where the oracle's own decision sat within 1e-11 of its threshold."""
    print(f"rows={rep.rows} exact={rep.exact} margin={rep.margin_rows} flagged={rep.flagged} "
          f"max_rel={rep.max_rel:.3g}", flush=True)
    assert not rep.mismatches, rep.mismatches[:10]
    assert len(rep.margin_rows) <= margin_rows, rep.margin_rows
    assert rep.exact + len(rep.margin_rows) == rep.rows


def test_c1_single_row_fp32():
    w = workloads.c1()
    gpu = run_gpu(w)
    check(compare(w, gpu))


def test_c2_penalised_rows():
    w = workloads.c2()
    gpu = run_gpu(w)
    check(compare(w, gpu))


def test_c3_metric_workload_all_rows():
    w = workloads.c3()
    gpu = run_gpu(w)
    check(compare(w, gpu))


def test_c5_stress_rows():
    w = workloads.c5()
    gpu = run_gpu(w, probs=None, kept=False)
    # Every greedy row at full size: the first argmax of the adjusted logits.
    V = w.logits.shape[1]
    for r in range(0, w.rows, 2):
        c = np.bincount(w.histories[r], minlength=V).astype(np.int32)
        v = O.adjusted_logits(w.logits[r], O.Policy(**w.policies[r]), c, c)
        assert gpu["tokens"][r] == int(np.argmax(v)) and gpu["consumed"][r] == 0 and gpu["status"][r] == 0
    # Every sampled row, from both families, against the full oracle.
    rows = list(range(1, w.rows, 2))
    sub = workloads.select_rows(w, rows)
    gpu_sub = {k: v[rows] for k, v in gpu.items()}
    check(compare(sub, gpu_sub))


def test_c5_near_tie_rows_with_probs_and_sets():
    w = workloads.select_rows(workloads.c5(), list(range(512, 544)))
    gpu = run_gpu(w)
    check(compare(w, gpu))


GOLD = np.load(os.path.join(HERE, "golden", "sampling_golden.npz"))
META = json.load(open(os.path.join(HERE, "golden", "sampling_golden.json")))


@pytest.mark.skip(reason="routing of history-less top-k rows to the top-k register path inside the "
                         "full-vocabulary kernel is not built: its one GPU run ended in a memory fault "
                         "whose cause was not found, so the routing was taken out")
def test_mixed_batch_of_history_and_top_k_rows():
    """One launch with bf16 rows that carry histories (no top-k) and rows with
    an empty history and a top-k: the latter take the top-k register path
    inside the full-vocabulary kernel, not the general path."""
    c2, c3 = workloads.c2(rows=8), workloads.c3(rows=8)
    logits = np.concatenate([c2.logits, c3.logits])
    pols = c2.policies + c3.policies
    hist = list(c2.histories) + [np.zeros(0, np.int64)] * 8
    w = workloads.Workload("mixed", "bf16", logits, pols, np.concatenate([c2.uniforms, c3.uniforms]),
                           histories=hist)
    gpu = run_gpu(w)
    check(compare(w, gpu))
    assert not (gpu["flags"][8:] & N.FLAG_GENERAL).any()
    assert not (gpu["flags"][:8] & N.FLAG_GENERAL).any()


def test_full_path_rows_with_many_equal_values():
    """bf16 rows with a history where more than 65,535 tokens share one value
    (a 16-bit key count would wrap): the register-resident path must hand them
    to the general path, and the result must still match the oracle."""
    rng = np.random.default_rng(5150)
    V, R = workloads.VOCAB, 4
    x = rng.normal(0, 1, (R, V))
    x[:, : 100_000] = 0.25                 # one bf16 value, 100k times
    x[1, 5] = 3.0                           # a clear maximum in one row
    logits = workloads.bf16_round(x)
    hist = [rng.choice(V, 300, replace=False) for _ in range(R)]
    pols = [dict(temperature=1.0, top_p=0.9, repetition_penalty=1.2, presence_penalty=0.4),
            dict(temperature=0.7, repetition_penalty=1.1, frequency_penalty=0.2),
            dict(temperature=0.0, presence_penalty=0.5),
            dict(temperature=1.3, top_p=0.5, min_p=0.01, frequency_penalty=0.3)]
    w = workloads.Workload("equal", "bf16", logits, pols, rng.random(R), histories=hist)
    gpu = run_gpu(w)
    check(compare(w, gpu))
    assert (gpu["flags"][[0, 1, 3]] & N.FLAG_GENERAL).all()  # sampled rows: the count check hands them over


@pytest.mark.parametrize("case", META["probabilities"], ids=lambda c: c["name"])
def test_golden_vectors_on_gpu(case):
    from test_oracle_golden import golden_case
    logits, counts, gen, bias, allowed = golden_case(case)
    n = case["name"]
    V = len(logits)
    dev = "cuda"
    x = torch.from_numpy(np.ascontiguousarray(logits)).to(dev).reshape(1, V)
    hist = None if counts is None else batch.HistoryTable.from_dense(counts[None], gen[None], device=dev)
    bt = None if bias is None else batch.BiasTable.from_dicts([bias], device=dev)
    allow = None if allowed is None else torch.from_numpy(batch.pack_allow(allowed[None]).view(np.int32)).to(dev)
    for u, want in zip(case["uniforms"], case["ids"]):
        res = batch.sample_rows(x, [case["policy"]], history=hist, bias=bt, allow_bits=allow,
                                uniforms=torch.tensor([u], dtype=torch.float64, device=dev), probs="f64")
        assert int(res.status.item()) == 0
        if int(res.tokens.item()) != want:
            # Tolerated only where the reference's own decision sat in the rounding band.
            ref = O.sample_row(logits, O.Policy(**case["policy"]), float(u), counts, gen, bias, allowed)
            assert ref.token == want and ref.margin < MARGIN, (n, u, int(res.tokens.item()), want)
        p = res.probs[0].cpu().numpy()
        if f"{n}/probs" in GOLD:
            ref = GOLD[f"{n}/probs"]
            np.testing.assert_array_equal(p > 0, ref > 0)
            np.testing.assert_allclose(p, ref, rtol=1e-12, atol=0)
        else:
            np.testing.assert_allclose(p[GOLD[f"{n}/probs_top_idx"]], GOLD[f"{n}/probs_top_val"], rtol=1e-12)
            assert abs(p.sum() - 1) < 1e-12


def _one(logits, policy, u=0.5, **kw):
    x = torch.as_tensor(np.asarray(logits)).to("cuda").reshape(1, -1)
    res = batch.sample_rows(x, [policy], uniforms=torch.tensor([u], dtype=torch.float64, device="cuda"),
                            probs="f64", **kw)
    return int(res.status.item()), int(res.tokens.item()), int(res.consumed.item()), res.probs[0].cpu().numpy()


def test_edge_cases_against_oracle():
    rng = np.random.default_rng(5)
    cases = [
        (np.array([0.5]), dict()),
        (np.array([1.0, 1.0]), dict()),
        (np.array([1.0, 1.0, 1.0]), dict(temperature=1e-320)),
        (np.log(np.array([.5, .3, .2])), dict(top_p=0.0)),
        (np.log(np.array([.5, .3, .2])), dict(min_p=1.0)),
        (np.array([-np.inf, 2.0, -np.inf]), dict(top_k=1)),
        (rng.normal(0, 1, 1000), dict(top_k=999, top_p=0.999999)),
        (rng.normal(0, 1, 1000), dict(top_k=1000)),
        (rng.normal(0, 1, 1000), dict(top_k=5000)),
        (np.round(rng.normal(0, 1, 777), 1), dict(top_k=37, top_p=0.6, temperature=0.3)),
        (rng.normal(0, 50, 4099), dict(temperature=100.0, min_p=0.9)),
        (np.zeros(64), dict(top_p=0.5)),
        (np.zeros(65), dict(top_k=3)),
    ]
    for logits, kw in cases:
        for dtype in (np.float64, np.float32):
            x = logits.astype(dtype)
            for u in (0.0, 0.37, np.nextafter(1.0, 0.0)):
                st, tok, used, p = _one(x, kw, float(u))
                ref = O.sample_row(x, O.Policy(**kw), float(u))
                assert st == ref.status, (kw, dtype)
                assert tok == ref.token and bool(used) == ref.consumed, (kw, dtype, u, tok, ref.token)
                np.testing.assert_allclose(p, ref.probs, rtol=1e-12, atol=1e-300)


def test_status_codes():
    assert _one(np.array([0.0, np.nan]), {})[0] == N.E_LOGITS
    assert _one(np.array([0.0, np.inf]), {})[0] == N.E_LOGITS
    assert _one(np.array([-np.inf, -np.inf]), {})[0] == N.E_MASKED
    allow = torch.zeros(1, 1, dtype=torch.int32, device="cuda")
    assert _one(np.array([1.0, 2.0]), {}, allow_bits=allow)[0] == N.E_MASKED
    assert _one(np.array([1.0, 2.0]), {}, u=1.0)[0] == N.E_UNIFORM
    assert _one(np.array([1.0, 2.0]), {}, u=-0.1)[0] == N.E_UNIFORM
    assert _one(np.array([1.0, 9.0]), {"temperature": 0}, u=7.0)[0] == 0   # no draw: the uniform is not read
    assert _one(np.array([1.0, 2.0]), {"temperature": -1.0})[0] == N.E_POLICY
    assert _one(np.array([1.0, 2.0]), {"top_k": -2})[0] == N.E_POLICY
    d = "cuda"
    h = batch.HistoryTable(torch.tensor([0, 1], device=d), torch.tensor([1], dtype=torch.int32, device=d),
                           torch.tensor([1], dtype=torch.int32, device=d), torch.tensor([2], dtype=torch.int32, device=d))
    assert _one(np.array([1.0, 2.0]), {}, history=h)[0] == N.E_GENERATED
    h.counts.fill_(2_000_000)
    assert _one(np.array([1.0, 2.0]), {}, history=h)[0] == N.E_COUNTS
    h = batch.HistoryTable(torch.tensor([0, 1], device=d), torch.tensor([5], dtype=torch.int32, device=d),
                           torch.tensor([1], dtype=torch.int32, device=d), torch.tensor([1], dtype=torch.int32, device=d))
    assert _one(np.array([1.0, 2.0]), {}, history=h)[0] == N.E_COUNTS
    b = batch.BiasTable(torch.tensor([0, 1], device=d), torch.tensor([0], dtype=torch.int32, device=d),
                        torch.tensor([101.0], dtype=torch.float64, device=d))
    assert _one(np.array([1.0, 2.0]), {}, bias=b)[0] == N.E_BIAS


def test_penalties_bias_mask_match_oracle_on_mixed_rows():
    rng = np.random.default_rng(9)
    V, B = 5000, 24
    logits = workloads.bf16_round(rng.normal(0, 2, (B, V)))
    dev = "cuda"
    counts = np.zeros((B, V), np.int32)
    gens = np.zeros((B, V), np.int32)
    biases, pols = [], []
    for r in range(B):
        h = rng.integers(0, V, int(rng.integers(0, 400)))
        counts[r] = np.bincount(h, minlength=V)
        gens[r] = np.minimum(counts[r], np.bincount(h[len(h) // 3:], minlength=V))
        ids = rng.choice(V, int(rng.integers(0, 20)), replace=False)
        biases.append({int(t): float(rng.uniform(-100, 100)) for t in ids})
        pols.append(dict(temperature=float(rng.choice([0.0, 0.5, 1.0, 1.7])), top_k=int(rng.choice([0, 1, 40, 4999])),
                         top_p=float(rng.choice([1.0, 0.9, 0.3])), min_p=float(rng.choice([0.0, 0.02])),
                         repetition_penalty=float(rng.uniform(0.5, 2)), presence_penalty=float(rng.uniform(-2, 2)),
                         frequency_penalty=float(rng.uniform(-2, 2))))
    allowed = rng.random((B, V)) < 0.8
    u = rng.random(B)
    x = torch.from_numpy(workloads.bf16_bits(logits).view(np.int16)).to(dev).view(torch.bfloat16)
    res = batch.sample_rows(x, pols, history=batch.HistoryTable.from_dense(counts, gens, device=dev),
                            bias=batch.BiasTable.from_dicts(biases, device=dev),
                            allow_bits=torch.from_numpy(batch.pack_allow(allowed).view(np.int32)).to(dev),
                            uniforms=torch.from_numpy(u).to(dev), probs="f64", kept=True)
    kept = batch.unpack_bits(res.kept_bits.cpu().numpy().view(np.uint32), V)
    probs = res.probs.cpu().numpy()
    for r in range(B):
        ref = O.sample_row(logits[r], O.Policy(**pols[r]), float(u[r]), counts[r], gens[r], biases[r], allowed[r])
        assert int(res.status[r]) == ref.status
        if ref.status:
            continue
        if ref.margin >= MARGIN:
            assert int(res.tokens[r]) == ref.token and bool(res.consumed[r]) == ref.consumed, r
        np.testing.assert_array_equal(kept[r], ref.topk_kept)
        np.testing.assert_allclose(probs[r], ref.probs, rtol=1e-12, atol=1e-300)


def test_strided_rows_and_odd_vocab():
    rng = np.random.default_rng(2)
    V, ld = 1001, 1040
    base = rng.normal(0, 1, (6, ld)).astype(np.float32)
    x = torch.from_numpy(base).to("cuda")[:, :V]
    assert x.stride(0) == ld
    pols = [dict(top_k=20, top_p=0.8, temperature=0.9)] * 6
    u = rng.random(6)
    res = batch.sample_rows(x, pols, uniforms=torch.from_numpy(u).to("cuda"))
    for r in range(6):
        ref = O.sample_row(base[r, :V], O.Policy(**pols[r]), float(u[r]))
        assert int(res.tokens[r]) == ref.token


def test_verify_c4_against_oracle():
    w = workloads.c4()
    e = w.extra
    dev = "cuda"
    R, K, V = e["target"].shape[0], e["K"], e["target"].shape[2]
    tgt = torch.from_numpy(e["target"]).to(dev)
    drf = torch.from_numpy(e["draft"]).to(dev)
    # Proposal step on the GPU: draft ids drawn from each draft row.
    draw = batch.sample_rows(drf.reshape(R * K, V), [dict()] * (R * K),
                             uniforms=torch.from_numpy(e["u_draft"].reshape(-1)).to(dev))
    ids = draw.tokens.reshape(R, K).contiguous()
    res = batch.verify_drafts(tgt, drf, ids, [dict()] * R, torch.from_numpy(e["u_accept"]).to(dev),
                              torch.from_numpy(e["u_target"]).to(dev), torch.from_numpy(e["limit"]).to(dev))
    torch.cuda.synchronize()
    ids_np = ids.cpu().numpy()
    hits = 0
    for r in range(R):
        ref = O.verify(e["target"][r], e["draft"][r], list(ids_np[r]), O.Policy(), e["u_accept"][r],
                       float(e["u_target"][r]), output_limit=10)
        assert int(res.status[r]) == ref.status == 0
        got = (int(res.accepted[r]), tuple(int(t) for t in res.ids[r, :int(res.count[r])].tolist()),
               None if int(res.pending[r]) < 0 else int(res.pending[r]), int(res.used_accept[r]),
               int(res.used_target[r]))
        want = (ref.accepted, ref.output_ids, ref.pending, ref.used_accept, ref.used_target)
        assert got == want, (r, got, want, ref.margin)
        hits += 1
    assert hits == R == 32


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_fast_and_general_paths_match_the_oracle(dtype):
    """Filter-free requests take the statistics-only verifier; an all-ones
    allow mask sends the same requests through the full-distribution path.
    Both must equal the oracle on every request; a decision may differ only
    where the oracle's own margin is below 1e-11."""
    rng = np.random.default_rng(11)
    R, K, V = 24, 3, 5003
    tgt_np = rng.normal(0, 2, (R, K + 1, V)).astype(np.float32)
    drf_np = tgt_np[:, :K] + rng.normal(0, 0.5, (R, K, V)).astype(np.float32)
    dev = "cuda"
    tgt = torch.from_numpy(tgt_np).to(dev).to(dtype)
    drf = torch.from_numpy(drf_np).to(dev).to(dtype)
    temps = [1.0, 0.7, 1.3, 0.0]
    pols = [dict(temperature=temps[r % 4]) for r in range(R)]
    # Draft ids from the draft rows themselves, so most are plausible.
    draw = batch.sample_rows(drf.reshape(R * K, V).contiguous(), [dict()] * (R * K),
                             uniforms=torch.from_numpy(rng.random(R * K)).to(dev))
    ids = draw.tokens.reshape(R, K).contiguous()
    # Greedy requests (every fourth) propose each draft row's argmax, so their
    # proposals have probability one.
    greedy = torch.arange(R, device=dev) % 4 == 3
    ids[greedy] = drf.float().argmax(dim=-1).to(torch.int32)[greedy]
    ua_np, ut_np = rng.random((R, K)), rng.random(R)
    ua, ut = torch.from_numpy(ua_np).to(dev), torch.from_numpy(ut_np).to(dev)
    limits = np.array([10, 2, 3, 10] * (R // 4), dtype=np.int32)
    lim = torch.from_numpy(limits).to(dev)
    eos_ids = ids[:, 1].contiguous()  # the second draft of each request is an EOS token
    eos_off = torch.arange(0, R + 1, dtype=torch.int64, device=dev)
    words = (V + 31) // 32
    ones = torch.full((R, K + 1, words), -1, dtype=torch.int32, device=dev)  # every bit set
    kw = dict(eos_offsets=eos_off, eos_ids=eos_ids)
    fast = batch.verify_drafts(tgt, drf, ids, pols, ua, ut, lim, **kw)
    gen = batch.verify_drafts(tgt, drf, ids, pols, ua, ut, lim, allow_bits=ones, **kw)
    torch.cuda.synchronize()
    # The oracle sees the logits the device sees (bf16 rows rounded once).
    tgt_seen = tgt.float().cpu().numpy()
    drf_seen = drf.float().cpu().numpy()
    ids_np, eos_np = ids.cpu().numpy(), eos_ids.cpu().numpy()
    waived = 0
    for r in range(R):
        ref = O.verify(tgt_seen[r], drf_seen[r], list(ids_np[r]), O.Policy(**pols[r]), ua_np[r], float(ut_np[r]),
                       eos_ids=(int(eos_np[r]),), output_limit=int(limits[r]))
        want = (ref.status, ref.accepted, ref.output_ids, ref.pending, ref.stop, ref.used_accept, ref.used_target)
        for res in (fast, gen):
            n = int(res.count[r])
            got = (int(res.status[r]), int(res.accepted[r]), tuple(res.ids[r, :n].tolist()),
                   None if int(res.pending[r]) < 0 else int(res.pending[r]),
                   {0: None, 1: "eos", 2: "length"}[int(res.stop[r])], int(res.used_accept[r]),
                   int(res.used_target[r]))
            if got != want:
                assert ref.margin < MARGIN, (r, got, want, ref.margin)
                waived += 1
    assert waived == 0
    assert int(fast.status.abs().sum()) == 0


@pytest.mark.parametrize("V", [5003, 5008])  # unaligned rows (element loads) and 16-byte aligned rows
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_fast_path_non_finite_and_masked_rows(V, dtype):
    """Filter-free requests whose rows hold NaN, +inf, -NaN or only -inf:
    every proposal row and the first target are checked up front, later
    targets only when the chain reaches them (sampling.py:264-272).  The
    kernel's statuses and decisions equal the oracle's on every request."""
    rng = np.random.default_rng(23 + V)
    R, K = 12, 3
    dev = "cuda"
    tgt_np = rng.normal(0, 2, (R, K + 1, V)).astype(np.float32)
    drf_np = (tgt_np[:, :K] + rng.normal(0, 0.5, (R, K, V))).astype(np.float32)
    greedy = np.arange(R) % 2 == 1
    ids_np = rng.integers(0, V, (R, K)).astype(np.int32)
    for r in np.flatnonzero(greedy):
        drf_np[r] = tgt_np[r, :K]
    pos = lambda: int(rng.integers(0, V))
    drf_np[0, 1, pos()] = np.nan              # a proposal row: checked up front
    tgt_np[1, 0, pos()] = np.inf              # the first target
    tgt_np[2, 2, pos()] = np.inf              # a later target, not reached (sampled request, rejected early or not)
    tgt_np[3, 2, pos()] = np.nan              # a later target, reached (greedy)
    drf_np[4, 0, :] = -np.inf                 # a fully masked proposal
    neg_nan = np.array([0xFFC00001], np.uint32).view(np.float32)[0]
    tgt_np[5, 1, pos()] = neg_nan             # -NaN in a reached target (greedy)
    tgt_np[6, 0, :V // 2] = -np.inf           # half masked: still a distribution
    tgt = torch.from_numpy(tgt_np).to(dev).to(dtype)
    drf = torch.from_numpy(drf_np).to(dev).to(dtype)
    tgt_seen, drf_seen = tgt.float().cpu().numpy(), drf.float().cpu().numpy()
    # Greedy requests propose the first argmax of the target rows as the
    # device sees them, so their chains reach every target.
    for r in np.flatnonzero(greedy):
        ids_np[r] = np.nan_to_num(tgt_seen[r, :K], nan=-np.inf).argmax(axis=1)
    pols = [dict(temperature=0.0) if greedy[r] else dict(temperature=1.0) for r in range(R)]
    ua_np, ut_np = rng.random((R, K)), rng.random(R)
    ids = torch.from_numpy(ids_np).to(dev)
    res = batch.verify_drafts(tgt, drf, ids, pols, torch.from_numpy(ua_np).to(dev), torch.from_numpy(ut_np).to(dev),
                              torch.full((R,), 10, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert res.args.hints == N.HINT_VERIFY_FAST
    for r in range(R):
        ref = O.verify(tgt_seen[r], drf_seen[r], list(ids_np[r]), O.Policy(**pols[r]), ua_np[r], float(ut_np[r]),
                       output_limit=10)
        assert int(res.status[r]) == ref.status, (r, int(res.status[r]), ref.status)
        if ref.status == 0:
            n = int(res.count[r])
            got = (int(res.accepted[r]), tuple(res.ids[r, :n].tolist()), int(res.used_accept[r]), int(res.used_target[r]))
            assert got == (ref.accepted, ref.output_ids, ref.used_accept, ref.used_target), (r, got, ref)
    st = res.status.cpu().numpy()
    assert st[0] == N.E_LOGITS and st[1] == N.E_LOGITS and st[3] == N.E_LOGITS and st[5] == N.E_LOGITS
    assert st[4] == N.E_MASKED and st[6] == 0


def test_verify_hint_broken_by_a_filter_is_reported():
    """DSR_HINT_VERIFY_FAST forced on requests that carry filters: the
    general-path launch is left out, so those requests get DSR_E_HINT and
    consume no draws, and every filter-free request decides as without the
    hint."""
    rng = np.random.default_rng(12)
    R, K, V = 8, 3, 5003
    dev = "cuda"
    tgt = torch.from_numpy(rng.normal(0, 2, (R, K + 1, V)).astype(np.float32)).to(dev)
    drf = (tgt[:, :K] + torch.from_numpy(rng.normal(0, 0.5, (R, K, V)).astype(np.float32)).to(dev)).contiguous()
    pols = [[dict(), dict(top_k=50), dict(top_p=0.9, temperature=0.8), dict(min_p=0.02)][r % 4] for r in range(R)]
    draw = batch.sample_rows(drf.reshape(R * K, V).contiguous(), [dict(top_k=50)] * (R * K),
                             uniforms=torch.from_numpy(rng.random(R * K)).to(dev))
    ids = draw.tokens.reshape(R, K).contiguous()
    ua, ut = torch.from_numpy(rng.random((R, K))).to(dev), torch.from_numpy(rng.random(R)).to(dev)
    lim = torch.full((R,), 10, dtype=torch.int32, device=dev)
    plain = batch.verify_drafts(tgt, drf, ids, pols, ua, ut, lim)
    forced = batch.verify_drafts(tgt, drf, ids, pols, ua, ut, lim, hints=N.HINT_VERIFY_FAST)
    torch.cuda.synchronize()
    assert plain.args.hints == 0
    fast = torch.arange(R, device=dev) % 4 == 0
    for k in ("status", "accepted", "ids", "count", "pending", "stop", "used_accept", "used_target", "flags"):
        assert torch.equal(getattr(plain, k)[fast], getattr(forced, k)[fast]), k
    assert (plain.status[fast] == 0).all() and (plain.status[1::4] == 0).all()
    assert (forced.status[~fast] == N.E_HINT).all()
    assert (forced.used_accept[~fast] == 0).all() and (forced.used_target[~fast] == 0).all()
    assert (forced.ids[~fast] == -1).all() and (forced.count[~fast] == 0).all()


@pytest.mark.parametrize("case", META["verify"], ids=lambda c: c["name"])
def test_verify_golden_on_gpu(case):
    dev = "cuda"
    tgt = torch.from_numpy(GOLD[f"{case['name']}/target"]).to(dev)[None]
    drf = torch.from_numpy(GOLD[f"{case['name']}/draft"]).to(dev)[None]
    ids = torch.tensor([case["ids"]], dtype=torch.int32, device=dev)
    eos = case["eos"]
    f64 = torch.float64
    res = batch.verify_drafts(tgt, drf, ids, [case["policy"]], torch.tensor([case["u_accept"]], dtype=f64, device=dev),
                              torch.tensor([case["u_target"]], dtype=f64, device=dev),
                              torch.tensor([case["limit"]], dtype=torch.int32, device=dev),
                              eos_offsets=torch.tensor([0, len(eos)], dtype=torch.int64, device=dev),
                              eos_ids=torch.tensor(eos, dtype=torch.int32, device=dev))
    assert int(res.status.item()) == 0
    n = int(res.count.item())
    stop = {0: None, 1: "eos", 2: "length"}[int(res.stop.item())]
    pending = int(res.pending.item())
    assert (int(res.accepted.item()), res.ids[0, :n].tolist(), None if pending < 0 else pending, stop) == (
        case["accepted"], case["output_ids"], case["pending"], case["stop"])
    assert int(res.used_accept.item()) == case["calls"].count("accept")
    assert int(res.used_target.item()) == case["calls"].count("target")
