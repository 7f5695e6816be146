"""Vocabulary projection with the verifier's row statistics in its epilogue
(dsr_vocab_head, dsr_verify_drafts_head).

The terminal stage computes logits = lm_head(norm(hidden)) in FP32, checks
torch.isfinite(logits).all() and verifies the drafts against those rows
(stage_graph.py:356-362 and :396, terminal_sampling.py:170-183).  Here:

- the logits equal the oracle's float64 product of the same bf16 inputs
  (oracle/head_oracle.py ``project``), and torch's FP32 matmul on the GPU,
  within the FP32 accumulation bound (dim / 16 + 16) * 2^-24 * sum_k |x_k w_k|:
  the kernel adds dim / 16 matrix core partial sums of 16 exact bf16 products
  into one FP32 accumulator;
- every (row, 128-column tile) record equals the oracle's ``records`` of the
  kernel's own logits: the maximum and the first column holding it bit for
  bit, the NaN / +inf / finite / -inf flags exactly, the exp sum within 1e-12
  relative;
- verifier decisions read from the records equal, field for field, those of
  the verifier that reads the logits, and the oracle's on the same FP32 rows
  (a decision may differ only where the oracle's own margin is below 1e-11).
"""
import ctypes

import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch
from oracle import head_oracle as H
from oracle import sampling_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TILE = 128


def bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)


def head_inputs(seed, rows, dim, vocab, scale=2.0):
    rng = np.random.default_rng(seed)
    x = bf16(rng.normal(0, 1, (rows, dim)))
    w = bf16(rng.normal(0, scale / np.sqrt(dim), (vocab, dim)))
    return x, w


def check_logits(x, w, got, cols=None):
    """``got`` [rows, vocab] (host float32) against the oracle's float64
    product, on the columns ``cols`` (all when None)."""
    want, scale = H.project(x.float().numpy(), (w if cols is None else w[cols]).float().numpy())
    g = got.astype(np.float64) if cols is None else got[:, cols].astype(np.float64)
    tol = (x.shape[1] // 16 + 16) * 2.0 ** -24 * scale + 1e-30
    err = np.abs(g - want)
    assert np.all(err <= tol), float(np.max(err / tol))


@pytest.mark.parametrize("rows,dim,vocab", [(1, 256, 128), (5, 256, 512), (32, 512, 2560), (33, 768, 1024),
                                            (100, 256, 896), (160, 1024, 1280), (200, 256, 4096), (256, 256, 2048)])
def test_logits_match_the_float64_product(rows, dim, vocab):
    x, w = head_inputs(rows * 7 + dim, rows, dim, vocab)
    for records in (False, True):
        res = batch.vocab_head(x.to(DEV), w.to(DEV), records=records)
        check_logits(x, w, res.logits.cpu().numpy())
    # torch's FP32 product of the same inputs on the GPU, within the same bound.
    ref = (x.to(DEV).float() @ w.to(DEV).float().T).cpu().double().numpy()
    scale = np.abs(x.double().numpy()) @ np.abs(w.double().numpy()).T
    assert np.all(np.abs(res.logits.cpu().double().numpy() - ref) <= 2 * (dim // 16 + 16) * 2.0 ** -24 * scale + 1e-30)


def device_weight(seed, vocab, dim):
    """bf16 weight q * 2^-10 with q uniform on [-64, 63], drawn on the device."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    q = torch.randint(-64, 64, (vocab, dim), generator=g, device=DEV, dtype=torch.int32)
    return (q.to(torch.bfloat16) * 2.0 ** -10).contiguous()


def test_full_vocabulary_logits_at_the_terminal_stage_width():
    """160 rows x dim 5,120 x vocab 129,280 (the terminal stage's lm_head,
    stage_graph.py:180-182), compared on 4,096 columns spread over the row."""
    x = bf16(np.random.default_rng(5).normal(0, 1, (160, 5120)))
    xd, wd = x.to(DEV), device_weight(5, 129280, 5120)
    res = batch.vocab_head(xd, wd, policies=[dict(temperature=1.0)] * 32, rows_per_policy=5)
    got = res.logits.cpu().numpy()
    cols = np.sort(np.random.default_rng(6).choice(129280, 4096, replace=False))
    check_logits(x, wd[torch.from_numpy(cols).to(DEV)].cpu(), got[:, cols])
    assert bool(res.finite_rows().all())
    plain = batch.vocab_head(xd, wd, records=False)
    assert torch.equal(plain.logits, res.logits)  # the epilogue changes no logit


def record_reference(logits, temps):
    """The oracle's records as the kernel stores them: (sum, max, info)."""
    sums, mx, first, flags = H.records(logits, temps, tile=TILE)
    info = (flags | (np.where(first >= 0, first, 0xFFFFFF) << 8)).astype(np.uint32).view(np.int32)
    return sums, mx, info


@pytest.mark.parametrize("rows,dim,vocab", [(7, 256, 1024), (40, 512, 2048), (200, 256, 1024)])
def test_records_equal_the_float64_statistics_of_the_logits(rows, dim, vocab):
    x, w = head_inputs(rows + 3 * dim, rows, dim, vocab)
    xn, wn = x.float().numpy(), w.float().numpy()
    xn[1, 0] = np.inf                 # row 1: +inf and -inf logits (the sign of w[:, 0])
    xn[2, 3] = np.nan                 # row 2: every logit NaN
    xn[3] = 0.0                       # row 3: every logit 0: maximum at each tile's column 0, sum 128
    wn[5] = wn[7] = 8.0 * np.sign(xn[4])  # row 4: the same maximum at columns 5 and 7
    wn[5, 0] = wn[7, 0] = 0.0         # (row 1's columns 5 and 7: inf * 0, NaN)
    x, w = bf16(xn), bf16(wn)
    temps = [1.0, 0.7, 0.0, 2.5, 1e-3, 100.0]
    pols = [dict(temperature=temps[i % len(temps)]) for i in range(-(-rows // 2))]
    res = batch.vocab_head(x.to(DEV), w.to(DEV), policies=pols, rows_per_policy=2)
    logits = res.logits.cpu().numpy()
    row_t = [pols[r // 2]["temperature"] for r in range(rows)]
    sums, mx, info = record_reference(logits, row_t)
    assert np.array_equal(res.part_max.cpu().numpy().view(np.uint32), mx.view(np.uint32))
    assert np.array_equal(res.part_info.cpu().numpy(), info)
    got = res.part_sum.cpu().numpy()
    np.testing.assert_allclose(got, sums, rtol=1e-12, atol=0)
    assert (info[3, 0] >> 8) & 0xFFFFFF == 0 and got[3, 0] == float(TILE) * (row_t[3] > 0)
    assert (info[4, 0] >> 8) & 0xFFFFFF == 5 and (info[2, 0] >> 8) & 0xFFFFFF == 0xFFFFFF
    finite = res.finite_rows().cpu().numpy()
    assert np.array_equal(finite, np.isfinite(logits).all(axis=1))
    assert not finite[1] and not finite[2]


def verify_case(seed, dim=256, R=32, K=4, V=129280, poison=None):
    """C4-shaped requests whose target and draft rows come from one head."""
    rng = np.random.default_rng(seed)
    w = device_weight(seed, V, dim) * (2.0 / np.sqrt(dim) / 0.036)
    xt_np = rng.normal(0, 1, (R * (K + 1), dim)).astype(np.float32)
    xd_np = xt_np.reshape(R, K + 1, dim)[:, :K].reshape(R * K, dim) + rng.normal(0, 0.35, (R * K, dim))
    if poison is not None:
        xt_np[poison] = np.nan
    xt, xd = bf16(xt_np).to(DEV), bf16(xd_np).to(DEV)
    temps = [1.0, 0.7, 1.3, 0.0]
    pols = [dict(temperature=temps[r % 4]) for r in range(R)]
    pols[5] = dict(temperature=0.8, top_k=50)   # a filtered request: the full-distribution path
    pt = batch.policy_tensor(pols, DEV)
    th = batch.vocab_head(xt, w, policies=pt, rows_per_policy=K + 1)
    dh = batch.vocab_head(xd, w, policies=pt, rows_per_policy=K)
    tgt, drf = th.logits.view(R, K + 1, V), dh.logits.view(R, K, V)
    draw = batch.sample_rows(dh.logits, [pols[r // K] for r in range(R * K)],
                             uniforms=torch.from_numpy(rng.random(R * K)).to(DEV))
    ids = draw.tokens.reshape(R, K).contiguous()
    greedy = torch.tensor([p["temperature"] == 0 for p in pols], device=DEV)
    ids[greedy] = drf.argmax(dim=-1).to(torch.int32)[greedy]
    ua_np, ut_np = rng.random((R, K)), rng.random(R)
    ua, ut = torch.from_numpy(ua_np).to(DEV), torch.from_numpy(ut_np).to(DEV)
    lim = torch.from_numpy(np.array([10, 2, 3, 10] * (R // 4), np.int32)).to(DEV)
    eos_ids = ids[:, 1].contiguous()
    eos_off = torch.arange(0, R + 1, dtype=torch.int64, device=DEV)
    kw = dict(eos_offsets=eos_off, eos_ids=eos_ids)
    by_logits = batch.verify_drafts(tgt, drf, ids, pt, ua, ut, lim, **kw)
    by_head = batch.verify_drafts(tgt, drf, ids, pt, ua, ut, lim, head=(th, dh), **kw)
    return dict(pols=pols, tgt=tgt, drf=drf, ids=ids, ua=ua_np, ut=ut_np, lim=lim, eos=eos_ids,
                a=by_logits, b=by_head, th=th)


FIELDS = ("accepted", "ids", "count", "pending", "stop", "used_accept", "used_target", "status", "flags")


def test_verify_from_head_records_equals_the_logits_path_and_the_oracle():
    c = verify_case(21)
    a, b = c["a"], c["b"]
    for f in FIELDS:
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    tgt, drf = c["tgt"].cpu().numpy(), c["drf"].cpu().numpy()
    ids, lim, eos = c["ids"].cpu().numpy(), c["lim"].cpu().numpy(), c["eos"].cpu().numpy()
    R = tgt.shape[0]
    waived = 0
    for r in range(R):
        p = c["pols"][r]
        ref = O.verify(tgt[r], drf[r], list(ids[r]), O.Policy(**p), c["ua"][r], float(c["ut"][r]),
                       output_limit=int(lim[r]), eos_ids=(int(eos[r]),))
        got = (int(b.status[r]), int(b.accepted[r]), tuple(int(t) for t in b.ids[r, :int(b.count[r])].tolist()),
               None if int(b.pending[r]) < 0 else int(b.pending[r]), int(b.used_accept[r]), int(b.used_target[r]))
        want = (ref.status, ref.accepted, ref.output_ids, ref.pending, ref.used_accept, ref.used_target)
        if got != want:
            assert ref.margin < 1e-11, (r, got, want, ref.margin)
            waived += 1
    assert waived == 0


def test_a_non_finite_head_row_is_reported_the_same_way():
    """Request 3's target row 1 is NaN: both verifiers report it (or not, when
    the chain ends first) exactly as the oracle does."""
    K = 4
    c = verify_case(22, R=8, poison=3 * (K + 1) + 1)
    a, b = c["a"], c["b"]
    for f in FIELDS:
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    tgt, drf = c["tgt"].cpu().numpy(), c["drf"].cpu().numpy()
    ids, lim, eos = c["ids"].cpu().numpy(), c["lim"].cpu().numpy(), c["eos"].cpu().numpy()
    ref = O.verify(tgt[3], drf[3], list(ids[3]), O.Policy(**c["pols"][3]), c["ua"][3], float(c["ut"][3]),
                   output_limit=int(lim[3]), eos_ids=(int(eos[3]),))
    assert int(b.status[3]) == ref.status
    finite = c["th"].finite_rows().cpu().numpy()
    assert not finite[3 * (K + 1) + 1] and finite.sum() == finite.size - 1


def test_head_arguments_are_checked_before_any_launch():
    x, w = head_inputs(1, 4, 256, 512)
    xd, wd = x.to(DEV), w.to(DEV)
    with pytest.raises(ValueError):
        batch.vocab_head(torch.zeros(257, 256, dtype=torch.bfloat16, device=DEV), wd)
    with pytest.raises(ValueError):
        batch.vocab_head(xd[:, :192].contiguous(), wd[:, :192].contiguous())
    with pytest.raises(ValueError):
        batch.vocab_head(xd, wd[:500].contiguous())
    lib = N.load()
    out = torch.empty(4, 512, dtype=torch.float32, device=DEV)
    a = N.HeadArgs()
    a.hidden, a.weight, a.logits = xd.data_ptr() + 2, wd.data_ptr(), out.data_ptr()  # misaligned hidden
    a.rows, a.dim, a.vocab = 4, 256, 512
    assert lib.dsr_vocab_head(ctypes.byref(a), None) == -1
    a.hidden, a.dim = xd.data_ptr(), 320
    assert lib.dsr_vocab_head(ctypes.byref(a), None) == -1
    a.dim, a.reserved = 256, 1
    assert lib.dsr_vocab_head(ctypes.byref(a), None) == -1
    a.reserved = 0
    assert lib.dsr_vocab_head(ctypes.byref(a), None) == 0   # the same call, valid
    torch.cuda.synchronize()
    check_logits(x, w, out.cpu().numpy())


def test_policy_tensors_off_the_device_are_refused():
    """A policy tensor the kernels cannot read (host memory, another dtype,
    a strided view) is refused before any launch, by every entry that takes one."""
    x, w = head_inputs(1, 4, 256, 512)
    xd, wd = x.to(DEV), w.to(DEV)
    pols = [dict(temperature=1.0)] * 4
    host = batch.policy_tensor(pols, "cpu")
    dev = batch.policy_tensor(pols, DEV)
    for bad in (host, dev.to(torch.int32), dev.view(4, -1)[:, ::2]):
        with pytest.raises(ValueError):
            batch.vocab_head(xd, wd, policies=bad)
        with pytest.raises(ValueError):
            batch.sample_rows(torch.zeros(4, 512, dtype=torch.float32, device=DEV), bad,
                              uniforms=torch.full((4,), 0.5, dtype=torch.float64, device=DEV))
    one = batch.policy_tensor([dict(temperature=1.0)] * 2, DEV)
    with pytest.raises(ValueError):   # two policies for four rows
        batch.sample_rows(torch.zeros(4, 512, dtype=torch.float32, device=DEV), one,
                          uniforms=torch.full((4,), 0.5, dtype=torch.float64, device=DEV))


def _sample_pair(logits, pols, u, parts, **kw):
    """The same rows sampled with and without the projection's records."""
    pt = batch.policy_tensor(pols, DEV)
    ud = torch.from_numpy(np.asarray(u, np.float64)).to(DEV)
    a = batch.sample_rows(logits, pt, uniforms=ud, head_parts=parts, probs="f64", kept=True, **kw)
    b = batch.sample_rows(logits, pt, uniforms=ud, probs="f64", kept=True, **kw)
    torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("rows,dim,vocab", [(6, 256, 129280), (16, 512, 8192), (3, 256, 1024)])
def test_top_k_rows_from_the_records_match_the_plain_path_and_the_oracle(rows, dim, vocab):
    """dsr_sample_rows_head: FP32 top-k rows start from the projection's
    per-tile maxima.  Tokens, consumption, statuses, flags, kept bits and
    float64 probabilities equal those of dsr_sample_rows on the same logits
    bit for bit, and the oracle's on the host copy of the logits; rows whose
    k exceeds the finite tiles or whose candidate tiles are too many take
    the full pass in the same launch."""
    x, w = head_inputs(71 + rows, rows, dim, vocab, scale=3.0)
    res = batch.vocab_head(x.to(DEV), w.to(DEV))
    logits = res.logits
    host = logits.cpu().numpy()
    rng = np.random.default_rng(5000 + vocab)
    ks = [1, 3, 50, 200, 1000, 1024]
    pols = []
    for r in range(rows):
        k = min(ks[r % len(ks)], vocab - 1)
        pols.append(dict(temperature=[0.6, 1.0, 1.7][r % 3], top_k=k, top_p=[1.0, 0.9, 0.5][r % 3],
                         min_p=0.02 if r % 4 == 3 else 0.0))
    pols[0] = dict(temperature=0.0, top_k=5)
    u = rng.random(rows)
    a, b = _sample_pair(logits, pols, u, res.parts)
    for f in ("tokens", "consumed", "status", "flags", "kept_bits"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    assert torch.equal(a.probs, b.probs)
    # A top-k near the count of a small vocabulary's quad pairs may overflow
    # the candidate lists and hand the row over, with or without records;
    # smaller ones stay on the FP32 kernel.
    fits = np.array([p["temperature"] == 0.0 or p["top_k"] <= vocab // 16 for p in pols])
    assert ((a.flags.cpu().numpy() & N.FLAG_F32_TOPK) != 0)[fits].all()
    tok = a.tokens.cpu().numpy()
    for r in range(rows):
        ref = O.sample_row(host[r], O.Policy(**pols[r]), float(u[r]))
        assert int(tok[r]) == ref.token, r
        np.testing.assert_allclose(a.probs[r].cpu().numpy(), ref.probs, rtol=1e-5, atol=1e-300)


def test_records_with_masks_infinities_or_other_paths_change_nothing():
    """A masked batch ignores the records; rows with -inf logits and rows
    whose every value is -inf take the records' route or hand over as the
    plain path does; device draws advance the same states."""
    rows, dim, vocab = 4, 256, 4096
    x, w = head_inputs(93, rows, dim, vocab)
    res = batch.vocab_head(x.to(DEV), w.to(DEV))
    logits = res.logits.clone()
    logits[1, 100:300] = -float("inf")
    logits[2, :] = -float("inf")
    # The edited rows' records (maximum, first column holding it, flags),
    # as dsr_vocab_head writes them, from the edited logits.
    host = logits.cpu().numpy()
    p = res.parts.cpu().numpy().reshape(rows, vocab // TILE, 4).copy()
    for r in (1, 2):
        t = host[r].reshape(-1, TILE)
        for tl in range(t.shape[0]):
            mx = t[tl].max()
            fin = np.isfinite(t[tl]).any()
            col = int(np.flatnonzero(t[tl] == mx)[0]) if fin else 0xFFFFFF
            flags = (2 if fin else 0) | (4 if np.isneginf(t[tl]).any() else 0)
            p[r, tl, 2] = np.array([mx], np.float32).view(np.int32)[0]
            p[r, tl, 3] = np.array([flags | (col << 8)], np.uint32).view(np.int32)[0]
    parts = torch.from_numpy(p).to(DEV)
    pols = [dict(temperature=0.8, top_k=20, top_p=0.9)] * rows
    u = np.random.default_rng(3).random(rows)
    a, b = _sample_pair(logits, pols, u, parts)
    for f in ("tokens", "consumed", "status", "flags", "kept_bits"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    assert torch.equal(a.probs, b.probs)
    allow = torch.from_numpy(batch.pack_allow(np.random.default_rng(4).random((rows, vocab)) < 0.7).view(np.int32)).to(DEV)
    a, b = _sample_pair(logits, pols, u, parts, allow_bits=allow)
    for f in ("tokens", "consumed", "status", "flags"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    gens = [np.random.default_rng(40 + r) for r in range(rows)]
    s1, s2 = batch.pcg64_states(gens, DEV), batch.pcg64_states(gens, DEV)
    pt = batch.policy_tensor(pols, DEV)
    r1 = batch.sample_rows(logits, pt, rng_state=s1, head_parts=parts)
    r2 = batch.sample_rows(logits, pt, rng_state=s2)
    torch.cuda.synchronize()
    assert torch.equal(r1.tokens, r2.tokens) and torch.equal(s1, s2)
