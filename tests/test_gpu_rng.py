"""Device PCG64 draws (dsr_sample_rows with rng_state) against host draws.

Sampling with each row's PCG64 state on the device must give the decisions
that sampling with that generator's next host draw gives, on every kernel
path, and must leave each state advanced by exactly the draws the row
consumed (sampling.py:120-125: a single positive token draws nothing)."""
import numpy as np
import pytest
import torch

from deepseekrpc_amd import batch, workloads
from oracle import pcg64_oracle as P

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1


def expected_states(before, consumed):
    words = before.cpu().numpy().view(np.uint64)
    out = words.copy()
    for r, c in enumerate(consumed):
        if c:
            s = int(words[r, 0]) | (int(words[r, 1]) << 64)
            inc = int(words[r, 2]) | (int(words[r, 3]) << 64)
            s, _ = P.random(s, inc)
            out[r, 0], out[r, 1] = s & M64, s >> 64
    return out


def device_vs_host(logits, policies, seed, **kw):
    rows = logits.shape[0]
    gens_dev = [np.random.default_rng(seed + r) for r in range(rows)]
    gens_host = [np.random.default_rng(seed + r) for r in range(rows)]
    states = batch.pcg64_states(gens_dev)
    before = states.clone()
    got = batch.sample_rows(logits, policies, rng_state=states, **kw)
    u = torch.tensor([g.random() for g in gens_host], dtype=torch.float64, device=logits.device)
    want = batch.sample_rows(logits, policies, uniforms=u, **kw)
    for f in ("tokens", "consumed", "status", "flags"):
        assert torch.equal(getattr(got, f), getattr(want, f)), f
    consumed = got.consumed.cpu().numpy()
    np.testing.assert_array_equal(states.cpu().numpy().view(np.uint64), expected_states(before, consumed))
    return got


def test_top_k_kernel_all_rows():
    w = workloads.c3()
    d = workloads.to_device(w)
    got = device_vs_host(d.logits, d.policies, 100, allow_bits=d.allow_bits)
    assert int(got.consumed.sum()) > 200


def test_full_vocabulary_kernel_rows():
    w = workloads.c2(rows=16)
    d = workloads.to_device(w)
    device_vs_host(d.logits, d.policies, 200, history=d.history)


def test_stress_rows_greedy_rows_draw_nothing():
    w = workloads.select_rows(workloads.c5(), list(range(0, 16)) + list(range(512, 528)))
    d = workloads.to_device(w)
    got = device_vs_host(d.logits, d.policies, 300, history=d.history)
    c = got.consumed.cpu().numpy()
    assert (c[0::2] == 0).all() and (c[1::2] == 1).all()  # even rows greedy


def test_general_kernel_and_hand_over_rows():
    # fp32 rows run the general kernel.  In a bf16 batch without histories,
    # the row with no top-k runs the full-vocabulary kernel and the one with
    # top-k 2000 is finished by the general path inside that kernel; the
    # top-k rows run the top-k register kernel.
    rng = np.random.default_rng(7)
    V = 129280
    x32 = torch.from_numpy(rng.normal(0, 2, (4, V)).astype(np.float32)).cuda()
    pols = [dict(temperature=0.7, top_k=50, top_p=0.9), dict(), dict(top_k=1), dict(temperature=0.0)]
    got = device_vs_host(x32, pols, 400)
    assert got.consumed.cpu().tolist() == [1, 1, 0, 0]
    xb = torch.from_numpy(workloads.bf16_bits(workloads.bf16_round(rng.normal(0, 1, (4, V)))).view(np.int16)).cuda()
    got = device_vs_host(xb.view(torch.bfloat16), [dict(), dict(top_k=2000, top_p=0.8), dict(top_k=1), dict(top_k=7)],
                         500)
    assert got.consumed.cpu().tolist() == [1, 1, 0, 1]
    flags = got.flags.cpu().numpy()
    assert not flags[0] & 2 and flags[1] & 2


def test_repeated_launches_continue_the_streams():
    # Three launches on the same states draw the generators' first three values.
    w = workloads.c3(rows=8)
    d = workloads.to_device(w)
    gens = [np.random.default_rng(900 + r) for r in range(8)]
    ref = [np.random.default_rng(900 + r) for r in range(8)]
    states = batch.pcg64_states(gens)
    for _ in range(3):
        got = batch.sample_rows(d.logits, d.policies, allow_bits=d.allow_bits, rng_state=states)
        u = torch.tensor([g.random() if c else 0.5 for g, c in zip(ref, got.consumed.cpu().tolist())],
                         dtype=torch.float64, device="cuda")
        want = batch.sample_rows(d.logits, d.policies, allow_bits=d.allow_bits, uniforms=u)
        assert torch.equal(got.tokens[got.consumed.bool()], want.tokens[got.consumed.bool()])
    batch.pcg64_restore(gens, states)
    assert [g.random() for g in gens] == [g.random() for g in ref]


def verify_device_vs_host(tgt, drf, ids, pols, limit, seed, **kw):
    rows, K = ids.shape
    acc_dev = [np.random.default_rng(seed + 2 * r) for r in range(rows)]
    tgt_dev = [np.random.default_rng(seed + 2 * r + 1) for r in range(rows)]
    acc_host = [np.random.default_rng(seed + 2 * r) for r in range(rows)]
    tgt_host = [np.random.default_rng(seed + 2 * r + 1) for r in range(rows)]
    sa, st = batch.pcg64_states(acc_dev), batch.pcg64_states(tgt_dev)
    sa0, st0 = sa.clone(), st.clone()
    got = batch.verify_drafts(tgt, drf, ids, pols, None, None, limit, rng_accept=sa, rng_target=st, **kw)
    ua = torch.tensor([[g.random() for _ in range(K)] for g in acc_host], dtype=torch.float64, device="cuda")
    ut = torch.tensor([g.random() for g in tgt_host], dtype=torch.float64, device="cuda")
    want = batch.verify_drafts(tgt, drf, ids, pols, ua.reshape(-1), ut, limit, **kw)
    for f in ("accepted", "ids", "count", "pending", "stop", "used_accept", "used_target", "status", "flags"):
        assert torch.equal(getattr(got, f), getattr(want, f)), f
    used_a, used_t = got.used_accept.cpu().numpy(), got.used_target.cpu().numpy()
    np.testing.assert_array_equal(sa.cpu().numpy().view(np.uint64), expected_states_n(sa0, used_a))
    np.testing.assert_array_equal(st.cpu().numpy().view(np.uint64), expected_states_n(st0, used_t))
    return got


def expected_states_n(before, steps):
    words = before.cpu().numpy().view(np.uint64)
    out = words.copy()
    for r, n in enumerate(steps):
        s = int(words[r, 0]) | (int(words[r, 1]) << 64)
        inc = int(words[r, 2]) | (int(words[r, 3]) << 64)
        for _ in range(int(n)):
            s, _ = P.random(s, inc)
        out[r, 0], out[r, 1] = s & M64, s >> 64
    return out


def test_verifier_fast_path_device_draws():
    w = workloads.c4(rows=16)
    e = w.extra
    R, K, V = e["target"].shape[0], e["K"], e["target"].shape[2]
    tgt = torch.from_numpy(e["target"]).cuda()
    drf = torch.from_numpy(e["draft"]).cuda()
    draw = batch.sample_rows(drf.reshape(R * K, V), [dict()] * (R * K),
                             uniforms=torch.from_numpy(e["u_draft"].reshape(-1)).cuda())
    ids = draw.tokens.reshape(R, K).contiguous()
    got = verify_device_vs_host(tgt, drf, ids, [dict()] * R, torch.from_numpy(e["limit"]).cuda(), 700)
    assert int(got.used_accept.sum()) > R and int(got.used_target.sum()) > 0


def test_verifier_general_path_and_greedy_device_draws():
    # Filtered policies take the general verifier; greedy requests draw nothing.
    rng = np.random.default_rng(31)
    R, K, V = 6, 3, 1000
    tgt = torch.from_numpy(rng.normal(0, 2, (R, K + 1, V)).astype(np.float32)).cuda()
    drf = torch.from_numpy(rng.normal(0, 2, (R, K, V)).astype(np.float32)).cuda()
    ids = torch.from_numpy(rng.integers(0, V, (R, K)).astype(np.int32)).cuda()
    pols = [dict(top_k=50), dict(top_p=0.9), dict(temperature=0.0), dict(min_p=0.05), dict(), dict(temperature=0.0)]
    limit = torch.full((R,), 10, dtype=torch.int32, device="cuda")
    got = verify_device_vs_host(tgt, drf, ids, pols, limit, 800)
    for r in (2, 5):
        assert int(got.used_accept[r]) == 0 and int(got.used_target[r]) == 0
