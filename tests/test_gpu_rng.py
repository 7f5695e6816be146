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
    # fp32 rows run the general kernel; bf16 rows with no top-k (or top-k 1)
    # in a batch without histories start in the top-k kernel and are
    # finished by the general path in the same workgroup.
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
    assert (got.flags.cpu().numpy()[:2] & 2).all()  # the first two were finished by the general path


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
