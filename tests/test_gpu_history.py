"""Device history tables (dsr_history_from_dense / dsr_history_append)
against the oracle: offsets, ids, counts, generated counts and statuses must
be bit-exact."""
import ctypes

import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch, workloads
from oracle import history_oracle as H

pytestmark = pytest.mark.gpu

DEV = "cuda"


def host(table, status):
    """(off, ids, count, gen, status) as NumPy from a device table."""
    return (table.offsets.cpu().numpy(), table.ids.cpu().numpy(), table.counts.cpu().numpy(),
            table.generated.cpu().numpy(), status.cpu().numpy())


def assert_same(got, want):
    names = ("offsets", "ids", "counts", "generated", "status")
    for name, g, w in zip(names, got, want):
        np.testing.assert_array_equal(np.asarray(g, np.int64), np.asarray(w, np.int64), err_msg=name)


def dense_case(rng, rows, vocab, density):
    counts = (rng.integers(1, 4, (rows, vocab)) * (rng.random((rows, vocab)) < density)).astype(np.int32)
    gen = (counts - rng.integers(0, 2, (rows, vocab)).clip(0, counts)).astype(np.int32)
    return counts, gen


@pytest.mark.parametrize("vocab", [129280, 1000, 33])
def test_from_dense_matches_oracle(vocab):
    rng = np.random.default_rng(vocab)
    counts, gen = dense_case(rng, 6, vocab, 0.05)
    counts[1, 3] = -1                      # sampling.py:56
    counts[2, :] = 0
    counts[2, 0] = H.MAX_COUNT              # the bound itself
    gen[2, 0] = 7
    gen[3, 1] = counts[3, 1] + 1            # :64
    counts[4, :2] = H.MAX_COUNT // 2 + 1    # :57 total above the bound
    t, st = batch.HistoryTable.from_dense_device(torch.from_numpy(counts).to(DEV), torch.from_numpy(gen).to(DEV))
    assert_same(host(t, st), H.from_dense(counts, gen))
    # Generated counts omitted: every count is generated.
    t, st = batch.HistoryTable.from_dense_device(torch.from_numpy(counts).to(DEV))
    assert_same(host(t, st), H.from_dense(counts))


def test_from_dense_row_stride_and_empty_batch():
    rng = np.random.default_rng(5)
    counts, gen = dense_case(rng, 3, 1000, 0.2)
    wide = np.zeros((3, 1040), np.int32)
    wide_g = np.zeros((3, 1040), np.int32)
    wide[:, :1000], wide_g[:, :1000] = counts, gen
    c = torch.from_numpy(wide).to(DEV)[:, :1000]
    g = torch.from_numpy(wide_g).to(DEV)[:, :1000]
    t, st = batch.HistoryTable.from_dense_device(c, g)
    assert_same(host(t, st), H.from_dense(counts, gen))
    t, st = batch.HistoryTable.from_dense_device(torch.zeros((0, 1000), dtype=torch.int32, device=DEV))
    assert t.offsets.cpu().tolist() == [0] and t.ids.numel() == 0


def device_table(off, ids, cnt, gen):
    return batch.HistoryTable(*(torch.from_numpy(np.asarray(x, dt)).to(DEV) for x, dt in
                                ((off, np.int64), (ids, np.int32), (cnt, np.int32), (gen, np.int32))))


def csr(rows):
    off = np.zeros(len(rows) + 1, np.int64)
    off[1:] = np.cumsum([len(r) for r in rows])
    flat = np.concatenate([np.asarray(r, np.int64) for r in rows]) if off[-1] else np.zeros(0, np.int64)
    return flat, off


@pytest.mark.parametrize("vocab", [129280, 300, 33])
def test_append_matches_oracle(vocab):
    rng = np.random.default_rng(17 + vocab)
    counts, gen = dense_case(rng, 8, vocab, 0.3 if vocab < 1000 else 0.02)
    counts[5] = 0                          # an empty table row
    gen[5] = 0
    base = H.from_dense(counts, gen)
    token_rows = [rng.integers(0, vocab, int(rng.integers(0, 200))).tolist() for _ in range(8)]
    token_rows[0] = []                     # nothing to add
    token_rows[1] = [vocab - 1] * 50 + [0] * 3
    token_rows[2] = list(range(vocab))[:H.MAX_APPEND]
    token_rows[3] = [int(i) for i in base[1][base[0][3]:base[0][4]]]  # only ids the row already holds
    gen_from = np.array([0, 10, -5, 3, 1000, 0, 2, 7], np.int64)
    table = device_table(*base[:4])
    flat, off = csr(token_rows)
    for gf in (None, gen_from):
        t, st = table.append(torch.from_numpy(flat.astype(np.int32)).to(DEV), torch.from_numpy(off).to(DEV),
                             None if gf is None else torch.from_numpy(gf).to(DEV), vocab=vocab)
        assert_same(host(t, st), H.append(*base[:4], token_rows, vocab, gen_from=gf))


def test_append_statuses_and_rejected_rows():
    vocab = 500
    good_ids, good_cnt, good_gen = [3, 7], [2, 1], [1, 0]
    rows = [
        (good_ids, good_cnt, good_gen, [7, 8], H.OK),
        (good_ids, good_cnt, good_gen, [vocab], H.E_HISTORY),        # token beyond the vocabulary
        (good_ids, good_cnt, good_gen, [-1], H.E_HISTORY),           # negative token
        ([7, 3], [1, 1], [0, 0], [1], H.E_HISTORY),                  # ids not increasing
        ([3], [0], [0], [1], H.E_HISTORY),                           # count below one
        ([3], [1], [2], [1], H.E_HISTORY),                           # generated above count
        ([3], [H.MAX_COUNT + 1], [0], [1], H.E_HISTORY),             # count above the bound
        (good_ids, good_cnt, good_gen, [4] * (H.MAX_APPEND + 1), H.E_APPEND),
        (good_ids, good_cnt, good_gen, [4] * H.MAX_APPEND, H.OK),
    ]
    ids, off = csr([r[0] for r in rows])
    cnt, _ = csr([r[1] for r in rows])
    gen, _ = csr([r[2] for r in rows])
    table = device_table(off, ids, cnt, gen)
    token_rows = [r[3] for r in rows]
    flat, toff = csr(token_rows)
    t, st = table.append(torch.from_numpy(flat.astype(np.int32)).to(DEV), torch.from_numpy(toff).to(DEV),
                         vocab=vocab)
    want = H.append(off, ids, cnt, gen, token_rows, vocab)
    assert want[4].tolist() == [r[4] for r in rows]
    assert_same(host(t, st), want)


def test_from_token_lists_device_equals_host_builder_on_stress_histories():
    # 64 rows of the 16,384-token generated histories of the 1,024-row stress
    # batch, plus rows longer than one append call (built in rounds) with a
    # prompt / output split.
    w = workloads.c5(rows=64)
    hist = [np.asarray(h) for h in w.histories]
    rng = np.random.default_rng(9)
    long_rows = [rng.integers(0, batch.VOCAB, n) for n in (16385, 40000, 0)]
    hist += long_rows
    start = [0] * 64 + [100, 20000, 0]
    t, st = batch.HistoryTable.from_token_lists_device(hist, generated_start=start)
    ref = batch.HistoryTable.from_token_lists(hist, generated_start=start, device="cpu")
    got = host(t, st)
    assert (got[4] == 0).all()
    for g, r in zip(got[:4], (ref.offsets, ref.ids, ref.counts, ref.generated)):
        np.testing.assert_array_equal(g, r.numpy())


def test_append_capacity_too_small_writes_nothing():
    lib = N.load()
    tok = torch.tensor([5, 5, 9, 1], dtype=torch.int32, device=DEV)
    toff = torch.tensor([0, 3, 4], dtype=torch.int64, device=DEV)
    off = torch.empty(3, dtype=torch.int64, device=DEV)
    st = torch.empty(2, dtype=torch.int32, device=DEV)
    outs = [torch.full((8,), -7, dtype=torch.int32, device=DEV) for _ in range(3)]
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.dsr_history_append(None, None, None, None, p(tok), p(toff), None, 2, 16, p(off),
                                *(p(o) for o in outs), 2, p(st), stream)
    assert rc == 0
    assert off.cpu().tolist() == [0, 2, 3] and st.cpu().tolist() == [0, 0]
    assert all((o.cpu() == -7).all() for o in outs)  # total 3 > cap 2: no entry written
    rc = lib.dsr_history_append(None, None, None, None, p(tok), p(toff), None, 2, 16, p(off),
                                *(p(o) for o in outs), 3, p(st), stream)
    assert rc == 0
    assert outs[0].cpu().tolist()[:3] == [5, 9, 1] and outs[1].cpu().tolist()[:3] == [2, 1, 1]


def test_device_tables_feed_the_sampler_like_host_tables():
    # The stress rows sampled with a device-built table (as workloads.to_device
    # builds it) and with the host-built one give identical decisions.
    w = workloads.select_rows(workloads.c5(), list(range(0, 32)) + list(range(512, 544)))
    d = workloads.to_device(w)
    host_table = batch.HistoryTable.from_token_lists(w.histories, device=DEV)
    a = batch.sample_rows(d.logits, w.policies, history=host_table, uniforms=d.uniforms)
    b = batch.sample_rows(d.logits, w.policies, history=d.history, uniforms=d.uniforms)
    for f in ("tokens", "consumed", "status", "flags"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f


def test_drop_in_count_validation_order_and_messages():
    from deepseekrpc_amd.jsonutil import ValidationError
    from deepseekrpc_amd.sampling import SamplingPolicy
    pol = SamplingPolicy(repetition_penalty=1.5, presence_penalty=0.5, frequency_penalty=0.25)
    x = np.linspace(-2, 2, 64).astype(np.float32)
    counts = np.zeros(64, np.int32)
    counts[[3, 9]] = [2, 1]
    bad = counts.copy()
    bad[4] = -1
    big = counts.astype(np.int64)
    big[5] = 1 << 40                       # out of range as int64; must stay out of range on the device
    over = counts.copy()
    over[[1, 2]] = H.MAX_COUNT // 2 + 1    # sampling.py:57 total above the bound
    cmsg, gmsg = "sampling frequency counts do not match", "generated token counts must be a subset"
    for c, g, msg in ((bad, None, cmsg), (big, None, cmsg), (over, None, cmsg),
                      (counts, counts + (np.arange(64) == 9), gmsg),
                      (bad, np.zeros(3, np.int32), cmsg),          # counts are validated first
                      (counts, np.zeros(3, np.int32), gmsg),
                      (counts[:10], None, cmsg)):
        with pytest.raises(ValidationError, match=msg):
            pol.probabilities(x, counts=c, generated_counts=g)
    # Device count tensors give the numbers the NumPy ones give.
    a = pol.probabilities(x, counts=counts, generated_counts=np.minimum(counts, 1))
    b = pol.probabilities(x, counts=torch.from_numpy(counts).to(DEV),
                          generated_counts=torch.from_numpy(np.minimum(counts, 1)).to(DEV))
    np.testing.assert_array_equal(a, b)


def test_prefix_distribution_equals_dense_prefix_counts():
    # terminal_sampling.py:127-136: the conditioned distribution uses counts
    # and generated counts with one added per prefix token.  The device path
    # appends the prefix to the transaction's table; the result must be
    # bit-identical to probabilities() on the dense vectors with the prefix
    # added on the host.
    from deepseekrpc_amd.sampling import SamplingPolicy
    from deepseekrpc_amd.terminal_sampling import TerminalSampler
    V = 129280
    rng = np.random.default_rng(12)
    counts = np.zeros(V, np.int32)
    ids = rng.choice(V, 3000, replace=False)
    counts[ids] = rng.integers(1, 4, 3000)
    gen = np.minimum(counts, rng.integers(0, 3, V)).astype(np.int32)
    pol = SamplingPolicy(temperature=0.9, top_p=0.95, repetition_penalty=1.2, presence_penalty=0.4,
                         frequency_penalty=0.2)
    logits = torch.from_numpy(rng.normal(0, 2, V).astype(np.float32)).to(DEV)
    sampler = TerminalSampler(seed=7, vocabulary=V)
    seed = int(ids[2])
    gen[seed] = counts[seed]          # the pending seed is published, generated history
    work = sampler.begin_verification(seed_token=seed, policy=pol, counts=counts, remaining=8, generated_counts=gen)
    for prefix in ([], [int(ids[0])], [5, 5, int(ids[1]), V - 1]):
        got = work.distribution(logits, prefix)
        c, g = counts.copy(), gen.copy()
        for t in prefix:
            c[t] += 1
            g[t] += 1
        want = pol.probabilities(logits, counts=c, generated_counts=g)
        assert torch.equal(got, want), prefix
    work.abort()
