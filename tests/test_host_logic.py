"""Host-side logic of the drop-in API (no GPU): RNG domains and transactions,
policy validation, canonical JSON, bit packing and the sparse history tables."""
from copy import deepcopy
import json
import os

import numpy as np
import pytest

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch, jsonutil, workloads
from deepseekrpc_amd.jsonutil import ValidationError
from deepseekrpc_amd.sampling import DOMAINS, RandomStreams, SamplingPolicy

HERE = os.path.dirname(os.path.abspath(__file__))
META = json.load(open(os.path.join(HERE, "golden", "sampling_golden.json")))


@pytest.mark.parametrize("case", META["rng"], ids=lambda c: str(c["seed"]))
def test_random_streams_match_reference_draws(case):
    # Absolute PCG64 draws and snapshots recorded from the reference (sampling.py:166-231).
    streams = RandomStreams(case["seed"])
    assert streams.snapshot() == case["snapshot"]
    txn = streams.begin()
    assert {d: [txn.random(d) for _ in range(8)] for d in DOMAINS} == case["draws"]
    assert txn.commit() == case["after"]


def test_rejection_keeps_draft_draws_and_abort_restores():
    # tests/test_sampling.py:110-131 (RNG part)
    streams = RandomStreams(42)
    before = streams.snapshot()
    txn = streams.begin()
    for _ in range(5):
        txn.random("draft")
    state = txn.prepared_state()["domains"]["draft"]
    txn.commit()
    assert streams.snapshot()["domains"]["draft"] == state and streams.snapshot() != before
    committed = streams.snapshot()
    txn = streams.begin()
    for d in DOMAINS:
        txn.random(d)
    with pytest.raises(ValidationError, match="idle"):
        streams.snapshot()
    txn.abort()
    assert streams.snapshot() == committed


def test_snapshot_restore_is_atomic():
    # tests/test_sampling.py:133-146
    first, restored = RandomStreams(9), RandomStreams(0)
    saved = first.snapshot()
    bad = deepcopy(saved)
    bad["domains"]["accept"]["increment"] = "0" * 32
    before = restored.snapshot()
    with pytest.raises(ValidationError, match="odd"):
        restored.restore(bad)
    assert restored.snapshot() == before
    restored.restore(saved)
    a, b = first.begin(), restored.begin()
    for d in ("draft", "accept", "target"):
        assert [a.random(d) for _ in range(5)] == [b.random(d) for _ in range(5)]
    assert a.commit() == b.commit()


def test_transaction_window_is_bounded():
    txn = RandomStreams(1).begin()
    for _ in range(64):
        txn.random("target")
    with pytest.raises(ValidationError):
        txn.random("target")
    with pytest.raises(ValidationError):
        txn.random("other")


def test_policy_bounds_and_types():
    SamplingPolicy(temperature=0, top_p=0, top_k=129280, min_p=1, repetition_penalty=0.01,
                   presence_penalty=-2, frequency_penalty=2)
    for kw in (dict(temperature=True), dict(temperature=100.5), dict(top_p=1.5), dict(top_k=-1), dict(top_k=1.0),
               dict(repetition_penalty=0.0), dict(min_p=float("nan")), dict(presence_penalty=3)):
        with pytest.raises(ValidationError):
            SamplingPolicy(**kw)
    assert SamplingPolicy(top_k=3).as_dict()["top_k"] == 3


def test_jsonutil():
    assert jsonutil.canonical({"b": 1, "a": [1.5, None]}) == b'{"a":[1.5,null],"b":1}'
    with pytest.raises(ValueError):
        jsonutil.canonical({"x": float("nan")})
    with pytest.raises(ValidationError):
        jsonutil.integer(True, "x", 0, 5)
    with pytest.raises(ValidationError):
        jsonutil.hex_id("ABC", 3, "x")
    assert jsonutil.hex_id("0a9f", 4, "x") == "0a9f"


def test_allow_bit_packing_round_trip():
    rng = np.random.default_rng(0)
    for V in (1, 31, 32, 33, 129280):
        a = rng.random((3, V)) < 0.5
        words = batch.pack_allow(a)
        assert words.shape == (3, (V + 31) // 32) and words.dtype == np.uint32
        np.testing.assert_array_equal(batch.unpack_bits(words, V), a)
        i = int(rng.integers(0, V))
        assert bool((words[1, i >> 5] >> (i & 31)) & 1) == a[1, i]


def test_history_table_from_token_lists_and_dense():
    h = [np.array([5, 3, 5, 9, 3, 5]), np.array([], np.int64), np.array([1, 1])]
    t = batch.HistoryTable.from_token_lists(h, generated_start=[2, 0, 1], device="cpu")
    assert t.offsets.tolist() == [0, 3, 3, 4]
    assert t.ids.tolist() == [3, 5, 9, 1]
    assert t.counts.tolist() == [2, 3, 1, 2]
    assert t.generated.tolist() == [1, 2, 1, 1]
    dense = np.zeros((2, 10), np.int32)
    dense[0, [2, 7]] = [4, 1]
    gen = np.zeros_like(dense)
    gen[0, 2] = 3
    d = batch.HistoryTable.from_dense(dense, gen, device="cpu")
    assert d.offsets.tolist() == [0, 2, 2] and d.ids.tolist() == [2, 7]
    assert d.counts.tolist() == [4, 1] and d.generated.tolist() == [3, 0]


def test_policy_packing_layout():
    arr = batch.policy_array([dict(temperature=0.5, top_k=7), SamplingPolicy(top_p=0.25)])
    assert arr.dtype.itemsize == 56
    assert arr[0]["temperature"] == 0.5 and arr[0]["top_k"] == 7 and arr[0]["top_p"] == 1.0
    assert arr[1]["top_p"] == 0.25 and arr[1]["repetition_penalty"] == 1.0


def _mixed_policies(rows=96):
    wp, cp = workloads.whole().policies, workloads.c3().policies
    return [wp[r] if r % 3 == 0 else cp[r] for r in range(rows)]


def test_hints_follow_the_policies():
    arr = batch.policy_array(workloads.whole().policies)
    assert batch.sample_hints(arr, 129280) == N.HINT_WHOLE_SOME | N.HINT_WHOLE_ALL
    # Every C3 row has 1 <= top_k <= 1024: the FP32 top-k kernel's hint.
    assert batch.sample_hints(batch.policy_array(workloads.c3().policies), 129280) == N.HINT_TOPK_ALL
    assert batch.sample_hints(batch.policy_array(_mixed_policies()), 129280) == N.HINT_WHOLE_SOME
    # Greedy rows and rows with a top-k the register kernel takes are not whole.
    arr = batch.policy_array([dict(temperature=0.0), dict(top_k=1024), dict(top_k=1025), dict(top_k=8, top_p=0.5)])
    assert batch.sample_hints(arr, 129280) == N.HINT_WHOLE_SOME
    assert batch.sample_hints(batch.policy_array([dict(top_k=8)]), 8) == N.HINT_WHOLE_ALL | N.HINT_WHOLE_SOME
    # TOPK_ALL needs every row greedy or with 1 <= top_k <= 1024 below V, and in bounds.
    assert batch.sample_hints(batch.policy_array([dict(temperature=0.0), dict(top_k=1024)]), 129280) == \
        N.HINT_TOPK_ALL
    assert batch.sample_hints(batch.policy_array([dict(top_k=50, temperature=101.0)]), 129280) & N.HINT_TOPK_ALL == 0


def test_verify_hint_needs_filter_free_policies_and_plain_inputs():
    arr = batch.policy_array([dict(), dict(temperature=0.5), dict(top_k=129280)])
    assert batch.verify_hints(arr, 129280, True) == N.HINT_VERIFY_FAST
    assert batch.verify_hints(arr, 129280, False) == 0
    for bad in (dict(top_k=50), dict(top_p=0.9), dict(min_p=0.1)):
        assert batch.verify_hints(batch.policy_array([dict(), bad]), 129280, True) == 0


def _frozen(v):
    from deepseekrpc_amd import terminal_sampling as T
    support = np.flatnonzero(v > 0)
    return T._Counts(support, v[support], v.size, v.dtype)


def _hash_in_child(q):
    from deepseekrpc_amd import terminal_sampling as T
    c = _frozen(np.arange(5, dtype=np.int64))
    q.put(T._hash_worker().submit(T._count_hashes, c, c).result(timeout=20)[0])


def test_count_hash_worker_runs_in_a_forked_child():
    """The digest's hash worker is per process: a child forked after the
    parent used it still gets its hashes."""
    import multiprocessing as mp
    from deepseekrpc_amd import terminal_sampling as T
    v = np.arange(5, dtype=np.int64)
    c = _frozen(v)
    want = T._hash_worker().submit(T._count_hashes, c, c).result(timeout=20)[0]
    ctx = mp.get_context("fork")
    q = ctx.Queue()
    p = ctx.Process(target=_hash_in_child, args=(q,))
    p.start()
    got = q.get(timeout=30)
    p.join(timeout=30)
    assert p.exitcode == 0 and got == want == T._sha256_i8(v)
    assert np.array_equal(c.dense(), v) and not c.dense().flags.writeable and c.at(3) == 3 and c.at(0) == 0
