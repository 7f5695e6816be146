"""The allocation-free entry point against dsr_sample_rows.

dsr_sample_rows_noalloc runs the same kernels with the library's own device
array as the workspace.  Two calls in a row (the second smaller, so the array
holds the first call's leftovers) must give exactly the outputs of
dsr_sample_rows on the same inputs, for rows that use the workspace: the
general path (fp32 rows with a top-k above 1,024), the split path (fp32 rows
with top-k 50), the full-vocabulary path (bf16 rows with histories) and the
register path (C3 rows).  Calls beyond the array's size are refused.
"""
import ctypes

import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch, workloads

pytestmark = pytest.mark.gpu
V = workloads.VOCAB
DEV = "cuda"


def outputs(res):
    torch.cuda.synchronize()
    out = {k: getattr(res, k).cpu().numpy() for k in ("tokens", "consumed", "status", "flags")}
    if res.probs is not None:
        out["probs"] = res.probs.cpu().numpy()
    if res.kept_bits is not None:
        out["kept"] = res.kept_bits.cpu().numpy()
    return out


def same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)


def fp32_rows(rows, seed, top_k):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.normal(0, 2, (rows, V)).astype(np.float32)).to(DEV)
    pols = [dict(temperature=float(rng.uniform(0.3, 1.5)), top_k=top_k, top_p=float(rng.uniform(0.6, 1.0)))
            for _ in range(rows)]
    u = torch.from_numpy(rng.random(rows)).to(DEV)
    return x, pols, u


@pytest.mark.parametrize("top_k,first,second", [(2000, 48, 5), (50, 16, 3)])
def test_two_calls_match_the_workspace_entry_point(top_k, first, second):
    for rows, seed in ((first, 1), (second, 2)):
        x, pols, u = fp32_rows(rows, seed + top_k, top_k)
        want = outputs(batch.sample_rows(x, pols, uniforms=u, probs="f64", kept=True))
        got = outputs(batch.sample_rows(x, pols, uniforms=u, probs="f64", kept=True, noalloc=True))
        same(got, want)
        assert (got["status"] == 0).all()
        path = N.FLAG_GENERAL if top_k > 1024 else N.FLAG_F32_TOPK
        assert (got["flags"] & path).all()


def test_history_and_register_rows():
    for w in (workloads.c2(rows=24), workloads.select_rows(workloads.c2(), list(range(6))),
              workloads.c3(), workloads.c3(rows=9)):
        d = workloads.to_device(w)
        kw = dict(history=d.history, allow_bits=d.allow_bits, uniforms=d.uniforms, probs="f32")
        want = outputs(batch.sample_rows(d.logits, d.policies, **kw))
        got = outputs(batch.sample_rows(d.logits, d.policies, noalloc=True, **kw))
        same(got, want)


def test_calls_beyond_the_array_are_refused():
    lib = N.load()
    assert lib.dsr_sample_workspace_bytes(259, V) <= N.NOALLOC_SCRATCH_BYTES < lib.dsr_sample_workspace_bytes(260, V)
    x, pols, u = fp32_rows(260, 3, 2000)
    with pytest.raises(ValueError, match="allocation-free"):
        batch.sample_rows(x, pols, uniforms=u, noalloc=True)
    # Through the C ABI: too large -> DSR_ERR_WORKSPACE, a caller workspace -> DSR_ERR_ARG; nothing launches.
    res = batch.sample_rows(x[:2], batch.policy_tensor(pols[:2], DEV), uniforms=u[:2])
    a = N.SampleArgs.from_buffer_copy(res.args)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a.rows = 260
    a.workspace, a.workspace_bytes = None, 0
    assert lib.dsr_sample_rows_noalloc(ctypes.byref(a), stream) == -3
    a.rows = 2
    b = N.SampleArgs.from_buffer_copy(res.args)
    assert b.workspace and lib.dsr_sample_rows_noalloc(ctypes.byref(b), stream) == -1
    assert lib.dsr_sample_rows_noalloc(ctypes.byref(a), stream) == 0
    torch.cuda.synchronize()
