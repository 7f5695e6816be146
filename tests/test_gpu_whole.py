"""bf16 rows whose filters keep the whole vocabulary (no top-k: the
reference's default policy, top-p only, min-p only; sampling.py:28-36,86-106)
on batches without a history.

The host derives DSR_HINT_WHOLE_* from the policies, and such rows then run
the full-vocabulary kernel instead of the general path.  Hints choose
launches only: forcing wrong hints, or none, must give the same outputs.
"""
import numpy as np
import pytest
import torch

from deepseekrpc_amd import _native as N
from deepseekrpc_amd import batch, workloads
from parity_util import compare, run_gpu

pytestmark = pytest.mark.gpu


def check(rep):
    print(f"rows={rep.rows} exact={rep.exact} margin={rep.margin_rows} flagged={rep.flagged}", flush=True)
    assert not rep.mismatches, rep.mismatches[:10]
    assert not rep.margin_rows
    assert rep.exact == rep.rows


def mixed(rows=96):
    """c3's rows with every third policy replaced by one of the whole family's."""
    w = workloads.c3(rows=rows)
    wp = workloads.whole().policies
    w.policies = [dict(wp[r]) if r % 3 == 0 else w.policies[r] for r in range(rows)]
    return w


def run(w, hints):
    d = workloads.to_device(w)
    res = batch.sample_rows(d.logits, d.policies, allow_bits=d.allow_bits, uniforms=d.uniforms, probs="f64",
                            kept=True, hints=hints)
    torch.cuda.synchronize()
    return {k: getattr(res, k).cpu().numpy() for k in ("tokens", "consumed", "status", "flags", "probs", "kept_bits")}


def test_whole_rows_run_the_full_vocabulary_kernel():
    w = workloads.whole()
    gpu = run_gpu(w)
    check(compare(w, gpu))
    general = int(((gpu["flags"] & N.FLAG_GENERAL) != 0).sum())
    print(f"general-path rows: {general}", flush=True)
    assert general == 0


def test_mixed_batch_splits_between_the_two_kernels():
    w = mixed()
    gpu = run_gpu(w)
    check(compare(w, gpu))
    assert not ((gpu["flags"] & N.FLAG_GENERAL) != 0).any()


@pytest.mark.parametrize("forced", [0, N.HINT_WHOLE_SOME, N.HINT_WHOLE_ALL | N.HINT_WHOLE_SOME])
def test_forced_hints_change_no_result(forced):
    """Wrong or missing hints reroute rows (some to the general path) but
    every output stays the same."""
    w = mixed(48)
    auto = run(w, None)
    other = run(w, forced)
    for k in ("tokens", "consumed", "status", "kept_bits"):
        np.testing.assert_array_equal(auto[k], other[k], err_msg=k)
    np.testing.assert_allclose(other["probs"], auto["probs"], rtol=1e-6, atol=1e-300)
    c3 = workloads.c3(rows=32)
    base, forced_c3 = run(c3, None), run(c3, forced)
    for k in ("tokens", "consumed", "status", "kept_bits"):
        np.testing.assert_array_equal(base[k], forced_c3[k], err_msg=k)


def test_whole_rows_with_device_draws_match_the_host_uniforms():
    w = workloads.select_rows(workloads.whole(), list(range(16)))
    d = workloads.to_device(w)
    gens = [np.random.default_rng(900 + r) for r in range(w.rows)]
    state = batch.pcg64_states(gens, "cuda")
    res = batch.sample_rows(d.logits, d.policies, allow_bits=d.allow_bits, rng_state=state)
    # The same rows with each row's next Generator.random() as its uniform.
    u = np.array([np.random.default_rng(900 + r).random() for r in range(w.rows)])
    ref = batch.sample_rows(d.logits, d.policies, allow_bits=d.allow_bits,
                            uniforms=torch.from_numpy(u).cuda())
    torch.cuda.synchronize()
    assert torch.equal(res.tokens, ref.tokens) and torch.equal(res.status, ref.status)
    assert torch.equal(res.consumed, ref.consumed)
