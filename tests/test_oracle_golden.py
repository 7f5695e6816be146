"""The oracle against the golden vectors written by the reference itself.

tests/golden/make_golden.py imported the reference's sampling module and
recorded float64 probability vectors (bitwise, or by SHA-256 for full
vocabularies), categorical ids, verifier decisions and PCG64 draws.  The
oracle must reproduce every probability vector bit for bit.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import sampling_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "sampling_golden.npz"))
META = json.load(open(os.path.join(HERE, "golden", "sampling_golden.json")))


def golden_case(case):
    n = case["name"]
    if f"{n}/logits" in GOLD:
        logits = GOLD[f"{n}/logits"]
    else:
        logits = (GOLD[f"{n}/logits_bf16"].astype(np.uint32) << 16).view(np.float32)
    V = len(logits)
    counts = GOLD[f"{n}/counts"] if f"{n}/counts" in GOLD else None
    gen = GOLD[f"{n}/generated"] if f"{n}/generated" in GOLD else None
    allowed = np.unpackbits(GOLD[f"{n}/allowed"])[:V].astype(bool) if f"{n}/allowed" in GOLD else None
    bias = None if case["bias"] is None else {int(t): b for t, b in case["bias"]}
    return logits, counts, gen, bias, allowed


@pytest.mark.parametrize("case", META["probabilities"], ids=lambda c: c["name"])
def test_probabilities_bitwise(case):
    logits, counts, gen, bias, allowed = golden_case(case)
    p = O.probabilities(logits, O.Policy(**case["policy"]), counts, gen, bias, allowed)
    n = case["name"]
    if f"{n}/probs" in GOLD:
        assert np.array_equal(p, GOLD[f"{n}/probs"])
    else:
        assert hashlib.sha256(p.tobytes()).hexdigest() == META["hashes"][n]
        np.testing.assert_array_equal(p[GOLD[f"{n}/probs_top_idx"]], GOLD[f"{n}/probs_top_val"])
    assert [O.categorical(p, u)[0] for u in case["uniforms"]] == case["ids"]


@pytest.mark.parametrize("case", META["verify"], ids=lambda c: c["name"])
def test_verify_decisions(case):
    tgt, drf = GOLD[f"{case['name']}/target"], GOLD[f"{case['name']}/draft"]
    pol = O.Policy(**case["policy"])
    K = len(case["ids"])
    res = O.verify(tgt, drf, case["ids"], pol, case["u_accept"], case["u_target"], eos_ids=case["eos"],
                   output_limit=case["limit"])
    assert res.status == O.OK
    assert (res.accepted, list(res.output_ids), res.pending, res.stop) == (
        case["accepted"], case["output_ids"], case["pending"], case["stop"])
    assert res.used_accept == case["calls"].count("accept")
    assert res.used_target == case["calls"].count("target")
    assert K == 4
