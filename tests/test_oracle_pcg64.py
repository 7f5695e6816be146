"""Pins the PCG64 oracle (oracle/pcg64_oracle.py) against the reference's
recorded RandomStreams (tests/golden/sampling_golden.json, written by
importing the reference's sampling module) and against NumPy's own PCG64.
Planted mistakes at the end are each caught."""
import json
import os

import numpy as np
import pytest

from oracle import pcg64_oracle as P

GOLD = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampling_golden.json")))


def test_reference_streams_from_snapshot_to_after():
    # Each fixture: the domain states of a fresh RandomStreams(seed), eight
    # draws per domain, and the states after them (sampling.py:142-231).
    n = 0
    for case in GOLD["rng"]:
        for dom, d in case["snapshot"]["domains"].items():
            state, inc = int(d["state"], 16), int(d["increment"], 16)
            end, values = P.draws(state, inc, len(case["draws"][dom]))
            assert values == case["draws"][dom], (case["seed"], dom)
            after = case["after"]["domains"][dom]
            assert end == int(after["state"], 16) and inc == int(after["increment"], 16)
            n += 1
    assert n == 9


def test_numpy_pcg64_on_random_states():
    rng = np.random.default_rng(3)
    for _ in range(20):
        g = np.random.Generator(np.random.PCG64(int(rng.integers(0, 2**63))))
        st = g.bit_generator.state["state"]
        state, inc = st["state"], st["inc"]
        end, values = P.draws(state, inc, 50)
        assert values == [g.random() for _ in range(50)]
        assert end == g.bit_generator.state["state"]["state"]


_good_random = P.random


def _old_state_output(state, inc):
    s = P.step(state, inc)
    return s, (P.output(state) >> 11) * 2.0 ** -53


def _wrong_shift(state, inc):
    s = P.step(state, inc)
    return s, (P.output(s) >> 12) * 2.0 ** -52


def _no_increment(state, inc):
    s = (state * P.MULT) & P.MASK128
    return s, (P.output(s) >> 11) * 2.0 ** -53


@pytest.mark.parametrize("bad", [_old_state_output, _wrong_shift, _no_increment])
def test_planted_mistakes_are_caught(bad, monkeypatch):
    monkeypatch.setattr(P, "random", bad)
    with pytest.raises(AssertionError):
        test_reference_streams_from_snapshot_to_after()
