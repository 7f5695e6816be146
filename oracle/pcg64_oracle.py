"""CPU oracle for the device PCG64 draw.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it; the product package
never does.

The reference draws every uniform with NumPy's ``Generator.random()`` on a
PCG64 bit generator per domain (src/deepseekrpc/sampling.py:159-162,171-172,
214).  ``random()`` is one step of PCG64 (O'Neill's PCG family: a 128-bit
linear congruential state with the XSL-RR 64-bit output) scaled to [0, 1):

    state <- state * M + inc  (mod 2^128)
    x     = hi64(state) ^ lo64(state)
    out   = rotr64(x, hi64(state) >> 58)
    u     = (out >> 11) * 2^-53

with M the published PCG 128-bit multiplier.  ``state`` and ``inc`` are the
integers of the bit generator's state dict.  Seeding (SeedSequence) stays on
the host, where NumPy itself does it.

Pinning (tests/test_oracle_pcg64.py): the reference's recorded streams in
tests/golden/ (state before and after eight draws of each domain, and the
draws, for three seeds), NumPy's own PCG64 on random states, and planted
mistakes (output from the old state, a wrong shift, a dropped increment).
"""
from __future__ import annotations

MULT = 0x2360ED051FC65DA44385DF649FCCF645
MASK128 = (1 << 128) - 1
MASK64 = (1 << 64) - 1


def step(state: int, inc: int) -> int:
    return (state * MULT + inc) & MASK128


def output(state: int) -> int:
    hi, lo = state >> 64, state & MASK64
    rot = hi >> 58
    x = hi ^ lo
    return ((x >> rot) | (x << ((64 - rot) & 63))) & MASK64


def random(state: int, inc: int):
    """(next state, Generator.random() value)."""
    s = step(state, inc)
    return s, (output(s) >> 11) * 2.0 ** -53


def draws(state: int, inc: int, n: int):
    """(state after n draws, the n values)."""
    out = []
    for _ in range(n):
        state, u = random(state, inc)
        out.append(u)
    return state, out
