"""Exact model of the Shoup-companion computation used to prepare fixed operands.

launch_prepare_pairs (provenloop_amd/csrc/poly.hip, shoup_companion) forms
floor(w 2^64 / q) for w < q from the Barrett constant r = floor((2^128 - 1) / q)
without a 128-bit division: est = w r_hi + hi64(w r_lo) is at most one short,
and the remainder w 2^64 - est q, exact modulo 2^64, drives the correction.
This model repeats those 64-bit steps with Python integers and checks the
result against the definition on edge and random values of every integer
limb prime the library uses.
"""
import numpy as np
import pytest

from provenloop_amd.params import CHAIN_N32768_L8

M64 = (1 << 64) - 1
PRIMES = sorted({q for q in [1152921504606748673, 1152921504606683137, 1152921504606830593, 1152921504606601217]
                 + CHAIN_N32768_L8 if q >= 1 << 41} | {(1 << 61) - 1})


def companion(w: int, q: int) -> int:
    r = ((1 << 128) - 1) // q
    r_hi, r_lo = r >> 64, r & M64
    est = (w * r_hi + ((w * r_lo) >> 64)) & M64
    rem = (-est * q) & M64
    steps = 0
    while rem >= q:
        est, rem, steps = est + 1, rem - q, steps + 1
    assert steps <= 1
    return est


@pytest.mark.parametrize("q", PRIMES)
def test_companion_matches_definition(q):
    rng = np.random.default_rng(q % 99991)
    ws = [0, 1, 2, q - 1, q - 2, q // 2, (q + 1) // 2, 1 << 32, (1 << 60) % q]
    ws += [int(v) % q for v in rng.integers(0, 1 << 63, 4000, dtype=np.uint64)]
    for w in ws:
        assert companion(w, q) == (w << 64) // q, (q, w)
