"""Exact model of the FP64 reduction the rescale's fused column kernel uses.

For a limb prime q below 2^41 the kernel reduces the coefficient-domain last
limb c (any c < 2^61) modulo q without 64-bit multiplies (reduce_u64_f64 in
provenloop_amd/csrc/th_device.h): with c = ch 2^32 + cl,

    r = mulmod_f64(ch, 2^32 mod q) + cl,   then r < 0 -> r + q, r >= q -> r - q

where mulmod_f64 is the exact FP64 product of the NTT butterflies
(hi = x w, lo = fma(x, w, -hi), quot = rint(x w/q), fma(-quot, q, hi) + lo).
This model performs the same IEEE-754 double operations (products and sums
rounded to nearest even by Python's floats, fused multiply-adds rounded once
from the exact rational value, rint ties to even) and checks the result
against c mod q, so a wrong constant, a dropped term or a missing correction
fails here; the GPU parity tests check the kernel's output bit for bit.
"""
from fractions import Fraction

import numpy as np
import pytest

from provenloop_amd.params import CHAIN_N32768_L8

DEFAULT_CHAIN_N16384 = [1152921504606748673, 1099510054913, 1099508121601, 1152921504606683137]


def fma(a: float, b: float, c: float) -> float:
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def mulmod_f64(x: float, w: float, wq: float, q: float) -> float:
    hi = x * w
    lo = fma(x, w, -hi)
    quot = float(round(x * wq))
    r = fma(-quot, q, hi)
    return r + lo


def reduce_u64_f64(c: int, q: int) -> float:
    qd = float(q)
    k32 = float((1 << 32) % q)
    k32q = k32 / qd
    ch, cl = float(c >> 32), float(c & 0xFFFFFFFF)
    r = mulmod_f64(ch, k32, k32q, qd) + cl
    r = r + qd if r < 0.0 else r
    return r - qd if r >= qd else r


FP_PRIMES = sorted({q for q in DEFAULT_CHAIN_N16384 + CHAIN_N32768_L8 if q < 1 << 41} | {2199023190017})


@pytest.mark.parametrize("q", FP_PRIMES)
def test_reduce_matches_mod(q):
    rng = np.random.default_rng(q % 1000003)
    edges = [0, 1, q - 1, q, q + 1, 2 * q - 1, (1 << 32) - 1, 1 << 32, (1 << 32) + 1,
             (1 << 60) - 1, 1 << 60, (1 << 61) - 1, 1152921504606683136, 1152921504606748672]
    # values whose high word makes ch (2^32 mod q) land on the rounding ties of rint
    k32 = (1 << 32) % q
    for t in range(1, 64):
        ch = (t * q) // k32 if k32 else t
        if ch < 1 << 29:
            edges += [ch << 32, (ch << 32) | 0xFFFFFFFF]
    values = edges + [int(v) for v in rng.integers(0, 1 << 61, 3000, dtype=np.uint64)]
    for c in values:
        r = reduce_u64_f64(c, q)
        assert r == float(c % q), (q, c, r)
        assert 0.0 <= r < q


def test_model_catches_a_dropped_low_word():
    """Dropping cl (or the correction) is caught on the same inputs."""
    q = 1099510054913
    c = (123456789 << 32) | 987654321
    qd = float(q)
    k32 = float((1 << 32) % q)
    wrong = mulmod_f64(float(c >> 32), k32, k32 / qd, qd)
    wrong = wrong + qd if wrong < 0.0 else wrong
    assert wrong != float(c % q)
    assert reduce_u64_f64(c, q) == float(c % q)
