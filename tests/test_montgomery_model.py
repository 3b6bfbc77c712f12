"""Exact model of the Montgomery products in the fused NTT loads.

mont_mul (provenloop_amd/csrc/th_device.h) returns a b 2^-64 mod q in [0, 2q)
for any 64-bit a and b < q from T = a b and k = T_lo (-q^{-1}) mod 2^64 as
t_hi + hi64(k q) + (T_lo != 0); -q^{-1} mod 2^64 comes from Newton's
iteration (runtime_common.hip, six steps from 1) and operands are put into
Montgomery form as w (2^64 mod q) mod q (k_to_montgomery). This model
repeats the 64-bit steps with Python integers and checks, for every limb
prime the library uses, the inverse, the bound, and that a product with a
converted operand is a w mod q.
"""
import numpy as np
import pytest

from provenloop_amd.params import CHAIN_N32768_L8

M64 = (1 << 64) - 1
PRIMES = sorted(set([1152921504606748673, 1099510054913, 1099508121601, 1152921504606683137,
                     1152921504606830593, 1099511480321, 1099510890497, 1152921504606601217]
                    + CHAIN_N32768_L8 + [(1 << 61) - 1, 97, 17]))


def neg_inverse(q: int) -> int:
    qi = 1
    for _ in range(6):
        qi = (qi * (2 - q * qi)) & M64
    return (-qi) & M64


def mont_mul(a: int, b: int, q: int, mq: int) -> int:
    t = a * b
    t_lo, t_hi = t & M64, t >> 64
    k = (t_lo * mq) & M64
    return (t_hi + ((k * q) >> 64) + (1 if t_lo else 0)) & M64


@pytest.mark.parametrize("q", PRIMES)
def test_montgomery_product(q):
    mq = neg_inverse(q)
    assert (q * mq) & M64 == M64  # q (-q^{-1}) = -1 mod 2^64
    r64 = (1 << 64) % q
    rng = np.random.default_rng(q % 65521)
    ws = [0, 1, q - 1, q // 2] + [int(v) % q for v in rng.integers(0, 1 << 63, 400, dtype=np.uint64)]
    xs = [0, 1, q - 1, q, 2 * q - 1, 4 * q - 1 if 4 * q <= M64 else q, M64] + \
         [int(v) for v in rng.integers(0, 1 << 63, 400, dtype=np.uint64)]
    for w in ws:
        wm = (w * r64) % q  # k_to_montgomery
        for x in xs[:60] if w else xs:
            r = mont_mul(x, wm, q, mq)
            assert r < 2 * q, (q, x, w)
            assert r % q == (x * w) % q, (q, x, w)
