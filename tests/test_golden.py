"""Golden fixtures (tests/golden/golden.json, written by make_golden.py).

CPU tests: the oracle reproduces every fixture, and the small NTT vectors
agree with a brute-force evaluation of the polynomial at the odd powers of
psi, so the fixture is tied to the mathematics and not only to the code that
wrote it. GPU tests: the HIP engine reproduces the seeded keygen ->
keygen_public -> encrypt_pk -> ct x pt -> rescale -> decrypt chain bit for bit
(SHA-256 over every limb of every object).
"""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

from oracle import oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

with open(os.path.join(HERE, "golden", "golden.json")) as _f:
    GOLDEN = json.load(_f)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _u64(vals):
    return np.array([int(v) for v in vals], dtype=np.uint64)


def _brv(x, bits):
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


@pytest.mark.parametrize("case", GOLDEN["ntt"], ids=lambda c: f"n{c['n']}")
def test_oracle_ntt_vectors(case):
    q = int(case["q"])
    x = _u64(case["x"])
    assert np.array_equal(orc.ntt_forward(x, q), _u64(case["forward"]))
    assert np.array_equal(orc.ntt_inverse(x, q), _u64(case["inverse"]))
    assert np.array_equal(orc.ntt_inverse(_u64(case["forward"]), q), x)


@pytest.mark.parametrize("case", [c for c in GOLDEN["ntt"] if c["n"] <= 16], ids=lambda c: f"n{c['n']}")
def test_ntt_vectors_brute_force(case):
    """Output j of the forward transform is a(psi^(2*brv(j)+1)) mod q: the
    negacyclic evaluation in bit-reversed order, computed here term by term."""
    n, q = case["n"], int(case["q"])
    bits = n.bit_length() - 1
    psi = orc.ntt_tables(n, q)["psi"]
    assert pow(psi, n, q) == q - 1
    x = [int(v) for v in case["x"]]
    want = []
    for j in range(n):
        r = pow(psi, 2 * _brv(j, bits) + 1, q)
        want.append(sum(x[i] * pow(r, i, q) for i in range(n)) % q)
    assert [int(v) for v in case["forward"]] == want
    # the inverse is the exact inverse map: interpolation back to x
    inv = [int(v) for v in case["inverse"]]
    back = []
    for j in range(n):
        r = pow(psi, 2 * _brv(j, bits) + 1, q)
        back.append(sum(inv[i] * pow(r, i, q) for i in range(n)) % q)
    assert back == x


def test_oracle_chacha_prefix():
    assert [int(v) for v in orc.rng_u32(42, 64)] == GOLDEN["chacha_seed42_u32"]


def test_oracle_encrypt_pk_randomness():
    got = orc.encrypt_pk_randomness(1234, 1024)
    for name, arr in zip(("u", "e0", "e1"), got):
        want = GOLDEN["encrypt_pk_randomness_seed1234_n1024"][name]
        assert [int(v) for v in arr[:8]] == want[0]
        assert [int(v) for v in arr[-8:]] == want[1]


@pytest.mark.parametrize("n", [8192, 16384])
def test_oracle_chain(n):
    assert make_golden.chain(n) == GOLDEN["chain"][str(n)]


@pytest.mark.gpu
@pytest.mark.parametrize("n", [8192, 16384])
def test_engine_chain(n):
    from provenloop_amd import tensafe_he

    g = GOLDEN["chain"][str(n)]
    eng = tensafe_he.CkksContext(n)
    z, p = make_golden.chain_inputs(n)
    sk = eng.keygen(seed=11)
    pk = eng.keygen_public(sk, seed=22)
    ct = eng.encrypt_pk(z, pk, seed=33)
    prod = eng.ct_pt_mul(ct, p)
    res = eng.rescale(prod)
    dec = eng.decrypt(res, sk)

    assert [str(q) for q in eng.moduli] == g["moduli"]
    assert _sha(eng.sk_download(sk)) == g["sk"]["sha256"]
    b, a = eng.pk_download(pk)
    assert _sha(np.concatenate([b.ravel(), a.ravel()])) == g["pk"]["sha256"]
    for name, c in (("ct", ct), ("ct_pt", prod), ("rescaled", res)):
        c0, c1 = eng.ct_download(c)
        assert c.num_limbs == g[name]["limbs"], name
        assert c.scale == g[name]["scale"], name
        assert _sha(np.concatenate([c0.ravel(), c1.ravel()])) == g[name]["sha256"], name
    assert _sha(dec) == g["decrypt"]["sha256"]
