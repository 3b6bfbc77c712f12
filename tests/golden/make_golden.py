"""Writes tests/golden/golden.json: fixed input/output vectors of the CKKS
path, produced by the oracle (a line-for-line C++ restatement of the
reference CPU backend, itself pinned by the reference's own known-answer
tests and closed-form checks).

The fixtures pin the oracle and the HIP engine against themselves across
commits and machines: NTT vectors (q = 97 at N = 8, 16, the reference's
60-bit q0 at N = 256), the ChaCha20 stream prefix of TenSafeRng::from_seed(42),
encrypt_pk's randomness for one seed, and for N = 8192 and 16384 the SHA-256
of every object of a seeded keygen -> keygen_public -> encrypt_pk -> ct x pt
-> rescale -> decrypt chain, with head and tail coefficients.

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

Q0 = 1152921504606748673


def chain_inputs(n):
    """The chain's inputs, shared with the tests."""
    s = n // 2
    z = np.cos(np.arange(s) * 0.01) * 0.5
    pt = np.sin(np.arange(s) * 0.02) * 0.25
    return z, pt


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def head_tail(a, k=4):
    a = np.ascontiguousarray(a).ravel()
    return [[int(v) for v in a[:k]], [int(v) for v in a[-k:]]]


def chain(n):
    ref = orc.Context(n)
    z, p = chain_inputs(n)
    sk = ref.keygen(11)
    pk = ref.keygen_public(sk, 22)
    ct = ref.encrypt_pk(z, pk, 33)
    prod = ref.ct_pt_mul(ct, p)
    res = ref.rescale(prod)
    dec = ref.decrypt(res, sk)
    out = {"moduli": [str(q) for q in ref.moduli]}
    s = ref.sk_data(sk)
    out["sk"] = {"sha256": sha(s), "head_tail": head_tail(s)}
    b, a = ref.pk_data(pk)
    out["pk"] = {"sha256": sha(np.concatenate([b.ravel(), a.ravel()])), "head_tail": head_tail(b)}
    for name, c in (("ct", ct), ("ct_pt", prod), ("rescaled", res)):
        c0, c1 = ref.ct_data(c)
        out[name] = {"sha256": sha(np.concatenate([c0.ravel(), c1.ravel()])), "limbs": int(c0.shape[0]),
                     "scale": c.scale, "c0_head_tail": head_tail(c0), "c1_head_tail": head_tail(c1)}
    out["decrypt"] = {"sha256": sha(dec), "head": [float(v) for v in dec[:4]]}
    return out


def main():
    g = {"generator": "tests/golden/make_golden.py (CPU oracle)"}
    ntt = []
    rng = np.random.default_rng(5)
    for n, q in ((8, 97), (16, 97), (256, Q0)):
        x = rng.integers(0, q, n, dtype=np.uint64)
        ntt.append({"n": n, "q": str(q), "x": [str(v) for v in x],
                    "forward": [str(v) for v in orc.ntt_forward(x, q)],
                    "inverse": [str(v) for v in orc.ntt_inverse(x, q)]})
    g["ntt"] = ntt
    g["chacha_seed42_u32"] = [int(v) for v in orc.rng_u32(42, 64)]
    r = orc.encrypt_pk_randomness(1234, 1024)
    g["encrypt_pk_randomness_seed1234_n1024"] = {k: head_tail(np.asarray(v), 8) for k, v in zip(("u", "e0", "e1"), r)}
    g["chain"] = {str(n): chain(n) for n in (8192, 16384)}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.json")
    with open(path, "w") as f:
        json.dump(g, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
