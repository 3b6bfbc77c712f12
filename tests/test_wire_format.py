"""The wire format, pinned independently of the oracle's serialiser.

serialize.rs fixes the byte layout:
  * an RnsPoly is its limbs in order, each N little-endian u64 (:13-24);
  * a PublicKey is [b | a] (:47-52);
  * a Ciphertext is [scale as f64 LE | c0 | c1] (:69-77).

Here the expected bytes are parsed with `struct` from that description alone
and tied to the mathematics of the objects, so a swapped c0/c1, an [a | b]
key, a coefficient-interleaved (instead of limb-major) layout, a big-endian
word or a misplaced scale fails:
  * a ciphertext's parsed (c0, c1) must satisfy the decryption identity: the
    inverse NTT of c0 + c1 s is congruent, on every limb, to one small
    integer vector (m + e), equal to the encoded message up to the noise;
  * a public key's parsed (b, a) must satisfy b + a s = e with |e| small on
    every limb (the RLWE relation of keygen_public, ciphertext.rs:114-154).
The arithmetic uses Python integers and the oracle's NTT only (pinned by the
closed-form and known-answer tests).
"""
import struct

import numpy as np
import pytest

N = 8192


def _parse_poly(buf, off, limbs, n):
    """limbs x n little-endian u64, limb-major, from buf[off:]."""
    words = struct.unpack_from("<%dQ" % (limbs * n), buf, off)
    return np.array(words, dtype=np.uint64).reshape(limbs, n)


def _centred(x, q):
    x = int(x)
    return x - q if x > q // 2 else x


def _decrypt_identity(orc, q, s_ntt, c0, c1):
    """Per limb: inverse NTT of c0 + c1 * s (NTT domain, Python-int products), centred."""
    out = []
    for l in range(c0.shape[0]):
        ql = q[l]
        prod = [(int(a) + int(b) * int(s)) % ql for a, b, s in zip(c0[l], c1[l], s_ntt[l])]
        coef = orc.ntt_inverse(np.array(prod, dtype=np.uint64), ql)
        out.append([_centred(v, ql) for v in coef])
    return np.array(out, dtype=object)


@pytest.fixture(scope="module")
def setup(orc):
    ctx = orc.Context(N)
    sk = ctx.keygen(101)
    pk = ctx.keygen_public(sk, 202)
    rng = np.random.default_rng(5)
    z = rng.normal(size=N // 2) * 0.05  # |m| = |round(z 2^40)| stays far below q_l / 2 on every limb
    return ctx, sk, pk, z


def test_ciphertext_layout_top_level(orc, setup):
    ctx, sk, pk, z = setup
    ct = ctx.encrypt_pk(z, pk, 303)
    L = ct.num_limbs
    buf = ctx.ct_to_bytes(ct)
    assert len(buf) == 8 + 2 * L * N * 8
    # the scale first, as f64 little-endian: 2^40 for a fresh ciphertext (ciphertext.rs:314-318)
    assert buf[:8] == struct.pack("<d", 2.0 ** 40)
    c0 = _parse_poly(buf, 8, L, N)
    c1 = _parse_poly(buf, 8 + L * N * 8, L, N)
    q = ctx.moduli
    for l in range(L):
        assert int(c0[l].max()) < q[l] and int(c1[l].max()) < q[l]
    v = _decrypt_identity(orc, q, ctx.sk_data(sk), c0, c1)
    # one integer vector m + e on every limb (CRT-consistent), close to the encoded message
    for l in range(1, L):
        assert np.array_equal(v[l], v[0]), f"limb {l} disagrees with limb 0"
    m = ctx.encode(z).astype(object)[0]
    m = np.array([_centred(x, q[0]) for x in m], dtype=object)
    noise = np.abs((v[0] - m).astype(np.float64))
    assert noise.max() < 2 ** 20  # encryption noise (u e + e0 + e1 s), not a scrambled layout


def test_ciphertext_layout_after_rescale(orc, setup):
    ctx, sk, pk, z = setup
    ct = ctx.encrypt_pk(z, pk, 404)
    pt = ctx.encode_to_ntt(np.full(N // 2, 0.5))
    r = ctx.rescale(ctx.ct_pt_mul_ntt(ct, pt))
    L = r.num_limbs
    assert L == ct.num_limbs - 1
    q = ctx.moduli
    buf = ctx.ct_to_bytes(r)
    assert len(buf) == 8 + 2 * L * N * 8
    assert buf[:8] == struct.pack("<d", 2.0 ** 80 / q[-1])  # ciphertext.rs:533
    c0 = _parse_poly(buf, 8, L, N)
    c1 = _parse_poly(buf, 8 + L * N * 8, L, N)
    v = _decrypt_identity(orc, q, ctx.sk_data(sk), c0, c1)
    for l in range(1, L):
        assert np.array_equal(v[l], v[0]), f"limb {l} disagrees with limb 0"
    # the rescaled message m * m_pt / q_last is about 2^80 * 0.5 z / q3 ~ 2^19 |z|: small against q
    assert max(abs(int(x)) for x in v[0]) < 2 ** 40
    # the bytes round-trip through the oracle's parser
    back = ctx.ct_from_bytes(buf, L)
    b0, b1 = ctx.ct_data(back)
    assert np.array_equal(b0, c0) and np.array_equal(b1, c1) and back.scale == r.scale


def test_public_key_layout(orc, setup):
    ctx, sk, pk, _ = setup
    buf = ctx.pk_to_bytes(pk)
    L = len(ctx.moduli)
    assert len(buf) == 2 * L * N * 8
    b = _parse_poly(buf, 0, L, N)
    a = _parse_poly(buf, L * N * 8, L, N)
    s = ctx.sk_data(sk)
    q = ctx.moduli
    # b + a s = e, one small Gaussian vector on every limb; with [a | b] this is not small
    v = _decrypt_identity(orc, q, s, b, a)
    for l in range(1, L):
        assert np.array_equal(v[l], v[0])
    assert max(abs(int(x)) for x in v[0]) < 64
    w = _decrypt_identity(orc, q, s, a, b)
    assert max(abs(int(x)) for x in w[0]) > 2 ** 30
