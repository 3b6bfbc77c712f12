"""Independent pins of the CPU oracle: closed forms, brute force and invariants.

The reference holds no golden ciphertext vectors, so beyond its own KATs
(test_oracle_reference_tests.py) the oracle is pinned here by mathematics that
a plausible slip (a dropped Barrett term, a transposed twiddle index, a wrong
sign in the rescale, a swapped RNG draw order) would break:

* Barrett multiply == exact (a*b) mod q on random and edge operands.
* Forward NTT == the O(N^2) closed form  A[k] = sum_j a_j psi^((2 brv(k)+1) j).
* psi is a primitive 2N-th root and the first one the documented search
  (rns.rs:124-155: g = 2, 3, ... ) reaches.
* ChaCha20 stream == RFC-pinned block function applied to the documented
  seed -> key layout, counter 0, 1, 2, ...
* Box-Muller Gaussians == numpy evaluation of the formula on the raw stream.
* decode == direct evaluation of the canonical embedding; encode == numpy FFT.
* keygen_public: b + a*s is a small error polynomial (RLWE invariant).
* encrypt_pk: c0 + c1*s == m + e0 + e*u + e1*s exactly (negacyclic products of
  small integer polynomials computed with integer convolution).
* rescale: c' * q_last == c - (c_last mod q_l)  (mod q_l) per coefficient.
* CRT decrypt: a constructed ciphertext with known ~2^90 coefficients decodes
  to the centred big-integer value.
"""
import math

import numpy as np
import pytest

CHAINS = {8192: None, 16384: None, 32768: None}


def _chain(orc, n):
    if CHAINS[n] is None:
        CHAINS[n] = orc.default_chain(n)
    return CHAINS[n]


def brv(x, bits):
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


def negacyclic_int(a, b):
    """Exact negacyclic product of two integer polynomials (int64 inputs, small)."""
    n = len(a)
    full = np.convolve(np.asarray(a, np.int64), np.asarray(b, np.int64))
    out = full[:n].copy()
    out[: n - 1] -= full[n:]
    return out


# ---------------------------------------------------------------- Barrett
@pytest.mark.parametrize("n", [8192, 16384, 32768])
def test_barrett_matches_exact_mod(orc, n):
    rng = np.random.default_rng(7)
    for q in _chain(orc, n):
        a = rng.integers(0, q, 20000, dtype=np.uint64)
        b = rng.integers(0, q, 20000, dtype=np.uint64)
        edge = np.array([0, 1, 2, q - 1, q - 2, q // 2, (q + 1) // 2], np.uint64)
        a = np.concatenate([a, edge, edge[::-1], np.full(7, q - 1, np.uint64)])
        b = np.concatenate([b, edge, edge, edge])
        got = orc.mod_mul_barrett(a, b, q)
        exp = [(int(x) * int(y)) % q for x, y in zip(a, b)]
        assert got.tolist() == exp


def test_barrett_reduce_128bit_inputs(orc):
    rng = np.random.default_rng(11)
    for q in _chain(orc, 16384):
        xs = [int(rng.integers(0, 2**62)) * int(rng.integers(0, 2**62)) % (q * q) for _ in range(5000)]
        xs += [q * q - 1, q * q - q, 2**64, 2**64 - 1, 0]
        lo = np.array([x & (2**64 - 1) for x in xs], np.uint64)
        hi = np.array([x >> 64 for x in xs], np.uint64)
        assert orc.barrett_reduce(lo, hi, q).tolist() == [x % q for x in xs]


# ---------------------------------------------------------------- NTT
def _closed_form_ntt(a, q, psi):
    n = len(a)
    bits = n.bit_length() - 1
    pw = [1] * (2 * n)
    for e in range(1, 2 * n):
        pw[e] = pw[e - 1] * psi % q
    a = [int(x) for x in a]
    out = []
    for k in range(n):
        r = 2 * brv(k, bits) + 1
        s = 0
        for j in range(n):
            s += a[j] * pw[(r * j) % (2 * n)]
        out.append(s % q)
    return out


@pytest.mark.parametrize("n", [8, 64, 256])
def test_ntt_forward_closed_form(orc, n):
    rng = np.random.default_rng(n)
    for q in [97 if n <= 8 else 7681, *_chain(orc, 16384)]:
        if q % (2 * n) != 1:
            continue
        a = rng.integers(0, q, n, dtype=np.uint64)
        psi = orc.ntt_tables(n, q)["psi"]
        assert orc.ntt_forward(a, q).tolist() == _closed_form_ntt(a, q, psi)
        # inverse closed form: the forward transform of the inverse is the input
        assert orc.ntt_forward(orc.ntt_inverse(a, q), q).tolist() == a.tolist()


def test_ntt_closed_form_n1024_real_primes(orc):
    n = 1024
    rng = np.random.default_rng(5)
    for q in (_chain(orc, 16384)[0], _chain(orc, 16384)[1]):
        a = rng.integers(0, q, n, dtype=np.uint64)
        psi = orc.ntt_tables(n, q)["psi"]
        # vectorised closed form with Python ints on an object array
        bits = 10
        pw = np.empty(2 * n, dtype=object)
        pw[0] = 1
        for e in range(1, 2 * n):
            pw[e] = pw[e - 1] * psi % q
        j = np.arange(n)
        aj = np.array([int(x) for x in a], dtype=object)
        got = orc.ntt_forward(a, q)
        for k in rng.choice(n, 64, replace=False):
            r = 2 * brv(int(k), bits) + 1
            assert int(got[k]) == int(np.sum(aj * pw[(r * j) % (2 * n)]) % q)


@pytest.mark.parametrize("n", [8192, 16384, 32768])
def test_psi_is_first_primitive_root_of_search(orc, n):
    for q in _chain(orc, n):
        t = orc.ntt_tables(n, q)
        psi = t["psi"]
        assert pow(psi, n, q) == q - 1 and pow(psi, 2 * n, q) == 1
        e = (q - 1) // (2 * n)
        for g in range(2, 10000):
            c = pow(g, e, q)
            if c > 1 and pow(c, n, q) == q - 1:
                assert c == psi
                break
        assert t["psi_inv"] * psi % q == 1
        assert t["n_inv"] * n % q == 1


def test_twiddle_tables_are_bit_reversed_powers(orc):
    n = 256
    q = _chain(orc, 16384)[0]
    t = orc.ntt_tables(n, q)
    for i in range(n):
        assert int(t["fwd"][brv(i, 8)]) == pow(t["psi"], i, q)
        assert int(t["inv"][brv(i, 8)]) == pow(t["psi_inv"], i, q)


def test_ntt_linearity_and_convolution_large(orc):
    """NTT(a)*NTT(b) -> iNTT == exact negacyclic product (small a, b), N=16384."""
    n = 16384
    rng = np.random.default_rng(3)
    a = rng.integers(-3, 4, n)
    b = rng.integers(-20, 21, n)
    exact = negacyclic_int(a, b)
    for q in _chain(orc, n):
        A = orc.ntt_forward(np.mod(a, q).astype(np.uint64), q)
        B = orc.ntt_forward(np.mod(b, q).astype(np.uint64), q)
        c = orc.ntt_inverse(orc.mod_mul_barrett(A, B, q), q)
        assert np.array_equal(c, np.mod(exact, q).astype(np.uint64))


# ---------------------------------------------------------------- RNG
def _state(seed, counter):
    lo, hi = seed & 0xFFFFFFFF, seed >> 32
    return np.array([0x61707865, 0x3320646E, 0x79622D32, 0x6B206574,
                     lo, hi, lo, hi, lo, hi, lo, hi, counter, 0, 0, 0], np.uint32)


@pytest.mark.parametrize("seed", [0, 42, 2**40 + 17, 2**64 - 1])
def test_seeded_stream_is_chacha_blocks(orc, seed):
    stream = orc.rng_u32(seed, 48)
    for blk in range(3):
        assert stream[16 * blk: 16 * blk + 16].tolist() == orc.chacha20_block(_state(seed, blk)).tolist()
    u64 = orc.rng_u64(seed, 8)
    assert u64.tolist() == [int(stream[2 * i]) | (int(stream[2 * i + 1]) << 32) for i in range(8)]


def test_range_sampling_consumes_stream(orc):
    # range_u64 rejects r < 2^64 mod q and returns r mod q (rng.rs:124-133)
    for q in (_chain(orc, 16384)[0], 2**63 + 1):  # the second rejects ~half the draws
        raw = [int(x) for x in orc.rng_u64(9, 4000)]
        thr = (2**64) % q
        exp = [r % q for r in raw if r >= thr]
        got = orc.rng_range_u64(9, q, len(exp))
        assert got.tolist() == exp
    assert len(exp) < 0.6 * len(raw)
    raw32 = orc.rng_u32(9, 4000).astype(np.int64)
    thr32 = (2**32) % 3_000_000_001
    exp32 = [r % 3_000_000_001 for r in raw32 if r >= thr32]
    assert orc.rng_range_u32(9, 3_000_000_001, len(exp32)).tolist() == exp32


def test_gaussian_matches_box_muller_on_stream(orc):
    seed, n = 77, 20000
    raw = orc.rng_u64(seed, 2 * n)
    u = ((raw >> np.uint64(11)).astype(np.float64) + 0.5) / float(2**53)
    assert np.array_equal(orc.rng_f64(seed, 2 * n), u)
    z = np.sqrt(-2.0 * np.log(u[0::2])) * np.cos(2.0 * math.pi * u[1::2]) * 3.19
    g = orc.rng_gaussian(seed, 3.19, n)
    assert np.max(np.abs(g - z)) < 1e-12
    # rounding to integers agrees except within 1e-9 of a .5 boundary
    safe = np.abs(np.abs(z - np.trunc(z)) - 0.5) > 1e-9
    signed = orc.sample_gaussian_signed(seed, n, 3.19)
    half_away = (np.sign(z) * np.floor(np.abs(z) + 0.5)).astype(np.int64)  # f64::round
    assert np.array_equal(signed[safe], half_away[safe])


def test_encrypt_pk_randomness_draw_order(orc):
    """u = N range_u32(3) draws, then e0, then e1 (ciphertext.rs:255-273)."""
    n, seed = 1024, 5
    u, e0, e1 = orc.encrypt_pk_randomness(seed, n)
    raw = orc.rng_u32(seed, n + 8 * n + 64)
    assert raw[:n].min() > 0  # no rejections on this seed: positions are fixed
    # sample_ternary(rng, n, 3) stores r=0 -> 2, r=1 -> 0, r=2 -> 1 (sampling.rs:17-29)
    assert u.tolist() == np.array([2, 0, 1])[raw[:n] % 3].tolist()
    words = raw[n: n + 8 * n].astype(np.uint64)
    u64 = words[0::2] | (words[1::2] << np.uint64(32))
    f = ((u64 >> np.uint64(11)).astype(np.float64) + 0.5) / float(2**53)
    z = np.sqrt(-2.0 * np.log(f[0::2])) * np.cos(2.0 * math.pi * f[1::2]) * 3.19
    zr = np.sign(z) * np.floor(np.abs(z) + 0.5)
    assert np.array_equal(np.concatenate([e0, e1]), zr.astype(np.int64))


# ---------------------------------------------------------------- encode / decode
def test_decode_is_canonical_embedding(orc):
    n = 8192
    ctx = orc.Context(n)
    rng = np.random.default_rng(1)
    c = rng.normal(size=n)
    got = ctx.decode_coefficients(c)
    k = np.arange(n // 2)[:, None]
    j = np.arange(n)[None, :]
    sel = np.arange(0, n // 2, 97)
    exp = (np.cos(np.pi * ((2 * k[sel] + 1) * j % (2 * n)) / n) * c).sum(axis=1)
    assert np.allclose(got[sel], exp, rtol=0, atol=1e-9)


def test_encode_matches_numpy_fft(orc):
    n = 8192
    ctx = orc.Context(n)
    rng = np.random.default_rng(2)
    z = rng.normal(size=n // 2) * 0.1
    zt = np.zeros(n)
    zt[: n // 2] = z
    zt[n - 1 - np.arange(n // 2)] = z
    a = np.fft.fft(zt) / n
    j = np.arange(n)
    coeff = a.real * np.cos(np.pi * j / n) + a.imag * np.sin(np.pi * j / n)
    exp = np.round(coeff * 2.0**40).astype(np.int64)
    enc = ctx.encode(z)
    q0 = ctx.moduli[0]
    got = np.where(enc[0] > q0 // 2, enc[0].astype(object) - q0, enc[0].astype(object)).astype(np.int64)
    # numpy's FFT differs from the radix-2 DIT by a few ulps: allow +-1 at the rounding step
    assert np.max(np.abs(got - exp)) <= 1
    for l, q in enumerate(ctx.moduli):
        assert np.array_equal(enc[l], np.mod(got.astype(object), q).astype(np.uint64))


# ---------------------------------------------------------------- keys and encryption
@pytest.fixture(scope="module")
def keys(orc):
    ctx = orc.Context(8192)
    sk = ctx.keygen(1234)
    pk = ctx.keygen_public(sk, 5678)
    # keygen: sample_ternary stores r -> {2, 0, 1}; the limb map sends 0 -> -1, 1 -> 0,
    # 2 -> +1 (ciphertext.rs:86-97), so the draw r=0 is +1, r=1 is -1 and r=2 is 0.
    s_raw = orc.rng_range_u32(1234, 3, 8192)
    s = np.array([1, -1, 0], np.int64)[s_raw]
    return ctx, sk, pk, s


def test_secret_key_is_ntt_of_ternary_draws(orc, keys):
    ctx, sk, pk, s = keys
    S = ctx.sk_data(sk)
    for l, q in enumerate(ctx.moduli):
        assert np.array_equal(orc.ntt_inverse(S[l], q), np.mod(s, q).astype(np.uint64))


def _pk_error(orc, ctx, sk, pk):
    b, a = ctx.pk_data(pk)
    S = ctx.sk_data(sk)
    es = []
    for l, q in enumerate(ctx.moduli):
        e = orc.ntt_inverse(np.array([(int(x) + int(y) * int(z)) % q for x, y, z in zip(b[l], a[l], S[l])], np.uint64), q)
        es.append(np.where(e > q // 2, e.astype(object) - q, e.astype(object)).astype(np.int64))
    return es


def test_public_key_is_rlwe_sample(orc, keys):
    ctx, sk, pk, s = keys
    es = _pk_error(orc, ctx, sk, pk)
    for e in es[1:]:
        assert np.array_equal(e, es[0])  # the same signed error in every limb
    assert np.abs(es[0]).max() < 40 and 2.5 < es[0].std() < 4.0


def test_encrypt_pk_closed_form(orc, keys):
    ctx, sk, pk, s = keys
    n = ctx.n
    e = _pk_error(orc, ctx, sk, pk)[0]
    z = np.random.default_rng(4).normal(size=n // 2) * 0.1
    u_raw, e0, e1 = orc.encrypt_pk_randomness(99, n)
    u = np.where(u_raw == 0, -1, np.where(u_raw == 1, 0, 1)).astype(np.int64)
    ct = ctx.encrypt_pk_with(z, pk, u_raw, e0, e1)
    ct_seeded = ctx.encrypt_pk(z, pk, 99)
    for x, y in zip(ctx.ct_data(ct), ctx.ct_data(ct_seeded)):
        assert np.array_equal(x, y)
    m = ctx.encode(z)
    noise = e0 + negacyclic_int(e, u) + negacyclic_int(e1, s)
    c0, c1 = ctx.ct_data(ct)
    S = ctx.sk_data(sk)
    for l, q in enumerate(ctx.moduli):
        dec = orc.ntt_inverse(np.array([(int(x) + int(y) * int(w)) % q for x, y, w in zip(c0[l], c1[l], S[l])], np.uint64), q)
        exp = (m[l].astype(object) + np.mod(noise, q).astype(object)) % q
        assert np.array_equal(dec, exp.astype(np.uint64))


def test_rescale_closed_form(orc, keys):
    ctx, sk, pk, s = keys
    n = ctx.n
    z = np.random.default_rng(6).normal(size=n // 2)
    ct = ctx.ct_pt_mul(ctx.encrypt_pk(z, pk, 7), np.full(100, 0.25))
    r = ctx.rescale(ct)
    assert r.num_limbs == 3 and r.scale == ct.scale / ctx.moduli[3]
    c = ctx.ct_data(ct)
    rc = ctx.ct_data(r)
    ql = ctx.moduli[3]
    for comp in range(2):
        last = orc.ntt_inverse(c[comp][3], ql)
        for l in range(3):
            q = ctx.moduli[l]
            cl = orc.ntt_inverse(c[comp][l], q).astype(object)
            new = orc.ntt_inverse(rc[comp][l], q).astype(object)
            lhs = (new * ql) % q
            rhs = (cl - (last.astype(object) % q)) % q
            assert np.array_equal(lhs, rhs)


def test_crt_decrypt_closed_form(orc, keys):
    ctx, sk, pk, s = keys
    n, q0, q1 = ctx.n, ctx.moduli[0], ctx.moduli[1]
    rng = np.random.default_rng(8)
    big = [int(x) * 2**40 + int(y) for x, y in zip(rng.integers(-2**49, 2**49, n), rng.integers(0, 2**40, n))]
    # c1 = 0, c0 = NTT(big mod q_l): decryption is big itself
    c0 = np.stack([orc.ntt_forward(np.array([v % q for v in big], np.uint64), q) for q in ctx.moduli])
    scale = 2.0**80
    ct = ctx.ct_from_data(c0, np.zeros_like(c0), scale)
    got = ctx.decrypt(ct, sk)
    Q = q0 * q1
    centred = [((v % Q) - Q if (v % Q) > Q // 2 else (v % Q)) for v in big]
    exp = ctx.decode_coefficients(np.array([float(v) / scale for v in centred]))
    assert np.array_equal(got, exp)
