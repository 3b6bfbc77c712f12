"""The reference's own unit tests (tensafe-he-core, 43 tests), run against the CPU oracle.

Each test names the Rust test it restates (file:line). These are the
authoritative known-answer and tolerance tests of the reference (its CI runs
`cargo test -p tensafe-he-core`).
"""
import numpy as np
import pytest

Q16384 = [1152921504606748673, 1099510054913, 1099508121601, 1152921504606683137]


# ---------------- params.rs:328-422 ----------------
def test_params_n16384(orc):  # params.rs:332-340
    ch = orc.default_chain(16384)
    assert len(ch) == 4
    ctx = orc.Context(16384)
    assert ctx.n == 16384 and ctx.num_slots == 8192


def test_modulus_ntt_friendly(orc):  # params.rs:342-359
    for n in (8192, 16384, 32768):
        for q in orc.default_chain(n):
            assert q % (2 * n) == 1


def test_modulus_primality(orc):  # params.rs:361-394 (trial division, independent of the oracle)
    def is_prime(n):
        if n < 2:
            return False
        if n in (2, 3):
            return True
        if n % 2 == 0 or n % 3 == 0:
            return False
        # deterministic Miller-Rabin for n < 3.3e24 (bases 2..41)
        d, s = n - 1, 0
        while d % 2 == 0:
            d //= 2
            s += 1
        for a in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37, 41):
            x = pow(a, d, n)
            if x in (1, n - 1):
                continue
            for _ in range(s - 1):
                x = x * x % n
                if x == n - 1:
                    break
            else:
                return False
        return True

    for n in (8192, 16384, 32768):
        for q in orc.default_chain(n):
            assert is_prime(q)
            assert orc.is_prime(q)


def test_barrett_constant(orc):  # params.rs:396-404
    for q in orc.default_chain(16384):
        hi, lo = orc.barrett_constant(q)
        full = (2**128 - 1) // q
        assert hi == full >> 64
        assert lo == full & (2**64 - 1)


def test_custom_params(orc):  # params.rs:406-422
    ch = orc.custom_chain(16384, [60, 40, 40, 60])
    assert len(ch) == 4
    for q in ch:
        assert q % 32768 == 1


# ---------------- rns.rs:272-372 ----------------
def test_mod_add(orc):  # rns.rs:276-283
    q = 17
    assert orc.mod_add(5, 7, q) == 12
    assert orc.mod_add(10, 10, q) == 3
    assert orc.mod_add(0, 0, q) == 0
    assert orc.mod_add(16, 1, q) == 0


def test_mod_sub(orc):  # rns.rs:285-291
    q = 17
    assert orc.mod_sub(10, 3, q) == 7
    assert orc.mod_sub(3, 10, q) == 10
    assert orc.mod_sub(0, 0, q) == 0


def test_mod_mul(orc):  # rns.rs:293-299
    q = 17
    assert orc.mod_mul(5, 3, q) == 15
    assert orc.mod_mul(5, 4, q) == 3
    assert orc.mod_mul(0, 10, q) == 0


def test_mod_pow(orc):  # rns.rs:301-307
    q = 17
    assert orc.mod_pow(2, 0, q) == 1
    assert orc.mod_pow(2, 4, q) == 16
    assert orc.mod_pow(3, 16, q) == 1


def test_mod_inv(orc):  # rns.rs:309-316
    q = 17
    for a in range(1, q):
        assert orc.mod_mul(a, orc.mod_inv(a, q), q) == 1


def test_bit_reverse(orc):  # rns.rs:318-324
    assert orc.bit_reverse(0b0000, 4) == 0b0000
    assert orc.bit_reverse(0b0001, 4) == 0b1000
    assert orc.bit_reverse(0b0110, 4) == 0b0110
    assert orc.bit_reverse(0b1010, 4) == 0b0101


def test_primitive_root(orc):  # rns.rs:326-337
    psi = orc.find_primitive_root(4, 17)
    assert pow(psi, 8, 17) == 1
    assert pow(psi, 4, 17) == 16


def test_primitive_root_large(orc):  # rns.rs:339-352
    q, n = Q16384[0], 16384
    psi = orc.find_primitive_root(n, q)
    assert pow(psi, 2 * n, q) == 1
    assert pow(psi, n, q) == q - 1


def test_rns_poly_add(orc):  # rns.rs:354-371 (RnsPoly::add == limb-wise mod_add)
    a0, b0 = [1, 2, 3, 4], [5, 6, 7, 8]
    a1, b1 = [10, 20, 30, 40], [50, 60, 70, 80]
    assert [orc.mod_add(x, y, Q16384[0]) for x, y in zip(a0, b0)] == [6, 8, 10, 12]
    assert [orc.mod_add(x, y, Q16384[1]) for x, y in zip(a1, b1)] == [60, 80, 100, 120]


# ---------------- ntt.rs:143-243 ----------------
def test_ntt_roundtrip_small(orc):  # ntt.rs:147-166
    orig = np.array([1, 2, 3, 4], np.uint64)
    a = orc.ntt_forward(orig, 17)
    assert not np.array_equal(a, orig)
    assert np.array_equal(orc.ntt_inverse(a, 17), orig)


def test_ntt_roundtrip_large_modulus(orc):  # ntt.rs:168-184
    orig = np.arange(16, dtype=np.uint64)
    assert np.array_equal(orc.ntt_inverse(orc.ntt_forward(orig, 97), 97), orig)


def test_ntt_polynomial_multiply(orc):  # ntt.rs:186-221 (exact KAT)
    q = 97
    a = orc.ntt_forward(np.array([1, 2, 3, 0, 0, 0, 0, 0], np.uint64), q)
    b = orc.ntt_forward(np.array([4, 5, 0, 0, 0, 0, 0, 0], np.uint64), q)
    c = orc.mod_mul_barrett(a, b, q)
    assert orc.ntt_inverse(c, q).tolist() == [4, 13, 22, 15, 0, 0, 0, 0]


def test_ntt_roundtrip_60bit_prime(orc):  # ntt.rs:223-242
    q = 1152921504606830593
    orig = np.arange(256, dtype=np.uint64)
    a = orc.ntt_forward(orig, q)
    assert not np.array_equal(a, orig)
    assert np.array_equal(orc.ntt_inverse(a, q), orig)


# ---------------- rng.rs:223-368 ----------------
def test_chacha20_rfc8439_vector(orc):  # rng.rs:227-271 (RFC 8439 §2.3.2)
    st = np.array([0x61707865, 0x3320646E, 0x79622D32, 0x6B206574,
                   0x03020100, 0x07060504, 0x0B0A0908, 0x0F0E0D0C,
                   0x13121110, 0x17161514, 0x1B1A1918, 0x1F1E1D1C,
                   0x00000001, 0x09000000, 0x4A000000, 0x00000000], np.uint32)
    exp = [0xE4E7F110, 0x15593BD1, 0x1FDD0F50, 0xC47120A3, 0xC7F4D1C7, 0x0368C033,
           0x9AAA2204, 0x4E6CD4C3, 0x466482D2, 0x09AA9F07, 0x05D7C214, 0xA2028BD9,
           0xD19C12B5, 0xB94E16DE, 0xE883D0CB, 0x4E3C50A2]
    assert orc.chacha20_block(st).tolist() == exp


def test_deterministic_seeding(orc):  # rng.rs:273-280
    assert np.array_equal(orc.rng_u64(42, 1000), orc.rng_u64(42, 1000))


def test_different_seeds_produce_different_output(orc):  # rng.rs:282-293
    assert int(np.sum(orc.rng_u64(42, 100) == orc.rng_u64(43, 100))) < 5


def test_range_u32_uniform(orc):  # rng.rs:295-315
    v = orc.rng_range_u32(42, 3, 30000)
    assert v.max() < 3
    counts = np.bincount(v, minlength=3)
    assert np.all(np.abs(counts - 10000) < 1500)


def test_range_u64_bounds(orc):  # rng.rs:317-325
    q = 1099511627777
    assert orc.rng_range_u64(42, q, 10000).max() < q


def test_gaussian_distribution_rng(orc):  # rng.rs:327-347
    s = orc.rng_gaussian(42, 3.19, 50000)
    assert abs(s.mean()) < 0.1
    assert abs(s.std() - 3.19) < 0.15


def test_next_f64_range(orc):  # rng.rs:349-357
    v = orc.rng_f64(42, 10000)
    assert v.min() > 0.0 and v.max() < 1.0


def test_from_entropy_produces_output(orc):  # rng.rs:359-367
    v = orc.rng_entropy_u64(2)
    assert v[0] != 0 or v[1] != 0


# ---------------- sampling.rs:66-150 ----------------
def test_ternary_distribution(orc):  # sampling.rs:72-104
    q, n = 97, 10000
    s = orc.sample_ternary(42, n, q)
    for val in (q - 1, 0, 1):
        assert abs(int(np.sum(s == val)) - n // 3) < 500
    assert set(np.unique(s).tolist()) <= {0, 1, q - 1}


def test_gaussian_distribution_sampling(orc):  # sampling.rs:106-140
    q, n = 1099511627777, 10000
    s = orc.sample_gaussian(42, n, q, 3.19).astype(object)
    signed = np.array([-(q - int(x)) if int(x) > q // 2 else int(x) for x in s], np.float64)
    assert abs(signed.mean()) < 0.2
    assert abs(signed.std() - 3.19) < 0.3


def test_uniform_range(orc):  # sampling.rs:142-149
    assert orc.sample_uniform(42, 1000, 97).max() < 97


# ---------------- encoding.rs:318-387 ----------------
def test_encode_decode_roundtrip(orc):  # encoding.rs:322-343
    ctx = orc.Context(8192)
    z = np.arange(10) * 0.1
    d = ctx.decode(ctx.encode(z), 2.0**40)
    assert np.all(np.abs(d[:10] - z) < 1e-5)


def test_encode_zeros(orc):  # encoding.rs:345-361
    ctx = orc.Context(8192)
    d = ctx.decode(ctx.encode(np.zeros(100)), 2.0**40)
    assert np.all(np.abs(d[:100]) < 1e-7)


def test_encode_large_values(orc):  # encoding.rs:363-386
    ctx = orc.Context(8192)
    z = (np.arange(50) - 25.0) * 100.0
    d = ctx.decode(ctx.encode(z), 2.0**40)[:50]
    err = np.abs(d - z)
    rel = np.where(np.abs(z) > 1e-10, err / np.maximum(np.abs(z), 1e-300), err)
    assert np.all((rel < 1e-5) | (err < 1e-5))


# ---------------- ciphertext.rs:548-798 ----------------
# The Rust tests draw consecutive encryptions from one TenSafeRng; here each
# encryption takes its own seed. The tolerance checks are unaffected.
@pytest.fixture(scope="module")
def ctx_sk(orc):  # ciphertext.rs:553-559
    ctx = orc.Context(8192)
    return ctx, ctx.keygen(42)


def test_encrypt_decrypt_roundtrip(orc, ctx_sk):  # ciphertext.rs:561-579
    ctx, sk = ctx_sk
    z = np.arange(10) * 0.5
    d = ctx.decrypt(ctx.encrypt(z, sk, 123), sk)
    assert np.all(np.abs(d[:10] - z) < 1e-4)


def test_ct_pt_multiply(orc, ctx_sk):  # ciphertext.rs:581-606
    ctx, sk = ctx_sk
    x = np.array([1.0, 2, 3, 4, 5])
    p = np.full(5, 0.5)
    d = ctx.decrypt(ctx.ct_pt_mul(ctx.encrypt(x, sk, 456), p), sk)
    assert np.all(np.abs(d[:5] - x * p) < 0.1)


def test_ct_pt_mul_with_cached_ntt(orc, ctx_sk):  # ciphertext.rs:608-633
    ctx, sk = ctx_sk
    x = np.arange(20) * 0.1
    p = 1.0 - np.arange(20) * 0.04
    pt = ctx.encode_to_ntt(p)
    d = ctx.decrypt(ctx.ct_pt_mul_ntt(ctx.encrypt(x, sk, 789), pt), sk)
    assert np.all(np.abs(d[:20] - x * p) < 0.1)


def test_crt_overflow_validation(orc, ctx_sk):  # ciphertext.rs:635-660
    ctx, sk = ctx_sk
    x = np.arange(50) * 10.0 - 250.0
    p = np.arange(50) * 5.0 - 125.0
    d = ctx.decrypt(ctx.ct_pt_mul(ctx.encrypt(x, sk, 999), p), sk)
    assert np.all(np.abs(d[:50] - x * p) < 10.0)


def test_ct_add(orc, ctx_sk):  # ciphertext.rs:662-685
    ctx, sk = ctx_sk
    a = np.arange(10) * 1.5
    b = 10.0 - np.arange(10) * 0.3
    d = ctx.decrypt(ctx.ct_add(ctx.encrypt(a, sk, 111), ctx.encrypt(b, sk, 112)), sk)
    assert np.all(np.abs(d[:10] - (a + b)) < 1e-4)


def test_ct_sub(orc, ctx_sk):  # ciphertext.rs:687-710
    ctx, sk = ctx_sk
    a = np.arange(10) * 2.0
    b = np.arange(10) * 0.5
    d = ctx.decrypt(ctx.ct_sub(ctx.encrypt(a, sk, 222), ctx.encrypt(b, sk, 223)), sk)
    assert np.all(np.abs(d[:10] - (a - b)) < 1e-4)


def test_pk_encrypt_decrypt_roundtrip(orc, ctx_sk):  # ciphertext.rs:712-731
    ctx, sk = ctx_sk
    pk = ctx.keygen_public(sk, 333)
    z = np.arange(10) * 0.5
    d = ctx.decrypt(ctx.encrypt_pk(z, pk, 334), sk)
    assert np.all(np.abs(d[:10] - z) < 1e-3)


def test_pk_encrypt_ct_pt_mul(orc, ctx_sk):  # ciphertext.rs:733-762
    ctx, sk = ctx_sk
    pk = ctx.keygen_public(sk, 444)
    h = np.array([1.0, 2, 3, 4, 5])
    w = np.full(5, 0.5)
    d = ctx.decrypt(ctx.ct_pt_mul(ctx.encrypt_pk(h, pk, 445), w), sk)
    assert np.all(np.abs(d[:5] - h * w) < 0.1)


def test_rescale(orc, ctx_sk):  # ciphertext.rs:764-797
    ctx, sk = ctx_sk
    x = np.array([1.0, 2, 3, 4, 5])
    p = np.full(5, 0.5)
    ct_mul = ctx.ct_pt_mul(ctx.encrypt(x, sk, 555), p)
    assert ct_mul.scale > 2.0**40 * 1.5
    assert ct_mul.num_limbs == 4
    r = ctx.rescale(ct_mul)
    assert r.num_limbs == 3
    d = ctx.decrypt(r, sk)
    assert np.all(np.abs(d[:5] - x * p) < 1.0)


# ---------------- serialize.rs:95-146 ----------------
def test_pk_serialize_roundtrip(orc, ctx_sk):  # serialize.rs:102-118
    ctx, sk = ctx_sk
    pk = ctx.keygen_public(sk, 42)
    pk2 = ctx.pk_from_bytes(ctx.pk_to_bytes(pk))
    for x, y in zip(ctx.pk_data(pk), ctx.pk_data(pk2)):
        assert np.array_equal(x, y)


def test_ct_serialize_roundtrip(orc, ctx_sk):  # serialize.rs:120-145
    ctx, sk = ctx_sk
    z = np.arange(10, dtype=np.float64)
    ct = ctx.encrypt(z, sk, 42)
    raw = ctx.ct_to_bytes(ct)
    assert len(raw) == 8 + 2 * 4 * 8192 * 8
    ct2 = ctx.ct_from_bytes(raw, 4)
    assert ct2.scale == ct.scale
    for x, y in zip(ctx.ct_data(ct), ctx.ct_data(ct2)):
        assert np.array_equal(x, y)
    d = ctx.decrypt(ct2, sk)
    assert np.all(np.abs(d[:10] - z) < 1e-4)
