"""GPU parity: the HIP engine against the CPU oracle, bit for bit.

Every integer result (NTT outputs, keys, ciphertexts, products, rescaled
ciphertexts, serialised bytes) must equal the oracle's exactly; decrypted
slots come from an f64 decode evaluated in the reference's order with the
reference's twiddles, so they must be bit-identical too. The LoRA segment
sums are reduced in a different order than numpy's, so they are held to the
bound on decoded deltas ||gpu - cpu|| / ||cpu|| <= 1e-3 (in practice ~1e-15).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import tensafe_he

pytestmark = pytest.mark.gpu

Q16384 = [1152921504606748673, 1099510054913, 1099508121601, 1152921504606683137]


@pytest.fixture(scope="module")
def eng16():
    return tensafe_he.CkksContext(16384)


@pytest.fixture(scope="module")
def ref16():
    return orc.Context(16384)


@pytest.fixture(scope="module")
def keys16(eng16, ref16):
    sk = eng16.keygen(seed=11)
    pk = eng16.keygen_public(sk, seed=22)
    rsk = ref16.keygen(11)
    rpk = ref16.keygen_public(rsk, 22)
    return sk, pk, rsk, rpk


def _ct_equal(eng, ref, ct, rct):
    c0, c1 = eng.ct_download(ct)
    r0, r1 = ref.ct_data(rct)
    assert ct.num_limbs == rct.num_limbs
    assert ct.scale == rct.scale
    assert np.array_equal(c0, r0)
    assert np.array_equal(c1, r1)


# ------------------------------------------------------------------ NTT
@pytest.mark.parametrize("n", [1024, 2048, 4096, 8192, 16384])
def test_ntt_matches_oracle(n):
    ctx = tensafe_he.CkksContext(n, moduli=Q16384)
    rng = np.random.default_rng(n)
    x = np.stack([rng.integers(0, q, (3, n), dtype=np.uint64) for q in Q16384], axis=1)  # [3, 4, n]
    x[0, :, :4] = 0
    x[1, :, -4:] = np.array(Q16384, np.uint64)[:, None] - 1  # edge residues
    fwd = ctx.ntt_forward(x)
    for l, q in enumerate(Q16384):
        assert np.array_equal(fwd[:, l], orc.ntt_forward(x[:, l], q)), f"forward limb {l}"
    inv = ctx.ntt_inverse(fwd)
    assert np.array_equal(inv, x)
    inv2 = ctx.ntt_inverse(x)
    for l, q in enumerate(Q16384):
        assert np.array_equal(inv2[:, l], orc.ntt_inverse(x[:, l], q)), f"inverse limb {l}"


@pytest.mark.parametrize("n", [8192, 32768])
def test_ntt_default_chains(n):
    ctx = tensafe_he.CkksContext(n)
    q = orc.default_chain(n)
    rng = np.random.default_rng(1)
    x = np.stack([rng.integers(0, qq, (2, n), dtype=np.uint64) for qq in q], axis=1)
    fwd = ctx.ntt_forward(x)
    for l, qq in enumerate(q):
        assert np.array_equal(fwd[:, l], orc.ntt_forward(x[:, l], qq))
    assert np.array_equal(ctx.ntt_inverse(fwd), x)


@pytest.mark.parametrize("n,polys", [(8192, 72), (16384, 72)])
def test_ntt_large_batch_matches_oracle(n, polys):
    """More than 256 transforms per launch: the column + row pass kernels."""
    q = orc.default_chain(n)
    ctx = tensafe_he.CkksContext(n)
    rng = np.random.default_rng(n + polys)
    x = np.stack([rng.integers(0, qq, (polys, n), dtype=np.uint64) for qq in q], axis=1)
    x[5, :, :7] = 0
    x[6, :, -7:] = np.array(q, np.uint64)[:, None] - 1
    fwd = ctx.ntt_forward(x)
    for p in (0, 5, 6, polys - 1):
        for l, qq in enumerate(q):
            assert np.array_equal(fwd[p, l], orc.ntt_forward(x[p, l], qq)), f"forward poly {p} limb {l}"
    inv = ctx.ntt_inverse(x)
    for p in (0, 6, polys - 1):
        for l, qq in enumerate(q):
            assert np.array_equal(inv[p, l], orc.ntt_inverse(x[p, l], qq)), f"inverse poly {p} limb {l}"
    assert np.array_equal(ctx.ntt_inverse(fwd), x)


@pytest.mark.parametrize("n", [16384, 32768])
def test_ntt_batched_microbench_shape(n):
    """64 polynomials x 4 limbs (the batched round-trip workload) on the reference chain for N."""
    q = orc.default_chain(n)
    ctx = tensafe_he.CkksContext(n)
    rng = np.random.default_rng(7)
    x = np.stack([rng.integers(0, qq, (64, n), dtype=np.uint64) for qq in q], axis=1)
    fwd = ctx.ntt_forward(x)
    for p in (0, 31, 63):
        for l, qq in enumerate(q):
            assert np.array_equal(fwd[p, l], orc.ntt_forward(x[p, l], qq))
    assert np.array_equal(ctx.ntt_inverse(fwd), x)


# ------------------------------------------------------------------ keys and encryption
def test_keys_match_oracle(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    assert np.array_equal(eng16.sk_download(sk), ref16.sk_data(rsk))
    b, a = eng16.pk_download(pk)
    rb, ra = ref16.pk_data(rpk)
    assert np.array_equal(a, ra)
    assert np.array_equal(b, rb)


def test_encrypt_pk_seeded_matches_oracle(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    z = np.random.default_rng(3).normal(size=8192) * 0.1
    _ct_equal(eng16, ref16, eng16.encrypt_pk(z, pk, seed=5), ref16.encrypt_pk(z, rpk, 5))


def test_encrypt_pk_explicit_matches_oracle(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    z = np.random.default_rng(4).normal(size=1536) * 0.1
    u, e0, e1 = orc.encrypt_pk_randomness(1234, 16384)
    _ct_equal(eng16, ref16, eng16.encrypt_pk_explicit(z, pk, u, e0, e1), ref16.encrypt_pk_with(z, rpk, u, e0, e1))


def test_encrypt_pk_batch_matches_oracle(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    rng = np.random.default_rng(5)
    zs = [rng.normal(size=7680) * 0.1 for _ in range(5)]
    cts = eng16.encrypt_pk_batch(zs, pk, [100 + i for i in range(5)])
    for i in (0, 4):
        _ct_equal(eng16, ref16, cts[i], ref16.encrypt_pk(zs[i], rpk, 100 + i))


@pytest.mark.parametrize("sampler", ["device", "host", "device-serial"])
def test_samplers_match_oracle(eng16, ref16, keys16, sampler):
    """Seeded encrypt_pk through each randomness path equals the oracle's, seed by seed."""
    sk, pk, rsk, rpk = keys16
    rng = np.random.default_rng(17)
    eng16.set_sampler("host" if sampler == "host" else "device")
    eng16._force_serial_sampler(sampler == "device-serial")
    try:
        seeds = [0, 1, 2**32 - 1, 2**32, 2**63 + 12345, 2**64 - 1] + [int(v) for v in rng.integers(0, 2**62, 6)]
        if sampler == "device-serial":
            seeds = seeds[:3]
        zs = [rng.normal(size=8192) * 0.1 for _ in seeds]
        cts = eng16.encrypt_pk_batch(zs, pk, seeds)
        for ct, z, sd in zip(cts, zs, seeds):
            _ct_equal(eng16, ref16, ct, ref16.encrypt_pk(z, rpk, sd))
    finally:
        eng16.set_sampler("device")
        eng16._force_serial_sampler(False)


def test_device_sampler_many_seeds(eng16, ref16, keys16):
    """112 device-sampled encryptions (3.7M Gaussian draws) against the oracle."""
    sk, pk, rsk, rpk = keys16
    z = np.zeros(8192)
    seeds = list(range(1000, 1112))
    cts = eng16.encrypt_pk_batch([z] * len(seeds), pk, seeds)
    for ct, sd in zip(cts, seeds):
        _ct_equal(eng16, ref16, ct, ref16.encrypt_pk(z, rpk, sd))


def test_encode_extremes_match_oracle(eng16, ref16):
    for z in (np.zeros(8192), np.full(8192, 1e6), np.linspace(-3e3, 3e3, 8192), np.full(3, 5e12),
              np.array([np.pi, -np.e, 1e-12, -1e-12])):
        assert np.array_equal(eng16.pt_download(eng16.encode_to_ntt(z)), ref16.poly_data(ref16.encode_to_ntt(z)))


def test_secret_key_encrypt_matches_oracle(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    z = np.arange(10) * 0.5
    _ct_equal(eng16, ref16, eng16.encrypt(z, sk, seed=123), ref16.encrypt(z, rsk, 123))


def test_input_padding_and_truncation(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    long = np.random.default_rng(6).normal(size=9000)  # lib.rs:124-126 truncates to N/2
    _ct_equal(eng16, ref16, eng16.encrypt_pk(long, pk, seed=9), ref16.encrypt_pk(long[:8192], rpk, 9))
    empty = np.zeros(0)
    _ct_equal(eng16, ref16, eng16.encrypt_pk(empty, pk, seed=10), ref16.encrypt_pk(empty, rpk, 10))


# ------------------------------------------------------------------ products, add, rescale
@pytest.fixture(scope="module")
def base_ct(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    h = np.random.default_rng(8).normal(size=1536) * 0.1
    rep = np.zeros(8192)
    for i in range(5):
        rep[i * 1536:(i + 1) * 1536] = h
    return eng16.encrypt_pk(rep, pk, seed=77), ref16.encrypt_pk(rep, rpk, 77), h


def _packed_rows(A, b, slots=8192, d=1536, cols=5):
    pt = np.zeros(slots)
    for i, r in enumerate(range(b * cols, min((b + 1) * cols, A.shape[0]))):
        pt[i * d:(i + 1) * d] = A[r]
    return pt


def test_ct_pt_mul_matches_oracle(eng16, ref16, base_ct):
    ct, rct, _ = base_ct
    A = np.random.default_rng(9).normal(size=(16, 1536)) * 0.02
    p = _packed_rows(A, 0)
    _ct_equal(eng16, ref16, eng16.ct_pt_mul(ct, p), ref16.ct_pt_mul(rct, p))
    _ct_equal(eng16, ref16, ct * p, ref16.ct_pt_mul(rct, p))
    pt = eng16.encode_to_ntt(p)
    assert np.array_equal(eng16.pt_download(pt), ref16.poly_data(ref16.encode_to_ntt(p)))
    outs = eng16.ct_pt_mul_ntt_batch([ct, ct], [pt, pt])
    _ct_equal(eng16, ref16, outs[1], ref16.ct_pt_mul(rct, p))


def test_add_sub_match_oracle(eng16, ref16, keys16):
    sk, pk, rsk, rpk = keys16
    a = np.arange(10) * 1.5
    b = 10.0 - np.arange(10) * 0.3
    ca, cb = eng16.encrypt_pk(a, pk, seed=1), eng16.encrypt_pk(b, pk, seed=2)
    ra, rb = ref16.encrypt_pk(a, rpk, 1), ref16.encrypt_pk(b, rpk, 2)
    _ct_equal(eng16, ref16, eng16.ct_add(ca, cb), ref16.ct_add(ra, rb))
    _ct_equal(eng16, ref16, ca - cb, ref16.ct_sub(ra, rb))
    sq = eng16.ct_pt_mul(ca, np.ones(4))
    with pytest.raises(ValueError, match="Scale mismatch in ct_add"):
        eng16.ct_add(ca, sq)


def test_rescale_chain_matches_oracle(eng16, ref16, base_ct):
    ct, rct, _ = base_ct
    p = np.full(100, 0.25)
    cur, rcur = eng16.ct_pt_mul(ct, p), ref16.ct_pt_mul(rct, p)
    for limbs in (3, 2, 1):
        cur, rcur = eng16.rescale(cur), ref16.rescale(rcur)
        assert cur.num_limbs == limbs
        _ct_equal(eng16, ref16, cur, rcur)
    with pytest.raises(RuntimeError, match="only 1 limb left"):
        eng16.rescale(cur)


def test_rescale_batch_matches_oracle(eng16, ref16, base_ct):
    ct, rct, _ = base_ct
    A = np.random.default_rng(10).normal(size=(16, 1536)) * 0.02
    pts = [_packed_rows(A, b) for b in range(4)]
    prods = eng16.ct_pt_mul_ntt_batch([ct] * 4, [eng16.encode_to_ntt(p) for p in pts])
    res = eng16.rescale_batch(prods)
    for b in (0, 3):
        _ct_equal(eng16, ref16, res[b], ref16.rescale(ref16.ct_pt_mul(rct, pts[b])))


@pytest.mark.parametrize("count", [48, 130])
def test_rescale_large_batch_matches_oracle(eng16, ref16, base_ct, count):
    """Batches whose forward transforms take the split kernels: the inverse column
    pass and the forward column passes run as one fused kernel."""
    ct, rct, _ = base_ct
    rng = np.random.default_rng(count)
    ps = [rng.normal(size=8192) * 0.02 for _ in range(3)]
    pts = [eng16.encode_to_ntt(p) for p in ps]
    prods = eng16.ct_pt_mul_ntt_batch([ct] * count, [pts[i % 3] for i in range(count)])
    res = eng16.rescale_batch(prods)
    for i in (0, 1, 2, count - 1):
        _ct_equal(eng16, ref16, res[i], ref16.rescale(ref16.ct_pt_mul(rct, ps[i % 3])))


def test_rescale_batch_n32768_eight_limbs():
    """The fused rescale kernels at N=32768 on the 8-limb chain (7 forward transforms per inverse)."""
    from provenloop_amd.params import CHAIN_N32768_L8

    eng, ref = tensafe_he.CkksContext(32768, moduli=CHAIN_N32768_L8), orc.Context(32768, CHAIN_N32768_L8)
    sk, rsk = eng.keygen(seed=5), ref.keygen(5)
    pk, rpk = eng.keygen_public(sk, seed=6), ref.keygen_public(rsk, 6)
    z = np.random.default_rng(7).normal(size=16384) * 0.1
    ct, rct = eng.encrypt_pk(z, pk, seed=8), ref.encrypt_pk(z, rpk, 8)
    ps = [np.random.default_rng(9 + i).normal(size=16384) * 0.02 for i in range(2)]
    pts = [eng.encode_to_ntt(p) for p in ps]
    prods = eng.ct_pt_mul_ntt_batch([ct] * 6, [pts[i % 2] for i in range(6)])
    res = eng.rescale_batch(prods)
    for i in (0, 5):
        _ct_equal(eng, ref, res[i], ref.rescale(ref.ct_pt_mul(rct, ps[i % 2])))


# ------------------------------------------------------------------ decryption
def test_decrypt_bit_exact_both_branches(eng16, ref16, keys16, base_ct):
    sk, pk, rsk, rpk = keys16
    ct, rct, _ = base_ct
    assert np.array_equal(eng16.decrypt(ct, sk), ref16.decrypt(rct, rsk))  # limb-0 branch, scale 2^40
    p = np.random.default_rng(11).normal(size=8192) * 0.02
    prod, rprod = eng16.ct_pt_mul(ct, p), ref16.ct_pt_mul(rct, p)
    assert prod.scale > 1.5 * 2.0**40
    assert np.array_equal(eng16.decrypt(prod, sk), ref16.decrypt(rprod, rsk))  # CRT branch
    r, rr = eng16.rescale(prod), ref16.rescale(rprod)
    assert np.array_equal(eng16.decrypt(r, sk), ref16.decrypt(rr, rsk))  # scale 2^20 after rescale


def test_batch_decrypt_and_segment_sums(eng16, ref16, keys16, base_ct):
    sk, pk, rsk, rpk = keys16
    ct, rct, h = base_ct
    A = np.random.default_rng(12).normal(size=(16, 1536)) * 0.02
    pts = [_packed_rows(A, b) for b in range(4)]
    res = eng16.rescale_batch(eng16.ct_pt_mul_ntt_batch([ct] * 4, [eng16.encode_to_ntt(p) for p in pts]))
    full = eng16.batch_decrypt(res, sk)
    ref = [ref16.decrypt(ref16.rescale(ref16.ct_pt_mul(rct, p)), rsk) for p in pts]
    for b in range(4):
        assert np.array_equal(full[b], ref[b])
    seg = eng16.batch_decrypt_segsum(res, sk, 1536, 5)
    ref_seg = np.array([[np.sum(r[i * 1536:(i + 1) * 1536]) for i in range(5)] for r in ref])
    assert np.linalg.norm(seg - ref_seg) / np.linalg.norm(ref_seg) <= 1e-3
    assert np.max(np.abs(seg - ref_seg)) < 1e-9


def test_single_delta_config(eng16, ref16, keys16):
    """encrypt_pk -> 4 x (ct x pt -> rescale -> decrypt) -> 16 segment sums (the single-delta workload)."""
    sk, pk, rsk, rpk = keys16
    rng = np.random.default_rng(2024)
    h = (rng.normal(size=1536) * 0.1).astype(np.float32).astype(np.float64)
    A = (rng.normal(size=(16, 1536)) * 0.02).astype(np.float32).astype(np.float64)
    rep = np.zeros(8192)
    for i in range(5):
        rep[i * 1536:(i + 1) * 1536] = h
    ct = eng16.encrypt_pk(rep, pk, seed=31)
    pts = [eng16.encode_to_ntt(_packed_rows(A, b)) for b in range(4)]
    res = eng16.rescale_batch(eng16.ct_pt_mul_ntt_batch([ct] * 4, pts))
    seg = eng16.batch_decrypt_segsum(res, sk, 1536, 5)
    gpu = np.concatenate([seg[b, :5] for b in range(3)] + [seg[3, :1]])
    rct = ref16.encrypt_pk(rep, rpk, 31)
    cpu = []
    for b in range(4):
        dec = ref16.decrypt(ref16.rescale(ref16.ct_pt_mul(rct, _packed_rows(A, b))), rsk)
        cols = 5 if b < 3 else 1
        cpu += [np.sum(dec[i * 1536:(i + 1) * 1536]) for i in range(cols)]
    cpu = np.array(cpu)
    assert gpu.shape == (16,)
    assert np.linalg.norm(gpu - cpu) / np.linalg.norm(cpu) <= 1e-3


def test_lora_a_pass_matches_composed_ops(eng16, ref16, keys16):
    """th_lora_a_pass == encrypt_pk -> ct x pt -> (rescale) -> decrypt -> segment sums, both branches."""
    sk, pk, rsk, rpk = keys16
    rng = np.random.default_rng(33)
    H = rng.normal(size=(3, 1536)) * 0.1
    A = rng.normal(size=(16, 1536)) * 0.02
    pts_f = [_packed_rows(A, b) for b in range(4)]
    pts = [eng16.encode_to_ntt(p) for p in pts_f]
    pin = [0, 0, 1, 2, 2, 2]
    use = [0, 1, 2, 3, 0, 1]
    seeds = [501, 502, 503]
    for rescale in (True, False):
        got = eng16.lora_a_pass(pk, sk, H, seeds, [pts[u] for u in use], pin, rescale=rescale)
        assert got.shape == (6, 5)
        rcts = [ref16.encrypt_pk(_packed_rows(np.tile(h, (5, 1)), 0), rpk, sd) for h, sd in zip(H, seeds)]
        for row, (i, u) in enumerate(zip(pin, use)):
            r = ref16.ct_pt_mul(rcts[i], pts_f[u])
            if rescale:
                r = ref16.rescale(r)
            dec = ref16.decrypt(r, rsk)
            exp = np.array([np.sum(dec[c * 1536:(c + 1) * 1536]) for c in range(5)])
            assert np.max(np.abs(got[row] - exp)) <= 1e-9 * max(1.0, np.max(np.abs(exp)))


# ------------------------------------------------------------------ wire format
def test_serialization_matches_oracle_bytes(eng16, ref16, keys16, base_ct):
    sk, pk, rsk, rpk = keys16
    ct, rct, _ = base_ct
    raw = ct.to_bytes()
    assert raw == ref16.ct_to_bytes(rct)
    back = eng16.ct_from_bytes(raw)
    _ct_equal(eng16, ref16, back, rct)
    assert pk.to_bytes() == ref16.pk_to_bytes(rpk)
    pk2 = eng16.pk_from_bytes(pk.to_bytes())
    assert [np.array_equal(x, y) for x, y in zip(eng16.pk_download(pk2), ref16.pk_data(rpk))] == [True, True]
    with pytest.raises(ValueError, match="bytes for Ciphertext"):
        eng16.ct_from_bytes(raw[:-8])


def test_other_degrees_roundtrip():
    for n in (8192, 32768):
        eng, ref = tensafe_he.CkksContext(n), orc.Context(n)
        sk, rsk = eng.keygen(seed=5), ref.keygen(5)
        pk, rpk = eng.keygen_public(sk, seed=6), ref.keygen_public(rsk, 6)
        z = np.arange(20) * 0.1
        ct, rct = eng.encrypt_pk(z, pk, seed=7), ref.encrypt_pk(z, rpk, 7)
        _ct_equal(eng, ref, ct, rct)
        r, rr = eng.rescale(eng.ct_pt_mul(ct, np.full(20, 0.5))), ref.rescale(ref.ct_pt_mul(rct, np.full(20, 0.5)))
        _ct_equal(eng, ref, r, rr)
        assert np.array_equal(eng.decrypt(r, sk), ref.decrypt(rr, rsk))
