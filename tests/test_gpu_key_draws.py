"""Key and secret-key-encryption randomness drawn on the device.

keygen (N x range_u32(3)), keygen_public (range_u64(q_l) on every limb, then
N Gaussians) and the secret-key encrypt (the same draws per input, one
stream across a batch_encrypt) come from the reference's seeded ChaCha20
stream (rng.rs:31-157, sampling.rs:17-64, ciphertext.rs:77-229) drawn on the
GPU; the keys and ciphertexts must equal the oracle's bit for bit.

Seed 3416's stream rejects a range_u64 word at limb 2 (q = 1099508121601,
coefficient 11051: its draws and every later one move by two words), so
keygen_public and batch_encrypt take the serial replay of that stretch and,
in the batch, draw the inputs after it in parallel from an offset that is
not a whole ChaCha20 block (the CPU test below pins the rejection on the
oracle's stream).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import tensafe_he

N = 16384
REJECT_SEED, REJECT_LIMB, REJECT_AT = 3416, 2, 11051


def test_rejection_seed_is_pinned_on_the_oracle_stream():
    q = orc.default_chain(N)
    v = orc.rng_u64(REJECT_SEED, 4 * N)
    thr = [((1 << 64) - x) % x for x in q]
    first = [(l, int(np.nonzero(v[l * N:(l + 1) * N] < np.uint64(thr[l]))[0][0]))
             for l in range(4) if np.any(v[l * N:(l + 1) * N] < np.uint64(thr[l]))]
    assert first[0] == (REJECT_LIMB, REJECT_AT)


@pytest.fixture(scope="module")
def env():
    return tensafe_he.CkksContext(N), orc.Context(N)


def _same_keys(eng, ref, sk, pk, rsk, rpk):
    assert np.array_equal(eng.sk_download(sk), ref.sk_data(rsk))
    b, a = eng.pk_download(pk)
    rb, ra = ref.pk_data(rpk)
    assert np.array_equal(a, ra) and np.array_equal(b, rb)


def _same_ct(eng, ref, ct, rct):
    assert ct.num_limbs == rct.num_limbs and ct.scale == rct.scale
    for x, y in zip(eng.ct_download(ct), ref.ct_data(rct)):
        assert np.array_equal(x, y)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [17, REJECT_SEED])
def test_keys_and_secret_key_encrypt_match_oracle(env, seed):
    eng, ref = env
    sk, rsk = eng.keygen(seed=seed), ref.keygen(seed)
    pk, rpk = eng.keygen_public(sk, seed=seed), ref.keygen_public(rsk, seed)
    _same_keys(eng, ref, sk, pk, rsk, rpk)
    z = np.random.default_rng(seed).normal(size=N // 2) * 0.1
    _same_ct(eng, ref, eng.encrypt(z, sk, seed=seed), ref.encrypt(z, rsk, seed))


@pytest.mark.gpu
def test_batch_encrypt_after_a_rejection_matches_oracle(env):
    """The first input's stretch holds the rejected word, so the three after it start two
    words later than their blocks: drawn in parallel from that offset."""
    eng, ref = env
    sk, rsk = eng.keygen(seed=5), ref.keygen(5)
    rng = np.random.default_rng(6)
    arrays = [rng.normal(size=N // 2) * 0.1, rng.normal(size=100) * 0.1, np.zeros(0), rng.normal(size=N) * 0.1]
    for c, rc in zip(eng.batch_encrypt(arrays, sk, seed=REJECT_SEED), ref.batch_encrypt(arrays, rsk, REJECT_SEED)):
        _same_ct(eng, ref, c, rc)


@pytest.mark.gpu
def test_forced_serial_key_draws_match_oracle(env):
    """Every stretch drawn by the serial replay kernel (ternary secret included)."""
    eng, ref = env
    eng._force_serial_sampler(True)
    try:
        sk, rsk = eng.keygen(seed=21), ref.keygen(21)
        pk, rpk = eng.keygen_public(sk, seed=22), ref.keygen_public(rsk, 22)
        arrays = [np.arange(7) * 0.25, np.ones(N // 2) * 0.01]
        cts = eng.batch_encrypt(arrays, sk, seed=23)
    finally:
        eng._force_serial_sampler(False)
    _same_keys(eng, ref, sk, pk, rsk, rpk)
    for c, rc in zip(cts, ref.batch_encrypt(arrays, rsk, 23)):
        _same_ct(eng, ref, c, rc)


@pytest.mark.gpu
def test_band_redraw_of_key_draws_matches_oracle(env):
    """A wide sampler band flags the Gaussian draws: keygen_public and the batch encrypt draw
    their randomness again on the host with glibc, with the same result."""
    eng, ref = env
    sk, rsk = eng.keygen(seed=31), ref.keygen(31)
    eng.set_sampler_band(-4)
    try:
        before = eng.redrawn_inputs()
        pk = eng.keygen_public(sk, seed=32)
        arrays = [np.arange(5) * 0.5, np.ones(3)]
        cts = eng.batch_encrypt(arrays, sk, seed=REJECT_SEED)
        assert eng.redrawn_inputs() - before == 3
    finally:
        eng.set_sampler_band(-36)
    _same_keys(eng, ref, sk, pk, rsk, ref.keygen_public(rsk, 32))
    for c, rc in zip(cts, ref.batch_encrypt(arrays, rsk, REJECT_SEED)):
        _same_ct(eng, ref, c, rc)


@pytest.mark.gpu
def test_unseeded_keys_decrypt(env):
    """Seeds from the OS (TenSafeRng::from_entropy): two keygens differ and still round-trip."""
    eng, _ = env
    sk1, sk2 = eng.keygen(), eng.keygen()
    assert not np.array_equal(eng.sk_download(sk1), eng.sk_download(sk2))
    z = np.random.default_rng(1).normal(size=64)
    pk = eng.keygen_public(sk1)
    dec = eng.decrypt(eng.encrypt_pk(z, pk), sk1)
    assert np.max(np.abs(dec[:64] - z)) < 1e-5
    dec2 = eng.decrypt(eng.encrypt(z, sk2), sk2)
    assert np.max(np.abs(dec2[:64] - z)) < 1e-5
