"""GPU parity below the top level and for the shared-stream batch encrypt.

The reference's element-wise ops run over the first operand's limbs
(RnsPoly::add/sub/hadamard_mul, rns.rs:217-254), so after a rescale (one limb
dropped, ciphertext.rs:476-535) a ciphertext can still be multiplied by a
full-chain plaintext (ct_pt_mul_ntt, ciphertext.rs:422-429) and added to a
ciphertext with more limbs. batch_encrypt draws every encryption from ONE
seeded stream in order (tensafe-he-python/src/lib.rs:230-258). All results
must equal the oracle's bit for bit; the serialised bytes of a reduced-level
ciphertext must equal the layout of serialize.rs:69-77 read independently.
"""
import struct

import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import tensafe_he

pytestmark = pytest.mark.gpu

N = 16384


@pytest.fixture(scope="module")
def env():
    eng, ref = tensafe_he.CkksContext(N), orc.Context(N)
    sk, rsk = eng.keygen(seed=31), ref.keygen(31)
    pk, rpk = eng.keygen_public(sk, seed=32), ref.keygen_public(rsk, 32)
    z = np.random.default_rng(33).normal(size=N // 2) * 0.1
    ct, rct = eng.encrypt_pk(z, pk, seed=34), ref.encrypt_pk(z, rpk, 34)
    p = np.random.default_rng(35).normal(size=N // 2) * 0.02
    r = eng.rescale(eng.ct_pt_mul(ct, p))
    rr = ref.rescale(ref.ct_pt_mul(rct, p))
    return eng, ref, sk, rsk, ct, rct, r, rr


def _same(eng, ref, ct, rct):
    c0, c1 = eng.ct_download(ct)
    r0, r1 = ref.ct_data(rct)
    assert ct.num_limbs == rct.num_limbs
    assert ct.scale == rct.scale
    assert np.array_equal(c0, r0) and np.array_equal(c1, r1)


def test_rescaled_operand_is_the_oracles(env):
    eng, ref, _, _, _, _, r, rr = env
    assert r.num_limbs == 3
    _same(eng, ref, r, rr)


def test_ct_pt_mul_of_rescaled_ciphertext(env):
    """ct x pt at 3 limbs with a 4-limb plaintext: uncached (encode inside) and cached."""
    eng, ref, sk, rsk, _, _, r, rr = env
    p2 = np.random.default_rng(36).normal(size=N // 2) * 0.5
    m, rm = eng.ct_pt_mul(r, p2), ref.ct_pt_mul(rr, p2)
    _same(eng, ref, m, rm)
    pt, rpt = eng.encode_to_ntt(p2), ref.encode_to_ntt(p2)
    m2, rm2 = eng.ct_pt_mul_ntt(r, pt), ref.ct_pt_mul_ntt(rr, rpt)
    _same(eng, ref, m2, rm2)
    # and on down the chain: rescale to 2 limbs, decrypt (CRT branch at scale^2/q)
    m3, rm3 = eng.rescale(m2), ref.rescale(rm2)
    _same(eng, ref, m3, rm3)
    assert np.array_equal(eng.decrypt(m3, sk), ref.decrypt(rm3, rsk))
    # the operator form (TenSafeCiphertext.__mul__, lib.rs:336-356) on the rescaled ciphertext
    _same(eng, ref, r * p2, rm)


def test_ct_pt_mul_batch_of_rescaled_ciphertexts(env):
    eng, ref, _, _, _, _, r, rr = env
    ps = [np.random.default_rng(40 + i).normal(size=N // 2) * 0.1 for i in range(3)]
    outs = eng.ct_pt_mul_ntt_batch([r] * 3, [eng.encode_to_ntt(p) for p in ps])
    for o, p in zip(outs, ps):
        _same(eng, ref, o, ref.ct_pt_mul_ntt(rr, ref.encode_to_ntt(p)))


def test_add_sub_first_operand_has_fewer_limbs(env):
    """a (3 limbs, rescaled) +- b (4 limbs, same scale): the result has a's limbs."""
    eng, ref, sk, rsk, ct, rct, r, rr = env
    c0, c1 = eng.ct_download(ct)
    b = eng.ct_upload(c0, c1, r.scale)  # a 4-limb ciphertext at the rescaled scale
    rb = ref.ct_from_data(c0, c1, rr.scale)
    for op in ("ct_add", "ct_sub"):
        o, ro = getattr(eng, op)(r, b), getattr(ref, op)(rr, rb)
        assert o.num_limbs == 3
        _same(eng, ref, o, ro)
    _same(eng, ref, r + b, ref.ct_add(rr, rb))
    _same(eng, ref, r - b, ref.ct_sub(rr, rb))


def test_add_sub_first_operand_has_more_limbs_is_refused(env):
    """The reference indexes the second operand's limbs past its end and panics."""
    eng, ref, _, _, ct, rct, r, rr = env
    c0, c1 = eng.ct_download(ct)
    b = eng.ct_upload(c0, c1, r.scale)
    rb = ref.ct_from_data(c0, c1, rr.scale)
    with pytest.raises(ValueError, match="fewer than"):
        eng.ct_add(b, r)
    with pytest.raises(ValueError, match="fewer than"):
        eng.ct_sub(b, r)
    with pytest.raises(orc.OracleError, match="out of bounds"):
        ref.ct_add(rb, rr)


def test_reduced_level_bytes_follow_the_wire_layout(env):
    eng, ref, _, _, _, _, r, rr = env
    buf = r.to_bytes()
    assert buf == ref.ct_to_bytes(rr)
    L = r.num_limbs
    assert len(buf) == 8 + 2 * L * N * 8
    assert struct.unpack_from("<d", buf, 0)[0] == r.scale
    c0, c1 = eng.ct_download(r)
    words = np.frombuffer(buf, dtype="<u8", offset=8)
    assert np.array_equal(words[: L * N].reshape(L, N), c0)
    assert np.array_equal(words[L * N:].reshape(L, N), c1)
    back = eng.ct_from_bytes(buf, L)
    _same(eng, ref, back, rr)


def test_batch_encrypt_shares_one_stream(env):
    eng, ref, sk, rsk, *_ = env
    rng = np.random.default_rng(50)
    arrays = [rng.normal(size=100) * 0.1, rng.normal(size=N // 2) * 0.1, np.zeros(0),
              rng.normal(size=N) * 0.1]  # short, full, empty, longer than the slots (truncated)
    cts = eng.batch_encrypt(arrays, sk, seed=51)
    rcts = ref.batch_encrypt(arrays, rsk, 51)
    assert len(cts) == len(rcts) == 4
    for c, rc in zip(cts, rcts):
        _same(eng, ref, c, rc)
    # the second encryption continues the stream: it differs from a fresh one with that seed
    fresh = eng.encrypt(arrays[1], sk, seed=51)
    assert not np.array_equal(eng.ct_download(fresh)[1], eng.ct_download(cts[1])[1])
    dec = eng.batch_decrypt(cts, sk)
    assert np.max(np.abs(dec[1] - arrays[1])) < 1e-6
