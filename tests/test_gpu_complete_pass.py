"""The complete LoRA-set token (th_lora_deltas without TH_LORA_SK_FUSED).

It runs the reference's client/server sequence (inference_engine.py:1477-1482,
:1272-1315): encrypt_pk of each input from the public key alone, then ct x pt
and the rescale without the secret key, each forming every limb of its
ciphertext (ciphertext.rs:240-319, :422-429, :476-535), then one batched
decrypt that reads only what it decodes (ciphertext.rs:327-400).

The ciphertexts a token formed are copied out of the set (th_lora_ct) and
compared with the oracle's composed operations bit for bit: the encrypt_pk
output of each input, and every batch's product (rescaled or not). The
token's segment sums equal those of the sk-fused shortcut bit for bit (the
same residues on the limbs a decryption reads), and its deltas match the
oracle within the 1e-3 relative bound on decoded deltas.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import tensafe_he, zero_moai

pytestmark = pytest.mark.gpu

K = 3  # CryptoMOE experts per projection


@pytest.fixture(scope="module")
def env():
    eng, ref = tensafe_he.CkksContext(16384), orc.Context(16384)
    sk, rsk = eng.keygen(seed=61), ref.keygen(61)
    pk, rpk = eng.keygen_public(sk, seed=62), ref.keygen_public(rsk, 62)
    return eng, ref, sk, pk, rsk, rpk


def _same_ct(eng, ref, got, exp):
    assert got.num_limbs == exp.num_limbs
    assert got.scale == exp.scale
    return all(np.array_equal(x, y) for x, y in zip(eng.ct_download(got), ref.ct_data(exp)))


def _check_token(eng, ref, rpk, ls, H, seeds, proj, rescale, layers):
    """The set's last token: input ciphertexts and every product of `layers` bit-exact."""
    S = ref.num_slots
    d = H.shape[1]
    batch = 0
    first = {}
    for j, (i, A, _) in enumerate(proj):
        first[j] = batch
        batch += len(zero_moai.pack_rows(A, S))
    for i in layers:
        rct = ref.encrypt_pk(zero_moai.replicate(H[i], S, d), rpk, int(seeds[i]))
        assert _same_ct(eng, ref, ls.ciphertext("input", i), rct), f"input {i}"
        for j, (ii, A, _) in enumerate(proj):
            if ii != i:
                continue
            for b, p in enumerate(zero_moai.pack_rows(A, S)):
                r = ref.ct_pt_mul(rct, p)
                if rescale:
                    r = ref.rescale(r)
                assert _same_ct(eng, ref, ls.ciphertext("product", first[j] + b), r), f"projection {j} batch {b}"


@pytest.mark.parametrize("rescale", [True, False])
def test_complete_token_ciphertexts_bitexact(env, rescale):
    """Two layers x {q, v} at the Qwen2.5-1.5B shape: every input ciphertext and every product
    (4 limbs, or 3 after the rescale) equals the oracle's; segment sums equal the sk-fused
    shortcut's bit for bit."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(31)
    H = rng.normal(size=(2, 1536)) * 0.1
    proj = [(l, rng.normal(size=(16, 1536)) * 0.02, rng.normal(size=(o, 16)) * 0.02)
            for l in range(2) for o in (1536, 256)]
    ls = zero_moai.LoraSet(eng, 2, proj)
    seeds = [3101, 3102]
    got_f, sums_f = ls.deltas(pk, sk, H, seeds, rescale=rescale, with_intermediates=True, sk_fused=True)
    with pytest.raises(RuntimeError, match="SK_FUSED"):
        ls.ciphertext("input", 0)
    got, sums = ls.deltas(pk, sk, H, seeds, rescale=rescale, with_intermediates=True)
    assert np.array_equal(sums, sums_f)
    for g, f in zip(got, got_f):
        assert np.array_equal(g, f)
    _check_token(eng, ref, rpk, ls, H, seeds, proj, rescale, layers=(0, 1))
    # the deltas against the oracle's decryption of those ciphertexts
    S, cols = 8192, 5
    for j, (i, A, B) in enumerate(proj):
        rct = ref.encrypt_pk(zero_moai.replicate(H[i], S, 1536), rpk, seeds[i])
        inter = np.zeros(16)
        for b, p in enumerate(zero_moai.pack_rows(A, S)):
            r = ref.ct_pt_mul(rct, p)
            dec = ref.decrypt(ref.rescale(r) if rescale else r, rsk)
            n = min(cols, 16 - b * cols)
            inter[b * cols:b * cols + n] = [np.sum(dec[c * 1536:(c + 1) * 1536]) for c in range(n)]
        e = B @ inter
        assert np.linalg.norm(got[j] - e) <= 1e-3 * np.linalg.norm(e)


def test_complete_token_full_shape(env):
    """28 layers x {q, v} (224 products, one round of decrypt workgroups): layers 0 and 27's
    ciphertexts bit-exact after a device-resident token, sums equal to the host-I/O token's and
    to the sk-fused shortcut's."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(32)
    H = rng.normal(size=(28, 1536)) * 0.1
    proj = [(l, rng.normal(size=(16, 1536)) * 0.02, rng.normal(size=(o, 16)) * 0.02)
            for l in range(28) for o in (1536, 256)]
    ls = zero_moai.LoraSet(eng, 28, proj)
    seeds = list(range(300, 328))
    _, sums_f = ls.deltas(pk, sk, H, seeds, with_intermediates=True, sk_fused=True)
    got, sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    assert np.array_equal(sums, sums_f)
    _check_token(eng, ref, rpk, ls, H, seeds, proj, True, layers=(0, 27))


@pytest.mark.parametrize("n,chain,d", [(8192, None, 1536), (32768, "L8", 3584)])
def test_complete_token_other_rings(n, chain, d):
    """The complete token at N=8192 (the reference chain, 3 limbs) and at N=32768 on the 8-limb
    chain of the Qwen2.5-7B saturation shape (a rescale forms 7 limbs of each product): one layer
    x {q, v}, every input ciphertext and rescaled product equal to the oracle's, sums equal to
    the sk-fused shortcut's."""
    from provenloop_amd.params import CHAIN_N32768_L8

    moduli = CHAIN_N32768_L8 if chain == "L8" else None
    eng = tensafe_he.CkksContext(n) if moduli is None else tensafe_he.CkksContext(n, moduli=moduli)
    ref = orc.Context(n, moduli=moduli)
    sk, rsk = eng.keygen(seed=71), ref.keygen(71)
    pk, rpk = eng.keygen_public(sk, seed=72), ref.keygen_public(rsk, 72)
    rng = np.random.default_rng(33)
    H = rng.normal(size=(1, d)) * 0.1
    proj = [(0, rng.normal(size=(16, d)) * 0.02, rng.normal(size=(o, 16)) * 0.02) for o in (d, 128)]
    ls = zero_moai.LoraSet(eng, 1, proj)
    seeds = [3301]
    _, sums_f = ls.deltas(pk, sk, H, seeds, with_intermediates=True, sk_fused=True)
    _, sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    assert np.array_equal(sums, sums_f)
    _check_token(eng, ref, rpk, ls, H, seeds, proj, True, layers=(0,))


def test_complete_moe_products_are_ct_add_of_expert_products(env):
    """CryptoMOE set: each batch's rescaled product equals the oracle's k expert products
    (ct_pt_mul with g_x A_x rows), folded with ct_add and rescaled, bit for bit
    (ciphertext.rs:422-450, :476-535); after set_gates too."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(33)
    H = rng.normal(size=(1, 1536)) * 0.1
    proj = [(0, rng.normal(size=(K, 16, 1536)) * 0.02, rng.normal(size=(K, o, 16)) * 0.02) for o in (1536, 256)]
    gates = np.array([zero_moai.softmax_gate(40 + j, K) for j in range(2)])
    ls = zero_moai.LoraSet(eng, 1, proj, gates=gates)
    S = 8192
    for t, g in enumerate((gates, np.array([zero_moai.softmax_gate(90 + j, K) for j in range(2)]))):
        if t:
            ls.set_gates(g)
        seeds = [5000 + t]
        _, sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
        _, sums_f = ls.deltas(pk, sk, H, seeds, with_intermediates=True, sk_fused=True)
        assert np.array_equal(sums, sums_f)
        ls.deltas(pk, sk, H, seeds)  # the complete token's ciphertexts stay in the set
        rct = ref.encrypt_pk(zero_moai.replicate(H[0], S, 1536), rpk, seeds[0])
        assert _same_ct(eng, ref, ls.ciphertext("input", 0), rct)
        batch = 0
        for j, (_, A, _) in enumerate(proj):
            packs = [zero_moai.pack_rows(A[x], S) for x in range(K)]
            for b in range(len(packs[0])):
                acc = None
                for x in range(K):
                    prod = ref.ct_pt_mul(rct, g[j][x] * packs[x][b])
                    acc = prod if acc is None else ref.ct_add(acc, prod)
                assert _same_ct(eng, ref, ls.ciphertext("product", batch), ref.rescale(acc)), (t, j, b)
                batch += 1


def test_lora_ct_errors(env):
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(34)
    proj = [(0, rng.normal(size=(3, 1536)) * 0.02, rng.normal(size=(4, 3)) * 0.02)]
    ls = zero_moai.LoraSet(eng, 1, proj)
    with pytest.raises(RuntimeError, match="no token"):
        ls.ciphertext("input", 0)
    ls.deltas(pk, sk, rng.normal(size=(1, 1536)) * 0.1, [1])
    with pytest.raises(ValueError, match="out of range"):
        ls.ciphertext("input", 1)
    with pytest.raises(ValueError, match="out of range"):
        ls.ciphertext("product", ls.n_batches)
    assert ls.ciphertext("product", 0).num_limbs == 3
