"""Saturation workload pieces at Qwen2.5-7B shape on the 8-limb N = 32768
chain: NTT, encrypt_pk, ct x pt, rescale and decrypt bit-exact against the
oracle on that chain, and LoRA sets (q, k, v, o at rank 32, hidden 3584)
serving several sessions, each with its own keys, on one context.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import _lib, tensafe_he, zero_moai
from provenloop_amd.params import CHAIN_N32768_L8

pytestmark = pytest.mark.gpu

N, D, RANK = 32768, 3584, 32
D_OUT = {"q": 3584, "k": 512, "v": 512, "o": 3584}


@pytest.fixture(scope="module")
def ctxs():
    return tensafe_he.CkksContext(N, moduli=CHAIN_N32768_L8), orc.Context(N, CHAIN_N32768_L8)


def test_chain8_ntt_matches_oracle(ctxs):
    eng, _ = ctxs
    assert eng.moduli == CHAIN_N32768_L8
    rng = np.random.default_rng(3)
    x = np.stack([rng.integers(0, q, (3, N), dtype=np.uint64) for q in CHAIN_N32768_L8], axis=1)
    x[1, :, -3:] = np.array(CHAIN_N32768_L8, np.uint64)[:, None] - 1
    fwd = eng.ntt_forward(x)
    for l, q in enumerate(CHAIN_N32768_L8):
        assert np.array_equal(fwd[:, l], orc.ntt_forward(x[:, l], q)), f"limb {l}"
    assert np.array_equal(eng.ntt_inverse(fwd), x)


def test_chain8_ciphertext_ops_bitexact(ctxs):
    eng, ref = ctxs
    sk, rsk = eng.keygen(seed=1), ref.keygen(1)
    pk, rpk = eng.keygen_public(sk, seed=2), ref.keygen_public(rsk, 2)
    assert np.array_equal(eng.sk_download(sk), ref.sk_data(rsk))
    rng = np.random.default_rng(4)
    z = zero_moai.replicate(rng.normal(size=D) * 0.1, N // 2, D)
    p = zero_moai.pack_rows(rng.normal(size=(4, D)) * 0.02, N // 2)[0]
    ct, rct = eng.encrypt_pk(z, pk, seed=3), ref.encrypt_pk(z, rpk, 3)
    prod, rprod = eng.ct_pt_mul(ct, p), ref.ct_pt_mul(rct, p)
    res, rres = eng.rescale(prod), ref.rescale(rprod)
    for a, b in ((ct, rct), (prod, rprod), (res, rres)):
        assert a.num_limbs == b.num_limbs and a.scale == b.scale
        for x, y in zip(eng.ct_download(a), ref.ct_data(b)):
            assert np.array_equal(x, y)
    assert res.num_limbs == 7
    # decrypt of the full-limb product (CRT branch) and of the rescaled one (limb-0 branch)
    assert np.array_equal(eng.decrypt(prod, sk), ref.decrypt(rprod, rsk))
    assert np.array_equal(eng.decrypt(res, sk), ref.decrypt(rres, rsk))


def _layer_projections(rng, layers):
    proj = []
    for l in range(layers):
        for name in "qkvo":
            inp = 2 * l + (1 if name == "o" else 0)  # q, k, v share the layer input; o has its own
            proj.append((inp, rng.normal(size=(RANK, D)) * 0.02, rng.normal(size=(D_OUT[name], RANK)) * 0.02))
    return proj


def _oracle_deltas(ref, rpk, rsk, H, seeds, proj):
    S = N // 2
    cols = S // D
    cts = [ref.encrypt_pk(zero_moai.replicate(h, S, D), rpk, int(s)) for h, s in zip(H, seeds)]
    out = []
    for i, A, B in proj:
        inter = np.zeros(RANK)
        for b, p in enumerate(zero_moai.pack_rows(A, S)):
            dec = ref.decrypt(ref.rescale(ref.ct_pt_mul(cts[i], p)), rsk)
            seg = [np.sum(dec[c * D:(c + 1) * D]) for c in range(cols)]
            n = min(cols, RANK - b * cols)
            inter[b * cols:b * cols + n] = seg[:n]
        out.append(B @ inter)
    return out


@pytest.mark.usefixtures("lora_mode")
def test_saturation_sessions_match_oracle(ctxs):
    """One layer of q/k/v/o (rank 32: 8 batches of 4 rows each) for two sessions with their own
    keys, hidden states and seeds, served by one LoRA set."""
    eng, ref = ctxs
    rng = np.random.default_rng(5)
    proj = _layer_projections(rng, 1)
    ls = zero_moai.LoraSet(eng, 2, proj)
    assert (ls.cols, ls.n_batches) == (4, 32)
    for s in range(2):
        sk, rsk = eng.keygen(seed=100 + s), ref.keygen(100 + s)
        pk, rpk = eng.keygen_public(sk, seed=200 + s), ref.keygen_public(rsk, 200 + s)
        H = rng.normal(size=(2, D)) * 0.1
        seeds = [300 + 2 * s, 301 + 2 * s]
        got = ls.deltas(pk, sk, H, seeds)
        exp = _oracle_deltas(ref, rpk, rsk, H, seeds, proj)
        for g, e in zip(got, exp):
            assert g.shape == e.shape
            assert np.linalg.norm(g - e) <= 1e-3 * np.linalg.norm(e)


@pytest.mark.usefixtures("lora_mode")
def test_saturation_full_layer_count(ctxs):
    """All 28 layers (56 inputs, 112 projections, 896 products of 8 limbs) in one set serving two
    sessions (own keys, hidden states and seeds) queued back to back with device-resident inputs
    and outputs and one synchronisation: each session's layer-27 q and o projections against the
    oracle, and the second session's host-I/O run equal to its device-resident one."""
    eng, ref = ctxs
    lib = _lib.load()
    rng = np.random.default_rng(6)
    proj = _layer_projections(rng, 28)
    ls = zero_moai.LoraSet(eng, 56, proj)
    assert ls.n_batches == 896
    sess = []
    for s in range(2):
        sk, rsk = eng.keygen(seed=7 + 10 * s), ref.keygen(7 + 10 * s)
        pk, rpk = eng.keygen_public(sk, seed=8 + 10 * s), ref.keygen_public(rsk, 8 + 10 * s)
        H = np.ascontiguousarray(rng.normal(size=(56, D)) * 0.1)
        sess.append((sk, pk, rsk, rpk, H, list(range(500 + 100 * s, 556 + 100 * s))))
    bufs = []
    try:
        for sk, pk, _, _, H, seeds in sess:
            hd, od = C.c_void_p(), C.c_void_p()
            _lib.check(lib.th_dev_alloc(eng._h, H.nbytes, C.byref(hd)))
            bufs.append(hd)
            _lib.check(lib.th_dev_alloc(eng._h, ls.n_deltas * 8, C.byref(od)))
            bufs.append(od)
            _lib.check(lib.th_memcpy_h2d(eng._h, hd, _lib.ptr(H), H.nbytes))
        eng.sync()
        for s, (sk, pk, _, _, H, seeds) in enumerate(sess):
            ls.deltas_device(pk, sk, bufs[2 * s].value, seeds, bufs[2 * s + 1].value)
        eng.sync()
        outs = []
        for s in range(2):
            out = np.empty(ls.n_deltas)
            _lib.check(lib.th_memcpy_d2h(eng._h, _lib.ptr(out), bufs[2 * s + 1], ls.n_deltas * 8))
            outs.append(out)
    finally:
        for b in bufs:
            _lib.check(lib.th_dev_free(eng._h, b))
    last = [(0 if i == 54 else 1, A, B) for i, A, B in (proj[108], proj[111])]
    for s, (sk, pk, rsk, rpk, H, seeds) in enumerate(sess):
        exp = _oracle_deltas(ref, rpk, rsk, H[54:56], seeds[54:56], last)
        for j, e in zip((108, 111), exp):
            g = outs[s][ls.offsets[j]:ls.offsets[j + 1]]
            assert np.linalg.norm(g - e) <= 1e-3 * np.linalg.norm(e), (s, j)
    sk, pk, _, _, H, seeds = sess[1]
    assert np.array_equal(np.concatenate(ls.deltas(pk, sk, H, seeds)), outs[1])
