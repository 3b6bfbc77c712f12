"""CryptoMOE LoRA sets (th_lora_create_moe) against the oracle.

The oracle side runs the combination literally with the reference
operations: for each packed batch, one ct_pt_mul per expert with its
gate-scaled rows g_x A_x, the products folded with ct_add, then rescale,
decrypt and the d-slot segment sums; deltas = (sum_x g_x B_x) @ intermediate.
The engine folds the experts' plaintexts into one per batch; the test shows
that this gives the ct_add of the products bit for bit, and that the set's
segment sums are those of that very ciphertext.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import tensafe_he, zero_moai

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("lora_mode")]

K = 3  # experts per projection


@pytest.fixture(scope="module")
def env():
    eng, ref = tensafe_he.CkksContext(16384), orc.Context(16384)
    sk, rsk = eng.keygen(seed=51), ref.keygen(51)
    pk, rpk = eng.keygen_public(sk, seed=52), ref.keygen_public(rsk, 52)
    return eng, ref, sk, pk, rsk, rpk


def _experts(rng, n_layers, d=1536, rank=16, d_outs=(1536, 256)):
    proj, gates = [], []
    for l in range(n_layers):
        for j, o in enumerate(d_outs):
            proj.append((l, rng.normal(size=(K, rank, d)) * 0.02, rng.normal(size=(K, o, rank)) * 0.02))
            gates.append(zero_moai.softmax_gate(1000 * l + j, K))
    return proj, np.array(gates)


def _oracle(ref, rpk, rsk, H, seeds, proj, gates):
    S = ref.num_slots
    d = H.shape[1]
    cols = S // d
    cts = [ref.encrypt_pk(zero_moai.replicate(h, S, d), rpk, int(sd)) for h, sd in zip(H, seeds)]
    deltas, sums = [], []
    for (i, A, B), g in zip(proj, gates):
        rank = A.shape[1]
        packs = [zero_moai.pack_rows(A[x], S) for x in range(K)]
        inter = np.zeros(rank)
        for b in range(len(packs[0])):
            acc = None
            for x in range(K):
                prod = ref.ct_pt_mul(cts[i], g[x] * packs[x][b])
                acc = prod if acc is None else ref.ct_add(acc, prod)
            dec = ref.decrypt(ref.rescale(acc), rsk)
            seg = np.array([np.sum(dec[c * d:(c + 1) * d]) for c in range(cols)])
            sums.append(seg)
            n = min(cols, rank - b * cols)
            inter[b * cols:b * cols + n] = seg[:n]
        bmix = sum(g[x] * B[x] for x in range(K))
        deltas.append(bmix @ inter)
    return deltas, np.array(sums)


def test_moe_set_matches_oracle(env):
    """Two layers x {q, v} at the Qwen2.5-1.5B shape with 3 rank-16 experts per projection."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(21)
    H = rng.normal(size=(2, 1536)) * 0.1
    proj, gates = _experts(rng, 2)
    ls = zero_moai.LoraSet(eng, 2, proj, gates=gates)
    assert (ls.n_experts, ls.n_batches, ls.cols) == (K, 16, 5)
    seeds = [71, 72]
    got, got_sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, gates)
    assert np.max(np.abs(got_sums - exp_sums)) <= 1e-9 * max(1.0, np.max(np.abs(exp_sums)))
    for g, e in zip(got, exp):
        assert np.linalg.norm(g - e) <= 1e-3 * np.linalg.norm(e)


def test_moe_fold_is_ct_add_of_products(env):
    """Engine primitives: k products + ct_add + rescale equal the oracle's bit for bit, and
    the set's segment sums are the segment sums of exactly that ciphertext."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(22)
    H = rng.normal(size=(1, 1536)) * 0.1
    proj, gates = _experts(rng, 1, d_outs=(64,))
    (_, A, _), g = proj[0], gates[0]
    S = eng.num_slots
    rep = zero_moai.replicate(H[0], S, 1536)
    ct = eng.encrypt_pk_batch([rep], pk, [81])[0]
    rct = ref.encrypt_pk(rep, rpk, 81)
    acc = racc = None
    for x in range(K):
        p = g[x] * zero_moai.pack_rows(A[x], S)[0]
        prod = eng.ct_pt_mul_ntt(ct, eng.encode_to_ntt(p))
        rprod = ref.ct_pt_mul(rct, p)
        acc = prod if acc is None else eng.ct_add(acc, prod)
        racc = rprod if racc is None else ref.ct_add(racc, rprod)
    res, rres = eng.rescale(acc), ref.rescale(racc)
    for a, b in zip(eng.ct_download(res), ref.ct_data(rres)):
        assert np.array_equal(a, b)
    assert res.scale == rres.scale
    ls = zero_moai.LoraSet(eng, 1, proj, gates=gates)
    _, sums = ls.deltas(pk, sk, H, [81], with_intermediates=True)
    direct = eng.batch_decrypt_segsum([res], sk, 1536, 5)
    assert np.array_equal(sums[0], direct[0])


def test_moe_single_gate_scales(env):
    """One expert with weight g: the same as a plain set whose A and B are scaled by g."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(23)
    H = rng.normal(size=(1, 1536)) * 0.1
    A, B = rng.normal(size=(16, 1536)) * 0.02, rng.normal(size=(32, 16)) * 0.02
    g = 0.375  # a power-of-two fraction: g * x is exact, so both sets encode the same values
    moe = zero_moai.LoraSet(eng, 1, [(0, A[None], B[None])], gates=[[g]])
    plain = zero_moai.LoraSet(eng, 1, [(0, g * A, g * B)])
    a, sa = moe.deltas(pk, sk, H, [5], with_intermediates=True)
    b, sb = plain.deltas(pk, sk, H, [5], with_intermediates=True)
    assert np.array_equal(sa, sb)
    assert np.array_equal(a[0], b[0])


def test_moe_argument_errors(env):
    eng = env[0]
    rng = np.random.default_rng(24)
    proj, gates = _experts(rng, 1, d_outs=(8,))
    with pytest.raises(ValueError):
        zero_moai.LoraSet(eng, 1, proj, gates=gates[:, :2])  # gates for 2 experts, matrices for 3
    bad = gates.copy()
    bad[0, 1] = np.nan
    with pytest.raises(ValueError, match="finite"):
        zero_moai.LoraSet(eng, 1, proj, gates=bad)
    with pytest.raises(ValueError):
        zero_moai.LoraSet(eng, 1, [(0, proj[0][1][0], proj[0][2][0])], gates=gates)  # 2-D A with gates


def test_moe_set_gates_equals_set_created_with_them(env):
    """A gate that changes per token (th_lora_set_gates): after regating, the set's deltas and
    segment sums equal, bit for bit, those of a set created with the new gates, and the old
    gates come back exactly."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(25)
    H = rng.normal(size=(2, 1536)) * 0.1
    proj, g1 = _experts(rng, 2)
    g2 = np.array([zero_moai.softmax_gate(777 + j, K) for j in range(len(proj))])
    ls = zero_moai.LoraSet(eng, 2, proj, gates=g1)
    a1, s1 = ls.deltas(pk, sk, H, [91, 92], with_intermediates=True)
    ls.set_gates(g2)
    a2, s2 = ls.deltas(pk, sk, H, [91, 92], with_intermediates=True)
    fresh = zero_moai.LoraSet(eng, 2, proj, gates=g2)
    b2, t2 = fresh.deltas(pk, sk, H, [91, 92], with_intermediates=True)
    assert np.array_equal(s2, t2)
    for x, y in zip(a2, b2):
        assert np.array_equal(x, y)
    assert not np.array_equal(s1, s2)
    ls.set_gates(g1)
    a3, s3 = ls.deltas(pk, sk, H, [91, 92], with_intermediates=True)
    assert np.array_equal(s1, s3)
    for x, y in zip(a1, a3):
        assert np.array_equal(x, y)


def test_moe_set_gates_matches_oracle_per_token(env):
    """Three tokens, each with its own seeded gate, against the oracle's literal k products +
    ct_add + rescale + decrypt with that token's gates (layer 0, q and v)."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(26)
    proj, g0 = _experts(rng, 1)
    ls = zero_moai.LoraSet(eng, 1, proj, gates=g0)
    for t in range(3):
        H = rng.normal(size=(1, 1536)) * 0.1
        gt = np.array([zero_moai.softmax_gate(100 * t + j, K) for j in range(len(proj))])
        ls.set_gates(gt)
        got, got_sums = ls.deltas(pk, sk, H, [200 + t], with_intermediates=True)
        exp, exp_sums = _oracle(ref, rpk, rsk, H, [200 + t], proj, gt)
        assert np.max(np.abs(got_sums - exp_sums)) <= 1e-9 * max(1.0, np.max(np.abs(exp_sums)))
        for g, e in zip(got, exp):
            assert np.linalg.norm(g - e) <= 1e-3 * np.linalg.norm(e)


def test_moe_set_gates_errors(env):
    eng = env[0]
    rng = np.random.default_rng(27)
    proj, gates = _experts(rng, 1, d_outs=(8,))
    ls = zero_moai.LoraSet(eng, 1, proj, gates=gates)
    with pytest.raises(ValueError):
        ls.set_gates(gates[:, :2])
    bad = gates.copy()
    bad[0, 1] = np.inf
    with pytest.raises(ValueError, match="finite"):
        ls.set_gates(bad)
    plain = zero_moai.LoraSet(eng, 1, [(0, proj[0][1][0], proj[0][2][0])])
    with pytest.raises(RuntimeError, match="without gates"):
        plain.set_gates(np.ones((1, 1)))


def test_moe_full_shape_two_tokens(env):
    """The full CryptoMOE shape: 28 layers x {q, v} x 3 rank-16 experts (224 batches, 672 expert
    encodes per regate), two successive tokens each with its own gates (th_lora_set_gates) and
    device-resident inputs and outputs; layers 0 and 27 of both tokens against the oracle's
    literal k products + ct_add + rescale + decrypt with that token's gates."""
    import ctypes as C

    from provenloop_amd import _lib

    eng, ref, sk, pk, rsk, rpk = env
    lib = _lib.load()
    rng = np.random.default_rng(28)
    proj, g0 = _experts(rng, 28)
    ls = zero_moai.LoraSet(eng, 28, proj, gates=g0)
    assert ls.n_batches == 224
    hd, od = C.c_void_p(), C.c_void_p()
    _lib.check(lib.th_dev_alloc(eng._h, 28 * 1536 * 8, C.byref(hd)))
    _lib.check(lib.th_dev_alloc(eng._h, ls.n_deltas * 8, C.byref(od)))
    try:
        for t in range(2):
            H = np.ascontiguousarray(rng.normal(size=(28, 1536)) * 0.1)
            gt = np.array([zero_moai.softmax_gate(5000 * t + j, K) for j in range(len(proj))])
            seeds = [700 + 50 * t + i for i in range(28)]
            _lib.check(lib.th_memcpy_h2d(eng._h, hd, _lib.ptr(H), H.nbytes))
            ls.set_gates(gt)
            ls.deltas_device(pk, sk, hd.value, seeds, od.value)
            eng.sync()
            out = np.empty(ls.n_deltas)
            _lib.check(lib.th_memcpy_d2h(eng._h, _lib.ptr(out), od, ls.n_deltas * 8))
            for l in (0, 27):
                sub = [(0, A, B) for _, A, B in proj[2 * l:2 * l + 2]]
                exp, _ = _oracle(ref, rpk, rsk, H[l:l + 1], seeds[l:l + 1], sub, gt[2 * l:2 * l + 2])
                for j, e in zip((2 * l, 2 * l + 1), exp):
                    g = out[ls.offsets[j]:ls.offsets[j + 1]]
                    assert np.linalg.norm(g - e) <= 1e-3 * np.linalg.norm(e), (t, l, j)
    finally:
        _lib.check(lib.th_dev_free(eng._h, hd))
        _lib.check(lib.th_dev_free(eng._h, od))
