"""LoRA sets (th_lora_create / th_lora_deltas): one token of the encrypted
LoRA path for every projection, on the device, against the oracle.

The oracle side composes the reference operations one by one
(inference_engine.py:1258-1392 with the reference CKKS core): encrypt_pk of
the replicated input, ct x pt with each packed batch, rescale, decrypt, sum
of each d-slot segment, then B @ intermediate. Segment sums are reduced in a
different order on the GPU, so they are held to 1e-9 absolute (relative to
their size) and the deltas to the 1e-3 relative bound on decoded deltas (in
practice ~1e-15); the ciphertext arithmetic under them is bit-exact (see
test_gpu_parity.py), and the set's segment sums equal th_lora_a_pass's bit
for bit.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import _lib, tensafe_he, zero_moai

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("lora_mode")]


@pytest.fixture(scope="module")
def env():
    eng, ref = tensafe_he.CkksContext(16384), orc.Context(16384)
    sk, rsk = eng.keygen(seed=41), ref.keygen(41)
    pk, rpk = eng.keygen_public(sk, seed=42), ref.keygen_public(rsk, 42)
    return eng, ref, sk, pk, rsk, rpk


def _oracle(ref, rpk, rsk, H, seeds, projections, rescale):
    S = ref.num_slots
    d = H.shape[1]
    cols = S // d
    cts = [ref.encrypt_pk(zero_moai.replicate(h, S, d), rpk, int(sd)) for h, sd in zip(H, seeds)]
    deltas, sums = [], []
    for i, A, B in projections:
        inter = np.zeros(A.shape[0])
        for b, p in enumerate(zero_moai.pack_rows(A, S)):
            r = ref.ct_pt_mul(cts[i], p)
            if rescale:
                r = ref.rescale(r)
            dec = ref.decrypt(r, rsk)
            seg = np.array([np.sum(dec[c * d:(c + 1) * d]) for c in range(cols)])
            sums.append(seg)
            n = min(cols, A.shape[0] - b * cols)
            inter[b * cols:b * cols + n] = seg[:n]
        deltas.append(B @ inter)
    return deltas, np.array(sums)


def _check(got, got_sums, exp, exp_sums):
    assert got_sums.shape == exp_sums.shape
    assert np.max(np.abs(got_sums - exp_sums)) <= 1e-9 * max(1.0, np.max(np.abs(exp_sums)))
    for g, e in zip(got, exp):
        assert g.shape == e.shape
        assert np.linalg.norm(g - e) <= 1e-3 * np.linalg.norm(e)
        assert np.max(np.abs(g - e)) <= 1e-9 * max(1.0, np.max(np.abs(e)))


def _projections(rng, n_inputs, d, ranks, d_outs):
    return [(j % n_inputs, rng.normal(size=(r, d)) * 0.02, rng.normal(size=(o, r)) * 0.02)
            for j, (r, o) in enumerate(zip(ranks, d_outs))]


@pytest.mark.parametrize("rescale", [True, False])
def test_lora_set_matches_oracle(env, rescale):
    """Two layers x {q, v} at the Qwen2.5-1.5B shape (d=1536, rank 16, B_q 1536x16, B_v 256x16)."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(7)
    H = rng.normal(size=(2, 1536)) * 0.1
    proj = [(l, rng.normal(size=(16, 1536)) * 0.02, rng.normal(size=(o, 16)) * 0.02)
            for l in range(2) for o in (1536, 256)]
    ls = zero_moai.LoraSet(eng, 2, proj)
    assert (ls.n_batches, ls.cols, ls.n_deltas) == (16, 5, 2 * (1536 + 256))
    seeds = [9001, 9002]
    got, got_sums = ls.deltas(pk, sk, H, seeds, rescale=rescale, with_intermediates=True)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, rescale)
    _check(got, got_sums, exp, exp_sums)
    # the same segment sums as th_lora_a_pass (same kernels), bit for bit
    pts = [eng.encode_to_ntt(p) for _, A, _ in proj for p in zero_moai.pack_rows(A, 8192)]
    pin = [i for i, A, _ in proj for _ in range(4)]
    assert np.array_equal(eng.lora_a_pass(pk, sk, H, seeds, pts, pin, rescale=rescale), got_sums)


@pytest.mark.parametrize("scale", [3e3, 1e7, 1e12])
def test_lora_set_large_inputs(env, scale):
    """Hidden states whose encoded coefficients |m| exceed the 40-bit primes (3e3: about 2^45, the
    FP64 residue step), straddle 2^53 (1e7: FP64 step and 64-bit Barrett fallback), or saturate the
    encoder's rounding (1e12): the encrypt transforms' fused residues (m + e0, e1, u formed in the
    loads) equal the encoder-written residues of th_lora_a_pass bit for bit, and the segment sums
    match the oracle's."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(int(scale) % 1000)
    H = rng.normal(size=(1, 1536)) * scale
    proj = [(0, rng.normal(size=(5, 1536)) * 0.02, rng.normal(size=(8, 5)) * 0.02)]
    ls = zero_moai.LoraSet(eng, 1, proj)
    seeds = [777]
    for rescale in (True, False):
        got, got_sums = ls.deltas(pk, sk, H, seeds, rescale=rescale, with_intermediates=True)
        pts = [eng.encode_to_ntt(p) for p in zero_moai.pack_rows(proj[0][1], 8192)]
        assert np.array_equal(eng.lora_a_pass(pk, sk, H, seeds, pts, [0], rescale=rescale), got_sums)
        exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, rescale)
        assert np.max(np.abs(got_sums - exp_sums)) <= 1e-9 * max(1.0, np.max(np.abs(exp_sums)))


def test_lora_set_full_token_shape(env):
    """28 layers x {q, v} (224 products: the launches take the split-NTT path); layers 0 and 27
    against the oracle, and the device-resident run equal to the host-I/O run."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(14)
    H = rng.normal(size=(28, 1536)) * 0.1
    proj = [(l, rng.normal(size=(16, 1536)) * 0.02, rng.normal(size=(o, 16)) * 0.02)
            for l in range(28) for o in (1536, 256)]
    ls = zero_moai.LoraSet(eng, 28, proj)
    seeds = list(range(100, 128))
    got, got_sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    for l in (0, 27):
        sub = proj[2 * l:2 * l + 2]
        exp, exp_sums = _oracle(ref, rpk, rsk, H[l:l + 1], seeds[l:l + 1], [(0, A, B) for _, A, B in sub], True)
        _check(got[2 * l:2 * l + 2], got_sums[8 * l:8 * l + 8], exp, exp_sums)


def test_lora_set_ragged_shapes(env):
    """Ranks that do not fill the last batch, d with cols = 8, uneven d_out, inputs shared unevenly."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(8)
    d = 1000
    H = rng.normal(size=(3, d)) * 0.1
    proj = _projections(rng, 3, d, ranks=[3, 13, 8, 1], d_outs=[7, 300, 1, 64])
    ls = zero_moai.LoraSet(eng, 3, proj)
    assert ls.cols == 8 and ls.n_batches == 1 + 2 + 1 + 1
    seeds = [1, 2, 3]
    got, got_sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, True)
    _check(got, got_sums, exp, exp_sums)


def test_lora_set_one_column_per_batch(env):
    """d > N/4: one segment per plaintext batch (cols = 1)."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(9)
    d = 5000
    H = rng.normal(size=(1, d)) * 0.1
    proj = _projections(rng, 1, d, ranks=[3], d_outs=[5])
    ls = zero_moai.LoraSet(eng, 1, proj)
    assert ls.cols == 1 and ls.n_batches == 3
    got, got_sums = ls.deltas(pk, sk, H, [77], with_intermediates=True)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, [77], proj, True)
    _check(got, got_sums, exp, exp_sums)


@pytest.mark.parametrize("d", [900, 640])
def test_lora_set_many_columns(env, d):
    """cols = 9 and 12: more segments than the decrypt transform's fused segment-sum epilogue
    takes (8), so the standalone segment-sum kernels run; both paths against the oracle."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(d)
    H = rng.normal(size=(2, d)) * 0.1
    proj = _projections(rng, 2, d, ranks=[16, 5], d_outs=[32, 7])
    ls = zero_moai.LoraSet(eng, 2, proj)
    assert ls.cols == 8192 // d and ls.cols > 8
    seeds = [41, 42]
    got, got_sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, True)
    _check(got, got_sums, exp, exp_sums)


def test_lora_set_device_io_matches_host_io(env):
    eng, ref, sk, pk, rsk, rpk = env
    L = _lib.load()
    rng = np.random.default_rng(10)
    H = rng.normal(size=(2, 1536)) * 0.1
    proj = _projections(rng, 2, 1536, ranks=[16, 16, 16], d_outs=[1536, 256, 100])
    ls = zero_moai.LoraSet(eng, 2, proj)
    host = np.concatenate(ls.deltas(pk, sk, H, [5, 6]))
    hd, od = C.c_void_p(), C.c_void_p()
    _lib.check(L.th_dev_alloc(eng._h, H.nbytes, C.byref(hd)))
    _lib.check(L.th_dev_alloc(eng._h, ls.n_deltas * 8, C.byref(od)))
    try:
        Hc = np.ascontiguousarray(H)
        _lib.check(L.th_memcpy_h2d(eng._h, hd, _lib.ptr(Hc), H.nbytes))
        for _ in range(2):  # the set's working memory is reused across tokens
            ls.deltas_device(pk, sk, hd.value, [5, 6], od.value)
            dev = np.empty(ls.n_deltas)
            _lib.check(L.th_memcpy_d2h(eng._h, _lib.ptr(dev), od, ls.n_deltas * 8))
            assert np.array_equal(dev, host)
    finally:
        _lib.check(L.th_dev_free(eng._h, hd))
        _lib.check(L.th_dev_free(eng._h, od))


def test_lora_set_tokens_are_independent(env):
    """A later token with other inputs and seeds gives its own result (no stale working memory)."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(11)
    proj = _projections(rng, 1, 1536, ranks=[16], d_outs=[64])
    ls = zero_moai.LoraSet(eng, 1, proj)
    H1, H2 = rng.normal(size=(1, 1536)) * 0.1, rng.normal(size=(1, 1536)) * 0.1
    a = ls.deltas(pk, sk, H1, [1])[0]
    b = ls.deltas(pk, sk, H2, [2])[0]
    a2 = ls.deltas(pk, sk, H1, [1])[0]
    assert np.array_equal(a, a2) and not np.array_equal(a, b)
    exp, _ = _oracle(ref, rpk, rsk, H2, [2], proj, True)
    assert np.linalg.norm(b - exp[0]) <= 1e-3 * np.linalg.norm(exp[0])


def test_lora_set_argument_errors(env):
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(12)
    proj = _projections(rng, 1, 1536, ranks=[4], d_outs=[8])
    with pytest.raises(ValueError, match="input_of"):
        zero_moai.LoraSet(eng, 1, [(1,) + proj[0][1:]])
    ls = zero_moai.LoraSet(eng, 1, proj)
    with pytest.raises(ValueError):
        ls.deltas(pk, sk, np.zeros((2, 1536)), [1])
    one = tensafe_he.CkksContext(16384, moduli=[1152921504606748673])
    osk = one.keygen(seed=1)
    opk = one.keygen_public(osk, seed=2)
    ols = zero_moai.LoraSet(one, 1, proj)
    with pytest.raises(RuntimeError, match="Cannot rescale"):
        ols.deltas(opk, osk, np.zeros((1, 1536)), [1], rescale=True)
    with pytest.raises(ValueError, match="different CkksContext|another context"):
        ols.deltas(pk, sk, np.zeros((1, 1536)), [1], rescale=False)
    # one limb without rescale: the non-CRT decrypt branch
    oref = orc.Context(16384, moduli=[1152921504606748673])
    orsk = oref.keygen(1)
    orpk = oref.keygen_public(orsk, 2)
    H = rng.normal(size=(1, 1536)) * 0.1
    got, got_sums = ols.deltas(opk, osk, H, [3], rescale=False, with_intermediates=True)
    exp, exp_sums = _oracle(oref, orpk, orsk, H, [3], proj, False)
    _check(got, got_sums, exp, exp_sums)


def test_lora_set_split_sizes_n8192():
    """N = 8192 with 24 inputs: 288 encrypt transforms, past the whole-polynomial kernel's batch,
    so the encrypt residues and the public-key combine run in the split kernels at log N = 13;
    every input's segment sums equal th_lora_a_pass's (unfused encrypt) bit for bit, and two
    inputs match the oracle."""
    eng, ref = tensafe_he.CkksContext(8192), orc.Context(8192)
    sk, rsk = eng.keygen(seed=5), ref.keygen(5)
    pk, rpk = eng.keygen_public(sk, seed=6), ref.keygen_public(rsk, 6)
    rng = np.random.default_rng(81)
    n_in, d = 24, 512
    H = rng.normal(size=(n_in, d)) * 0.1
    proj = _projections(rng, n_in, d, ranks=[8] * n_in, d_outs=[16] * n_in)
    ls = zero_moai.LoraSet(eng, n_in, proj)
    assert ls.cols == 8 and ls.n_batches == n_in
    seeds = list(range(300, 300 + n_in))
    got, got_sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    pts = [eng.encode_to_ntt(p) for _, A, _ in proj for p in zero_moai.pack_rows(A, 4096)]
    assert np.array_equal(eng.lora_a_pass(pk, sk, H, seeds, pts, list(range(n_in))), got_sums)
    for i in (0, n_in - 1):
        exp, exp_sums = _oracle(ref, rpk, rsk, H[i:i + 1], seeds[i:i + 1], [(0, proj[i][1], proj[i][2])], True)
        _check(got[i:i + 1], got_sums[i:i + 1], exp, exp_sums)


@pytest.mark.parametrize("n_in", [64, 65])
def test_lora_set_sampler_in_encoder_launch_limit(n_in):
    """Up to 64 inputs (one launch's seeds) the encoder's first launch also draws the
    randomness (the sampler's workgroups beside the encoder's, two blocks per thread at
    this size); 65 take the sampler's own launches. Either way every input's segment sums
    equal th_lora_a_pass's (its own sampler launch) bit for bit, and the first and last
    inputs match the oracle."""
    eng, ref = tensafe_he.CkksContext(8192), orc.Context(8192)
    sk, rsk = eng.keygen(seed=7), ref.keygen(7)
    pk, rpk = eng.keygen_public(sk, seed=8), ref.keygen_public(rsk, 8)
    rng = np.random.default_rng(90 + n_in)
    d = 512
    H = rng.normal(size=(n_in, d)) * 0.1
    proj = _projections(rng, n_in, d, ranks=[4] * n_in, d_outs=[8] * n_in)
    ls = zero_moai.LoraSet(eng, n_in, proj)
    seeds = list(range(700, 700 + n_in))
    got, got_sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    pts = [eng.encode_to_ntt(p) for _, A, _ in proj for p in zero_moai.pack_rows(A, 4096)]
    assert np.array_equal(eng.lora_a_pass(pk, sk, H, seeds, pts, list(range(n_in))), got_sums)
    for i in (0, n_in - 1):
        exp, exp_sums = _oracle(ref, rpk, rsk, H[i:i + 1], seeds[i:i + 1], [(0, proj[i][1], proj[i][2])], True)
        _check(got[i:i + 1], got_sums[i:i + 1], exp, exp_sums)


@pytest.mark.parametrize("n_in", [4, 5])
def test_lora_set_host_io_paths(env, n_in):
    """Host hidden states of 4 x 1024 doubles (32 KiB) are read by the encoder from the set's
    mapped staging pages, 5 x 1024 are copied to the device first; host deltas are written into
    the staging pages by the last kernel. Every combination of host and device input and output
    gives the same deltas bit for bit, twice in a row."""
    eng, ref, sk, pk, rsk, rpk = env
    L = _lib.load()
    rng = np.random.default_rng(500 + n_in)
    d = 1024
    H = np.ascontiguousarray(rng.normal(size=(n_in, d)) * 0.1)
    proj = _projections(rng, n_in, d, ranks=[6] * n_in, d_outs=[33] * n_in)
    ls = zero_moai.LoraSet(eng, n_in, proj)
    seeds = np.arange(900, 900 + n_in, dtype=np.uint64)
    hd, od = C.c_void_p(), C.c_void_p()
    _lib.check(L.th_dev_alloc(eng._h, H.nbytes, C.byref(hd)))
    _lib.check(L.th_dev_alloc(eng._h, ls.n_deltas * 8, C.byref(od)))
    try:
        _lib.check(L.th_memcpy_h2d(eng._h, hd, _lib.ptr(H), H.nbytes))
        results = []
        for _ in range(2):
            for hin in (0, 1):
                for hout in (0, 1):
                    out = np.full(ls.n_deltas, np.nan)
                    dst = out.ctypes.data if hout else od.value
                    src = H.ctypes.data if hin else hd.value
                    _lib.check(L.th_lora_deltas(eng._h, ls._h, pk._h, sk._h, src, 0 if hin else 1,
                                                seeds.ctypes.data, 1, dst, 0 if hout else 1, None))
                    eng.sync()
                    if not hout:
                        _lib.check(L.th_memcpy_d2h(eng._h, _lib.ptr(out), od, out.nbytes))
                    results.append(out)
        for r in results[1:]:
            assert np.array_equal(results[0], r)
        exp, _ = _oracle(ref, rpk, rsk, H[:1], seeds[:1], [(0, proj[0][1], proj[0][2])], True)
        got0 = results[0][ls.offsets[0]:ls.offsets[1]]
        assert np.linalg.norm(got0 - exp[0]) <= 1e-9 * max(1.0, np.linalg.norm(exp[0]))
    finally:
        _lib.check(L.th_dev_free(eng._h, hd))
        _lib.check(L.th_dev_free(eng._h, od))


def test_lora_set_crt_branch_after_rescale():
    """A chain whose last prime is 30-bit: the rescaled scale is ~2^50 > 1.5 * 2^40, so the
    decrypt takes the CRT branch over limbs 0 and 1 (ciphertext.rs:351)."""
    q = [1152921504606748673, 1099510054913, 1073643521]
    eng, ref = tensafe_he.CkksContext(16384, moduli=q), orc.Context(16384, moduli=q)
    sk, rsk = eng.keygen(seed=3), ref.keygen(3)
    pk, rpk = eng.keygen_public(sk, seed=4), ref.keygen_public(rsk, 4)
    rng = np.random.default_rng(13)
    H = rng.normal(size=(1, 1536)) * 0.1
    proj = _projections(rng, 1, 1536, ranks=[16], d_outs=[32])
    ls = zero_moai.LoraSet(eng, 1, proj)
    got, got_sums = ls.deltas(pk, sk, H, [21], with_intermediates=True)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, [21], proj, True)
    _check(got, got_sums, exp, exp_sums)


@pytest.mark.parametrize("n, moduli, d", [
    (16384, [1125899904679937, 1099507695617, 1152921504598720513], 1536),
    (16384, [1099507695617, 1099506515969, 1152921504598720513], 1536),
    (4096, [1152921504606584833, 1099507695617, 1152921504598720513], 512),
])
def test_lora_set_rescale_decrypt_chains(n, moduli, d):
    """Rescaled sets whose decryption reads limb 0 rescale and decrypt each batch in one kernel
    after the last limb's inverse transforms: INTT(D pt - NTT(r1) s) - r0, times q_last^-1.
    Chains: a 50-bit limb 0 below a 60-bit last prime (the last limb's values are reduced by
    Barrett, not passed through), a 40-bit limb 0 (FP64 transforms), and N=4096. The segment
    sums equal th_lora_a_pass's (the full rescale, then the decryption) bit for bit, and the
    deltas match the oracle's."""
    eng, ref = tensafe_he.CkksContext(n, moduli=moduli), orc.Context(n, moduli=moduli)
    sk, rsk = eng.keygen(seed=5), ref.keygen(5)
    pk, rpk = eng.keygen_public(sk, seed=6), ref.keygen_public(rsk, 6)
    rng = np.random.default_rng(n + moduli[0] % 1000)
    H = rng.normal(size=(2, d)) * 0.1
    proj = _projections(rng, 2, d, ranks=[16, 7], d_outs=[24, 9])
    ls = _set_with(eng, "whole", 2, proj)
    seeds = [31, 32]
    got, got_sums = ls.deltas(pk, sk, H, seeds, rescale=True, with_intermediates=True)
    packs = [(i, zero_moai.pack_rows(A, n // 2)) for i, A, _ in proj]
    pts = [eng.encode_to_ntt(p) for _, ps in packs for p in ps]
    pin = [i for i, ps in packs for _ in ps]
    assert np.array_equal(eng.lora_a_pass(pk, sk, H, seeds, pts, pin, rescale=True), got_sums)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, True)
    _check(got, got_sums, exp, exp_sums)


@pytest.mark.parametrize("n, d", [(1024, 128), (2048, 256)])
def test_lora_set_small_rings(n, d):
    """N = 1024 and 2048 on the default chain's primes (one and two encoder parts, the
    sampler's workgroups in the same launch, whole-polynomial transforms everywhere): the
    segment sums equal th_lora_a_pass's bit for bit and the deltas match the oracle's."""
    q = [1152921504606748673, 1099510054913, 1099508121601, 1152921504606683137]
    eng, ref = tensafe_he.CkksContext(n, moduli=q), orc.Context(n, moduli=q)
    sk, rsk = eng.keygen(seed=9), ref.keygen(9)
    pk, rpk = eng.keygen_public(sk, seed=10), ref.keygen_public(rsk, 10)
    rng = np.random.default_rng(n)
    H = rng.normal(size=(3, d)) * 0.1
    proj = _projections(rng, 3, d, ranks=[8, 3, 5], d_outs=[10, 4, 7])
    ls = zero_moai.LoraSet(eng, 3, proj)
    seeds = [41, 42, 43]
    for rescale in (True, False):
        got, got_sums = ls.deltas(pk, sk, H, seeds, rescale=rescale, with_intermediates=True)
        packs = [(i, zero_moai.pack_rows(A, n // 2)) for i, A, _ in proj]
        pts = [eng.encode_to_ntt(p) for _, ps in packs for p in ps]
        pin = [i for i, ps in packs for _ in ps]
        assert np.array_equal(eng.lora_a_pass(pk, sk, H, seeds, pts, pin, rescale=rescale), got_sums)
        exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, rescale)
        _check(got, got_sums, exp, exp_sums)


def test_lora_set_many_batches_rescale(env):
    """260 batches, more than one round of one-workgroup-per-product kernels: the rescale and
    decryption run on the split kernels. A batch's sums depend only on its input, plaintext
    and keys, so the first 256 batches equal, bit for bit, those of a set of the first 64
    projections (one workgroup per product); all of them match th_lora_a_pass (which sums
    the segments in another order) to 1e-12, and the first two projections the oracle."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(17)
    H = rng.normal(size=(2, 1536)) * 0.1
    proj = _projections(rng, 2, 1536, ranks=[20] * 65, d_outs=[4] * 65)
    ls = zero_moai.LoraSet(eng, 2, proj)
    assert ls.n_batches == 260
    seeds = [51, 52]
    got, got_sums = ls.deltas(pk, sk, H, seeds, rescale=True, with_intermediates=True)
    first = zero_moai.LoraSet(eng, 2, proj[:64])
    assert first.n_batches == 256
    f_got, f_sums = first.deltas(pk, sk, H, seeds, rescale=True, with_intermediates=True)
    assert np.array_equal(f_sums, got_sums[:256])
    assert all(np.array_equal(a, b) for a, b in zip(f_got, got[:64]))
    packs = [(i, zero_moai.pack_rows(A, 8192)) for i, A, _ in proj]
    pts = [eng.encode_to_ntt(p) for _, ps in packs for p in ps]
    pin = [i for i, ps in packs for _ in ps]
    comp = eng.lora_a_pass(pk, sk, H, seeds, pts, pin, rescale=True)
    assert np.max(np.abs(comp - got_sums)) <= 1e-12 * np.max(np.abs(comp))
    exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj[:2], True)
    _check(got[:2], got_sums[:8], exp, exp_sums)


def _set_with(eng, kernels, n_inputs, proj):
    eng._rescale_decrypt_kernels(kernels)
    try:
        return zero_moai.LoraSet(eng, n_inputs, proj)
    finally:
        eng._rescale_decrypt_kernels("auto")


def test_lora_set_split_rescale_decrypt_equals_whole(env):
    """The split-kernel rescale-decrypt and the one-workgroup kernel (each forced) give the same
    segment sums and deltas, bit for bit, and the same as th_lora_a_pass, at the full token
    shape's 4 batches per projection."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(19)
    H = rng.normal(size=(3, 1536)) * 0.1
    proj = _projections(rng, 3, 1536, ranks=[16, 16, 7], d_outs=[64, 32, 5])
    whole = _set_with(eng, "whole", 3, proj)
    split = _set_with(eng, "split", 3, proj)
    seeds = [61, 62, 63]
    gw, sw = whole.deltas(pk, sk, H, seeds, with_intermediates=True)
    gs, ss = split.deltas(pk, sk, H, seeds, with_intermediates=True)
    assert np.array_equal(sw, ss)
    assert all(np.array_equal(a, b) for a, b in zip(gw, gs))
    packs = [(i, zero_moai.pack_rows(A, 8192)) for i, A, _ in proj]
    pts = [eng.encode_to_ntt(p) for _, ps in packs for p in ps]
    pin = [i for i, ps in packs for _ in ps]
    assert np.array_equal(eng.lora_a_pass(pk, sk, H, seeds, pts, pin, rescale=True), ss)
    # without a rescale the option changes nothing
    assert np.array_equal(whole.deltas(pk, sk, H, seeds, rescale=False, with_intermediates=True)[1],
                          split.deltas(pk, sk, H, seeds, rescale=False, with_intermediates=True)[1])


@pytest.mark.parametrize("n, moduli", [
    (8192, None),
    (32768, None),
    (16384, [1099507695617, 1099506515969, 1152921504598720513]),
])
def test_lora_set_split_rescale_decrypt_matches_oracle(n, moduli):
    """The split-kernel rescale-decrypt at log N = 13 and 15 (default chains) and on a 40-bit
    limb 0 (FP64 transforms, last-limb values reduced by Barrett) against the oracle."""
    eng = tensafe_he.CkksContext(n, moduli=moduli)
    ref = orc.Context(n, moduli=moduli) if moduli else orc.Context(n)
    sk, rsk = eng.keygen(seed=7), ref.keygen(7)
    pk, rpk = eng.keygen_public(sk, seed=8), ref.keygen_public(rsk, 8)
    rng = np.random.default_rng(n % 1000 + 3)
    d = {8192: 512, 16384: 1536, 32768: 2048}[n]  # cols = 8, 5, 8
    H = rng.normal(size=(2, d)) * 0.1
    proj = _projections(rng, 2, d, ranks=[9, 4], d_outs=[12, 6])
    ls = _set_with(eng, "split", 2, proj)
    seeds = [71, 72]
    got, got_sums = ls.deltas(pk, sk, H, seeds, with_intermediates=True)
    exp, exp_sums = _oracle(ref, rpk, rsk, H, seeds, proj, True)
    _check(got, got_sums, exp, exp_sums)


def test_lora_set_serial_sampler_path(env):
    """Forcing every input through the serial replay (the path a rejected range_u32 word
    takes) gives the same deltas, and the per-input reject flags are cleared afterwards."""
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(15)
    H = rng.normal(size=(3, 1536)) * 0.1
    proj = _projections(rng, 3, 1536, ranks=[16, 16, 16], d_outs=[40, 40, 40])
    ls = zero_moai.LoraSet(eng, 3, proj)
    base = np.concatenate(ls.deltas(pk, sk, H, [7, 8, 9]))
    eng._force_serial_sampler(True)
    try:
        forced = np.concatenate(ls.deltas(pk, sk, H, [7, 8, 9]))
    finally:
        eng._force_serial_sampler(False)
    again = np.concatenate(ls.deltas(pk, sk, H, [7, 8, 9]))
    assert np.array_equal(base, forced) and np.array_equal(base, again)
