"""The device sampler's boundary band (TH_OPT_SAMPLER_BAND) and its host redraw.

A rounded Gaussian draw round(z * 3.19) (rng.rs:152-157, sampling.rs:51-58)
could round differently on the device than with glibc only when z * 3.19 is
within a few ulps of k + 1/2. The device flags every draw within the band of
a boundary, and the host then draws that input's randomness again with glibc.
Widening the band makes the flagged path run on (nearly) every input, so
these tests exercise it: every result must equal the oracle's, and equal the
result of the default band bit for bit. The band is read when a call queues
its work, so one context can queue flagged and unflagged tokens in turn.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc
from provenloop_amd import _lib, tensafe_he, zero_moai

pytestmark = pytest.mark.gpu

N = 8192
WIDE, NARROW, DEFAULT = -4, -40, -36  # log2 of the band: nearly every input / (almost) none / the default


@pytest.fixture(scope="module")
def env():
    eng, ref = tensafe_he.CkksContext(N), orc.Context(N)
    sk, rsk = eng.keygen(seed=61), ref.keygen(61)
    pk, rpk = eng.keygen_public(sk, seed=62), ref.keygen_public(rsk, 62)
    yield eng, ref, sk, pk, rsk, rpk
    eng.set_sampler_band(DEFAULT)


def _same_ct(eng, ref, ct, rct):
    c0, c1 = eng.ct_download(ct)
    r0, r1 = ref.ct_data(rct)
    assert np.array_equal(c0, r0) and np.array_equal(c1, r1)


def test_band_option_range(env):
    eng = env[0]
    for bad in (0, -41, -53, 5):
        with pytest.raises(ValueError, match="band"):
            eng.set_sampler_band(bad)
    eng.set_sampler_band(DEFAULT)


def test_encrypt_pk_batch_redraw_matches_oracle(env):
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(63)
    zs = [rng.normal(size=N // 2) * 0.1 for _ in range(3)]
    seeds = [101, 102, 103]
    eng.set_sampler_band(WIDE)
    before = eng.redrawn_inputs()
    cts = eng.encrypt_pk_batch(zs, pk, seeds)
    assert eng.redrawn_inputs() - before == 3  # every input drawn again on the host
    eng.set_sampler_band(DEFAULT)
    for c, z, s in zip(cts, zs, seeds):
        _same_ct(eng, ref, c, ref.encrypt_pk(z, rpk, s))
    ct1 = eng.encrypt_pk(zs[0], pk, seed=seeds[0])  # default band: the device's own draws
    _same_ct(eng, ref, ct1, ref.encrypt_pk(zs[0], rpk, seeds[0]))


def test_lora_a_pass_redraw_equals_default(env):
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(64)
    d = 1024
    H = rng.normal(size=(2, d)) * 0.1
    A = rng.normal(size=(8, d)) * 0.02
    pts = [eng.encode_to_ntt(p) for p in zero_moai.pack_rows(A, N // 2)]
    args = (pk, sk, H, [7, 8], pts, [0, 1])
    plain = eng.lora_a_pass(*args, rescale=True)
    eng.set_sampler_band(WIDE)
    before = eng.redrawn_inputs()
    wide = eng.lora_a_pass(*args, rescale=True)
    assert eng.redrawn_inputs() - before == 2
    eng.set_sampler_band(DEFAULT)
    assert np.array_equal(plain, wide)


def _lora(eng, rng):
    d = 1024
    proj = [(0, rng.normal(size=(8, d)) * 0.02, rng.normal(size=(64, 8)) * 0.02),
            (1, rng.normal(size=(8, d)) * 0.02, rng.normal(size=(32, 8)) * 0.02)]
    return zero_moai.LoraSet(eng, 2, proj), proj


def test_lora_set_sync_redraw_matches_oracle(env):
    eng, ref, sk, pk, rsk, rpk = env
    rng = np.random.default_rng(65)
    ls, proj = _lora(eng, rng)
    H = rng.normal(size=(2, 1024)) * 0.1
    plain = np.concatenate(ls.deltas(pk, sk, H, [11, 12]))
    eng.set_sampler_band(WIDE)
    before = eng.redrawn_inputs()
    wide = np.concatenate(ls.deltas(pk, sk, H, [11, 12]))
    assert eng.redrawn_inputs() - before == 2
    eng.set_sampler_band(DEFAULT)
    assert np.array_equal(plain, wide)
    # and the oracle, composed from the reference operations
    S, d = N // 2, 1024
    cols = S // d
    cts = [ref.encrypt_pk(zero_moai.replicate(h, S, d), rpk, s) for h, s in zip(H, [11, 12])]
    exp = []
    for i, A, B in proj:
        inter = np.zeros(A.shape[0])
        for b, p in enumerate(zero_moai.pack_rows(A, S)):
            dec = ref.decrypt(ref.rescale(ref.ct_pt_mul(cts[i], p)), rsk)
            n = min(cols, A.shape[0] - b * cols)
            inter[b * cols:b * cols + n] = [np.sum(dec[c * d:(c + 1) * d]) for c in range(n)]
        exp.append(B @ inter)
    exp = np.concatenate(exp)
    assert np.linalg.norm(wide - exp) <= 1e-3 * np.linalg.norm(exp)


def test_lora_set_async_tokens_are_settled_at_sync(env):
    """Four tokens queued without waiting, the second with the wide band: the
    sync queues it again from glibc draws, and the two after it again from the
    device, so every output equals the synchronous result."""
    eng, ref, sk, pk, rsk, rpk = env
    L = _lib.load()
    rng = np.random.default_rng(66)
    ls, _ = _lora(eng, rng)
    tokens = 4
    Hs = [rng.normal(size=(2, 1024)) * 0.1 for _ in range(tokens)]
    seeds = [[100 + 2 * t, 101 + 2 * t] for t in range(tokens)]
    expect = [np.concatenate(ls.deltas(pk, sk, Hs[t], seeds[t])) for t in range(tokens)]
    hd, od = C.c_void_p(), C.c_void_p()
    hb, ob = 2 * 1024 * 8, ls.n_deltas * 8
    _lib.check(L.th_dev_alloc(eng._h, tokens * hb, C.byref(hd)))
    _lib.check(L.th_dev_alloc(eng._h, tokens * ob, C.byref(od)))
    try:
        Hc = np.ascontiguousarray(np.stack(Hs))
        _lib.check(L.th_memcpy_h2d(eng._h, hd, _lib.ptr(Hc), Hc.nbytes))
        zero = np.zeros(tokens * ls.n_deltas)
        _lib.check(L.th_memcpy_h2d(eng._h, od, _lib.ptr(zero), zero.nbytes))
        before = eng.redrawn_inputs()
        for t in range(tokens):
            eng.set_sampler_band(WIDE if t == 1 else NARROW)
            ls.deltas_device(pk, sk, hd.value + t * hb, seeds[t], od.value + t * ob)
        eng.set_sampler_band(DEFAULT)
        eng.sync()
        assert eng.redrawn_inputs() - before == 2  # token 1's two inputs
        got = np.empty(tokens * ls.n_deltas)
        _lib.check(L.th_memcpy_d2h(eng._h, _lib.ptr(got), od, got.nbytes))
        for t in range(tokens):
            assert np.array_equal(got[t * ls.n_deltas:(t + 1) * ls.n_deltas], expect[t]), f"token {t}"
        # without an explicit sync, reading the outputs settles the queued tokens too
        eng.set_sampler_band(WIDE)
        ls.deltas_device(pk, sk, hd.value, seeds[0], od.value)
        eng.set_sampler_band(DEFAULT)
        first = np.empty(ls.n_deltas)
        _lib.check(L.th_memcpy_d2h(eng._h, _lib.ptr(first), od, ob))
        assert np.array_equal(first, expect[0])
    finally:
        eng.set_sampler_band(DEFAULT)
        _lib.check(L.th_dev_free(eng._h, hd))
        _lib.check(L.th_dev_free(eng._h, od))


@pytest.mark.parametrize("sk_fused", [False, True])
def test_no_sync_token_exposes_only_nan_or_exact_deltas(env, sk_fused):
    """A token queued without a synchronisation whose inputs are flagged (wide band), its input
    and output in ROCm torch tensors: a torch copy of its deltas ordered after it on the context
    stream (a stream-ordered consumer, made before any settling call) holds NaN for every delta
    of a flagged input's projections and the exact delta otherwise, never another value; after
    th_ctx_sync the token's own output is exact. A later host-to-device copy into the token's
    input (th_memcpy_h2d) settles the token first, so its redo reads the input it was queued
    with."""
    import torch

    eng, ref, sk, pk, rsk, rpk = env
    L = _lib.load()
    rng = np.random.default_rng(67)
    ls, _ = _lora(eng, rng)
    H = np.ascontiguousarray(rng.normal(size=(2, 1024)) * 0.1)
    H2 = np.ascontiguousarray(rng.normal(size=(2, 1024)) * 0.1)
    seeds = np.ascontiguousarray([410, 411], np.uint64)
    expect = np.concatenate(ls.deltas(pk, sk, H, seeds))
    dev = torch.device("cuda:0")
    ht = torch.from_numpy(H).to(dev)
    out = torch.zeros(ls.n_deltas, dtype=torch.float64, device=dev)
    torch.cuda.synchronize()
    stream = C.c_void_p()
    _lib.check(L.th_ctx_stream(eng._h, C.byref(stream)))
    mode = zero_moai.LoraSet._mode(True, sk_fused)
    before = eng.redrawn_inputs()
    eng.set_sampler_band(WIDE)
    try:
        _lib.check(L.th_lora_deltas(eng._h, ls._h, eng._own(pk), eng._own(sk), ht.data_ptr(), 1, _lib.ptr(seeds),
                                    mode, out.data_ptr(), 1, None))
    finally:
        eng.set_sampler_band(DEFAULT)
    with torch.cuda.stream(torch.cuda.ExternalStream(stream.value)):
        seen = out.clone()  # a consumer ordered after the token on its stream
    _lib.check(L.th_memcpy_h2d(eng._h, C.c_void_p(ht.data_ptr()), _lib.ptr(H2), H2.nbytes))
    assert eng.redrawn_inputs() - before == 2
    eng.sync()
    torch.cuda.synchronize()
    seen_h, final = seen.cpu().numpy(), out.cpu().numpy()
    assert np.array_equal(final, expect)
    assert np.all(np.isnan(seen_h) | (seen_h == expect))
    assert np.all(np.isnan(seen_h))  # both inputs flagged: every projection reads one of them
