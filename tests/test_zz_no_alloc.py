"""th_batch_decrypt_segsum_noalloc against th_batch_decrypt_segsum, through the C ABI.

The no-allocation entry point keeps its working memory in a static device
array per GPU; its results must equal the allocating entry point's bit for
bit on each decrypt path (sums in the decrypt transform's epilogue, the
segment-sum kernels, the full decode), on two calls in a row with the second
smaller (the array keeps the first call's contents), and it must refuse a
batch that does not fit its array.
"""
import ctypes as C

import numpy as np
import pytest

from provenloop_amd import _lib, tensafe_he, zero_moai

pytestmark = pytest.mark.gpu

N = 16384


@pytest.fixture(scope="module")
def env():
    ctx = tensafe_he.CkksContext(N)
    sk = ctx.keygen(seed=71)
    pk = ctx.keygen_public(sk, seed=72)
    rng = np.random.default_rng(73)
    cts = ctx.encrypt_pk_batch([rng.normal(size=N // 2) * 0.1 for _ in range(3)], pk, [74, 75, 76])
    pts = [ctx.encode_to_ntt(rng.normal(size=N // 2) * 0.02) for _ in range(4)]
    prods = ctx.ct_pt_mul_ntt_batch([cts[i % 3] for i in range(12)], [pts[i % 4] for i in range(12)])
    rescaled = ctx.rescale_batch(prods)  # 3 limbs, scale 2^80 / q3: the limb-0 branch
    return ctx, sk, prods, rescaled


def _both(ctx, sk, cts, d, cols):
    L = _lib.load()
    arr = _lib.handle_array([ctx._own(c) for c in cts])
    ref = np.full((len(cts), cols), np.nan)
    got = np.full((len(cts), cols), np.nan)
    _lib.check(L.th_batch_decrypt_segsum(ctx._h, arr, len(cts), ctx._own(sk), d, cols, _lib.ptr(ref)))
    _lib.check(L.th_batch_decrypt_segsum_noalloc(ctx._h, arr, len(cts), ctx._own(sk), d, cols, _lib.ptr(got)))
    return ref, got


@pytest.mark.parametrize("path,d,cols", [
    ("epilogue", 1536, 5),      # limb-0 branch, at most 8 segments: sums in the decrypt transform
    ("segsum-kernels", 512, 16),  # more than 8 segments: segment-sum kernels on the coefficients
    ("full-decode", 256, 32),   # more than 16 segments: the slot decode, summed
])
def test_noalloc_equals_segsum_on_rescaled(env, path, d, cols):
    ctx, sk, _, rescaled = env
    for batch in (rescaled, rescaled[:5]):  # the second call smaller than the first
        ref, got = _both(ctx, sk, batch, d, cols)
        assert np.all(np.isfinite(ref))
        assert np.array_equal(got, ref), path


def test_noalloc_crt_branch(env):
    """Products at scale 2^80 decrypt through the CRT of limbs 0 and 1."""
    ctx, sk, prods, _ = env
    for batch in (prods[:7], prods[:2]):
        ref, got = _both(ctx, sk, batch, 1536, 5)
        assert np.array_equal(got, ref)


def test_noalloc_matches_lora_pass(env):
    """One projection's packed batches: the sums equal th_lora_a_pass's."""
    ctx, sk, _, _ = env
    pk = ctx.keygen_public(sk, seed=77)
    rng = np.random.default_rng(78)
    h = rng.normal(size=(1, 1536)) * 0.1
    A = rng.normal(size=(16, 1536)) * 0.02
    pts = [ctx.encode_to_ntt(p) for p in zero_moai.pack_rows(A, N // 2)]
    sums = ctx.lora_a_pass(pk, sk, h, [79], pts, [0] * len(pts))
    ct = ctx.encrypt_pk(zero_moai.replicate(h[0], N // 2, 1536), pk, seed=79)
    res = ctx.rescale_batch(ctx.ct_pt_mul_ntt_batch([ct] * len(pts), pts))
    _, got = _both(ctx, sk, res, 1536, 5)
    assert np.array_equal(got, sums)


def test_noalloc_refuses_batches_beyond_its_scratch(env):
    ctx, sk, _, rescaled = env
    L = _lib.load()
    big = (rescaled * 6)[:70]  # 70 full decodes need 70 x 512 KiB of scratch
    arr = _lib.handle_array([ctx._own(c) for c in big])
    out = np.zeros((len(big), 32))
    rc = L.th_batch_decrypt_segsum_noalloc(ctx._h, arr, len(big), ctx._own(sk), 256, 32, _lib.ptr(out))
    assert rc == _lib.TH_EINVAL
    assert "scratch" in _lib.last_error()
    # the entry point still works afterwards
    ref, got = _both(ctx, sk, rescaled[:3], 1536, 5)
    assert np.array_equal(got, ref)
