"""Handle lifetimes through the C ABI.

The reference's keys and ciphertexts are plain values that outlive the
CkksContext that made them, so a binding may drop the context first. Here
every handle holds a reference to its context: after th_ctx_free the context
refuses new work (TH_ESTATE), the handles stay valid to free, and the device
memory goes when the last one is released. th_dev_free accepts only live
th_dev_alloc buffers, so a double free cannot hand one buffer to two owners.
"""
import ctypes as C

import numpy as np
import pytest

from provenloop_amd import _lib

pytestmark = pytest.mark.gpu

N = 8192


def _ctx():
    L = _lib.load()
    out = C.c_void_p()
    _lib.check(L.th_ctx_create(N, None, 0, 40, 0, C.byref(out)))
    return L, out


def _out():
    return C.c_void_p()


def test_context_freed_before_its_handles():
    L, ctx = _ctx()
    sk, pk, ct, pt = _out(), _out(), _out(), _out()
    _lib.check(L.th_keygen(ctx, 1, 1, C.byref(sk)))
    _lib.check(L.th_keygen_public(ctx, sk, 2, 1, C.byref(pk)))
    z = np.linspace(-0.5, 0.5, N // 2)
    _lib.check(L.th_encrypt_pk(ctx, pk, _lib.ptr(z), z.size, 3, 1, C.byref(ct)))
    _lib.check(L.th_encode_to_ntt(ctx, _lib.ptr(z), z.size, C.byref(pt)))
    dec = np.zeros(N // 2)
    _lib.check(L.th_decrypt(ctx, ct, sk, _lib.ptr(dec)))
    assert np.max(np.abs(dec - z)) < 1e-6
    assert L.th_ctx_free(ctx) == _lib.TH_OK
    # the context is closed: new work is refused, not a use-after-free
    other = _out()
    rc = L.th_encrypt_pk(ctx, pk, _lib.ptr(z), z.size, 4, 1, C.byref(other))
    assert rc == _lib.TH_ESTATE and "freed" in _lib.last_error()
    assert L.th_ctx_free(ctx) == _lib.TH_ESTATE  # a second free is refused while handles hold it
    # the handles free cleanly, the last one releasing the context
    for fn, h in (("th_ct_free", ct), ("th_pt_free", pt), ("th_pk_free", pk), ("th_sk_free", sk)):
        assert getattr(L, fn)(h) == _lib.TH_OK


def test_context_freed_before_a_lora_set():
    from provenloop_amd import tensafe_he, zero_moai

    ctx = tensafe_he.CkksContext(N)
    sk = ctx.keygen(seed=5)
    pk = ctx.keygen_public(sk, seed=6)
    rng = np.random.default_rng(7)
    d = 1024
    proj = [(0, rng.normal(size=(4, d)) * 0.02, rng.normal(size=(8, 4)) * 0.02)]
    lora = zero_moai.LoraSet(ctx, 1, proj)
    h = rng.normal(size=(1, d)) * 0.1
    first = lora.deltas(pk, sk, h, [9])
    L = _lib.load()
    assert L.th_ctx_free(ctx._h) == _lib.TH_OK
    ctx._h = None  # the Python object must not free it again
    # the set and keys still free without touching freed memory
    assert L.th_lora_free(lora._h) == _lib.TH_OK
    lora._h = None
    assert L.th_pk_free(pk._h) == _lib.TH_OK and L.th_sk_free(sk._h) == _lib.TH_OK
    pk._h = sk._h = None
    assert np.all(np.isfinite(np.concatenate(first)))


def test_dev_free_refuses_double_and_foreign_pointers():
    L, ctx = _ctx()
    p = C.c_void_p()
    _lib.check(L.th_dev_alloc(ctx, 4096, C.byref(p)))
    assert L.th_dev_free(ctx, p) == _lib.TH_OK
    assert L.th_dev_free(ctx, p) == _lib.TH_EINVAL  # already freed
    assert "already freed" in _lib.last_error()
    # two later allocations of the size get distinct buffers
    a, b = C.c_void_p(), C.c_void_p()
    _lib.check(L.th_dev_alloc(ctx, 4096, C.byref(a)))
    _lib.check(L.th_dev_alloc(ctx, 4096, C.byref(b)))
    assert a.value != b.value
    x = np.arange(4096 // 8, dtype=np.uint64)
    _lib.check(L.th_memcpy_h2d(ctx, a, _lib.ptr(x), 4096))
    y = np.zeros_like(x)
    _lib.check(L.th_memcpy_h2d(ctx, b, _lib.ptr(y), 4096))
    back = np.empty_like(x)
    _lib.check(L.th_memcpy_d2h(ctx, _lib.ptr(back), a, 4096))
    assert np.array_equal(back, x)
    host = np.zeros(8, np.uint64)
    assert L.th_dev_free(ctx, C.c_void_p(host.ctypes.data)) == _lib.TH_EINVAL  # not from th_dev_alloc
    _lib.check(L.th_dev_free(ctx, a))
    _lib.check(L.th_dev_free(ctx, b))
    _lib.check(L.th_ctx_free(ctx))
