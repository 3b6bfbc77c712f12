"""Python-facing CKKS backend with the reference's `tensafe_he` interface.

Mirrors the PyO3 module of tensafe-he/crates/tensafe-he-python/src/lib.rs
(classes CkksContext, TenSafeCiphertext, TenSafeSecretKey, TenSafePublicKey;
same method names, argument meaning, padding, seed semantics and error
types), backed by the gfx950 HIP engine through the C ABI of
include/tensafe_he.h. Key, ciphertext and plaintext data stay in HBM.

Beyond the reference surface it adds the batched calls the encrypted-LoRA
path needs (encrypt_pk_batch, encode_to_ntt, ct_pt_mul_ntt(_batch),
rescale_batch, batch_decrypt_segsum, batch_decrypt_to_device) and parity
hooks (encrypt_pk_explicit, download / upload, serialisation).

There is no CPU path: constructing a context without a gfx950 device, or
without the built library, raises.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

from . import _lib

__all__ = ["CkksContext", "TenSafeCiphertext", "TenSafeSecretKey", "TenSafePublicKey", "TenSafePlaintext"]

_VERSION = "0.1.0"


def _as_f64_vector(data, what="data") -> np.ndarray:
    """PyReadonlyArray1<f64> + as_slice() semantics (lib.rs:119-123)."""
    if not isinstance(data, np.ndarray):
        raise TypeError(f"argument '{what}': expected a numpy.ndarray of float64")
    if data.dtype != np.float64:
        raise TypeError(f"argument '{what}': expected float64, got {data.dtype}")
    if data.ndim != 1:
        raise TypeError(f"argument '{what}': expected a 1-dimensional array, got {data.ndim} dimensions")
    if not data.flags.c_contiguous:
        raise ValueError("The given array is not contiguous")
    return data


def _seed_args(seed: Optional[int]):
    if seed is None:
        return 0, 0
    if seed < 0 or seed >= 1 << 64:
        raise OverflowError("seed must fit in an unsigned 64-bit integer")
    return int(seed), 1


class _Handle:
    __slots__ = ("_h", "_ctx", "__weakref__")
    _free_fn = ""

    def __init__(self, h, ctx):
        self._h = h
        self._ctx = ctx

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and getattr(_lib, "_lib", None) is not None:
            getattr(_lib._lib, self._free_fn)(h)
            self._h = None


class TenSafeSecretKey(_Handle):
    """Secret key s in the NTT domain (lib.rs:297-301)."""

    __slots__ = ()
    _free_fn = "th_sk_free"


class TenSafePublicKey(_Handle):
    """Public key (b, a) (lib.rs:303-307)."""

    __slots__ = ()
    _free_fn = "th_pk_free"

    def to_bytes(self) -> bytes:
        """serialize.rs:48-52 layout: [b | a]."""
        return self._ctx._export(self, "th_pk_export")


class TenSafePlaintext(_Handle):
    """Encoded plaintext in the NTT domain (ciphertext.rs:539-545), resident in HBM."""

    __slots__ = ()
    _free_fn = "th_pt_free"


class TenSafeCiphertext(_Handle):
    """CKKS ciphertext (lib.rs:309-395)."""

    __slots__ = ()
    _free_fn = "th_ct_free"

    def _info(self):
        limbs, scale = C.c_uint32(), C.c_double()
        _lib.check(_lib.load().th_ct_info(self._h, C.byref(limbs), C.byref(scale)))
        return limbs.value, scale.value

    @property
    def scale(self) -> float:
        return self._info()[1]

    @property
    def num_limbs(self) -> int:
        return self._info()[0]

    def __mul__(self, other):
        """ct x pt, no rescale (lib.rs:336-356)."""
        if isinstance(other, TenSafePlaintext):
            return self._ctx.ct_pt_mul_ntt(self, other)
        return self._ctx.ct_pt_mul(self, other)

    def __add__(self, other):
        return self._ctx.ct_add(self, other)

    def __sub__(self, other):
        return self._ctx.ct_sub(self, other)

    def download(self):
        """(c0, c1) residues as uint64 arrays of shape [num_limbs, N]."""
        return self._ctx.ct_download(self)

    def to_bytes(self) -> bytes:
        """serialize.rs:71-77 layout: [scale | c0 | c1]."""
        return self._ctx._export(self, "th_ct_export")


class CkksContext:
    """CKKS context on one gfx950 device (lib.rs:18-295)."""

    def __init__(self, poly_mod_degree: int = 16384, *, moduli: Optional[Sequence[int]] = None,
                 device: int = 0):
        L = _lib.load()
        if moduli is None and poly_mod_degree not in (8192, 16384, 32768):
            raise ValueError(f"Unsupported poly_mod_degree: {poly_mod_degree}. Use 8192, 16384, or 32768.")
        out = C.c_void_p()
        if moduli is None:
            _lib.check(L.th_ctx_create(poly_mod_degree, None, 0, 40, device, C.byref(out)))
        else:
            m = np.ascontiguousarray(moduli, dtype=np.uint64)
            _lib.check(L.th_ctx_create(poly_mod_degree, _lib.ptr(m), m.size, 40, device, C.byref(out)))
        self._h = out
        n, nl = C.c_uint32(), C.c_uint32()
        q = np.zeros(16, np.uint64)
        _lib.check(L.th_ctx_info(self._h, C.byref(n), C.byref(nl), _lib.ptr(q)))
        self._n = n.value
        self._limbs = nl.value
        self.moduli = [int(v) for v in q[: nl.value]]
        self._device = device

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and getattr(_lib, "_lib", None) is not None:
            _lib._lib.th_ctx_free(h)
            self._h = None

    # ------------------------------------------------------------ reference surface
    @staticmethod
    def for_depth(depth: int = 3) -> "CkksContext":
        """lib.rs:62-76."""
        table = {1: 8192, 2: 16384, 3: 32768, 4: 32768, 5: 32768}
        if depth not in table:
            raise ValueError(f"Unsupported depth: {depth}. Use 1-5.")
        return CkksContext(table[depth])

    @property
    def num_slots(self) -> int:
        return self._n // 2

    @property
    def poly_mod_degree(self) -> int:
        return self._n

    @property
    def num_limbs(self) -> int:
        return self._limbs

    @property
    def device(self) -> int:
        """HIP device index the context's buffers and stream live on."""
        return self._device

    def _new(self, cls, fn, *args):
        out = C.c_void_p()
        _lib.check(fn(*args, C.byref(out)))
        return cls(out, self)

    def _pad(self, data, what="data") -> np.ndarray:
        return _as_f64_vector(data, what)[: self.num_slots]

    def keygen(self, seed: Optional[int] = None) -> TenSafeSecretKey:
        s, has = _seed_args(seed)
        return self._new(TenSafeSecretKey, _lib.load().th_keygen, self._h, s, has)

    def keygen_public(self, sk: TenSafeSecretKey, seed: Optional[int] = None) -> TenSafePublicKey:
        s, has = _seed_args(seed)
        return self._new(TenSafePublicKey, _lib.load().th_keygen_public, self._h, self._own(sk), s, has)

    def encrypt(self, data, sk: TenSafeSecretKey, seed: Optional[int] = None) -> TenSafeCiphertext:
        z = self._pad(data)
        s, has = _seed_args(seed)
        return self._new(TenSafeCiphertext, _lib.load().th_encrypt, self._h, self._own(sk), _lib.ptr(z), z.size,
                         s, has)

    def encrypt_pk(self, data, pk: TenSafePublicKey, seed: Optional[int] = None) -> TenSafeCiphertext:
        z = self._pad(data)
        s, has = _seed_args(seed)
        return self._new(TenSafeCiphertext, _lib.load().th_encrypt_pk, self._h, self._own(pk), _lib.ptr(z),
                         z.size, s, has)

    def decrypt(self, ct: TenSafeCiphertext, sk: TenSafeSecretKey) -> np.ndarray:
        out = np.zeros(self.num_slots, np.float64)
        _lib.check(_lib.load().th_decrypt(self._h, self._own(ct), self._own(sk), _lib.ptr(out)))
        return out

    def ct_pt_mul(self, ct: TenSafeCiphertext, plaintext) -> TenSafeCiphertext:
        p = self._pad(plaintext, "plaintext")
        return self._new(TenSafeCiphertext, _lib.load().th_ct_pt_mul, self._h, self._own(ct), _lib.ptr(p), p.size)

    def ct_add(self, ct_a: TenSafeCiphertext, ct_b: TenSafeCiphertext) -> TenSafeCiphertext:
        return self._new(TenSafeCiphertext, _lib.load().th_ct_add, self._h, self._own(ct_a), self._own(ct_b))

    def ct_sub(self, ct_a: TenSafeCiphertext, ct_b: TenSafeCiphertext) -> TenSafeCiphertext:
        return self._new(TenSafeCiphertext, _lib.load().th_ct_sub, self._h, self._own(ct_a), self._own(ct_b))

    def rescale(self, ct: TenSafeCiphertext) -> TenSafeCiphertext:
        return self._new(TenSafeCiphertext, _lib.load().th_rescale, self._h, self._own(ct))

    def batch_encrypt(self, arrays, sk: TenSafeSecretKey, seed: Optional[int] = None):
        """lib.rs:230-258: one RNG stream shared by the whole batch."""
        zs = [self._pad(a, "arrays") for a in arrays]
        if not zs:
            return []
        S = self.num_slots
        flat = np.zeros((len(zs), S), np.float64)
        lens = np.array([z.size for z in zs], np.uint64)
        for i, z in enumerate(zs):
            flat[i, : z.size] = z
        s, has = _seed_args(seed)
        outs = (C.c_void_p * len(zs))()
        _lib.check(_lib.load().th_encrypt_batch(self._h, self._own(sk), _lib.ptr(flat), _lib.ptr(lens), S,
                                                len(zs), s, has, outs))
        return [TenSafeCiphertext(outs[i], self) for i in range(len(zs))]

    def batch_decrypt(self, cts, sk: TenSafeSecretKey):
        """lib.rs:261-273, as one GPU batch with a single device-to-host copy."""
        cts = list(cts)
        out = np.zeros((len(cts), self.num_slots), np.float64)
        if cts:
            arr = _lib.handle_array([self._own(c) for c in cts])
            _lib.check(_lib.load().th_batch_decrypt(self._h, arr, len(cts), self._own(sk), _lib.ptr(out)))
        return [out[i] for i in range(len(cts))]

    @staticmethod
    def is_available() -> bool:
        """True when the HIP library loads and a GPU is visible (lib.rs:276-279)."""
        try:
            return _lib.device_count() > 0
        except Exception:
            return False

    def get_backend_info(self) -> dict:
        """lib.rs:282-294."""
        return {
            "backend": "tensafe-he-mi355x",
            "version": _VERSION,
            "language": "C++/HIP (gfx950)",
            "gpu_accelerated": True,
            "poly_mod_degree": self._n,
            "num_slots": self.num_slots,
            "num_limbs": self._limbs,
            "device": self._device,
        }

    # ------------------------------------------------------------ batched encrypted-LoRA path
    def encrypt_pk_batch(self, arrays, pk: TenSafePublicKey, seeds: Sequence[int]):
        """encrypt_pk of each array with its own seed, as one batch."""
        arrays = list(arrays)
        if len(seeds) != len(arrays):
            raise ValueError("need one seed per array")
        if not arrays:
            return []
        S = self.num_slots
        flat = np.zeros((len(arrays), S), np.float64)
        for i, a in enumerate(arrays):
            z = self._pad(a, "arrays")
            flat[i, : z.size] = z
        sd = np.ascontiguousarray(seeds, dtype=np.uint64)
        outs = (C.c_void_p * len(arrays))()
        _lib.check(_lib.load().th_encrypt_pk_batch(self._h, self._own(pk), _lib.ptr(flat), S, S, len(arrays),
                                                   _lib.ptr(sd), outs))
        return [TenSafeCiphertext(outs[i], self) for i in range(len(arrays))]

    def encrypt_pk_explicit(self, data, pk: TenSafePublicKey, u, e0, e1) -> TenSafeCiphertext:
        """encrypt_pk with caller-supplied (u, e0, e1) (values as sample_ternary / the Gaussian sampler give them)."""
        z = self._pad(data)
        n = self._n
        u = np.ascontiguousarray(u, dtype=np.uint8)
        e0 = np.ascontiguousarray(e0, dtype=np.int64)
        e1 = np.ascontiguousarray(e1, dtype=np.int64)
        if u.size != n or e0.size != n or e1.size != n:
            raise ValueError(f"u, e0 and e1 must have {n} entries")
        return self._new(TenSafeCiphertext, _lib.load().th_encrypt_pk_explicit, self._h, self._own(pk),
                         _lib.ptr(z), z.size, _lib.ptr(u), _lib.ptr(e0), _lib.ptr(e1))

    def encode_to_ntt(self, data) -> TenSafePlaintext:
        z = _as_f64_vector(data)
        if z.size > self.num_slots:
            raise ValueError(f"Input length {z.size} exceeds slot count {self.num_slots}")
        return self._new(TenSafePlaintext, _lib.load().th_encode_to_ntt, self._h, _lib.ptr(z), z.size)

    def ct_pt_mul_ntt(self, ct: TenSafeCiphertext, pt: TenSafePlaintext) -> TenSafeCiphertext:
        return self._new(TenSafeCiphertext, _lib.load().th_ct_pt_mul_ntt, self._h, self._own(ct), self._own(pt))

    def ct_pt_mul_ntt_batch(self, cts, pts):
        cts, pts = list(cts), list(pts)
        if len(cts) != len(pts):
            raise ValueError("cts and pts must have the same length")
        if not cts:
            return []
        outs = (C.c_void_p * len(cts))()
        _lib.check(_lib.load().th_ct_pt_mul_ntt_batch(self._h, _lib.handle_array([self._own(c) for c in cts]),
                                                      _lib.handle_array([self._own(p) for p in pts]), len(cts),
                                                      outs))
        return [TenSafeCiphertext(outs[i], self) for i in range(len(cts))]

    def rescale_batch(self, cts):
        cts = list(cts)
        if not cts:
            return []
        outs = (C.c_void_p * len(cts))()
        _lib.check(_lib.load().th_rescale_batch(self._h, _lib.handle_array([self._own(c) for c in cts]),
                                                len(cts), outs))
        return [TenSafeCiphertext(outs[i], self) for i in range(len(cts))]

    def batch_decrypt_segsum(self, cts, sk: TenSafeSecretKey, d: int, cols: int) -> np.ndarray:
        """[len(cts), cols] segment sums of the decrypted slots, one host sync."""
        cts = list(cts)
        out = np.zeros((len(cts), cols), np.float64)
        if cts:
            _lib.check(_lib.load().th_batch_decrypt_segsum(self._h, _lib.handle_array([self._own(c) for c in cts]),
                                                           len(cts), self._own(sk), d, cols, _lib.ptr(out)))
        return out

    def lora_a_pass(self, pk: TenSafePublicKey, sk: TenSafeSecretKey, hidden: np.ndarray, seeds, pts,
                    pt_input, rescale: bool = True) -> np.ndarray:
        """Whole encrypted LoRA-A pass in one call (see th_lora_a_pass).

        hidden: [n_inputs, d] float64; seeds: n_inputs encrypt_pk seeds; pts: cached
        plaintext batches; pt_input[j]: the input that pts[j] multiplies. Returns the
        [len(pts), (N/2)//d] segment sums of the decrypted products.
        """
        h = np.ascontiguousarray(hidden, dtype=np.float64)
        if h.ndim != 2:
            raise ValueError("hidden must be [n_inputs, d]")
        n_in, d = h.shape
        sd = np.ascontiguousarray(seeds, dtype=np.uint64)
        pin = np.ascontiguousarray(pt_input, dtype=np.uint32)
        if sd.size != n_in or pin.size != len(pts):
            raise ValueError("need one seed per input and one input index per plaintext")
        cols = self.num_slots // d
        out = np.zeros((len(pts), cols), np.float64)
        _lib.check(_lib.load().th_lora_a_pass(self._h, self._own(pk), self._own(sk), _lib.ptr(h), n_in, d,
                                              _lib.ptr(sd), _lib.handle_array([self._own(p) for p in pts]),
                                              _lib.ptr(pin), len(pts), int(rescale), _lib.ptr(out)))
        return out

    def batch_decrypt_to_device(self, cts, sk: TenSafeSecretKey, dev_ptr: int):
        """Decrypt into device memory at dev_ptr (len(cts) x num_slots float64)."""
        cts = list(cts)
        if cts:
            _lib.check(_lib.load().th_batch_decrypt_device(self._h, _lib.handle_array([self._own(c) for c in cts]),
                                                           len(cts), self._own(sk), C.c_void_p(dev_ptr)))

    # ------------------------------------------------------------ data movement (tests, wire format)
    def ct_download(self, ct: TenSafeCiphertext):
        limbs = ct.num_limbs
        c0 = np.zeros((limbs, self._n), np.uint64)
        c1 = np.zeros((limbs, self._n), np.uint64)
        _lib.check(_lib.load().th_ct_download(self._h, self._own(ct), _lib.ptr(c0), _lib.ptr(c1)))
        return c0, c1

    def ct_upload(self, c0, c1, scale: float) -> TenSafeCiphertext:
        c0 = np.ascontiguousarray(c0, dtype=np.uint64)
        c1 = np.ascontiguousarray(c1, dtype=np.uint64)
        if c0.shape != c1.shape or c0.ndim != 2 or c0.shape[1] != self._n:
            raise ValueError("c0 and c1 must both have shape [limbs, N]")
        return self._new(TenSafeCiphertext, _lib.load().th_ct_upload, self._h, _lib.ptr(c0), _lib.ptr(c1),
                         c0.shape[0], float(scale))

    def sk_download(self, sk: TenSafeSecretKey) -> np.ndarray:
        out = np.zeros((self._limbs, self._n), np.uint64)
        _lib.check(_lib.load().th_sk_download(self._h, self._own(sk), _lib.ptr(out)))
        return out

    def pk_download(self, pk: TenSafePublicKey):
        b = np.zeros((self._limbs, self._n), np.uint64)
        a = np.zeros((self._limbs, self._n), np.uint64)
        _lib.check(_lib.load().th_pk_download(self._h, self._own(pk), _lib.ptr(b), _lib.ptr(a)))
        return b, a

    def pt_download(self, pt: TenSafePlaintext) -> np.ndarray:
        out = np.zeros((self._limbs, self._n), np.uint64)
        _lib.check(_lib.load().th_pt_download(self._h, self._own(pt), _lib.ptr(out)))
        return out

    def _export(self, obj, fn) -> bytes:
        n = C.c_size_t()
        f = getattr(_lib.load(), fn)
        _lib.check(f(self._h, self._own(obj), None, 0, C.byref(n)))
        buf = np.zeros(n.value, np.uint8)
        _lib.check(f(self._h, self._own(obj), _lib.ptr(buf), buf.size, C.byref(n)))
        return buf.tobytes()

    def ct_from_bytes(self, data: bytes, num_limbs: Optional[int] = None) -> TenSafeCiphertext:
        """serialize.rs:80-93 (num_limbs defaults to the context's chain length)."""
        b = np.frombuffer(data, np.uint8).copy()
        limbs = self._limbs if num_limbs is None else num_limbs
        return self._new(TenSafeCiphertext, _lib.load().th_ct_import, self._h, _lib.ptr(b), b.size, limbs)

    def pk_from_bytes(self, data: bytes) -> TenSafePublicKey:
        b = np.frombuffer(data, np.uint8).copy()
        return self._new(TenSafePublicKey, _lib.load().th_pk_import, self._h, _lib.ptr(b), b.size)

    def ntt_forward(self, polys: np.ndarray) -> np.ndarray:
        """Forward NTT of [count, limbs, N] (or [limbs, N]) uint64 residues; returns a copy."""
        return self._ntt(polys, "th_ntt_forward_batch")

    def ntt_inverse(self, polys: np.ndarray) -> np.ndarray:
        return self._ntt(polys, "th_ntt_inverse_batch")

    def _ntt(self, polys, fn):
        x = np.array(polys, dtype=np.uint64, order="C", copy=True)
        if x.shape[-1] != self._n:
            raise ValueError(f"last dimension must be N={self._n}")
        limbs = x.shape[-2] if x.ndim >= 2 else 1
        count = x.size // (limbs * self._n)
        _lib.check(getattr(_lib.load(), fn)(self._h, _lib.ptr(x), count, limbs, 0))
        return x

    def sync(self):
        rc = _lib.load().th_ctx_sync(self._h)
        if rc:
            _lib.check(rc)

    def set_sampler(self, where: str):
        """Where seeded encrypt_pk draws its randomness: "device" (default) or "host"."""
        value = {"device": _lib.TH_SAMPLER_DEVICE, "host": _lib.TH_SAMPLER_HOST}.get(where)
        if value is None:
            raise ValueError("sampler must be 'device' or 'host'")
        _lib.check(_lib.load().th_ctx_set_option(self._h, _lib.TH_OPT_SAMPLER, value))

    def set_sampler_band(self, log2_band: int):
        """Band of the device sampler's boundary check: Gaussian draws whose
        z * 3.19 lies within 2**log2_band of a rounding boundary are drawn
        again on the host with glibc (default -36)."""
        _lib.check(_lib.load().th_ctx_set_option(self._h, _lib.TH_OPT_SAMPLER_BAND, int(log2_band)))

    def redrawn_inputs(self) -> int:
        """How many encrypt_pk inputs the host has drawn again after the band check."""
        v = C.c_uint64()
        _lib.check(_lib.load().th_ctx_stats(self._h, C.byref(v)))
        return v.value

    def _rescale_decrypt_kernels(self, which: str):
        """Testing hook: the kernels LoRA sets created afterwards rescale and
        decrypt with: "auto" (default), "split" or "whole" (one workgroup per
        product wherever it serves); the results are the same bit for bit."""
        value = {"auto": _lib.TH_RD_AUTO, "split": _lib.TH_RD_SPLIT, "whole": _lib.TH_RD_WHOLE}[which]
        _lib.check(_lib.load().th_ctx_set_option(self._h, _lib.TH_OPT_RESCALE_DECRYPT, value))

    def _force_serial_sampler(self, on: bool):
        """Testing hook: replay every device stream serially (the rejection path)."""
        _lib.check(_lib.load().th_ctx_set_option(self._h, _lib.TH_OPT_FORCE_SERIAL_SAMPLER, int(on)))

    def _own(self, obj):
        if obj is None or not isinstance(obj, _Handle):
            raise TypeError("expected a tensafe_he key, plaintext or ciphertext object")
        if obj._ctx is not self:
            raise ValueError("object belongs to a different CkksContext")
        return obj._h
