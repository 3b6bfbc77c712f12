"""ctypes wrapper of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY. The oracle is a C++ restatement of the reference CPU
CKKS backend (tensafe-he/crates/tensafe-he-core/src/*.rs). It is imported only
by tests/, by ``__graft_entry__.smoke()`` and by bench.py's CPU-baseline leg,
always as the source of expected results or the timed baseline, never as the
thing measured or shipped. The product path (provenloop_amd) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB selects another build of the same sources (the sanitizer build)
_LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
VP = C.c_void_p
SZ = C.c_size_t
U64 = C.c_uint64


class OracleError(RuntimeError):
    pass


def build():
    """Compile liboracle.so with the committed Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise OracleError(f"{_LIB_PATH} is not built; run `make -C oracle`")
    L = C.CDLL(_LIB_PATH)
    sig = {
        "orc_last_error": (C.c_char_p, []),
        "orc_default_chain": (C.c_int, [SZ, u64p, C.POINTER(SZ)]),
        "orc_custom_chain": (C.c_int, [SZ, u32p, SZ, u64p]),
        "orc_modulus": (C.c_int, [U64, C.POINTER(U64), C.POINTER(U64)]),
        "orc_is_prime": (C.c_int, [U64]),
        "orc_mod_add": (U64, [U64, U64, U64]),
        "orc_mod_sub": (U64, [U64, U64, U64]),
        "orc_mod_mul": (U64, [U64, U64, U64]),
        "orc_mod_pow": (U64, [U64, U64, U64]),
        "orc_mod_inv": (C.c_int, [U64, U64, C.POINTER(U64)]),
        "orc_bit_reverse": (C.c_uint32, [C.c_uint32, C.c_uint32]),
        "orc_find_primitive_root": (C.c_int, [SZ, U64, C.POINTER(U64)]),
        "orc_barrett_reduce": (C.c_int, [u64p, u64p, SZ, U64, u64p]),
        "orc_mod_mul_barrett": (C.c_int, [u64p, u64p, SZ, U64, u64p]),
        "orc_ntt_tables": (C.c_int, [SZ, U64, u64p, u64p, C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
        "orc_ntt_forward": (C.c_int, [u64p, SZ, SZ, U64]),
        "orc_ntt_inverse": (C.c_int, [u64p, SZ, SZ, U64]),
        "orc_chacha20_block": (None, [u32p, u32p]),
        "orc_rng_u32": (C.c_int, [U64, SZ, u32p]),
        "orc_rng_u64": (C.c_int, [U64, SZ, u64p]),
        "orc_rng_range_u32": (C.c_int, [U64, C.c_uint32, SZ, u32p]),
        "orc_rng_range_u64": (C.c_int, [U64, U64, SZ, u64p]),
        "orc_rng_f64": (C.c_int, [U64, SZ, f64p]),
        "orc_rng_gaussian": (C.c_int, [U64, C.c_double, SZ, f64p]),
        "orc_rng_entropy_u64": (C.c_int, [SZ, u64p]),
        "orc_sample_ternary": (C.c_int, [U64, SZ, U64, u64p]),
        "orc_sample_gaussian": (C.c_int, [U64, SZ, U64, C.c_double, u64p]),
        "orc_sample_gaussian_signed": (C.c_int, [U64, SZ, C.c_double, i64p]),
        "orc_sample_uniform": (C.c_int, [U64, SZ, U64, u64p]),
        "orc_encrypt_pk_randomness": (C.c_int, [U64, SZ, u8p, i64p, i64p]),
        "orc_ctx_new": (C.c_int, [SZ, VP, SZ, C.POINTER(VP)]),
        "orc_ctx_free": (None, [VP]),
        "orc_sk_free": (None, [VP]),
        "orc_pk_free": (None, [VP]),
        "orc_ct_free": (None, [VP]),
        "orc_poly_free": (None, [VP]),
        "orc_fft_tables": (C.c_int, [VP, f64p, f64p, f64p, f64p]),
        "orc_encode": (C.c_int, [VP, f64p, SZ, u64p]),
        "orc_decode": (C.c_int, [VP, u64p, SZ, C.c_double, f64p]),
        "orc_decode_coefficients": (C.c_int, [VP, f64p, f64p]),
        "orc_keygen": (C.c_int, [VP, U64, C.POINTER(VP)]),
        "orc_sk_data": (C.c_int, [VP, u64p]),
        "orc_keygen_public": (C.c_int, [VP, VP, U64, C.POINTER(VP)]),
        "orc_pk_data": (C.c_int, [VP, u64p, u64p]),
        "orc_encrypt": (C.c_int, [VP, f64p, SZ, VP, U64, C.POINTER(VP)]),
        "orc_encrypt_pk": (C.c_int, [VP, f64p, SZ, VP, U64, C.POINTER(VP)]),
        "orc_batch_encrypt": (C.c_int, [VP, f64p, VP, SZ, SZ, VP, U64, VP]),
        "orc_encrypt_pk_with": (C.c_int, [VP, f64p, SZ, VP, u8p, i64p, i64p, C.POINTER(VP)]),
        "orc_ct_info": (C.c_int, [VP, C.POINTER(SZ), C.POINTER(C.c_double)]),
        "orc_ct_data": (C.c_int, [VP, u64p, u64p]),
        "orc_ct_from_data": (C.c_int, [VP, u64p, u64p, SZ, C.c_double, C.POINTER(VP)]),
        "orc_decrypt": (C.c_int, [VP, VP, VP, f64p]),
        "orc_ct_pt_mul": (C.c_int, [VP, VP, f64p, SZ, C.POINTER(VP)]),
        "orc_encode_to_ntt": (C.c_int, [VP, f64p, SZ, C.POINTER(VP)]),
        "orc_poly_data": (C.c_int, [VP, u64p]),
        "orc_ct_pt_mul_ntt": (C.c_int, [VP, VP, VP, C.POINTER(VP)]),
        "orc_ct_add": (C.c_int, [VP, VP, VP, C.POINTER(VP)]),
        "orc_ct_sub": (C.c_int, [VP, VP, VP, C.POINTER(VP)]),
        "orc_rescale": (C.c_int, [VP, VP, C.POINTER(VP)]),
        "orc_ct_to_bytes": (C.c_int, [VP, VP, SZ, C.POINTER(SZ)]),
        "orc_ct_from_bytes": (C.c_int, [u8p, SZ, SZ, SZ, C.POINTER(VP)]),
        "orc_pk_to_bytes": (C.c_int, [VP, VP, SZ, C.POINTER(SZ)]),
        "orc_pk_from_bytes": (C.c_int, [u8p, SZ, SZ, SZ, C.POINTER(VP)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _check(rc):
    if rc != 0:
        raise OracleError(lib().orc_last_error().decode())


def _f64(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64).ravel())


# ---------------------------------------------------------------------------
# parameters and scalar arithmetic (params.rs, rns.rs)
# ---------------------------------------------------------------------------
def default_chain(n):
    out = np.zeros(16, np.uint64)
    L = SZ()
    _check(lib().orc_default_chain(n, out, C.byref(L)))
    return [int(v) for v in out[: L.value]]


def custom_chain(n, bits):
    b = np.asarray(bits, np.uint32)
    out = np.zeros(len(b), np.uint64)
    _check(lib().orc_custom_chain(n, b, len(b), out))
    return [int(v) for v in out]


def barrett_constant(q):
    hi, lo = U64(), U64()
    _check(lib().orc_modulus(q, C.byref(hi), C.byref(lo)))
    return hi.value, lo.value


def is_prime(n):
    return bool(lib().orc_is_prime(n))


def mod_add(a, b, q):
    return lib().orc_mod_add(a, b, q)


def mod_sub(a, b, q):
    return lib().orc_mod_sub(a, b, q)


def mod_mul(a, b, q):
    return lib().orc_mod_mul(a, b, q)


def mod_pow(a, e, q):
    return lib().orc_mod_pow(a, e, q)


def mod_inv(a, q):
    out = U64()
    _check(lib().orc_mod_inv(a, q, C.byref(out)))
    return out.value


def bit_reverse(x, bits):
    return lib().orc_bit_reverse(x, bits)


def find_primitive_root(n, q):
    out = U64()
    _check(lib().orc_find_primitive_root(n, q, C.byref(out)))
    return out.value


def barrett_reduce(lo, hi, q):
    lo = np.ascontiguousarray(lo, np.uint64)
    hi = np.ascontiguousarray(hi, np.uint64)
    out = np.zeros(lo.size, np.uint64)
    _check(lib().orc_barrett_reduce(lo, hi, lo.size, q, out))
    return out


def mod_mul_barrett(a, b, q):
    a = np.ascontiguousarray(a, np.uint64)
    b = np.ascontiguousarray(b, np.uint64)
    out = np.zeros(a.size, np.uint64)
    _check(lib().orc_mod_mul_barrett(a, b, a.size, q, out))
    return out


# ---------------------------------------------------------------------------
# NTT (ntt.rs)
# ---------------------------------------------------------------------------
def ntt_tables(n, q):
    fwd = np.zeros(n, np.uint64)
    inv = np.zeros(n, np.uint64)
    psi, psi_inv, n_inv = U64(), U64(), U64()
    _check(lib().orc_ntt_tables(n, q, fwd, inv, C.byref(psi), C.byref(psi_inv), C.byref(n_inv)))
    return dict(fwd=fwd, inv=inv, psi=psi.value, psi_inv=psi_inv.value, n_inv=n_inv.value)


def ntt_forward(a, q):
    """Forward negacyclic NTT of each row of `a` (shape [..., N]) mod q; returns a copy."""
    x = np.array(a, dtype=np.uint64, order="C", copy=True)
    n = x.shape[-1]
    _check(lib().orc_ntt_forward(x.reshape(-1), x.size // n, n, q))
    return x


def ntt_inverse(a, q):
    x = np.array(a, dtype=np.uint64, order="C", copy=True)
    n = x.shape[-1]
    _check(lib().orc_ntt_inverse(x.reshape(-1), x.size // n, n, q))
    return x


# ---------------------------------------------------------------------------
# RNG and sampling (rng.rs, sampling.rs)
# ---------------------------------------------------------------------------
def chacha20_block(state):
    s = np.ascontiguousarray(state, np.uint32)
    out = np.zeros(16, np.uint32)
    lib().orc_chacha20_block(s, out)
    return out


def rng_u32(seed, count):
    out = np.zeros(count, np.uint32)
    _check(lib().orc_rng_u32(seed, count, out))
    return out


def rng_u64(seed, count):
    out = np.zeros(count, np.uint64)
    _check(lib().orc_rng_u64(seed, count, out))
    return out


def rng_range_u32(seed, mx, count):
    out = np.zeros(count, np.uint32)
    _check(lib().orc_rng_range_u32(seed, mx, count, out))
    return out


def rng_range_u64(seed, mx, count):
    out = np.zeros(count, np.uint64)
    _check(lib().orc_rng_range_u64(seed, mx, count, out))
    return out


def rng_f64(seed, count):
    out = np.zeros(count, np.float64)
    _check(lib().orc_rng_f64(seed, count, out))
    return out


def rng_gaussian(seed, sigma, count):
    out = np.zeros(count, np.float64)
    _check(lib().orc_rng_gaussian(seed, sigma, count, out))
    return out


def rng_entropy_u64(count):
    out = np.zeros(count, np.uint64)
    _check(lib().orc_rng_entropy_u64(count, out))
    return out


def sample_ternary(seed, n, q):
    out = np.zeros(n, np.uint64)
    _check(lib().orc_sample_ternary(seed, n, q, out))
    return out


def sample_gaussian(seed, n, q, sigma):
    out = np.zeros(n, np.uint64)
    _check(lib().orc_sample_gaussian(seed, n, q, sigma, out))
    return out


def sample_gaussian_signed(seed, n, sigma):
    out = np.zeros(n, np.int64)
    _check(lib().orc_sample_gaussian_signed(seed, n, sigma, out))
    return out


def sample_uniform(seed, n, q):
    out = np.zeros(n, np.uint64)
    _check(lib().orc_sample_uniform(seed, n, q, out))
    return out


def encrypt_pk_randomness(seed, n):
    """(u, e0, e1) that encrypt_pk draws from TenSafeRng::from_seed(seed).

    u holds the values sample_ternary(rng, n, 3) returns, v in {0, 1, 2}, which
    ciphertext.rs:261-266 maps to v=0 -> -1, v=1 -> 0, v=2 -> +1."""
    u = np.zeros(n, np.uint8)
    e0 = np.zeros(n, np.int64)
    e1 = np.zeros(n, np.int64)
    _check(lib().orc_encrypt_pk_randomness(seed, n, u, e0, e1))
    return u, e0, e1


# ---------------------------------------------------------------------------
# CKKS context (ciphertext.rs, encoding.rs, serialize.rs)
# ---------------------------------------------------------------------------
class _Handle:
    _free = None

    def __init__(self, ptr):
        self.ptr = ptr

    def __del__(self):
        if self.ptr and _lib is not None:
            getattr(_lib, self._free)(self.ptr)
            self.ptr = None


class SecretKey(_Handle):
    _free = "orc_sk_free"


class PublicKey(_Handle):
    _free = "orc_pk_free"


class Poly(_Handle):
    _free = "orc_poly_free"


class Ciphertext(_Handle):
    _free = "orc_ct_free"

    @property
    def num_limbs(self):
        L, s = SZ(), C.c_double()
        _check(lib().orc_ct_info(self.ptr, C.byref(L), C.byref(s)))
        return L.value

    @property
    def scale(self):
        L, s = SZ(), C.c_double()
        _check(lib().orc_ct_info(self.ptr, C.byref(L), C.byref(s)))
        return s.value


class Context:
    """Oracle CkksContext (ciphertext.rs:49-546). moduli=None selects for_degree(n)."""

    def __init__(self, n=16384, moduli=None):
        out = VP()
        if moduli is None:
            _check(lib().orc_ctx_new(n, None, 0, C.byref(out)))
            self.moduli = default_chain(n)
        else:
            m = np.ascontiguousarray(moduli, np.uint64)
            _check(lib().orc_ctx_new(n, m.ctypes.data, m.size, C.byref(out)))
            self.moduli = [int(v) for v in m]
        self.ptr = out
        self.n = n
        self.num_slots = n // 2
        self.L = len(self.moduli)

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.orc_ctx_free(self.ptr)
            self.ptr = None

    def _new(self, cls, fn, *args):
        out = VP()
        _check(fn(*args, C.byref(out)))
        return cls(out)

    def fft_tables(self):
        n = self.n
        tr, ti = np.zeros(n), np.zeros(n)
        sr, si = np.zeros(n - 1), np.zeros(n - 1)
        _check(lib().orc_fft_tables(self.ptr, tr, ti, sr, si))
        return tr, ti, sr, si

    def encode(self, z):
        z = _f64(z)
        out = np.zeros((self.L, self.n), np.uint64)
        _check(lib().orc_encode(self.ptr, z, z.size, out.reshape(-1)))
        return out

    def decode(self, poly, scale):
        p = np.ascontiguousarray(poly, np.uint64)
        out = np.zeros(self.num_slots)
        _check(lib().orc_decode(self.ptr, p.reshape(-1), p.shape[0], scale, out))
        return out

    def decode_coefficients(self, coeffs):
        c = _f64(coeffs)
        out = np.zeros(self.num_slots)
        _check(lib().orc_decode_coefficients(self.ptr, c, out))
        return out

    def keygen(self, seed):
        return self._new(SecretKey, lib().orc_keygen, self.ptr, seed)

    def sk_data(self, sk):
        out = np.zeros((self.L, self.n), np.uint64)
        _check(lib().orc_sk_data(sk.ptr, out.reshape(-1)))
        return out

    def keygen_public(self, sk, seed):
        return self._new(PublicKey, lib().orc_keygen_public, self.ptr, sk.ptr, seed)

    def pk_data(self, pk):
        b = np.zeros((self.L, self.n), np.uint64)
        a = np.zeros((self.L, self.n), np.uint64)
        _check(lib().orc_pk_data(pk.ptr, b.reshape(-1), a.reshape(-1)))
        return b, a

    def encrypt(self, z, sk, seed):
        z = _f64(z)
        return self._new(Ciphertext, lib().orc_encrypt, self.ptr, z, z.size, sk.ptr, seed)

    def batch_encrypt(self, arrays, sk, seed):
        """lib.rs:230-258: one seeded stream shared by every encryption, in order."""
        arrays = [_f64(a) for a in arrays]
        if not arrays:
            return []
        width = max(a.size for a in arrays)
        flat = np.zeros((len(arrays), max(width, 1)), np.float64)
        for i, a in enumerate(arrays):
            flat[i, : a.size] = a
        lens = np.array([a.size for a in arrays], np.uint64)
        outs = (VP * len(arrays))()
        _check(lib().orc_batch_encrypt(self.ptr, flat.reshape(-1), lens.ctypes.data, flat.shape[1],
                                       len(arrays), sk.ptr, seed, outs))
        return [Ciphertext(outs[i]) for i in range(len(arrays))]

    def encrypt_pk(self, z, pk, seed):
        z = _f64(z)
        return self._new(Ciphertext, lib().orc_encrypt_pk, self.ptr, z, z.size, pk.ptr, seed)

    def encrypt_pk_with(self, z, pk, u, e0, e1):
        z = _f64(z)
        return self._new(
            Ciphertext, lib().orc_encrypt_pk_with, self.ptr, z, z.size, pk.ptr,
            np.ascontiguousarray(u, np.uint8), np.ascontiguousarray(e0, np.int64),
            np.ascontiguousarray(e1, np.int64),
        )

    def ct_data(self, ct):
        L = ct.num_limbs
        c0 = np.zeros((L, self.n), np.uint64)
        c1 = np.zeros((L, self.n), np.uint64)
        _check(lib().orc_ct_data(ct.ptr, c0.reshape(-1), c1.reshape(-1)))
        return c0, c1

    def ct_from_data(self, c0, c1, scale):
        c0 = np.ascontiguousarray(c0, np.uint64)
        c1 = np.ascontiguousarray(c1, np.uint64)
        return self._new(Ciphertext, lib().orc_ct_from_data, self.ptr, c0.reshape(-1),
                         c1.reshape(-1), c0.shape[0], scale)

    def decrypt(self, ct, sk):
        out = np.zeros(self.num_slots)
        _check(lib().orc_decrypt(self.ptr, ct.ptr, sk.ptr, out))
        return out

    def ct_pt_mul(self, ct, pt):
        p = _f64(pt)
        return self._new(Ciphertext, lib().orc_ct_pt_mul, self.ptr, ct.ptr, p, p.size)

    def encode_to_ntt(self, z):
        z = _f64(z)
        return self._new(Poly, lib().orc_encode_to_ntt, self.ptr, z, z.size)

    def poly_data(self, p):
        out = np.zeros((self.L, self.n), np.uint64)
        _check(lib().orc_poly_data(p.ptr, out.reshape(-1)))
        return out

    def ct_pt_mul_ntt(self, ct, pt):
        return self._new(Ciphertext, lib().orc_ct_pt_mul_ntt, self.ptr, ct.ptr, pt.ptr)

    def ct_add(self, a, b):
        return self._new(Ciphertext, lib().orc_ct_add, self.ptr, a.ptr, b.ptr)

    def ct_sub(self, a, b):
        return self._new(Ciphertext, lib().orc_ct_sub, self.ptr, a.ptr, b.ptr)

    def rescale(self, ct):
        return self._new(Ciphertext, lib().orc_rescale, self.ptr, ct.ptr)

    def ct_to_bytes(self, ct):
        n = SZ()
        _check(lib().orc_ct_to_bytes(ct.ptr, None, 0, C.byref(n)))
        buf = np.zeros(n.value, np.uint8)
        _check(lib().orc_ct_to_bytes(ct.ptr, buf.ctypes.data, buf.size, C.byref(n)))
        return buf.tobytes()

    def ct_from_bytes(self, data, limbs):
        b = np.frombuffer(data, np.uint8).copy()
        return self._new(Ciphertext, lib().orc_ct_from_bytes, b, b.size, self.n, limbs)

    def pk_to_bytes(self, pk):
        n = SZ()
        _check(lib().orc_pk_to_bytes(pk.ptr, None, 0, C.byref(n)))
        buf = np.zeros(n.value, np.uint8)
        _check(lib().orc_pk_to_bytes(pk.ptr, buf.ctypes.data, buf.size, C.byref(n)))
        return buf.tobytes()

    def pk_from_bytes(self, data):
        b = np.frombuffer(data, np.uint8).copy()
        return self._new(PublicKey, lib().orc_pk_from_bytes, b, b.size, self.n, self.L)
