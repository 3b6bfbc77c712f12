"""ctypes binding of libtensafe_he_hip.so (the C ABI in include/tensafe_he.h).

The library is loaded from this package directory only. There is no fallback:
if the library is missing or no gfx950 device is present, the calls fail with
an error naming the problem.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtensafe_he_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "tensafe_he.h")

TH_OK, TH_EINVAL, TH_EDEVICE, TH_ENOMEM, TH_ESTATE = 0, -1, -2, -3, -4
TH_OPT_SAMPLER, TH_OPT_FORCE_SERIAL_SAMPLER, TH_OPT_SAMPLER_BAND, TH_OPT_RESCALE_DECRYPT = 1, 2, 3, 4
TH_RD_AUTO, TH_RD_SPLIT, TH_RD_WHOLE = 0, 1, 2
TH_SAMPLER_DEVICE, TH_SAMPLER_HOST = 0, 1
TH_LORA_RESCALE, TH_LORA_SK_FUSED = 1, 2
TH_LORA_CT_INPUT, TH_LORA_CT_PRODUCT = 0, 1

VP = C.c_void_p
SZ = C.c_size_t
U32 = C.c_uint32
U64 = C.c_uint64
I32 = C.c_int
PVP = C.POINTER(C.c_void_p)

_SIGS = {
    "th_last_error": (C.c_char_p, []),
    "th_version": (C.c_char_p, []),
    "th_device_count": (I32, [C.POINTER(I32)]),
    "th_ctx_create": (I32, [U32, VP, U32, U32, I32, PVP]),
    "th_ctx_free": (I32, [VP]),
    "th_ctx_info": (I32, [VP, C.POINTER(U32), C.POINTER(U32), VP]),
    "th_ctx_sync": (I32, [VP]),
    "th_ctx_stream": (I32, [VP, PVP]),
    "th_ctx_set_option": (I32, [VP, I32, C.c_int64]),
    "th_ctx_stats": (I32, [VP, C.POINTER(U64)]),
    "th_keygen": (I32, [VP, U64, I32, PVP]),
    "th_keygen_public": (I32, [VP, VP, U64, I32, PVP]),
    "th_sk_free": (I32, [VP]),
    "th_pk_free": (I32, [VP]),
    "th_sk_download": (I32, [VP, VP, VP]),
    "th_pk_download": (I32, [VP, VP, VP, VP]),
    "th_encrypt": (I32, [VP, VP, VP, SZ, U64, I32, PVP]),
    "th_encrypt_batch": (I32, [VP, VP, VP, VP, SZ, SZ, U64, I32, VP]),
    "th_encrypt_pk": (I32, [VP, VP, VP, SZ, U64, I32, PVP]),
    "th_encrypt_pk_explicit": (I32, [VP, VP, VP, SZ, VP, VP, VP, PVP]),
    "th_encrypt_pk_batch": (I32, [VP, VP, VP, SZ, SZ, SZ, VP, VP]),
    "th_encode_to_ntt": (I32, [VP, VP, SZ, PVP]),
    "th_pt_free": (I32, [VP]),
    "th_pt_download": (I32, [VP, VP, VP]),
    "th_ct_pt_mul": (I32, [VP, VP, VP, SZ, PVP]),
    "th_ct_pt_mul_ntt": (I32, [VP, VP, VP, PVP]),
    "th_ct_pt_mul_ntt_batch": (I32, [VP, VP, VP, SZ, VP]),
    "th_ct_add": (I32, [VP, VP, VP, PVP]),
    "th_ct_sub": (I32, [VP, VP, VP, PVP]),
    "th_rescale": (I32, [VP, VP, PVP]),
    "th_rescale_batch": (I32, [VP, VP, SZ, VP]),
    "th_decrypt": (I32, [VP, VP, VP, VP]),
    "th_batch_decrypt": (I32, [VP, VP, SZ, VP, VP]),
    "th_batch_decrypt_segsum": (I32, [VP, VP, SZ, VP, U32, U32, VP]),
    "th_batch_decrypt_device": (I32, [VP, VP, SZ, VP, VP]),
    "th_batch_decrypt_segsum_noalloc": (I32, [VP, VP, SZ, VP, U32, U32, VP]),
    "th_lora_a_pass": (I32, [VP, VP, VP, VP, U32, U32, VP, VP, VP, U32, I32, VP]),
    "th_lora_create": (I32, [VP, U32, U32, U32, VP, VP, VP, VP, VP, PVP]),
    "th_lora_create_moe": (I32, [VP, U32, U32, U32, VP, VP, VP, U32, VP, VP, VP, PVP]),
    "th_lora_set_gates": (I32, [VP, VP, VP]),
    "th_lora_free": (I32, [VP]),
    "th_lora_info": (I32, [VP, C.POINTER(U64), C.POINTER(U32), C.POINTER(U32)]),
    "th_lora_deltas": (I32, [VP, VP, VP, VP, VP, I32, VP, I32, VP, I32, VP]),
    "th_lora_ct": (I32, [VP, VP, I32, U32, PVP]),
    "th_ct_free": (I32, [VP]),
    "th_ct_info": (I32, [VP, C.POINTER(U32), C.POINTER(C.c_double)]),
    "th_ct_download": (I32, [VP, VP, VP, VP]),
    "th_ct_upload": (I32, [VP, VP, VP, U32, C.c_double, PVP]),
    "th_ct_export": (I32, [VP, VP, VP, SZ, C.POINTER(SZ)]),
    "th_ct_import": (I32, [VP, VP, SZ, U32, PVP]),
    "th_pk_export": (I32, [VP, VP, VP, SZ, C.POINTER(SZ)]),
    "th_pk_import": (I32, [VP, VP, SZ, PVP]),
    "th_ntt_forward_batch": (I32, [VP, VP, SZ, U32, I32]),
    "th_ntt_inverse_batch": (I32, [VP, VP, SZ, U32, I32]),
    "th_dev_alloc": (I32, [VP, SZ, PVP]),
    "th_dev_free": (I32, [VP, VP]),
    "th_memcpy_h2d": (I32, [VP, VP, VP, SZ]),
    "th_memcpy_d2h": (I32, [VP, VP, VP, SZ]),
    "th_ntt_time": (I32, [VP, VP, SZ, U32, I32, I32, C.POINTER(C.c_float)]),
}

_lib = None


class HipEngineError(RuntimeError):
    """A failure reported by the HIP engine (device missing, HIP error, bad state)."""


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Function names declared in include/tensafe_he.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(th_[a-z0-9_]+)\s*\(", text)))


def _share_hip_runtime_with_torch():
    """Make the library and PyTorch use ONE HIP runtime in this process.

    PyTorch-ROCm wheels carry their own libamdhip64 / libhsa-runtime64 and
    load them under the unversioned name, while this library links the
    system ROCm's libamdhip64.so.7. Loaded in that order, a process would hold
    two HIP runtimes and the second to initialise finds no GPU. PyTorch's copy
    has the same soname (libamdhip64.so.7), so importing torch first lets the
    dynamic loader bind this library to the runtime already in the process.
    Without torch installed the system runtime is used.
    """
    if "torch" in sys.modules:
        return
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load():
    """Load the library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipEngineError(
            f"{LIB_PATH} is missing: build it with `make -C provenloop_amd/csrc` "
            "(or __graft_entry__.build()); there is no CPU fallback")
    _share_hip_runtime_with_torch()
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    return load().th_last_error().decode(errors="replace")


def check(rc: int):
    if rc == TH_OK:
        return
    msg = last_error()
    if rc == TH_EINVAL:
        raise ValueError(msg)
    if rc == TH_ESTATE:
        raise RuntimeError(msg)
    if rc == TH_ENOMEM:
        raise MemoryError(msg)
    raise HipEngineError(msg)


def device_count() -> int:
    n = I32(0)
    check(load().th_device_count(C.byref(n)))
    return n.value


def ptr(a: np.ndarray):
    return VP(a.ctypes.data)  # half the cost of a.ctypes.data_as(VP) per call


def handle_array(objs) -> C.Array:
    arr = (VP * max(1, len(objs)))()
    for i, o in enumerate(objs):
        arr[i] = o
    return arr
