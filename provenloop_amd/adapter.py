"""Engine-facing adapter over the HIP CKKS engine.

Keeps the contract of the engine's `_TenSafeHEAdapter`
(demonstrator/server/inference_engine.py:148-220): `encrypt_vector`,
`decrypt_vector`, `decrypt_to_gpu`, `status()` and the same metrics keys,
so `_he_lora_delta` (:1244-1405) runs unchanged on top of it. Differences,
all toward the GPU:

  * `decrypt_to_gpu` returns a float64 torch tensor on the context's ROCm
    device, written by the GPU decrypt + decode kernels (no host round trip);
  * `batch_decrypt_to_gpu` decrypts a list of ciphertexts into one
    [n, slots] device tensor with a single launch sequence;
  * `status()` reports the GPU engine.

`init_tensafe_he` mirrors the "Try 0" block of `_init_ckks` (:626-652).
"""
from __future__ import annotations

import os
import time
from typing import Optional, Sequence

import numpy as np

from . import tensafe_he
from .tensafe_he import CkksContext, TenSafeCiphertext, TenSafeSecretKey


class TenSafeHEAdapter:
    def __init__(self, ctx: CkksContext, sk: TenSafeSecretKey):
        self._ctx = ctx
        self._sk = sk
        self._slots = ctx.num_slots
        self._metrics = {
            "total_encryptions": 0,
            "total_decryptions": 0,
            "total_encrypt_ms": 0.0,
            "total_decrypt_ms": 0.0,
        }

    @property
    def context(self) -> CkksContext:
        return self._ctx

    def encrypt_vector(self, data: np.ndarray) -> TenSafeCiphertext:
        """Secret-key encryption of the flattened data, zero-padded to the slot count (:166-176)."""
        self._metrics["total_encryptions"] += 1
        t0 = time.perf_counter()
        padded = np.zeros(self._slots, dtype=np.float64)
        flat = np.asarray(data).flatten().astype(np.float64)
        n = min(len(flat), self._slots)
        padded[:n] = flat[:n]
        ct = self._ctx.encrypt(padded, self._sk)
        self._metrics["total_encrypt_ms"] += (time.perf_counter() - t0) * 1000
        return ct

    def decrypt_vector(self, ct: TenSafeCiphertext) -> np.ndarray:
        """Decrypt + decode to a host float64 vector of `slots` values (:178-188)."""
        self._metrics["total_decryptions"] += 1
        t0 = time.perf_counter()
        result = np.asarray(self._ctx.decrypt(ct, self._sk), dtype=np.float64)
        self._metrics["total_decrypt_ms"] += (time.perf_counter() - t0) * 1000
        return result

    def _device(self):
        import torch

        return torch.device("cuda", self._ctx.device)

    def batch_decrypt_to_gpu(self, cts: Sequence[TenSafeCiphertext]):
        """Decrypt every ciphertext into one [len(cts), slots] float64 device tensor."""
        import torch

        cts = list(cts)
        self._metrics["total_decryptions"] += len(cts)
        t0 = time.perf_counter()
        out = torch.empty((len(cts), self._slots), dtype=torch.float64, device=self._device())
        if cts:
            # the allocation is ordered on torch's stream; finish it before the engine's stream writes
            torch.cuda.current_stream(out.device).synchronize()
            self._ctx.batch_decrypt_to_device(cts, self._sk, out.data_ptr())
        self._metrics["total_decrypt_ms"] += (time.perf_counter() - t0) * 1000
        return out

    def decrypt_to_gpu(self, ct: TenSafeCiphertext):
        """Decrypt and keep the slots on the GPU as a float64 torch tensor (:190-205, :262-275)."""
        return self.batch_decrypt_to_gpu([ct])[0]

    def status(self) -> dict:
        info = self._ctx.get_backend_info()
        return {
            "backend": info.get("backend", "tensafe-he-hip"),
            "version": info.get("version"),
            "initialized": True,
            "gpu_available": True,
            "gpu_enabled": True,
            "gpu_accelerated": True,
            "gpu_device": info.get("device"),
            "poly_mod_degree": self._slots * 2,
            "emulated": False,
            "metrics": dict(self._metrics),
        }


def init_tensafe_he(poly_modulus_degree: int = 16384, device: int = 0, sk_seed: Optional[int] = None):
    """Mirror of `_init_ckks` Try 0 (:630-652): context, secret key, adapter.

    TENSAFE_POLY_N overrides the degree when it names a supported one.
    Returns (adapter, simd_slots). Raises if the HIP engine cannot run here
    (no gfx950 device, library not built): the engine then falls through to
    its next tier exactly as it does when `import tensafe_he` fails.
    """
    poly_n = int(os.environ.get("TENSAFE_POLY_N", "0"))
    if poly_n not in (8192, 16384, 32768):
        poly_n = poly_modulus_degree
    ctx = tensafe_he.CkksContext(poly_mod_degree=poly_n, device=device)
    sk = ctx.keygen(sk_seed)
    adapter = TenSafeHEAdapter(ctx, sk)
    return adapter, ctx.num_slots
