"""ZeRo-MOAI column-packed ct x pt LoRA-A matvec on the HIP engine.

Restates the encrypted branch of the engine's `_he_lora_delta`
(demonstrator/server/inference_engine.py:1244-1405) and its plaintext cache
(`_precompute_he_cache`, :1037-1074; spec docs/ZERO_MOAI.md:45-165):

  cols_per_ct = S // d            (:1258)
  n_batches   = ceil(rank / cols) (:1259)
  replicate h into cols segments of d slots, encrypt once         (:1266-1272)
  pt_b packs rows b*cols .. into the same segments                (:1300-1308)
  ct_b = ct_rep * pt_b  (no rotation)                             (:1311)
  intermediate[r] = sum of segment i of decrypt(ct_b)             (:1379-1386)
  delta = B @ intermediate                                        (:1392)

Here all inputs of a token go through one encrypt_pk batch, all products
through one launch, the optional rescale through one batch, and all
decryptions through one GPU batch that returns only the segment sums.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Sequence

import numpy as np

from .tensafe_he import CkksContext, TenSafePlaintext, TenSafePublicKey, TenSafeSecretKey


def layout(simd_slots: int, d_model: int, rank: int):
    cols = max(1, simd_slots // d_model)
    return cols, math.ceil(rank / cols)


def replicate(h: np.ndarray, simd_slots: int, d_model: int) -> np.ndarray:
    """[h | h | ... | 0] with cols copies (inference_engine.py:1266-1269)."""
    cols = max(1, simd_slots // d_model)
    out = np.zeros(simd_slots, np.float64)
    hv = np.asarray(h, np.float64).ravel()[:d_model]
    for i in range(cols):
        out[i * d_model: i * d_model + hv.size] = hv
    return out


def pack_rows(lora_a: np.ndarray, simd_slots: int) -> List[np.ndarray]:
    """Packed plaintext batches of LoRA-A rows (inference_engine.py:1037-1074)."""
    rank, d = lora_a.shape
    cols, nb = layout(simd_slots, d, rank)
    pts = []
    for b in range(nb):
        p = np.zeros(simd_slots, np.float64)
        for i, r in enumerate(range(b * cols, min((b + 1) * cols, rank))):
            p[i * d:(i + 1) * d] = lora_a[r].astype(np.float64)
        pts.append(p)
    return pts


@dataclass
class Adapter:
    """One projection's LoRA pair with its cached NTT-domain plaintext batches."""

    lora_a: np.ndarray  # [rank, d]
    lora_b: np.ndarray  # [d_out, rank]
    pts: List[TenSafePlaintext] = field(default_factory=list)

    @property
    def rank(self) -> int:
        return self.lora_a.shape[0]

    @property
    def d_model(self) -> int:
        return self.lora_a.shape[1]


def prepare_adapter(ctx: CkksContext, lora_a: np.ndarray, lora_b: np.ndarray) -> Adapter:
    a = np.asarray(lora_a, np.float64)
    ad = Adapter(a, np.asarray(lora_b, np.float64))
    ad.pts = [ctx.encode_to_ntt(p) for p in pack_rows(a, ctx.num_slots)]
    return ad


def lora_deltas(ctx: CkksContext, pk: TenSafePublicKey, sk: TenSafeSecretKey, hidden: Sequence[np.ndarray],
                seeds: Sequence[int], adapters: Sequence[Sequence[Adapter]], rescale: bool = True):
    """Encrypted LoRA deltas for a set of inputs.

    hidden[i] is input i (length d); adapters[i] lists the projections that
    read input i (e.g. q and v of one layer share the layer input). Returns
    (deltas, intermediates): deltas[i][j] = B_ij @ (A_ij h_i) with A_ij h_i
    computed under encryption. The whole set is one th_lora_a_pass call: one
    encrypt_pk batch, one product launch, one rescale batch and one GPU
    decrypt with a single device-to-host copy.
    """
    d = adapters[0][0].d_model
    S = ctx.num_slots
    cols = max(1, S // d)
    pts, pin, index = [], [], []
    for i, ads in enumerate(adapters):
        for j, ad in enumerate(ads):
            if ad.d_model != d:
                raise ValueError("all adapters must share d_model")
            for b, pt in enumerate(ad.pts):
                pts.append(pt)
                pin.append(i)
                index.append((i, j, b))
    H = np.stack([np.asarray(h, np.float64).ravel()[:d] for h in hidden])
    sums = ctx.lora_a_pass(pk, sk, H, seeds, pts, pin, rescale)
    inter: Dict = {}
    for row, (i, j, b) in enumerate(index):
        ad = adapters[i][j]
        vec = inter.setdefault((i, j), np.zeros(ad.rank))
        r0 = b * cols
        n = min(cols, ad.rank - r0)
        vec[r0:r0 + n] = sums[row, :n]
    deltas = [[adapters[i][j].lora_b @ inter[(i, j)] for j in range(len(adapters[i]))] for i in range(len(adapters))]
    return deltas, inter
