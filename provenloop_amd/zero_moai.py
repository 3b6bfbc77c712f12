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
decryptions through one GPU batch that returns only the segment sums
(`lora_deltas`, one th_lora_a_pass call). `LoraSet` keeps the plaintexts,
the LoRA-B matrices and the token's working memory on the device and also
applies B on the GPU (th_lora_create / th_lora_deltas), so a token is one
call with one stream synchronisation and, if the caller keeps its hidden
states and deltas in HBM, no host transfer at all.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field
from typing import Dict, List, Sequence

import numpy as np

from . import _lib
from .tensafe_he import CkksContext, TenSafeCiphertext, TenSafePlaintext, TenSafePublicKey, TenSafeSecretKey


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


def softmax_gate(seed: int, n_experts: int) -> np.ndarray:
    """CryptoMOE gate: softmax over a seeded logit vector.

    The reference routes each query to one adapter by keyword step-gates
    (inference_engine.py:1155-1171) and has no gated combination; this rule
    is the library's own: logits ~ N(0, 1) from numpy's PCG64 stream seeded
    with `seed`, g = exp(l - max l) / sum exp(l - max l)."""
    logits = np.random.default_rng(seed).standard_normal(n_experts)
    w = np.exp(logits - logits.max())
    return w / w.sum()


class LoraSet:
    """LoRA projections resident on the device (th_lora_create).

    `projections` lists (input_index, lora_a [rank, d], lora_b [d_out, rank])
    for every projection; projections that read the same input (q and v of
    one layer) share that input's ciphertext. `deltas()` runs one token of
    the encrypted path for all of them with one stream synchronisation:
    encrypt_pk per input, ct x pt per packed batch, rescale, batched decrypt
    with segment sums and B @ intermediate, all on the GPU.

    CryptoMOE (th_lora_create_moe): with `gates` [n_proj, k], lora_a is
    [k, rank, d] and lora_b [k, d_out, rank] (k expert adapters per
    projection). Each batch's ciphertext is then the ct_add of the k
    experts' products with their gate-scaled plaintexts g_x A_x, so the
    decrypted intermediate is sum_x g_x A_x h, and the deltas are
    (sum_x g_x B_x) @ intermediate. `set_gates()` replaces the gates (a gate
    that changes per token) on the device.
    """

    def __init__(self, ctx: CkksContext, n_inputs: int, projections, gates=None):
        self._ctx = ctx
        self._lib = _lib.load()
        projections = list(projections)
        if not projections:
            raise ValueError("need at least one projection")
        self.n_inputs = int(n_inputs)
        A = [np.ascontiguousarray(a, np.float64) for _, a, _ in projections]
        B = [np.ascontiguousarray(b, np.float64) for _, _, b in projections]
        if gates is None:
            k = 1
            A = [a[None] for a in A]
            B = [b[None] for b in B]
        else:
            G = np.ascontiguousarray(gates, np.float64)
            if G.ndim != 2 or G.shape[0] != len(A):
                raise ValueError("gates must be [n_proj, n_experts]")
            k = G.shape[1]
        if any(a.ndim != 3 or a.shape[0] != k for a in A) or any(b.ndim != 3 or b.shape[0] != k for b in B):
            raise ValueError("with gates, lora_a must be [k, rank, d] and lora_b [k, d_out, rank]")
        d = A[0].shape[2]
        for a, b in zip(A, B):
            if a.shape[2] != d:
                raise ValueError("every lora_a must be [rank, d] with the same d")
            if b.shape[2] != a.shape[1]:
                raise ValueError("lora_b must be [d_out, rank]")
        self.d = d
        self.n_experts = k
        self.d_out = [b.shape[1] for b in B]
        self.offsets = np.concatenate([[0], np.cumsum(self.d_out)]).astype(int)
        inp = np.array([int(i) for i, _, _ in projections], np.uint32)
        ranks = np.array([a.shape[1] for a in A], np.uint32)
        dout = np.array(self.d_out, np.uint32)
        aptr = (C.c_void_p * (len(A) * k))(*[a[x].ctypes.data for a in A for x in range(k)])
        bptr = (C.c_void_p * (len(B) * k))(*[b[x].ctypes.data for b in B for x in range(k)])
        self._keep = (A, B)
        out = C.c_void_p()
        if gates is None:
            _lib.check(self._lib.th_lora_create(ctx._h, self.n_inputs, d, len(A), _lib.ptr(inp), _lib.ptr(ranks),
                                                _lib.ptr(dout), aptr, bptr, C.byref(out)))
        else:
            _lib.check(self._lib.th_lora_create_moe(ctx._h, self.n_inputs, d, len(A), _lib.ptr(inp),
                                                    _lib.ptr(ranks), _lib.ptr(dout), k, _lib.ptr(G), aptr, bptr,
                                                    C.byref(out)))
        self._h = out
        nd, nb, cols = C.c_uint64(), C.c_uint32(), C.c_uint32()
        _lib.check(self._lib.th_lora_info(self._h, C.byref(nd), C.byref(nb), C.byref(cols)))
        self.n_deltas, self.n_batches, self.cols = nd.value, nb.value, cols.value

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and getattr(_lib, "_lib", None) is not None:
            _lib._lib.th_lora_free(h)
            self._h = None

    def set_gates(self, gates):
        """Replace the gates [n_proj, k] of a set created with gates
        (th_lora_set_gates): queued on the context stream, so the next
        deltas()/deltas_device() call uses them, bit for bit as a set created
        with these gates."""
        G = np.ascontiguousarray(gates, np.float64)
        if G.shape != (len(self.d_out), self.n_experts):
            raise ValueError(f"gates must be [{len(self.d_out)}, {self.n_experts}]")
        _lib.check(self._lib.th_lora_set_gates(self._ctx._h, self._h, _lib.ptr(G)))

    @staticmethod
    def _mode(rescale: bool, sk_fused: bool) -> int:
        return (_lib.TH_LORA_RESCALE if rescale else 0) | (_lib.TH_LORA_SK_FUSED if sk_fused else 0)

    def deltas(self, pk: TenSafePublicKey, sk: TenSafeSecretKey, hidden, seeds, rescale: bool = True,
               with_intermediates: bool = False, sk_fused: bool = False):
        """Host in, host out: hidden [n_inputs, d] -> list of per-projection deltas.

        By default the token forms every ciphertext of the reference's
        client/server sequence (encrypt_pk, ct x pt and rescale without the
        secret key; the batched decrypt reads only what it decodes).
        sk_fused=True takes the single-party shortcut (TH_LORA_SK_FUSED): the
        same deltas bit for bit, no complete ciphertext formed."""
        H = np.ascontiguousarray(hidden, np.float64)
        if H.shape != (self.n_inputs, self.d):
            raise ValueError(f"hidden must be [{self.n_inputs}, {self.d}]")
        sd = np.ascontiguousarray(seeds, np.uint64)
        if sd.shape != (self.n_inputs,):
            raise ValueError("need one seed per input")
        out = np.empty(self.n_deltas, np.float64)
        inter = np.empty((self.n_batches, self.cols), np.float64) if with_intermediates else None
        _lib.check(self._lib.th_lora_deltas(self._ctx._h, self._h, self._ctx._own(pk), self._ctx._own(sk),
                                            _lib.ptr(H), 0, _lib.ptr(sd), self._mode(rescale, sk_fused), _lib.ptr(out), 0,
                                            None if inter is None else _lib.ptr(inter)))
        parts = [out[self.offsets[j]:self.offsets[j + 1]] for j in range(len(self.d_out))]
        return (parts, inter) if with_intermediates else parts

    def deltas_device(self, pk: TenSafePublicKey, sk: TenSafeSecretKey, hidden_dev: int, seeds, dev_out: int,
                      rescale: bool = True, sk_fused: bool = False):
        """Device in, device out: hidden_dev points at n_inputs x d doubles in
        HBM, dev_out receives n_deltas doubles. Only queues the token on the
        context stream (no host synchronisation): call ctx.sync(), or order
        later work after ctx's stream, before reading dev_out."""
        sd = np.ascontiguousarray(seeds, np.uint64)
        if sd.shape != (self.n_inputs,):
            raise ValueError("need one seed per input")
        # plain ints for the pointer arguments (the binding declares them
        # c_void_p): this call is on the per-token path
        rc = self._lib.th_lora_deltas(self._ctx._h, self._h, self._ctx._own(pk), self._ctx._own(sk), hidden_dev, 1,
                                      sd.ctypes.data, self._mode(rescale, sk_fused), dev_out, 1, None)
        if rc:
            _lib.check(rc)

    def ciphertext(self, which: str, index: int) -> TenSafeCiphertext:
        """A copy of a ciphertext the last token formed (th_lora_ct): which =
        "input" (the encrypt_pk output of input `index`) or "product" (batch
        `index`'s ct x pt, rescaled if the token rescaled). Raises
        RuntimeError after a sk_fused token, which forms none."""
        w = {"input": _lib.TH_LORA_CT_INPUT, "product": _lib.TH_LORA_CT_PRODUCT}[which]
        out = C.c_void_p()
        _lib.check(self._lib.th_lora_ct(self._ctx._h, self._h, w, int(index), C.byref(out)))
        return TenSafeCiphertext(out, self._ctx)
