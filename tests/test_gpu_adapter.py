"""The engine adapter on the GPU: the `_TenSafeHEAdapter` contract
(demonstrator/server/inference_engine.py:148-220) and the `_he_lora_delta`
flow that uses it (:1258-1392): replicate h, encrypt once, multiply by each
packed LoRA-A batch with `ct * pt` (no rescale), decrypt on the GPU, sum the
segments.
"""
import math

import numpy as np
import pytest

from provenloop_amd import adapter as ad
from provenloop_amd import zero_moai

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def adp():
    a, slots = ad.init_tensafe_he(16384, sk_seed=5)
    assert slots == 8192
    return a


def test_round_trip_and_metrics(adp):
    rng = np.random.default_rng(0)
    x = rng.normal(size=3000) * 0.1
    ct = adp.encrypt_vector(x.reshape(30, 100))  # flattened like the engine does
    y = adp.decrypt_vector(ct)
    assert y.shape == (8192,)
    assert np.max(np.abs(y[:3000] - x)) < 1e-4  # ciphertext.rs encrypt/decrypt tolerance
    assert np.max(np.abs(y[3000:])) < 1e-4
    m = adp.status()["metrics"]
    assert m["total_encryptions"] == 1 and m["total_decryptions"] == 1
    st = adp.status()
    assert st["gpu_accelerated"] and not st["emulated"] and st["poly_mod_degree"] == 16384


def test_decrypt_to_gpu_matches_host_decrypt(adp):
    import torch

    rng = np.random.default_rng(1)
    cts = [adp.encrypt_vector(rng.normal(size=8192)) for _ in range(3)]
    host = [adp.decrypt_vector(c) for c in cts]
    one = adp.decrypt_to_gpu(cts[0])
    assert one.is_cuda and one.dtype == torch.float64 and tuple(one.shape) == (8192,)
    assert np.array_equal(one.cpu().numpy(), host[0])
    many = adp.batch_decrypt_to_gpu(cts)
    assert tuple(many.shape) == (3, 8192)
    for i in range(3):
        assert np.array_equal(many[i].cpu().numpy(), host[i])


def test_he_lora_delta_flow(adp):
    """inference_engine.py:1258-1392 with the adapter: segment sums equal A @ h."""
    import torch

    ctx = adp.context
    d, rank = 1536, 16
    rng = np.random.default_rng(2)
    h = rng.normal(size=d) * 0.1
    A = rng.normal(size=(rank, d)) * 0.02
    B = rng.normal(size=(d, rank)) * 0.02
    cols = max(1, adp._slots // d)
    n_batches = math.ceil(rank / cols)
    ct_rep = adp.encrypt_vector(zero_moai.replicate(h, adp._slots, d))
    packed = zero_moai.pack_rows(A, adp._slots)
    assert len(packed) == n_batches == 4
    decs = [adp.decrypt_to_gpu(ct_rep * p) for p in packed]  # scale 2^80: CRT decrypt branch
    stacked = torch.stack(decs).cpu().numpy()
    inter = np.zeros(rank)
    for b in range(n_batches):
        for i, r in enumerate(range(b * cols, min((b + 1) * cols, rank))):
            inter[r] = stacked[b, i * d:(i + 1) * d].sum()
    ref = A @ h
    assert np.linalg.norm(inter - ref) / np.linalg.norm(ref) < 1e-3
    delta = B @ inter
    assert np.linalg.norm(delta - B @ ref) / np.linalg.norm(B @ ref) < 1e-3
