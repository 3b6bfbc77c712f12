import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (checker only)."""
    from oracle import oracle as o

    if not os.path.exists(o._LIB_PATH):
        o.build()
    return o


@pytest.fixture(params=["complete", "sk_fused"])
def lora_mode(request, monkeypatch):
    """Runs a LoRA-set test in both token modes: the complete pass (every
    ciphertext of the reference's client/server sequence formed) and the
    sk-fused shortcut (TH_LORA_SK_FUSED). The mode is set for every
    LoraSet.deltas / deltas_device call of the test."""
    if request.param == "sk_fused":
        from provenloop_amd import zero_moai

        mode = zero_moai.LoraSet._mode
        monkeypatch.setattr(zero_moai.LoraSet, "_mode", staticmethod(lambda rescale, sk_fused: mode(rescale, True)))
    return request.param
