"""CPU-side checks of the drop-in boundary (no GPU needed, no compute calls).

* the built C-ABI library loads and exports every function include/tensafe_he.h declares;
* the ctypes binding covers exactly those functions;
* without a GPU the product path fails loudly (no CPU fallback);
* argument validation that happens before any device work mirrors the reference's errors.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from provenloop_amd import _lib, tensafe_he

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"


def test_exports_every_header_symbol():
    declared = _lib.header_symbols()
    assert len(declared) >= 40
    exported = _exported(_lib.LIB_PATH)
    missing = [s for s in declared if s not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_matches_header():
    declared = set(_lib.header_symbols())
    assert set(_lib._SIGS) == declared


def test_library_loads_and_reports_version():
    L = _lib.load()
    assert b"gfx950" in L.th_version()
    assert _lib.last_error() == ""


def test_no_gpu_fails_loudly():
    if _lib.device_count() > 0:
        pytest.skip("a GPU is visible; this checks the no-device path")
    with pytest.raises(_lib.HipEngineError, match="no HIP device"):
        tensafe_he.CkksContext(16384)
    assert tensafe_he.CkksContext.is_available() is False


def test_reference_argument_errors():
    # lib.rs:42-46 and :69-73 raise ValueError before any device work
    with pytest.raises(ValueError, match="Unsupported poly_mod_degree: 4096"):
        tensafe_he.CkksContext(4096)
    with pytest.raises(ValueError, match="Unsupported depth: 9"):
        tensafe_he.CkksContext.for_depth(9)


def test_c_abi_rejects_bad_context_arguments():
    L = _lib.load()
    out = ctypes.c_void_p()
    rc = L.th_ctx_create(3000, None, 0, 40, 0, ctypes.byref(out))
    assert rc == _lib.TH_EINVAL and "Unsupported poly_mod_degree" in _lib.last_error()
    rc = L.th_ctx_create(16384, None, 0, 30, 0, ctypes.byref(out))
    assert rc == _lib.TH_EINVAL and "scale_bits" in _lib.last_error()
    bad = np.array([1152921504606748673, 1152921504606748673], np.uint64)
    rc = L.th_ctx_create(16384, _lib.ptr(bad), 2, 40, 0, ctypes.byref(out))
    assert rc == _lib.TH_EINVAL and "distinct" in _lib.last_error()
    notfriendly = np.array([1152921504606748673, 1099511627791], np.uint64)
    rc = L.th_ctx_create(16384, _lib.ptr(notfriendly), 2, 40, 0, ctypes.byref(out))
    assert rc == _lib.TH_EINVAL and "not 1 mod 2N" in _lib.last_error()
    wide = np.array([1152921504606748673, (1 << 61) + 1], np.uint64)  # the lazy NTT ranges need 8q < 2^64
    rc = L.th_ctx_create(16384, _lib.ptr(wide), 2, 40, 0, ctypes.byref(out))
    assert rc == _lib.TH_EINVAL and "below 2^61" in _lib.last_error()
    assert not out.value


def test_product_never_imports_oracle():
    """The product package must not reach the oracle (checker-only code)."""
    pkg = os.path.join(ROOT, "provenloop_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "from oracle" not in text, f
                assert "liboracle" not in text, f


def test_adapter_init_fails_loudly_without_gpu():
    from provenloop_amd import adapter

    if _lib.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(_lib.HipEngineError, match="no HIP device"):
        adapter.init_tensafe_he(16384)


def test_one_hip_runtime_per_process():
    """The library binds to the HIP runtime PyTorch already loaded (same soname), so a
    process using both never holds two runtimes (the second would find no GPU)."""
    import re

    _lib.load()
    maps = open("/proc/self/maps").read()
    assert len(set(re.findall(r"/\S*/libamdhip64\.so\S*", maps))) == 1
    assert len(set(re.findall(r"/\S*/libhsa-runtime64\.so\S*", maps))) == 1
