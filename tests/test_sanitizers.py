"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the host-side C++.

* The engine's host arithmetic (provenloop_amd/csrc/host_math.cpp: chains,
  primality, roots, the ChaCha20 stream and samplers, the encoder tables, the
  segment weights) is built with g++ -fsanitize=address,undefined and driven
  by host_math_check.cpp; any sanitizer report fails the run, and its values
  must equal the oracle's (the weights a numpy closed form's).
* The oracle itself is rebuilt the same way (liboracle_san.so) and the CPU
  test files that exercise it run again on that build, in a child process
  with libasan preloaded (Python itself is not instrumented).
"""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "provenloop_amd", "csrc")
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _f64(hexes):
    return np.array([int(h, 16) for h in hexes], dtype=np.uint64).view(np.float64)


@pytest.fixture(scope="module")
def host_math_out():
    subprocess.run(["make", "-s", "-f", os.path.join(CSRC, "Makefile.san")], check=True)
    env = dict(os.environ, **SAN_ENV)
    r = subprocess.run([os.path.join(CSRC, "_build", "host_math_check")], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    return {ln.split()[0]: ln.split()[1:] for ln in r.stdout.splitlines() if ln.strip()}


def test_host_math_chains_and_roots(host_math_out, orc):
    o = host_math_out
    for n in (8192, 16384, 32768):
        q = [int(v) for v in o[f"chain_{n}"]]
        assert q == orc.default_chain(n)
        assert [int(v) for v in o[f"psi_{n}"]] == [orc.find_primitive_root(n, p) for p in q]
        assert [int(v) for v in o[f"inv3_{n}"]] == [orc.mod_inv(3, p) for p in q]
        assert o[f"isprime_{n}"] == ["1"] * len(q)
    assert o["isprime_composites"] == ["0"] * 6
    assert int(o["powmod"][0]) == pow(3, 1000000, 1152921504606748673)
    assert int(o["powmod"][1]) == pow(2, 64, 1099510054913)


def test_host_math_stream_and_samplers(host_math_out, orc):
    o = host_math_out
    assert np.array_equal(np.array(o["chacha_u32_42"], dtype=np.uint64), orc.rng_u32(42, 64).astype(np.uint64))
    assert np.array_equal(np.array(o["below_u64_9"], dtype=np.uint64),
                          orc.rng_range_u64(9, 1152921504606748673, 256))
    assert np.array_equal(_f64(o["normal_11"]), orc.rng_gaussian(11, 3.19, 256))
    u, e0, e1 = orc.encrypt_pk_randomness(7, 1024)
    assert np.array_equal(np.array(o["pk_u_7"], dtype=np.int64), u.astype(np.int64))
    assert np.array_equal(np.array(o["pk_e0_7"], dtype=np.int64), e0)
    assert np.array_equal(np.array(o["pk_e1_7"], dtype=np.int64), e1)


def test_host_math_encoder_tables(host_math_out, orc):
    o = host_math_out
    # the encoder tables depend on N only: the oracle's at N = 1024 (any NTT-friendly prime)
    tr, ti, sr, si = orc.Context(1024, [12289]).fft_tables()
    assert np.array_equal(_f64(o["twist_re_1024"]), tr)
    assert np.array_equal(_f64(o["twist_im_1024"]), ti)
    assert np.array_equal(_f64(o["stage_re_1024"])[: sr.size], sr)
    assert np.array_equal(_f64(o["stage_im_1024"])[: si.size], si)


def test_host_math_segment_weights(host_math_out):
    o = host_math_out
    n, d, cols = 1024, 100, 5
    w = _f64(o["segw_1024_100_5"]).reshape(cols, n)
    j = np.arange(n)
    for c in range(cols):
        k = np.arange(c * d, (c + 1) * d)
        exp = np.cos(np.pi * np.outer(j, 2 * k + 1) / n).sum(axis=1)  # sum of the segment's slot weights
        assert np.max(np.abs(w[c] - exp)) < 1e-9
    p = _f64(o["segp_1024_100"]).reshape(n, 2)
    assert np.max(np.abs(p[:, 0] - w[0])) < 1e-12
    phi = np.pi * j * d / n
    assert np.max(np.abs(p[1:, 1] - 2 * np.cos(2 * phi[1:]))) < 1e-12


def test_oracle_tests_under_sanitizers():
    subprocess.run(["make", "-s", "-f", os.path.join(ROOT, "oracle", "Makefile.san")], check=True)
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    ubsan = subprocess.run(["gcc", "-print-file-name=libubsan.so"], capture_output=True, text=True).stdout.strip()
    env = dict(os.environ, **SAN_ENV, LD_PRELOAD=f"{asan}:{ubsan}",
               ORACLE_LIB=os.path.join(ROOT, "oracle", "liboracle_san.so"))
    files = ["tests/test_oracle_reference_tests.py", "tests/test_oracle_pins.py", "tests/test_golden.py",
             "tests/test_wire_format.py", "tests/test_params.py"]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider"] + files,
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr, tail


def test_sampler_band_predicate(host_math_out):
    """The device sampler's boundary-band test (band.h, constexpr, the same definition the GPU
    runs) against exact rational arithmetic: flagged iff t is not finite, |t| >= 2^52, or t lies
    strictly within the band of k + 1/2."""
    from fractions import Fraction

    o = host_math_out
    t = _f64(o["band_t"])
    for key, band in (("band_flag_36", Fraction(1, 2 ** 36)), ("band_flag_40", Fraction(1, 2 ** 40))):
        got = [int(v) for v in o[key]]
        exp = []
        for v in t:
            if not np.isfinite(v) or abs(v) >= 2.0 ** 52:
                exp.append(1)
                continue
            f = Fraction(float(v))
            frac = f - (f.numerator // f.denominator)
            exp.append(int(abs(frac - Fraction(1, 2)) < band))
        assert got == exp, (key, got, exp)
    assert sum(int(v) for v in o["band_flag_36"]) >= 8  # the test values do reach both sides
