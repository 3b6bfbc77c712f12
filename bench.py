#!/usr/bin/env python3
"""Benchmark of the encrypted LoRA-delta path on one MI355X.

Step = one per-token HE-LoRA pass at Qwen2.5-1.5B shape, N = 16384, the
reference's 4-limb chain, scale 2^40: 28 layers x {q, v} projections
(hidden 1536, rank 16, B_q [1536,16], B_v [256,16]). Per token, the
reference's client/server sequence (inference_engine.py:1477-1482): 28
encrypt_pk of the replicated layer inputs, each forming every limb of c0 and
c1 from the public key; 224 column-packed ct x pt products (4 batches per
projection), each fused into a rescale that forms every limb of the
rescaled product, without the secret key; then one batched decrypt that
reads limb 0 of each product with the secret key and writes segment sums;
then B @ intermediate; all on the GPU (one LoRA-set call, one stream
synchronisation). Hidden states are in HBM before the timed region starts
and the deltas stay in HBM; the same pass with host inputs and outputs is
reported beside it as pcie_inclusive. 56 encrypted LoRA deltas per token;
value = deltas/s. The input ciphertexts and rescaled products of layers 0
and 27 of the last timed token are copied out of the set (th_lora_ct) and
compared with the oracle bit for bit. Order on the GPU: the roofline
microbench, the warm-up tokens, the pipelined, reference-sequence and
sk-fused tokens, the timed tokens, the host-I/O tokens, then the other
figures.

Also measured in the same run:
  * roofline: the batched NTT (64 polynomials x 4 limbs, N = 16384, forward
    and inverse as separate launches, coefficients range_u64(q_l) from one
    seeded ChaCha20 stream in (polynomial, limb, coefficient) order), timed
    with HIP events on the engine's stream before the token passes;
    algorithmic bytes = read + write of every limb-polynomial; the same
    round trip at N = 32768 (reference chain for that degree) is reported
    beside it as ntt_n32768;
  * sk_fused: the same tokens through the single-party shortcut
    (TH_LORA_SK_FUSED: only the limbs the decryptions read, the secret key
    inside the encryption, no complete ciphertext); reported beside value,
    never as it;
  * single_delta: the latency of one encrypted LoRA delta (encrypt_pk, 4
    column-packed ct x pt, rescale, decrypt to 16 floats), host in and out;
  * moe: the CryptoMOE variant with a gate that changes every token (3
    experts per projection, the gated plaintexts re-encoded on the device per
    token);
  * saturation: 32 sessions at Qwen2.5-7B shape, N = 32768, 8 limbs;
  * parity: one layer of the timed pass re-run on the CPU oracle (bit-exact
    ciphertexts, deltas within 1e-3 relative), the NTT round trip and a
    forward transform checked against the oracle;
  * cpu_baseline: the CPU oracle (a line-for-line C++ restatement of the
    reference CPU backend, which is Rust and cannot be built here) on the
    same per-layer workload, on the host's cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
import types

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "encrypted LoRA deltas/s at N=16384; NTT achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
N = 16384
LAYERS, D, RANK, D_V = 28, 1536, 16, 256


def make_workload(seed=1234):
    rng = np.random.default_rng(seed)
    A = {(l, p): (rng.normal(size=(RANK, D)) * 0.02).astype(np.float32) for l in range(LAYERS) for p in "qv"}
    B = {(l, "q"): (rng.normal(size=(D, RANK)) * 0.02).astype(np.float32) for l in range(LAYERS)}
    B.update({(l, "v"): (rng.normal(size=(D_V, RANK)) * 0.02).astype(np.float32) for l in range(LAYERS)})
    return A, B


def hidden_states(token, seed=99):
    rng = np.random.default_rng(seed + 7919 * token)
    return [(rng.normal(size=D) * 0.1).astype(np.float32).astype(np.float64) for _ in range(LAYERS)]


def seeds_for(token):
    return [1_000_003 * token + l + 1 for l in range(LAYERS)]


# ------------------------------------------------------------------ seeded inputs
NTT_SEED = 2024


def _chacha_blocks(seed, first, count):
    """ChaCha20 blocks first .. first+count-1 of TenSafeRng::from_seed(seed)
    (rng.rs:38-68, :163-206: key words (lo, hi) x 4, block counter in word
    12, nonce 0), as a [count, 16] uint32 array."""
    lo, hi = seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF
    st = np.zeros((16, count), np.uint32)
    st[0:4] = np.array([0x61707865, 0x3320646E, 0x79622D32, 0x6B206574], np.uint32)[:, None]
    st[4:12:2], st[5:12:2] = lo, hi
    st[12] = (np.arange(first, first + count, dtype=np.uint64) & 0xFFFFFFFF).astype(np.uint32)
    w = st.copy()

    def rotl(x, r):
        return (x << np.uint32(r)) | (x >> np.uint32(32 - r))

    def qr(a, b, c, d):
        w[a] += w[b]; w[d] ^= w[a]; w[d] = rotl(w[d], 16)
        w[c] += w[d]; w[b] ^= w[c]; w[b] = rotl(w[b], 12)
        w[a] += w[b]; w[d] ^= w[a]; w[d] = rotl(w[d], 8)
        w[c] += w[d]; w[b] ^= w[c]; w[b] = rotl(w[b], 7)

    for _ in range(10):
        qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15)
        qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14)
    return (w + st).T


def seeded_residues(seed, moduli, polys, n):
    """[polys, len(moduli), n] uint64: coefficient (p, l, i) = range_u64(q_l) of
    one TenSafeRng::from_seed(seed) stream, drawn in (p, l, i) order
    (rng.rs:99-103 next_u64 = lo | hi << 32; rng.rs:124-133 rejects
    r < (2^64 - q) % q and returns r % q)."""
    q = np.asarray(moduli, np.uint64)
    L = q.size
    total = polys * L * n
    mods = np.broadcast_to(np.repeat(q, n)[None, :], (polys, L * n)).reshape(-1)
    thr = np.array([((1 << 64) - int(x)) % int(x) for x in q], np.uint64)
    thr_seq = np.broadcast_to(np.repeat(thr, n)[None, :], (polys, L * n)).reshape(-1)
    blocks = (total + 7) // 8  # 8 u64 per block
    words = _chacha_blocks(seed, 0, blocks).reshape(-1).astype(np.uint64)
    r = words[0::2] | (words[1::2] << np.uint64(32))
    r = r[:total]
    if not np.any(r < thr_seq):
        return (r % mods).reshape(polys, L, n)
    # a rejection shifts every later draw: consume the stream one draw at a time
    out = np.empty(total, np.uint64)
    pos, have, blk = 0, r, blocks
    for k in range(total):
        while True:
            if pos >= have.size:
                more = _chacha_blocks(seed, blk, 64).reshape(-1).astype(np.uint64)
                have = np.concatenate([have, more[0::2] | (more[1::2] << np.uint64(32))])
                blk += 64
            x = have[pos]
            pos += 1
            if x >= thr_seq[k]:
                out[k] = x % mods[k]
                break
    return out.reshape(polys, L, n)


# ------------------------------------------------------------------ GPU side
def gpu_setup(A, B):
    from provenloop_amd import tensafe_he, zero_moai

    ctx = tensafe_he.CkksContext(N)
    sk = ctx.keygen(seed=11)
    pk = ctx.keygen_public(sk, seed=22)
    # projection 2l = q of layer l, 2l+1 = v of layer l; both read layer l's input
    proj = [(l, A[(l, p)], B[(l, p)]) for l in range(LAYERS) for p in "qv"]
    lora = zero_moai.LoraSet(ctx, LAYERS, proj)
    ctx.sync()
    return ctx, sk, pk, lora


class DeviceInputs:
    """Every step's hidden states uploaded to HBM before the timed region, and
    an HBM output slot per step for its deltas."""

    def __init__(self, ctx, lora, hidden_by_step):
        from provenloop_amd import _lib

        self.ctx, self.L, self.lora = ctx, _lib.load(), lora
        self.steps = len(hidden_by_step)
        self.h_stride = lora.n_inputs * lora.d * 8
        self.o_stride = lora.n_deltas * 8
        self.h, self.o = C.c_void_p(), C.c_void_p()
        _lib.check(self.L.th_dev_alloc(ctx._h, self.steps * self.h_stride, C.byref(self.h)))
        _lib.check(self.L.th_dev_alloc(ctx._h, self.steps * self.o_stride, C.byref(self.o)))
        Hs = np.ascontiguousarray(np.stack([np.stack(h) for h in hidden_by_step]), np.float64)
        _lib.check(self.L.th_memcpy_h2d(ctx._h, self.h, _lib.ptr(Hs), Hs.nbytes))
        ctx.sync()

    def run(self, pk, sk, step, seeds, rescale=True, sk_fused=False):
        self.lora.deltas_device(pk, sk, self.h.value + step * self.h_stride, seeds, self.o.value + step * self.o_stride,
                                rescale=rescale, sk_fused=sk_fused)

    def deltas(self, step):
        from provenloop_amd import _lib

        out = np.empty(self.lora.n_deltas, np.float64)
        _lib.check(self.L.th_memcpy_d2h(self.ctx._h, _lib.ptr(out), C.c_void_p(self.o.value + step * self.o_stride),
                                        self.o_stride))
        return out

    def free(self):
        from provenloop_amd import _lib

        _lib.check(self.L.th_dev_free(self.ctx._h, self.h))
        _lib.check(self.L.th_dev_free(self.ctx._h, self.o))


class NttRoofline:
    """Batched NTT: 64 polys x 4 limbs at the context's N, forward and inverse
    launches timed with HIP events on the engine's stream (time()); the
    round trip and one forward launch checked against the oracle afterwards
    (check()), so that the timing can run right before the token pass."""

    def __init__(self, ctx):
        from provenloop_amd import _lib

        self.ctx, self.L = ctx, _lib.load()
        self.q = ctx.moduli[:4]
        self.n = ctx.poly_mod_degree
        self.seed = NTT_SEED
        self.host = seeded_residues(self.seed, self.q, 64, self.n)
        self.dev = C.c_void_p()
        _lib.check(self.L.th_dev_alloc(ctx._h, self.host.nbytes, C.byref(self.dev)))
        _lib.check(self.L.th_memcpy_h2d(ctx._h, self.dev, _lib.ptr(self.host), self.host.nbytes))

    def time(self, reps=20, inner=10):
        """warm-up round trips, then `reps` runs of `inner` back-to-back forward
        launches followed by as many inverse launches (which bring the data
        back exactly); each sample is the average launch time of one run"""
        from provenloop_amd import _lib

        t_f, t_i = C.c_float(), C.c_float()
        h, L = self.ctx._h, self.L
        for _ in range(3):
            _lib.check(L.th_ntt_time(h, self.dev, 64, 4, 0, 1, C.byref(t_f)))
            _lib.check(L.th_ntt_time(h, self.dev, 64, 4, 1, 1, C.byref(t_i)))
        fwd_ms, inv_ms = [], []
        for _ in range(reps):
            _lib.check(L.th_ntt_time(h, self.dev, 64, 4, 0, inner, C.byref(t_f)))
            fwd_ms.append(t_f.value)
            _lib.check(L.th_ntt_time(h, self.dev, 64, 4, 1, inner, C.byref(t_i)))
            inv_ms.append(t_i.value)
        self.fwd, self.inv = float(np.median(fwd_ms)), float(np.median(inv_ms))

    def check(self):
        from provenloop_amd import _lib
        from oracle import oracle as orc

        h, L, nbytes = self.ctx._h, self.L, self.host.nbytes
        back = np.empty_like(self.host)
        _lib.check(L.th_memcpy_d2h(h, _lib.ptr(back), self.dev, nbytes))
        roundtrip_ok = bool(np.array_equal(back, self.host))
        # one forward launch checked against the oracle on polynomial 0
        _lib.check(L.th_ntt_forward_batch(h, self.dev, 64, 4, 1))
        _lib.check(L.th_memcpy_d2h(h, _lib.ptr(back), self.dev, nbytes))
        fwd_ok = all(np.array_equal(back[0, l], orc.ntt_forward(self.host[0, l], self.q[l])) for l in range(4))
        _lib.check(L.th_dev_free(h, self.dev))
        f, i = self.fwd, self.inv
        per_launch = 2 * nbytes  # read + write of every limb-polynomial
        return {
            "polys": 64, "limbs": 4, "N": self.n, "bytes_per_launch": per_launch,
            "input": f"range_u64(q_l) of TenSafeRng::from_seed({self.seed}), (polynomial, limb, coefficient) order",
            "fwd_ms": f, "inv_ms": i,
            "fwd_GBs": per_launch / (f * 1e-3) / 1e9, "inv_GBs": per_launch / (i * 1e-3) / 1e9,
            "roundtrip_ms": f + i, "roundtrip_GBs": 2 * per_launch / ((f + i) * 1e-3) / 1e9,
            "roundtrip_bitexact": roundtrip_ok, "forward_matches_oracle": bool(fwd_ok),
        }


def ntt_roofline(ctx, reps=20):
    r = NttRoofline(ctx)
    r.time(reps)
    return r.check()


def ntt_traffic():
    """HBM bytes per launch of the batched NTT (mean of forward and inverse),
    from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of
    `bench.py --ntt-only`, scaled by the calibration copy's factor; None if
    the summary is absent."""
    path = os.path.join(ROOT, "profiles", "ntt_64x4_n16384_hbm_traffic.json")
    try:
        with open(path) as f:
            p = json.load(f)
    except (OSError, ValueError):
        return None
    k = p["calibration"]["factor"]
    per = [(p[d]["fetch_kib"] + p[d]["write_kib"]) * 1024 * k for d in ("forward", "inverse")]
    return int(sum(per) / len(per))


def roofline_block(ntt):
    """The line's roofline object for the batched NTT. `bound` names the
    resource closer to saturation by the committed counters: "hbm" when the
    achieved share of 8 TB/s is at least the VALU-busy share, else "valu"
    (VALU issue; there is no MFMA work)."""
    frac = ntt["roundtrip_GBs"] / HBM_PEAK_GBS
    valu = ntt_valu_busy()
    bound = "hbm" if valu is None or frac >= valu else "valu"
    return {
        "kernel": "ntt (batched forward + inverse, 64 polys x 4 limbs, N=16384)",
        "bound": bound,
        "achieved": round(ntt["roundtrip_GBs"], 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(frac, 4),
        "traffic": ntt_traffic(),
        "valu_busy": valu,
        "limiter": "neither HBM nor VALU saturated: per CU the loads, the 60-bit limbs' integer arithmetic, "
                   "the LDS exchanges and the stores follow one another (one polynomial per CU at this "
                   "batch); bound = the larger of the HBM and VALU-busy shares; no MFMA work",
    }


def ntt_valu_busy():
    """VALU-busy fraction of the batched NTT launches (mean of forward and
    inverse) from the committed rocprofv3 counter summary of
    `bench.py --ntt-only` (SQ_ACTIVE_INST_VALU over the CUs' active cycles);
    None if the summary is absent."""
    path = os.path.join(ROOT, "profiles", "ntt_64x4_n16384_valu.json")
    try:
        with open(path) as f:
            p = json.load(f)
        return round((p["forward"]["valu_busy"] + p["inverse"]["valu_busy"]) / 2, 4)
    except (OSError, ValueError, KeyError):
        return None


# ------------------------------------------------------------------ CPU oracle side
class CpuLayer:
    """One layer of the per-token pass on the CPU oracle (checker / baseline only)."""

    def __init__(self, A, B):
        from oracle import oracle as orc
        from provenloop_amd.zero_moai import pack_rows

        self.orc = orc
        self.ctx = orc.Context(N)
        self.sk = self.ctx.keygen(11)
        self.pk = self.ctx.keygen_public(self.sk, 22)
        self.pts = {k: [self.ctx.encode_to_ntt(p) for p in pack_rows(np.asarray(A[k], np.float64), N // 2)] for k in A}
        self.B = B

    def run(self, layer, h, seed, rescale=True):
        from provenloop_amd.zero_moai import replicate

        cols = (N // 2) // D
        ct = self.ctx.encrypt_pk(replicate(h, N // 2, D), self.pk, seed)
        out, cts = {}, {}
        for p in "qv":
            inter = np.zeros(RANK)
            for b, pt in enumerate(self.pts[(layer, p)]):
                r = self.ctx.ct_pt_mul_ntt(ct, pt)
                if rescale:
                    r = self.ctx.rescale(r)
                cts[(p, b)] = r
                dec = self.ctx.decrypt(r, self.sk)
                for i in range(min(cols, RANK - b * cols)):
                    inter[b * cols + i] = np.sum(dec[i * D:(i + 1) * D])
            out[p] = np.asarray(self.B[(layer, p)], np.float64) @ inter
        return out, cts, ct


def cpu_share():
    """Cores this process may run on: the host's count, the affinity mask and the
    cgroup CPU quota (a one-GPU job gets a share of the host), and the share."""
    host = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = host
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    share = aff if quota is None else max(1, min(aff, int(quota)))
    return {"host_cores": host, "affinity_cores": aff, "cgroup_quota_cores": quota, "share": share}


def _cpu_worker(w, workers, ready, go, stop_at, out):
    """One CPU-baseline process: its own oracle context and plaintexts, then
    layers w, w + workers, ... of token 0 until stop_at (time.time())."""
    A, B = make_workload()
    cpu = CpuLayer(A, B)
    hs, seeds = hidden_states(0), seeds_for(0)
    ready.put(w)
    go.wait()
    k = w
    done = 0
    while time.time() < stop_at.value:
        cpu.run(k % LAYERS, hs[k % LAYERS], seeds[k % LAYERS])
        done += 1
        k += workers
    out.put(done)


def cpu_baseline(cpu, budget_s=12.0):
    """Deltas/s of the oracle on this host: one thread in this process, then one
    process per core of the CPU share (each its own oracle context; the
    reference core is single-threaded per operation, so the layers run side
    by side)."""
    import multiprocessing as mp

    hs = hidden_states(0)
    seeds = seeds_for(0)
    t0 = time.perf_counter()
    n1 = 0
    while time.perf_counter() - t0 < budget_s / 3 or n1 == 0:
        cpu.run(n1 % LAYERS, hs[n1 % LAYERS], seeds[n1 % LAYERS])
        n1 += 1
    single = 2 * n1 / (time.perf_counter() - t0)
    share = cpu_share()
    workers = share["share"]
    ctx = mp.get_context("spawn")  # fresh interpreters: no GPU runtime is inherited
    ready, out, go = ctx.Queue(), ctx.Queue(), ctx.Event()
    stop_at = ctx.Value("d", 0.0)
    procs = [ctx.Process(target=_cpu_worker, args=(w, workers, ready, go, stop_at, out)) for w in range(workers)]
    def collect(q, what, limit):
        got, deadline = [], time.time() + limit
        while len(got) < len(procs):
            try:
                got.append(q.get(timeout=1.0))
            except Exception:  # queue.Empty: check that every worker is still alive
                dead = [p.exitcode for p in procs if p.exitcode not in (None, 0)]
                if dead or time.time() > deadline:
                    for p in procs:
                        p.kill()
                    raise RuntimeError(f"CPU baseline workers failed while {what} (exit codes {dead})")
        return got

    for p in procs:
        p.start()
    collect(ready, "setting up", 600)
    span = 2 * budget_s / 3
    start = time.time()
    stop_at.value = start + span
    go.set()
    total = sum(collect(out, "running", 600 + span))
    elapsed = time.time() - start
    for p in procs:
        p.join(timeout=60)
    multi = 2 * total / elapsed
    return single, multi, workers, n1, total, share


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_calibration(ctx, nbytes, reps=3):
    """A plain device-to-device copy of nbytes (the HIP runtime's blit kernel):
    it reads and writes exactly nbytes of HBM, so its FETCH_SIZE / WRITE_SIZE
    counters give the counter scale."""
    from provenloop_amd import _lib

    L = _lib.load()
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipDeviceSynchronize.argtypes = []
    src, dst = C.c_void_p(), C.c_void_p()
    _lib.check(L.th_dev_alloc(ctx._h, nbytes, C.byref(src)))
    _lib.check(L.th_dev_alloc(ctx._h, nbytes, C.byref(dst)))
    host = np.arange(nbytes // 8, dtype=np.uint64)
    _lib.check(L.th_memcpy_h2d(ctx._h, src, _lib.ptr(host), nbytes))
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        if hip.hipMemcpy(dst, src, nbytes, 3) != 0:  # hipMemcpyDeviceToDevice
            raise RuntimeError("hipMemcpy device-to-device failed")
    if hip.hipDeviceSynchronize() != 0:
        raise RuntimeError("hipDeviceSynchronize failed")
    ms = (time.perf_counter() - t0) / reps * 1e3
    back = np.empty_like(host)
    _lib.check(L.th_memcpy_d2h(ctx._h, _lib.ptr(back), dst, nbytes))
    if not np.array_equal(back, host):
        raise RuntimeError("calibration copy mismatch")
    _lib.check(L.th_dev_free(ctx._h, src))
    _lib.check(L.th_dev_free(ctx._h, dst))
    return ms


# The four largest primes q = 1 mod 2N (N = 16384) below 2^60 and below 2^40:
# chains that exercise only the integer (60-bit) or only the FP64 (< 2^41)
# butterfly path of the NTT.
NTT_CHAINS = {
    "default": None,
    "int60": [1152921504606748673, 1152921504606683137, 1152921504606584833, 1152921504605962241],
    "fp40": [1099510054913, 1099508121601, 1099507695617, 1099506515969],
}


def ntt_only(chain="default", n=N):
    from provenloop_amd import tensafe_he

    q = NTT_CHAINS[chain]
    if q is not None and n != N:
        raise SystemExit("--ntt-chain other than default is defined for N=16384 only")
    ctx = tensafe_he.CkksContext(n) if q is None else tensafe_he.CkksContext(n, moduli=q)
    ntt = ntt_roofline(ctx, reps=60)
    copy_ms = copy_calibration(ctx, ntt["bytes_per_launch"] // 2)
    print(json.dumps({
        "metric": f"batched NTT achieved GB/s (64 polys x 4 limbs, N={n})",
        "chain": chain, "moduli": ctx.moduli,
        "ntt": {k: (round(v, 5) if isinstance(v, float) else v) for k, v in ntt.items()},
        "copy_calibration": {"bytes": ntt["bytes_per_launch"] // 2, "ms": round(copy_ms, 4)},
    }), flush=True)


# ------------------------------------------------------------------ secondary workloads
def _timed_sessions(ctx, lora, sessions, dev_by_session, steps, warmup, seeds_fn, sk_fused=False):
    """Time `steps` steps; a step queues one token of every session (its own keys,
    HBM-resident inputs and outputs) and synchronises the stream once."""
    for w in range(warmup):
        for s, (pk, sk) in enumerate(sessions):
            dev_by_session[s].run(pk, sk, steps + w, seeds_fn(s, 10_000 + w), sk_fused=sk_fused)
    ctx.sync()
    seeds = {(s, t): np.asarray(seeds_fn(s, t), np.uint64) for s in range(len(sessions)) for t in range(steps)}
    t0 = time.perf_counter()
    for t in range(steps):
        for s, (pk, sk) in enumerate(sessions):
            dev_by_session[s].run(pk, sk, t, seeds[(s, t)], sk_fused=sk_fused)
        ctx.sync()
    return time.perf_counter() - t0


def moe_gates(t, n_proj, k):
    """The CryptoMOE gate of token t: a softmax over a seeded logit vector per projection."""
    from provenloop_amd import zero_moai

    return np.array([zero_moai.softmax_gate(1_000_003 * t + 7919 * j + 17, k) for j in range(n_proj)])


def moe_workload(steps, warmup):
    """CryptoMOE variant of the per-token pass (Qwen2.5-1.5B shape): 3 rank-16
    expert adapters per projection and a softmax gate that changes every
    token. Per token: th_lora_set_gates (the k gate-scaled plaintexts of every
    batch encoded, transformed and folded, and sum_x g_x B_x, on the device),
    then the token pass; one synchronisation per token. Parity: layer 0 (q and
    v) of the last token against the oracle's literal k products + ct_add +
    rescale + decrypt with that token's gates."""
    from oracle import oracle as orc
    from provenloop_amd import tensafe_he, zero_moai

    K = 3
    rng = np.random.default_rng(4321)
    proj = []
    for l in range(LAYERS):
        for o in (D, D_V):
            proj.append((l, rng.normal(size=(K, RANK, D)) * 0.02, rng.normal(size=(K, o, RANK)) * 0.02))
    ctx = tensafe_he.CkksContext(N)
    sk = ctx.keygen(seed=11)
    pk = ctx.keygen_public(sk, seed=22)
    order = list(range(steps)) + [10_000 + w for w in range(warmup)]
    gates = {t: moe_gates(t, len(proj), K) for t in order}
    lora = zero_moai.LoraSet(ctx, LAYERS, proj, gates=gates[order[0]])
    hidden = {t: hidden_states(t) for t in order}
    dev = DeviceInputs(ctx, lora, [hidden[t] for t in order])
    seeds = {t: np.asarray(seeds_for(t), np.uint64) for t in order}
    for w in range(warmup):
        t = 10_000 + w
        lora.set_gates(gates[t])
        dev.run(pk, sk, steps + w, seeds[t])
        ctx.sync()
    t0 = time.perf_counter()
    for t in range(steps):
        lora.set_gates(gates[t])
        dev.run(pk, sk, t, seeds[t])
        ctx.sync()
    elapsed = time.perf_counter() - t0
    last = steps - 1
    flat = dev.deltas(last)
    t1 = time.perf_counter()
    for t in range(steps):
        lora.set_gates(gates[t])
        dev.run(pk, sk, t, seeds[t], sk_fused=True)
        ctx.sync()
    fused_elapsed = time.perf_counter() - t1
    fused_equal = bool(np.array_equal(dev.deltas(last), flat))
    dev.free()
    ref = orc.Context(N)
    rsk = ref.keygen(11)
    rpk = ref.keygen_public(rsk, 22)
    S, cols = N // 2, (N // 2) // D
    rct = ref.encrypt_pk(zero_moai.replicate(hidden[last][0], S, D), rpk, int(seeds[last][0]))
    rel = []
    for j in range(2):
        _, A, Bm = proj[j]
        g = gates[last][j]
        packs = [zero_moai.pack_rows(A[x], S) for x in range(K)]
        inter = np.zeros(RANK)
        for b in range(len(packs[0])):
            acc = None
            for x in range(K):
                prod = ref.ct_pt_mul(rct, g[x] * packs[x][b])
                acc = prod if acc is None else ref.ct_add(acc, prod)
            dec = ref.decrypt(ref.rescale(acc), rsk)
            n = min(cols, RANK - b * cols)
            inter[b * cols:b * cols + n] = [np.sum(dec[c * D:(c + 1) * D]) for c in range(n)]
        e = sum(g[x] * Bm[x] for x in range(K)) @ inter
        gj = flat[lora.offsets[j]:lora.offsets[j + 1]]
        rel.append(float(np.linalg.norm(gj - e) / np.linalg.norm(e)))
    deltas = LAYERS * 2 * steps
    return {
        "value": round(deltas / elapsed, 3), "unit": "deltas/s", "steps": steps, "warmup": warmup,
        "ms_per_step": round(elapsed / steps * 1e3, 4), "experts": K,
        "workload": "CryptoMOE per-token pass, Qwen2.5-1.5B shape: 28 layers x {q,v} x 3 rank-16 experts, a "
                    "softmax gate per projection drawn for every token; per token the gate-scaled expert "
                    "plaintexts are encoded, transformed and folded on the device (th_lora_set_gates), then "
                    "encrypt_pk (every limb), one product per batch (the ct_add of the experts' products, bit "
                    "for bit) fused into a rescale that forms every limb, one batched decrypt of limb 0; hidden "
                    "states and deltas resident in HBM",
        "sk_fused": {"value": round(deltas / fused_elapsed, 3), "ms_per_step": round(fused_elapsed / steps * 1e3, 4),
                     "deltas_equal": fused_equal},
        "parity": {"delta_rel_err_max_layer0": max(rel)},
    }


def run_moe(args):
    r = moe_workload(args.steps, args.warmup)
    print(json.dumps(dict({
        "metric": "encrypted LoRA deltas/s, CryptoMOE variant (3 experts per projection, per-token gate) at N=16384",
        "n_gpus": 1, "higher_is_better": True, "dtype": "u64",
        "data": "synthetic (seeded N(0,1)*0.1 hidden states, N(0,0.02) expert A/B, seeded per-token gates)",
        "config": {"workload": r.pop("workload"), "experts": r.pop("experts"), "N": N},
    }, **r)), flush=True)


def saturation_workload(steps, warmup, parity_checks=((0, 4 * 27), (0, 4 * 27 + 3), (31, 4 * 27), (31, 4 * 27 + 3))):
    """Saturation run at Qwen2.5-7B shape: 32 sessions (own
    keys), hidden 3584, 28 layers x {q,k,v,o}, rank 32, N=32768 on the 8-limb
    chain; one step = one token of every session, queued back to back with
    one synchronisation. Parity: (session, projection) pairs of the last step
    against the oracle."""
    from oracle import oracle as orc
    from provenloop_amd import tensafe_he, zero_moai
    from provenloop_amd.params import CHAIN_N32768_L8

    n, d, rank, sessions, layers = 32768, 3584, 32, 32, 28
    d_out = {"q": 3584, "k": 512, "v": 512, "o": 3584}
    rng = np.random.default_rng(777)
    proj = [(2 * l + (p == "o"), rng.normal(size=(rank, d)) * 0.02, rng.normal(size=(d_out[p], rank)) * 0.02)
            for l in range(layers) for p in "qkvo"]
    ctx = tensafe_he.CkksContext(n, moduli=CHAIN_N32768_L8)
    lora = zero_moai.LoraSet(ctx, 2 * layers, proj)
    keys = []
    for s in range(sessions):
        sk = ctx.keygen(seed=1000 + s)
        keys.append((ctx.keygen_public(sk, seed=2000 + s), sk))
    steps_all = steps + warmup

    def hidden(s, t):
        r = np.random.default_rng(100_003 * s + t)
        return [(r.normal(size=d) * 0.1).astype(np.float32).astype(np.float64) for _ in range(2 * layers)]

    devs = [DeviceInputs(ctx, lora, [hidden(s, t) for t in range(steps_all)]) for s in range(sessions)]

    def seeds_fn(s, t):
        return [(7_000_003 * s + 1_000_003 * t + i + 1) % (1 << 63) for i in range(2 * layers)]

    fused_elapsed = _timed_sessions(ctx, lora, keys, devs, steps, warmup, seeds_fn, sk_fused=True)
    fused_last = devs[0].deltas(steps - 1)
    elapsed = _timed_sessions(ctx, lora, keys, devs, steps, warmup, seeds_fn)
    fused_equal = bool(np.array_equal(devs[0].deltas(steps - 1), fused_last))
    ref = orc.Context(n, CHAIN_N32768_L8)
    S, cols = n // 2, (n // 2) // d
    last = steps - 1
    rel = []
    for s, j in parity_checks:
        flat = devs[s].deltas(last)
        rsk = ref.keygen(1000 + s)
        rpk = ref.keygen_public(rsk, 2000 + s)
        hs, sd = hidden(s, last), seeds_fn(s, last)
        i, A, Bm = proj[j]
        rct = ref.encrypt_pk(zero_moai.replicate(hs[i], S, d), rpk, sd[i])
        inter = np.zeros(rank)
        for b, p in enumerate(zero_moai.pack_rows(A, S)):
            dec = ref.decrypt(ref.rescale(ref.ct_pt_mul(rct, p)), rsk)
            k = min(cols, rank - b * cols)
            inter[b * cols:b * cols + k] = [np.sum(dec[c * d:(c + 1) * d]) for c in range(k)]
        e = Bm @ inter
        gj = flat[lora.offsets[j]:lora.offsets[j + 1]]
        rel.append(float(np.linalg.norm(gj - e) / np.linalg.norm(e)))
    for dv in devs:
        dv.free()
    per_step = sessions * 4 * layers
    return {
        "value": round(per_step * steps / elapsed, 3), "unit": "deltas/s", "steps": steps, "warmup": warmup,
        "ms_per_step": round(elapsed / steps * 1e3, 4),
        "session_tokens_per_s": round(sessions * steps / elapsed, 3),
        "workload": "32 concurrent sessions, Qwen2.5-7B shape: 28 layers x {q,k,v,o}, hidden 3584, rank 32 "
                    "(8 batches of 4 rows), N=32768, 8-limb chain, scale 2^40; per session token 56 encrypt_pk "
                    "(every limb), 896 ct x pt fused into rescales that form every limb (7), one batched decrypt "
                    "of limb 0; all sessions queued as one batch per step with one host synchronisation",
        "sk_fused": {"value": round(per_step * steps / fused_elapsed, 3),
                     "ms_per_step": round(fused_elapsed / steps * 1e3, 4), "deltas_equal_session0": fused_equal},
        "sessions": sessions, "N": n, "moduli": CHAIN_N32768_L8,
        "parity": {"delta_rel_err_max": max(rel), "checked": [list(c) for c in parity_checks]},
    }


def run_saturation(args):
    r = saturation_workload(args.steps, args.warmup)
    print(json.dumps(dict({
        "metric": "encrypted LoRA deltas/s, saturation at Qwen2.5-7B shape (32 sessions), N=32768, 8 limbs",
        "n_gpus": 1, "higher_is_better": True, "dtype": "u64",
        "data": "synthetic (seeded N(0,1)*0.1 hidden states, N(0,0.02) LoRA A/B, per-session seeded keys)",
        "config": {"workload": r.pop("workload"), "sessions": r.pop("sessions"), "N": r.pop("N"),
                   "moduli": r.pop("moduli"), "session_tokens_per_s": r.pop("session_tokens_per_s")},
    }, **r)), flush=True)


def single_delta_workload(ctx, sk, pk, cpu, reps=100, warm=10):
    """One encrypted LoRA delta at N=16384: encrypt_pk of the replicated
    hidden state, 4 column-packed ct x pt products with cached plaintexts,
    rescale, decrypt with segment sums: 16 floats, host input and output, one
    synchronisation per delta. Latency = median over `reps` calls; parity and
    the oracle's own time for the same delta on one host thread."""
    from provenloop_amd import zero_moai

    rng = np.random.default_rng(4242)
    A = (rng.normal(size=(RANK, D)) * 0.02).astype(np.float32).astype(np.float64)
    h = (rng.normal(size=D) * 0.1).astype(np.float32).astype(np.float64)
    lora = zero_moai.LoraSet(ctx, 1, [(0, A, np.eye(RANK))])  # B = I: the deltas are the 16 intermediates
    H = h[None]

    def latency(sk_fused):
        times = []
        for t in range(warm + reps):
            t0 = time.perf_counter()
            out = lora.deltas(pk, sk, H, [50_000 + t], sk_fused=sk_fused)
            times.append(time.perf_counter() - t0)
        return float(np.median(times[warm:])), out

    lat_f, out_f = latency(True)
    lat, out = latency(False)
    S, cols = N // 2, (N // 2) // D
    t0 = time.perf_counter()
    rct = cpu.ctx.encrypt_pk(zero_moai.replicate(h, S, D), cpu.pk, 50_000 + warm + reps - 1)
    inter = np.zeros(RANK)
    for b, p in enumerate(zero_moai.pack_rows(A, S)):
        dec = cpu.ctx.decrypt(cpu.ctx.rescale(cpu.ctx.ct_pt_mul_ntt(rct, cpu.ctx.encode_to_ntt(p))), cpu.sk)
        n = min(cols, RANK - b * cols)
        inter[b * cols:b * cols + n] = [np.sum(dec[c * D:(c + 1) * D]) for c in range(n)]
    cpu_ms = (time.perf_counter() - t0) * 1e3
    rel = float(np.linalg.norm(out[0] - inter) / np.linalg.norm(inter))
    return {
        "latency_ms": round(lat * 1e3, 4), "deltas_per_s": round(1.0 / lat, 3), "reps": reps, "warmup": warm,
        "workload": "one encrypted LoRA delta, N=16384, 4-limb chain, scale 2^40: encrypt_pk of the replicated "
                    "1536-dim hidden state (every limb, public key only), 4 ct x pt with cached plaintexts of "
                    "LoRA-A [16,1536] fused into rescales that form every limb of each product, decrypt of limb 0 "
                    "with segment sums -> 16 floats; host input and output, one synchronisation",
        "sk_fused_latency_ms": round(lat_f * 1e3, 4),
        "sk_fused_equal": bool(np.array_equal(out[0], out_f[0])),
        "cpu_oracle_ms_1thread": round(cpu_ms, 2),
        "cpu_oracle_note": "the same delta on the CPU oracle, one host thread, plaintext encoding included "
                           "(the reference's Python path encodes uncached)",
        "parity": {"rel_err": rel},
    }


def drop_in_workload(ctx, sk, A, B, hidden, steps=3, warm=1):
    """The reference's own per-token call sequence through the drop-in Python
    module (provenloop_amd.adapter / tensafe_he), one call at a time as the
    engine makes them (inference_engine.py:1244-1392): per projection of each
    of the 28 layers, encrypt_vector of the replicated hidden state (secret-key
    encrypt, :166-176, :1266-1272), then per packed LoRA-A batch
    `ct_rep * packed_pt` (ct x pt with the plaintext encoded on the fly,
    lib.rs:336-356) and decrypt_to_gpu (:1311-1315), the batches' slots
    stacked on the GPU and copied to the host once, the segment sums and
    B @ intermediate on the host (:1379-1392). ms per token and deltas/s, and
    the deltas against B (A h) in plaintext."""
    import torch

    from provenloop_amd import zero_moai
    from provenloop_amd.adapter import TenSafeHEAdapter

    adp = TenSafeHEAdapter(ctx, sk)
    S, cols = N // 2, (N // 2) // D
    packed = {k: zero_moai.pack_rows(np.asarray(A[k], np.float64), S) for k in A}  # the engine's _packed_pts

    def token(hs):
        out = {}
        for l in range(LAYERS):
            for p in "qv":
                ct_rep = adp.encrypt_vector(zero_moai.replicate(hs[l], S, D))
                decs = [adp.decrypt_to_gpu(ct_rep * pt) for pt in packed[(l, p)]]
                all_dec = torch.stack(decs).cpu().numpy()
                inter = np.zeros(RANK)
                for b in range(len(decs)):
                    for i, r in enumerate(range(b * cols, min((b + 1) * cols, RANK))):
                        inter[r] = np.sum(all_dec[b, i * D:(i + 1) * D])
                out[(l, p)] = np.asarray(B[(l, p)], np.float64) @ inter
        return out

    for w in range(warm):
        token(hidden[w % len(hidden)])
    t0 = time.perf_counter()
    for t in range(steps):
        got = token(hidden[t % len(hidden)])
    elapsed = time.perf_counter() - t0
    hs = hidden[(steps - 1) % len(hidden)]
    rel = []
    for l in (0, LAYERS - 1):
        for p in "qv":
            e = np.asarray(B[(l, p)], np.float64) @ (np.asarray(A[(l, p)], np.float64) @ hs[l])
            rel.append(float(np.linalg.norm(got[(l, p)] - e) / np.linalg.norm(e)))
    return {
        "value": round(LAYERS * 2 * steps / elapsed, 3), "unit": "deltas/s", "ms_per_step": round(elapsed / steps * 1e3, 3),
        "steps": steps, "warmup": warm,
        "workload": "the reference's per-token call sequence through the drop-in module, one call at a time: per "
                    "projection of 28 layers, adapter.encrypt_vector (secret key, unseeded), 4 x ct_rep * packed_pt "
                    "(plaintext encoded per call) and decrypt_to_gpu, one stack and host copy, segment sums and "
                    "B @ intermediate on the host (inference_engine.py:1244-1392); 56 encryptions, 224 products "
                    "and 224 decryptions with their host synchronisations per token",
        "parity": {"delta_rel_err_vs_plaintext_max_layers_0_27": max(rel)},
    }


def run_single(args):
    """Only the single-delta figure (one encrypted delta), for a kernel trace of its
    launches: the same calls as the reported line's single_delta."""
    from oracle import oracle as orc
    from provenloop_amd import tensafe_he

    ctx = tensafe_he.CkksContext(N)
    sk = ctx.keygen(seed=11)
    pk = ctx.keygen_public(sk, seed=22)
    cpu = types.SimpleNamespace(ctx=orc.Context(N))
    cpu.sk = cpu.ctx.keygen(11)
    cpu.pk = cpu.ctx.keygen_public(cpu.sk, 22)
    r = single_delta_workload(ctx, sk, pk, cpu, reps=args.steps, warm=args.warmup)
    print(json.dumps(dict({
        "metric": "latency of one encrypted LoRA delta at N=16384 (host in, host out)",
        "n_gpus": 1, "higher_is_better": False, "dtype": "u64",
        "data": "synthetic (seeded N(0,1)*0.1 hidden state, N(0,0.02) LoRA A)",
        "config": {"workload": r.pop("workload"), "N": N},
    }, **r)), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 100 tokens; 20 steps for the saturation workload)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default 20 tokens; 3 steps for the saturation workload)")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU-oracle baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the single-delta, CryptoMOE and saturation figures of the reported line")
    ap.add_argument("--ntt-only", action="store_true",
                    help="only the batched-NTT launches plus a plain device copy of the same size "
                         "(the copy calibrates HBM byte counters); prints one JSON line")
    ap.add_argument("--ntt-chain", choices=sorted(NTT_CHAINS), default="default",
                    help="modulus chain of the --ntt-only launches: the default 4-limb chain, or four "
                         "60-bit (integer butterfly path) or four 40-bit (FP64 butterfly path) primes")
    ap.add_argument("--ntt-n", type=int, choices=(16384, 32768), default=N,
                    help="ring degree of the --ntt-only launches (reference chain for that degree)")
    ap.add_argument("--workload", choices=("token", "moe", "saturation", "single", "dropin"), default="token",
                    help="token: the per-token Qwen2.5-1.5B pass (the reported line); moe: its CryptoMOE "
                         "variant with a per-token gate; saturation: 32 sessions at Qwen2.5-7B shape on "
                         "N=32768 with 8 limbs; single: one encrypted delta's latency; dropin: the reference's "
                         "per-token call sequence through the drop-in module")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 20 if args.workload == "saturation" else 100
    if args.warmup is None:
        args.warmup = {"saturation": 3, "single": 10}.get(args.workload, 20)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path shards by session/token "
              "with no cross-GPU exchange, so N GPUs scale the one-GPU figure)", file=sys.stderr)
        sys.exit(2)
    if args.ntt_only:
        ntt_only(args.ntt_chain, args.ntt_n)
        return
    if args.workload == "moe":
        run_moe(args)
        return
    if args.workload == "saturation":
        run_saturation(args)
        return
    if args.workload == "single":
        run_single(args)
        return
    if args.workload == "dropin":
        from provenloop_amd import tensafe_he

        A, B = make_workload()
        ctx = tensafe_he.CkksContext(N)
        sk = ctx.keygen(seed=11)
        r = drop_in_workload(ctx, sk, A, B, [hidden_states(t) for t in range(args.steps)], steps=args.steps,
                             warm=args.warmup)
        print(json.dumps(dict({
            "metric": "encrypted LoRA deltas/s through the drop-in module in the reference's call sequence",
            "n_gpus": 1, "higher_is_better": True, "dtype": "u64", "data": "synthetic (seeded, as the token pass)",
            "config": {"workload": r.pop("workload"), "N": N},
        }, **r)), flush=True)
        return

    A, B = make_workload()
    ctx, sk, pk, lora = gpu_setup(A, B)
    # synthetic inputs for every step, generated and uploaded to HBM before the timed region
    warm = [10_000 + w for w in range(args.warmup)]
    order = list(range(args.steps)) + warm
    hidden = {t: hidden_states(t) for t in order}
    dev = DeviceInputs(ctx, lora, [hidden[t] for t in order])
    seeds = {t: seeds_for(t) for t in range(args.steps)}
    seed_arr = {t: np.asarray(seeds[t], np.uint64) for t in range(args.steps)}  # prepared like the inputs
    warm_seeds = [np.asarray(seeds_for(t), np.uint64) for t in warm]
    ntt16 = NttRoofline(ctx)
    # Order: the roofline microbench, the warm-up tokens, the pipelined and the
    # reference-sequence figures, then the timed synchronised tokens. After
    # an idle second (or a host-bound stretch such as building a LoRA set) a
    # synchronised token runs up to 8 % slower for about its first 100
    # tokens (the GPU's clocks ramp under load; a power-management state,
    # not set-up: it returns after every idle second); the measurements
    # before the timed tokens keep the device busy up to them.
    ntt16.time(reps=60)
    for w in range(args.warmup):
        dev.run(pk, sk, args.steps + w, warm_seeds[w])
    ctx.sync()

    # the same tokens queued back to back (host launches overlap the GPU; one sync at the end)
    t2 = time.perf_counter()
    for t in range(args.steps):
        dev.run(pk, sk, t, seed_arr[t])
    ctx.sync()
    piped = time.perf_counter() - t2

    # the reference's own call sequence: ct x pt, then decrypt without a rescale
    # (inference_engine.py:1311-1315; the CRT branch of ciphertext.rs:351-396)
    t3 = time.perf_counter()
    for t in range(args.steps):
        dev.run(pk, sk, t, seed_arr[t], rescale=False)
        ctx.sync()
    norescale_elapsed = time.perf_counter() - t3
    flat_nr = dev.deltas(args.steps - 1)

    # the single-party shortcut (TH_LORA_SK_FUSED): reported beside value, never as it
    t4 = time.perf_counter()
    for t in range(args.steps):
        dev.run(pk, sk, t, seed_arr[t], sk_fused=True)
        ctx.sync()
    fused_elapsed = time.perf_counter() - t4
    flat_fused = dev.deltas(args.steps - 1)

    tok = []
    t0 = time.perf_counter()
    for t in range(args.steps):
        dev.run(pk, sk, t, seed_arr[t])
        ctx.sync()  # one host synchronisation per token
        tok.append(time.perf_counter())
    elapsed = time.perf_counter() - t0
    deltas_per_token = LAYERS * 2
    value = deltas_per_token * args.steps / elapsed
    tok_ms = np.diff(np.concatenate([[t0], tok])) * 1e3
    flat_timed = dev.deltas(args.steps - 1)
    # the ciphertexts the last timed token formed: the encrypt_pk output of
    # layers 0 and 27 and their 8 rescaled products each (copies queued now,
    # before any other token reuses the set's working memory)
    check_layers = (0, LAYERS - 1)
    timed_cts = {("input", l): lora.ciphertext("input", l) for l in check_layers}
    for l in check_layers:
        for j, p in enumerate("qv"):
            for b in range(4):
                timed_cts[(p, l, b)] = lora.ciphertext("product", (2 * l + j) * 4 + b)

    # the same pass with host inputs and outputs (PCIe included): reported beside value
    t1 = time.perf_counter()
    for t in range(args.steps):
        host_out = lora.deltas(pk, sk, np.stack(hidden[t]), seeds[t])
    pcie_elapsed = time.perf_counter() - t1

    # parity on layers 0 and 27 of token steps-1 against the oracle (the
    # host-I/O pass left that token's deltas in host_out; the device-I/O run of
    # the same token is compared with them)
    last = args.steps - 1
    flat = np.concatenate(host_out)
    dev.run(pk, sk, last, seed_arr[last])
    ctx.sync()
    dev_host_equal = bool(np.array_equal(dev.deltas(last), flat))
    dev.free()
    cpu = CpuLayer(A, B)
    hs, sd = hidden[last], seeds[last]
    rel, rel_nr = [], []
    n_ct_checked, n_ct_exact = 0, 0
    for l in check_layers:
        ref, r_prods, r_in = cpu.run(l, hs[l], sd[l])
        for j, p in enumerate("qv"):
            k = 2 * l + j
            g, c = flat[lora.offsets[k]:lora.offsets[k + 1]], ref[p]
            rel.append(float(np.linalg.norm(g - c) / np.linalg.norm(c)))
        pairs = [(timed_cts[("input", l)], r_in)] + [(timed_cts[(p, l, b)], r_prods[(p, b)]) for p in "qv"
                                                     for b in range(4)]
        for g_ct, r_ct in pairs:
            n_ct_checked += 1
            n_ct_exact += int(g_ct.num_limbs == r_ct.num_limbs and g_ct.scale == r_ct.scale and all(
                np.array_equal(x, y) for x, y in zip(ctx.ct_download(g_ct), cpu.ctx.ct_data(r_ct))))
    ref_nr, _, _ = cpu.run(0, hs[0], sd[0], rescale=False)
    for j, p in enumerate("qv"):
        g, c = flat_nr[lora.offsets[j]:lora.offsets[j + 1]], ref_nr[p]
        rel_nr.append(float(np.linalg.norm(g - c) / np.linalg.norm(c)))
    # bit-exact ciphertext check of one encrypt_pk + product + rescale
    from provenloop_amd import zero_moai

    rep = zero_moai.replicate(hs[0], N // 2, D)
    g_ct = ctx.encrypt_pk_batch([rep], pk, [sd[0]])[0]
    g_pt = ctx.encode_to_ntt(zero_moai.pack_rows(np.asarray(A[(0, "q")], np.float64), N // 2)[0])
    g_r = ctx.rescale(ctx.ct_pt_mul_ntt(g_ct, g_pt))
    r_ct = cpu.ctx.encrypt_pk(rep, cpu.pk, sd[0])
    r_r = cpu.ctx.rescale(cpu.ctx.ct_pt_mul_ntt(r_ct, cpu.pts[(0, "q")][0]))
    ct_exact = all(np.array_equal(x, y) for x, y in zip(ctx.ct_download(g_ct), cpu.ctx.ct_data(r_ct)))
    rs_exact = all(np.array_equal(x, y) for x, y in zip(ctx.ct_download(g_r), cpu.ctx.ct_data(r_r)))

    ntt = ntt16.check()
    from provenloop_amd import tensafe_he

    ctx32 = tensafe_he.CkksContext(2 * N)
    ntt32 = ntt_roofline(ctx32)
    del ctx32

    # the timed token's deltas equal the host-I/O token's and the shortcut's (same residues)
    timed_equal_fused = bool(np.array_equal(flat_timed, flat_fused))
    timed_equal_host = bool(np.array_equal(flat_timed, flat))

    extra = {}
    if not args.no_extra:
        extra["single_delta"] = single_delta_workload(ctx, sk, pk, cpu)
        extra["drop_in_sequence"] = drop_in_workload(ctx, sk, A, B, [hidden[t] for t in range(args.steps)])
        del lora
        extra["moe"] = moe_workload(steps=10, warmup=2)
        extra["saturation"] = saturation_workload(steps=3, warmup=1)

    if args.no_cpu:
        cpu_single = cpu_multi = None
        threads = n1 = nm = 0
        share = cpu_share()
    else:
        cpu_single, cpu_multi, threads, n1, nm, share = cpu_baseline(cpu, args.cpu_budget)

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "deltas/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic (seeded N(0,1)*0.1 hidden states, N(0,0.02) LoRA A/B, random-init)",
        "config": {
            "workload": "per-token HE-LoRA pass, Qwen2.5-1.5B shape: 28 layers x {q,v}, hidden 1536, rank 16, "
                        "N=16384, 4-limb chain [60,40,40,60], scale 2^40; the reference's client/server sequence: "
                        "28 encrypt_pk (every limb of c0 and c1, public key only), 224 column-packed ct x pt fused "
                        "into rescales that form every limb of each product (no secret key), one batched decrypt "
                        "of limb 0 per token (secret key), B @ intermediate on the GPU; hidden states and deltas "
                        "resident in HBM, one host synchronisation per token",
            "N": N, "layers": LAYERS, "hidden": D, "rank": RANK, "deltas_per_token": deltas_per_token,
            "tokens_per_s": round(args.steps / elapsed, 3),
        },
        "roofline": roofline_block(ntt),
        "token_ms": {"median": round(float(np.median(tok_ms)), 4), "first": round(float(tok_ms[0]), 4),
                     "last": round(float(tok_ms[-1]), 4), "min": round(float(tok_ms.min()), 4)},
        "reference_sequence": {
            "value": round(deltas_per_token * args.steps / norescale_elapsed, 3), "unit": "deltas/s",
            "ms_per_step": round(norescale_elapsed / args.steps * 1e3, 4),
            "workload": "the same tokens through the reference's own call sequence (inference_engine.py:1311-1315): "
                        "ct x pt, then decrypt without a rescale (scale 2^80: the CRT branch over limbs 0 and 1), "
                        "segment sums, B @ intermediate; one host synchronisation per token",
            "parity": {"delta_rel_err_max_layer0": max(rel_nr)},
        },
        "sk_fused": {
            "value": round(deltas_per_token * args.steps / fused_elapsed, 3), "unit": "deltas/s",
            "ms_per_step": round(fused_elapsed / args.steps * 1e3, 4),
            "workload": "the same tokens through the single-party shortcut (TH_LORA_SK_FUSED): only the limbs the "
                        "decryptions read, c0 + c1 s formed with the secret key inside the encryption, the rescale "
                        "fused into the decryption; no complete ciphertext exists, so a server without the secret "
                        "key cannot run it; not the reference's architecture and never the value",
            "deltas_equal_complete_pass": timed_equal_fused,
        },
        "pipelined": {
            "value": round(deltas_per_token * args.steps / piped, 3), "unit": "deltas/s",
            "ms_per_step": round(piped / args.steps * 1e3, 4),
            "io": "same HBM-resident tokens queued back to back, one host synchronisation at the end",
        },
        "pcie_inclusive": {
            "value": round(deltas_per_token * args.steps / pcie_elapsed, 3), "unit": "deltas/s",
            "ms_per_step": round(pcie_elapsed / args.steps * 1e3, 4),
            "io": "hidden states from host memory, deltas to host memory (one device-to-host copy per token)",
        },
        "ntt": {k: (round(v, 5) if isinstance(v, float) else v) for k, v in ntt.items()},
        "ntt_n32768": dict({k: (round(v, 5) if isinstance(v, float) else v) for k, v in ntt32.items()},
                           frac=round(ntt32["roundtrip_GBs"] / HBM_PEAK_GBS, 4)),
        "parity": {
            "delta_rel_err_max": max(rel),
            "timed_pass_ciphertexts_bitexact": n_ct_exact == n_ct_checked,
            "timed_pass_ciphertexts_checked": f"{n_ct_exact} of {n_ct_checked} bit-exact: the encrypt_pk output "
                                              f"(4 limbs) and the 8 rescaled products (3 limbs) of layers 0 and 27 "
                                              f"of the last timed token, copied out of the set (th_lora_ct)",
            "timed_deltas_equal_host_io": timed_equal_host,
            "device_io_equals_host_io": dev_host_equal,
            "encrypt_pk_bitexact": bool(ct_exact),
            "ctpt_rescale_bitexact": bool(rs_exact),
            "ntt_roundtrip_bitexact": ntt["roundtrip_bitexact"],
            "ntt_forward_bitexact": ntt["forward_matches_oracle"],
            "ntt_n32768_roundtrip_bitexact": ntt32["roundtrip_bitexact"],
            "ntt_n32768_forward_bitexact": ntt32["forward_matches_oracle"],
        },
        "cpu_baseline": None if cpu_multi is None else {
            "value": round(cpu_multi, 3),
            "unit": "deltas/s",
            "cores": threads,
            "kind": "port",
            "sample": f"CPU oracle, one layer (encrypt_pk + 2 projections x 4 x (ct x pt, rescale, decrypt)) "
                      f"of token 0 repeated: {n1} layers on 1 thread, then {nm} layers in {threads} processes "
                      f"(one per core of this job's CPU share) over {2 * args.cpu_budget / 3:.0f} s",
            "single_thread_value": round(cpu_single, 3),
            "host_cores": share["host_cores"],
            "affinity_cores": share["affinity_cores"],
            "cgroup_quota_cores": share["cgroup_quota_cores"],
            "cpu_model": cpu_model(),
            "gpu_over_cpu": round(value / cpu_multi, 1),
        },
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
