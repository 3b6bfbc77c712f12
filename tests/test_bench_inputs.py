"""The batched-NTT microbench's seeded inputs (bench.seeded_residues): one
TenSafeRng::from_seed(seed) stream, range_u64(q_l) drawn in (polynomial,
limb, coefficient) order, equal to the oracle's ChaCha20 stream with the
reference's rejection rule (rng.rs:99-133)."""
import numpy as np

import bench
from oracle import oracle as orc


def _reference(seed, moduli, polys, n):
    stream = orc.rng_u64(seed, 4 * polys * len(moduli) * n + 64)
    out, k = [], 0
    for _ in range(polys):
        for q in moduli:
            thr = ((1 << 64) - q) % q
            for _ in range(n):
                while True:
                    r = int(stream[k])
                    k += 1
                    if r >= thr:
                        out.append(r % q)
                        break
    return np.array(out, np.uint64).reshape(polys, len(moduli), n)


def test_default_chain_order():
    q = orc.default_chain(16384)
    assert np.array_equal(bench.seeded_residues(11, q, 3, 40), _reference(11, q, 3, 40))


def test_rejections_shift_the_stream():
    # q = 2^63 + 1 rejects about half of the draws, so the slow path runs
    q = [(1 << 63) + 1, 97]
    assert np.array_equal(bench.seeded_residues(5, q, 2, 32), _reference(5, q, 2, 32))
    assert np.array_equal(bench.seeded_residues(5, [q[0]], 1, 64).reshape(-1), orc.rng_range_u64(5, q[0], 64))


def test_block_boundaries_and_seed_words():
    # seeds with both 32-bit halves set; lengths that end inside a block
    for seed in (0, 1, (1 << 40) + 3, (1 << 64) - 1):
        got = bench.seeded_residues(seed, [1099510054913], 1, 37)
        assert np.array_equal(got.reshape(-1), orc.rng_range_u64(seed, 1099510054913, 37))
