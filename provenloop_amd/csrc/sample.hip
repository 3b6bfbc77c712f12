// GPU sampling of encrypt_pk's randomness (tensafe-he-core/src/ciphertext.rs
// :255-273) from the reference's seeded ChaCha20 stream (rng.rs:31-157).
//
// Stream layout: word p of TenSafeRng::from_seed(seed) is word p % 16 of the
// RFC 8439 block with counter p / 16 (key = seed words (lo, hi) x 4, nonce 0).
// encrypt_pk draws, in order:
//   u:  N x range_u32(3)  -> one word each; a word is rejected only if it is 0
//       (threshold 2^32 mod 3 = 1), stored as sample_ternary's {2, 0, 1}[r % 3]
//   e0: N x gaussian(3.19) -> two next_u64 = four words each
//   e1: N more.
// Without a rejection (probability 1 - N * 2^-32 per encryption) u occupies
// words [0, N) and each 16-word block past it holds exactly four Gaussian
// draws, so one thread per block produces its outputs independently. A check
// kernel regenerates the u words; if any is 0 it replays the whole stream
// serially, exactly as the reference consumes it.
//
// Box-Muller uses the device log/cos. Its rounded integer equals glibc's
// unless z * 3.19 lies within a few ulps of a .5 boundary; every draw within
// the band (BandArgs, default 2^-36) of a boundary raises its job's band flag
// in host-visible memory, and the host redraws that job's randomness with
// glibc before the result is returned, so the draws equal the reference's.
#include "sample_device.h"

namespace th {

// One thread per 16-word block of the stream.
__global__ void k_sample_blocks(const SampleJob* __restrict__ jobs, uint32_t n, SeedBlock sb, int use_sb,
                                BandArgs band) {
  const SampleJob jb = jobs[blockIdx.y];
  sample_block(jb, job_seed(jb, sb, use_sb, blockIdx.y), n, blockIdx.x * blockDim.x + threadIdx.x, band.band,
               flag_of(band, blockIdx.y));
}

// One workgroup per job: re-derive the u words; if any was rejected (== 0),
// or force_serial is set, lane 0 rewrites u, e0 and e1 by the serial walk.
__global__ __launch_bounds__(256) void k_sample_check(const SampleJob* __restrict__ jobs, uint32_t n, int force_serial,
                                                      SeedBlock sb, int use_sb, BandArgs band) {
  const SampleJob jb = jobs[blockIdx.x];
  const uint64_t seed = job_seed(jb, sb, use_sb, blockIdx.x);
  int bad = 0;
  for (uint32_t b = threadIdx.x; b < n / 16; b += blockDim.x) {
    uint32_t w[16];
    chacha20((uint32_t)seed, (uint32_t)(seed >> 32), b, w);
#pragma unroll
    for (int i = 0; i < 16; ++i) bad |= (w[i] == 0);
  }
  bad = __syncthreads_or(bad) | force_serial;
  if (!bad || threadIdx.x != 0) return;
  serial_replay(jb, seed, n, flag_of(band, blockIdx.x), band.band);
}

// One thread per job with a reject flag: replay flagged (or forced) jobs
// serially, then clear the flag for the next launch.
__global__ void k_sample_fix(const SampleJob* __restrict__ jobs, uint32_t njobs, uint32_t n, int force_serial,
                             SeedBlock sb, int use_sb, BandArgs band) {
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= njobs) return;
  const SampleJob jb = jobs[j];
  sample_fix_job(jb, job_seed(jb, sb, use_sb, j), n, force_serial, flag_of(band, j), band.band);
}

hipError_t launch_sample_pk(const SampleJob* jobs, uint32_t njobs, uint32_t n, int force_serial, hipStream_t s,
                            const uint64_t* seeds, bool flagged, bool fix_later, BandArgs band) {
  if (!njobs) return hipSuccess;
  if (n % 16) return hipErrorInvalidValue;
  const uint32_t nblocks = 9 * (n / 16);
  SeedBlock sb{};
  for (uint32_t first = 0; first < njobs; first += SEEDS_PER_LAUNCH) {
    const uint32_t cnt = njobs - first < SEEDS_PER_LAUNCH ? njobs - first : SEEDS_PER_LAUNCH;
    if (seeds)
      for (uint32_t i = 0; i < cnt; ++i) sb.v[i] = seeds[first + i];
    const BandArgs bf = band_from(band, first);
    hipLaunchKernelGGL(k_sample_blocks, dim3((nblocks + 255) / 256, cnt), dim3(256), 0, s, jobs + first, n, sb,
                       seeds != nullptr, bf);
    if (flagged && fix_later)
      continue;  // the caller's next launch replays flagged jobs and clears the flags
    if (flagged)
      hipLaunchKernelGGL(k_sample_fix, dim3((cnt + 63) / 64), dim3(64), 0, s, jobs + first, cnt, n, force_serial, sb,
                         seeds != nullptr, bf);
    else
      hipLaunchKernelGGL(k_sample_check, dim3(cnt), dim3(256), 0, s, jobs + first, n, force_serial, sb,
                         seeds != nullptr, bf);
  }
  return hipGetLastError();
}

}  // namespace th
