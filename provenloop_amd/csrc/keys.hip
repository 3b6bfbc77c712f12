// Key and secret-key-encryption randomness on the device (launch_key_draws,
// launch_key_replay, declared with the sampler in encode_sample.h):
// keygen's ternary secret, and keygen_public's and the secret-key
// encryption's uniform a on every limb followed by the Gaussian e, from the
// reference's seeded ChaCha20 stream (tensafe-he-core/src/rng.rs:31-157,
// sampling.rs:17-64, ciphertext.rs:77-229).
//
// Stream layout without a rejection: keygen's N range_u32(3) draws take one
// word each; each range_u64(q_l) takes two (next_u64 = lo | hi << 32,
// rng.rs:99-103) and each Gaussian four (two next_u64, rng.rs:139-157), so a
// stretch of L x N uniform draws and N Gaussians takes 2 L N + 4 N words.
// Thread b of a job produces the draws in words [16 b, 16 b + 16) of the
// stretch, which start at stream word word0 (a whole number of blocks unless
// an earlier rejection moved the stretch): 16 ternary values, or 8 uniform
// values of one limb (N is a multiple of 8), or 4 Gaussians.
#include "sample_device.h"

namespace th {

// Stream words [w, w + 16) of the stream of `seed` (one or two blocks).
static __device__ __forceinline__ void stream_words(uint64_t seed, uint64_t w, uint32_t out[16]) {
  const uint32_t lo = (uint32_t)seed, hi = (uint32_t)(seed >> 32);
  const uint32_t blk = (uint32_t)(w >> 4), sh = (uint32_t)(w & 15);
  if (sh == 0) {
    chacha20(lo, hi, blk, out);
    return;
  }
  uint32_t a[16], b[16];
  chacha20(lo, hi, blk, a);
  chacha20(lo, hi, blk + 1, b);
#pragma unroll
  for (uint32_t i = 0; i < 16; ++i) out[i] = i + sh < 16 ? a[(i + sh) & 15] : b[(i + sh) & 15];
}

__global__ __launch_bounds__(256) void k_key_draws(const KeyDrawJob* __restrict__ jobs, uint32_t n, uint32_t L,
                                                   const BarrettConst* __restrict__ bc, uint32_t* reject,
                                                   BandArgs band) {
  const KeyDrawJob jb = jobs[blockIdx.y];
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if ((uint64_t)16 * b >= key_draw_words(jb.kind, n, L)) return;
  uint32_t w[16];
  stream_words(jb.seed, jb.word0 + (uint64_t)16 * b, w);
  bool rejected = false;
  if (jb.kind == KEY_TERNARY) {
    // range_u32(3) rejects 0 (rng.rs:109-120); sample_ternary's {2, 0, 1}
    // mapped by keygen to +1, -1, 0 (sampling.rs:17-29, ciphertext.rs:86-97)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t r = w[i] % 3;
      gst(jb.s)[16 * b + i] = r == 0 ? 1 : (r == 1 ? -1 : 0);
      rejected |= w[i] == 0;
    }
  } else if (b < 2 * L * n / 16) {
    const uint32_t d0 = 8 * b, l = d0 / n, i0 = d0 % n;
    const BarrettConst c = bc[l];
    const uint64_t thr = mulmod_barrett(0 - c.q, 1, c);  // (2^64 - q) mod q (rng.rs:124-133)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t r = (uint64_t)w[2 * j] | ((uint64_t)w[2 * j + 1] << 32);
      rejected |= r < thr;
      gst(jb.a)[(size_t)l * n + i0 + j] = mulmod_barrett(r, 1, c);
    }
  } else {
    const uint32_t g0 = (16 * b - 2 * L * n) / 4;
    bool any = false;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      bool near;
      gst(jb.e)[g0 + t] = gaussian_rounded(w[4 * t], w[4 * t + 1], w[4 * t + 2], w[4 * t + 3], band.band, near);
      any |= near;
    }
    if (any) flag_of(band, blockIdx.y).raise();
  }
  if (rejected) atomicMin(reject, blockIdx.y);
}

// One thread: the job's draws from word word0 on, serially in the
// reference's order (a rejected word is skipped and the draw takes the next
// one); *end receives the word after the last one used.
__global__ void k_key_replay(const KeyDrawJob* __restrict__ job, uint32_t n, uint32_t L,
                             const BarrettConst* __restrict__ bc, uint64_t* end, BandArgs band) {
  const KeyDrawJob jb = *job;
  SerialStream st(jb.seed, (uint32_t)(jb.word0 >> 4));
  for (uint32_t i = 0; i < (uint32_t)(jb.word0 & 15); ++i) (void)st.next();
  uint64_t used = jb.word0;
  constexpr uint32_t kGuard = 1u << 20;  // bounds the walk over a stream of rejected words
  if (jb.kind == KEY_TERNARY) {
    for (uint32_t i = 0; i < n; ++i) {
      uint32_t r = st.next();
      ++used;
      for (uint32_t g = 0; r == 0 && g < kGuard; ++g, ++used) r = st.next();
      r %= 3;
      jb.s[i] = r == 0 ? 1 : (r == 1 ? -1 : 0);
    }
  } else {
    for (uint32_t l = 0; l < L; ++l) {
      const BarrettConst c = bc[l];
      const uint64_t thr = mulmod_barrett(0 - c.q, 1, c);
      for (uint32_t i = 0; i < n; ++i) {
        uint64_t r = 0;
        for (uint32_t g = 0; g < kGuard; ++g) {
          const uint64_t lo = st.next();
          r = lo | ((uint64_t)st.next() << 32);
          used += 2;
          if (r >= thr) break;
        }
        jb.a[(size_t)l * n + i] = mulmod_barrett(r, 1, c);
      }
    }
    bool any = false;
    for (uint32_t g = 0; g < n; ++g) {
      const uint32_t w0 = st.next(), w1 = st.next(), w2 = st.next(), w3 = st.next();
      used += 4;
      bool near;
      jb.e[g] = gaussian_rounded(w0, w1, w2, w3, band.band, near);
      any |= near;
    }
    if (any) flag_of(band, 0).raise();
  }
  *end = used;
}

hipError_t launch_key_draws(const KeyDrawJob* jobs, uint32_t njobs, uint32_t n, uint32_t L, const BarrettConst* bc,
                            uint32_t* reject, BandArgs band, hipStream_t s) {
  if (!njobs) return hipSuccess;
  if (n % 16) return hipErrorInvalidValue;
  const uint64_t threads = key_draw_words(KEY_UNIFORM_GAUSS, n, L) / 16;  // the longer kind
  hipLaunchKernelGGL(k_key_draws, dim3((uint32_t)((threads + 255) / 256), njobs), dim3(256), 0, s, jobs, n, L, bc,
                     reject, band);
  return hipGetLastError();
}

hipError_t launch_key_replay(const KeyDrawJob* job, uint32_t n, uint32_t L, const BarrettConst* bc, uint64_t* end,
                             BandArgs band, hipStream_t s) {
  hipLaunchKernelGGL(k_key_replay, dim3(1), dim3(1), 0, s, job, n, L, bc, end, band);
  return hipGetLastError();
}

}  // namespace th
