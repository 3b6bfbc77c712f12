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
// Box-Muller uses the device log/cos; its rounded integer equals glibc's
// unless the two libraries' results straddle a .5 boundary (an event of
// probability ~1e-15 per sample). Parity runs use host-supplied randomness.
#include "encode_sample.h"

namespace th {

#define TH_QR(a, b, c, d)                                             \
  a += b; d ^= a; d = __builtin_rotateleft32(d, 16);                   \
  c += d; b ^= c; b = __builtin_rotateleft32(b, 12);                   \
  a += b; d ^= a; d = __builtin_rotateleft32(d, 8);                    \
  c += d; b ^= c; b = __builtin_rotateleft32(b, 7);

__device__ __forceinline__ void chacha20(uint32_t lo, uint32_t hi, uint32_t counter, uint32_t out[16]) {
  const uint32_t k0 = 0x61707865u, k1 = 0x3320646eu, k2 = 0x79622d32u, k3 = 0x6b206574u;
  uint32_t x0 = k0, x1 = k1, x2 = k2, x3 = k3, x4 = lo, x5 = hi, x6 = lo, x7 = hi;
  uint32_t x8 = lo, x9 = hi, x10 = lo, x11 = hi, x12 = counter, x13 = 0, x14 = 0, x15 = 0;
#pragma unroll 1
  for (int r = 0; r < 10; ++r) {
    TH_QR(x0, x4, x8, x12) TH_QR(x1, x5, x9, x13) TH_QR(x2, x6, x10, x14) TH_QR(x3, x7, x11, x15)
    TH_QR(x0, x5, x10, x15) TH_QR(x1, x6, x11, x12) TH_QR(x2, x7, x8, x13) TH_QR(x3, x4, x9, x14)
  }
  out[0] = x0 + k0; out[1] = x1 + k1; out[2] = x2 + k2; out[3] = x3 + k3;
  out[4] = x4 + lo; out[5] = x5 + hi; out[6] = x6 + lo; out[7] = x7 + hi;
  out[8] = x8 + lo; out[9] = x9 + hi; out[10] = x10 + lo; out[11] = x11 + hi;
  out[12] = x12 + counter; out[13] = x13; out[14] = x14; out[15] = x15;
}
#undef TH_QR

__device__ __forceinline__ uint8_t ternary_value(uint32_t w) {
  const uint32_t r = w % 3;  // sampling.rs:20-25: r=0 -> 2 (q-1 with q=3), 1 -> 0, 2 -> 1
  return r == 0 ? 2 : (r == 1 ? 0 : 1);
}

__device__ __forceinline__ double unit_open(uint32_t w0, uint32_t w1) {
  const uint64_t v = (uint64_t)w0 | ((uint64_t)w1 << 32);  // next_u64: lo word first (rng.rs:99-103)
  return ((double)(v >> 11) + 0.5) / 9007199254740992.0;     // rng.rs:139-144
}

__device__ __forceinline__ int64_t gaussian_rounded(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  const double u1 = unit_open(w0, w1);
  const double u2 = unit_open(w2, w3);
  constexpr double kTwoPi = 2.0 * 3.14159265358979323846264338327950288;  // 2.0 * PI, exact doubling
  const double z = sqrt(-2.0 * log(u1)) * cos(kTwoPi * u2);                // rng.rs:155
  const double r = round(z * 3.19);                                      // sampling.rs:54-55
  if (r != r) return 0;
  if (r >= 9223372036854775808.0) return INT64_MAX;
  if (r < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)r;
}

// Seeds of up to SEEDS_PER_LAUNCH jobs passed with the launch itself, so a
// caller whose job arrays stay in device memory needs no copy per call.
constexpr uint32_t SEEDS_PER_LAUNCH = 64;
struct SeedBlock {
  uint64_t v[SEEDS_PER_LAUNCH];
};

__device__ __forceinline__ uint64_t job_seed(const SampleJob& jb, const SeedBlock& sb, int use_sb, uint32_t j) {
  return use_sb ? sb.v[j] : jb.seed;
}

// One thread per 16-word block of the stream.
__global__ void k_sample_blocks(const SampleJob* __restrict__ jobs, uint32_t n, SeedBlock sb, int use_sb) {
  const SampleJob jb = jobs[blockIdx.y];
  const uint64_t seed = job_seed(jb, sb, use_sb, blockIdx.y);
  const uint32_t nblocks = 9 * (n / 16);
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  uint32_t w[16];
  chacha20((uint32_t)seed, (uint32_t)(seed >> 32), b, w);
  if (b < n / 16) {
    bool zero = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      gst(jb.u)[16 * b + i] = ternary_value(w[i]);
      zero |= w[i] == 0;
    }
    if (zero && jb.reject) atomicOr(jb.reject, 1u);  // range_u32 rejects 0 (rng.rs:112-119)
  } else {
    const uint32_t g0 = (16 * b - n) / 4;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t g = g0 + t;
      const int64_t e = gaussian_rounded(w[4 * t], w[4 * t + 1], w[4 * t + 2], w[4 * t + 3]);
      if (g < n)
        gst(jb.e0)[g] = e;
      else
        gst(jb.e1)[g - n] = e;
    }
  }
}

// Serial replay of the reference's consumption order for one stream.
struct SerialStream {
  uint32_t lo, hi, counter, pos, w[16];
  __device__ explicit SerialStream(uint64_t seed) : lo((uint32_t)seed), hi((uint32_t)(seed >> 32)), counter(0), pos(16) {}
  __device__ uint32_t next() {
    if (pos == 16) {
      chacha20(lo, hi, counter, w);
      ++counter;
      pos = 0;
    }
    return w[pos++];
  }
};

// The reference's consumption order for one stream, walked serially
// (handles range_u32 rejections: rng.rs:109-133, ciphertext.rs:255-273).
__device__ void serial_replay(const SampleJob& jb, uint64_t seed, uint32_t n) {
  SerialStream st(seed);
  for (uint32_t i = 0; i < n; ++i) {
    uint32_t r = st.next();
    for (uint32_t guard = 0; r < 1 && guard < (1u << 20); ++guard) r = st.next();  // rng.rs:112-119
    jb.u[i] = ternary_value(r);
  }
  for (uint32_t i = 0; i < 2 * n; ++i) {
    const uint32_t w0 = st.next(), w1 = st.next(), w2 = st.next(), w3 = st.next();
    const int64_t e = gaussian_rounded(w0, w1, w2, w3);
    if (i < n)
      jb.e0[i] = e;
    else
      jb.e1[i - n] = e;
  }
}

// One workgroup per job: re-derive the u words; if any was rejected (== 0),
// or force_serial is set, lane 0 rewrites u, e0 and e1 by the serial walk.
__global__ __launch_bounds__(256) void k_sample_check(const SampleJob* __restrict__ jobs, uint32_t n, int force_serial,
                                                      SeedBlock sb, int use_sb) {
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
  serial_replay(jb, seed, n);
}

// One thread per job with a reject flag: replay flagged (or forced) jobs
// serially, then clear the flag for the next launch.
__global__ void k_sample_fix(const SampleJob* __restrict__ jobs, uint32_t njobs, uint32_t n, int force_serial,
                             SeedBlock sb, int use_sb) {
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= njobs) return;
  const SampleJob jb = jobs[j];
  if (*jb.reject || force_serial) serial_replay(jb, job_seed(jb, sb, use_sb, j), n);
  *jb.reject = 0;
}

hipError_t launch_sample_pk(const SampleJob* jobs, uint32_t njobs, uint32_t n, int force_serial, hipStream_t s,
                            const uint64_t* seeds, bool flagged) {
  if (!njobs) return hipSuccess;
  if (n % 16) return hipErrorInvalidValue;
  const uint32_t nblocks = 9 * (n / 16);
  SeedBlock sb{};
  for (uint32_t first = 0; first < njobs; first += SEEDS_PER_LAUNCH) {
    const uint32_t cnt = njobs - first < SEEDS_PER_LAUNCH ? njobs - first : SEEDS_PER_LAUNCH;
    if (seeds)
      for (uint32_t i = 0; i < cnt; ++i) sb.v[i] = seeds[first + i];
    hipLaunchKernelGGL(k_sample_blocks, dim3((nblocks + 255) / 256, cnt), dim3(256), 0, s, jobs + first, n, sb,
                       seeds != nullptr);
    if (flagged)
      hipLaunchKernelGGL(k_sample_fix, dim3((cnt + 63) / 64), dim3(64), 0, s, jobs + first, cnt, n, force_serial, sb,
                         seeds != nullptr);
    else
      hipLaunchKernelGGL(k_sample_check, dim3(cnt), dim3(256), 0, s, jobs + first, n, force_serial, sb,
                         seeds != nullptr);
  }
  return hipGetLastError();
}

}  // namespace th
