// Device side of the encrypt_pk sampler (tensafe-he-core/src/rng.rs:31-157,
// sampling.rs:17-64, ciphertext.rs:255-273), shared by the sampler kernels
// and by the encoder's kernels, which can draw a token's randomness beside the
// encoding and finish the sampler's rejection handling.
#pragma once
#include "band.h"
#include "encode_sample.h"

namespace th {

#define TH_QR(a, b, c, d)                                             \
  a += b; d ^= a; d = __builtin_rotateleft32(d, 16);                   \
  c += d; b ^= c; b = __builtin_rotateleft32(b, 12);                   \
  a += b; d ^= a; d = __builtin_rotateleft32(d, 8);                    \
  c += d; b ^= c; b = __builtin_rotateleft32(b, 7);

static __device__ __forceinline__ void chacha20(uint32_t lo, uint32_t hi, uint32_t counter, uint32_t out[16]) {
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

static __device__ __forceinline__ uint8_t ternary_value(uint32_t w) {
  const uint32_t r = w % 3;  // sampling.rs:20-25: r=0 -> 2 (q-1 with q=3), 1 -> 0, 2 -> 1
  return r == 0 ? 2 : (r == 1 ? 0 : 1);
}

static __device__ __forceinline__ double unit_open(uint32_t w0, uint32_t w1) {
  const uint64_t v = (uint64_t)w0 | ((uint64_t)w1 << 32);  // next_u64: lo word first (rng.rs:99-103)
  return ((double)(v >> 11) + 0.5) / 9007199254740992.0;     // rng.rs:139-144
}

static __device__ __forceinline__ int64_t gaussian_rounded(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                                           double band, bool& near) {
  const double u1 = unit_open(w0, w1);
  const double u2 = unit_open(w2, w3);
  constexpr double kTwoPi = 2.0 * 3.14159265358979323846264338327950288;  // 2.0 * PI, exact doubling
  const double z = sqrt(-2.0 * log(u1)) * cos(kTwoPi * u2);                // rng.rs:155
  const double t = z * 3.19;
  near = near_rounding_boundary(t, band);
  const double r = round(t);  // sampling.rs:54-55
  if (r != r) return 0;
  if (r >= 9223372036854775808.0) return INT64_MAX;
  if (r < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)r;
}

// Block b (one ChaCha20 block of 16 words) of job jb's stream: the u values
// of words [16 b, 16 b + 16) while they lie below n, else four Gaussian draws
// (g = (16 b - n) / 4 onwards, e0 then e1). A zero u word sets the job's
// reject flag; a draw within `band` of a rounding boundary raises `flag`.
static __device__ __forceinline__ void sample_block(const SampleJob& jb, uint64_t seed, uint32_t n, uint32_t b,
                                                    double band, const FlagOut& flag) {
  if (b >= 9 * (n / 16)) return;
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
    bool any = false;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t g = g0 + t;
      bool near;
      const int64_t e = gaussian_rounded(w[4 * t], w[4 * t + 1], w[4 * t + 2], w[4 * t + 3], band, near);
      any |= near;
      if (g < n)
        gst(jb.e0)[g] = e;
      else
        gst(jb.e1)[g - n] = e;
    }
    if (any) flag.raise();  // plain stores; rare
  }
}

// Seeds of up to SEEDS_PER_LAUNCH jobs passed with the launch itself, so a
// caller whose job arrays stay in device memory needs no copy per call.
struct SeedBlock {
  uint64_t v[SEEDS_PER_LAUNCH];
};

static __device__ __forceinline__ uint64_t job_seed(const SampleJob& jb, const SeedBlock& sb, int use_sb, uint32_t j) {
  return use_sb ? sb.v[j] : jb.seed;
}

// Serial replay of the reference's consumption order for one stream.
struct SerialStream {
  uint32_t lo, hi, counter, pos, w[16];
  __device__ explicit SerialStream(uint64_t seed, uint32_t block = 0)
      : lo((uint32_t)seed), hi((uint32_t)(seed >> 32)), counter(block), pos(16) {}
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
// flag: this job's band flag outputs.
static __device__ void serial_replay(const SampleJob& jb, uint64_t seed, uint32_t n, const FlagOut& flag,
                                     double band) {
  SerialStream st(seed);
  for (uint32_t i = 0; i < n; ++i) {
    uint32_t r = st.next();
    for (uint32_t guard = 0; r < 1 && guard < (1u << 20); ++guard) r = st.next();  // rng.rs:112-119
    jb.u[i] = ternary_value(r);
  }
  bool any = false;
  for (uint32_t i = 0; i < 2 * n; ++i) {
    const uint32_t w0 = st.next(), w1 = st.next(), w2 = st.next(), w3 = st.next();
    bool near;
    const int64_t e = gaussian_rounded(w0, w1, w2, w3, band, near);
    any |= near;
    if (i < n)
      jb.e0[i] = e;
    else
      jb.e1[i - n] = e;
  }
  if (any) flag.raise();
}

// The end of a flagged sampler launch for job j: replay the stream serially
// if a u word was rejected (or force_serial), then clear the flag. Run by one
// thread, in a launch ordered after the block kernel.
inline __device__ void sample_fix_job(const SampleJob& jb, uint64_t seed, uint32_t n, int force_serial,
                                      const FlagOut& flag, double band) {
  if (*jb.reject || force_serial) serial_replay(jb, seed, n, flag, band);
  *jb.reject = 0;
}

}  // namespace th
