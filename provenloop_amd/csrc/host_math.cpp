// Host-side arithmetic of the engine (see host_math.h). Compiled with
// -ffp-contract=off: the encoder's f64 operations must round exactly as the
// reference's do.
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include "host_math.h"

#include <math.h>

#include <algorithm>
#include <stdio.h>
#include <string.h>

namespace th {

static const double kPi = 3.14159265358979323846264338327950288;

bool default_chain(uint32_t n, std::vector<uint64_t>& q) {
  switch (n) {
    case 8192:  // params.rs:69-74
      q = {1152921504606830593ULL, 1099511480321ULL, 1099510890497ULL, 1152921504606601217ULL};
      return true;
    case 16384:  // params.rs:91-96
      q = {1152921504606748673ULL, 1099510054913ULL, 1099508121601ULL, 1152921504606683137ULL};
      return true;
    case 32768:  // params.rs:112-117
      q = {1152921504606584833ULL, 1099507695617ULL, 1099506515969ULL, 1152921504598720513ULL};
      return true;
    default:
      return false;
  }
}

uint64_t powmod(uint64_t b, uint64_t e, uint64_t q) {
  uint64_t r = 1 % q;
  b %= q;
  while (e) {
    if (e & 1) r = (uint64_t)(((u128)r * b) % q);
    b = (uint64_t)(((u128)b * b) % q);
    e >>= 1;
  }
  return r;
}

uint64_t invmod(uint64_t a, uint64_t q) { return powmod(a, q - 2, q); }

bool is_prime(uint64_t n) {
  if (n < 2) return false;
  static const uint64_t small[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  for (uint64_t p : small) {
    if (n == p) return true;
    if (n % p == 0) return false;
  }
  uint64_t d = n - 1;
  int s = 0;
  while ((d & 1) == 0) {
    d >>= 1;
    ++s;
  }
  for (uint64_t a : small) {  // deterministic for n < 3.3e24
    uint64_t x = powmod(a, d, n);
    if (x == 1 || x == n - 1) continue;
    bool comp = true;
    for (int r = 1; r < s; ++r) {
      x = (uint64_t)(((u128)x * x) % n);
      if (x == n - 1) {
        comp = false;
        break;
      }
    }
    if (comp) return false;
  }
  return true;
}

uint64_t primitive_2n_root(uint32_t n, uint64_t q) {
  const uint64_t two_n = 2ULL * n;
  if (q % two_n != 1) return 0;
  const uint64_t e = (q - 1) / two_n;
  for (uint64_t g = 2; g < 10000 && g < q; ++g) {
    uint64_t psi = powmod(g, e, q);
    if (psi <= 1) continue;
    if (powmod(psi, n, q) == q - 1) return psi;
  }
  return 0;
}

// ---------------------------------------------------------------- ChaCha20
#define TH_QR(a, b, c, d)                 \
  a += b; d ^= a; d = (d << 16) | (d >> 16); \
  c += d; b ^= c; b = (b << 12) | (b >> 20); \
  a += b; d ^= a; d = (d << 8) | (d >> 24);  \
  c += d; b ^= c; b = (b << 7) | (b >> 25);

ChaChaStream::ChaChaStream(uint64_t seed) {
  // rng.rs:38-68: key words alternate (lo, hi) of the seed, counter and nonce zero,
  // the first block is produced at construction.
  for (int i = 0; i < 4; ++i) {
    key_[2 * i] = (uint32_t)seed;
    key_[2 * i + 1] = (uint32_t)(seed >> 32);
  }
  counter_ = 0;
  next_block();
}

uint64_t os_entropy_seed() {
  uint64_t seed = 0;
  FILE* f = fopen("/dev/urandom", "rb");
  bool ok = false;
  if (f) {
    ok = fread(&seed, 1, 8, f) == 8;
    fclose(f);
  }
  if (!ok) seed = (uint64_t)(uintptr_t)&seed ^ 0xdeadbeefcafebabeULL;
  return seed;
}

ChaChaStream ChaChaStream::from_os_entropy() { return ChaChaStream(os_entropy_seed()); }

void ChaChaStream::next_block() {
  const uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                           key_[0], key_[1], key_[2], key_[3], key_[4], key_[5], key_[6], key_[7],
                           counter_, 0u, 0u, 0u};
  uint32_t x0 = in[0], x1 = in[1], x2 = in[2], x3 = in[3], x4 = in[4], x5 = in[5], x6 = in[6],
           x7 = in[7], x8 = in[8], x9 = in[9], x10 = in[10], x11 = in[11], x12 = in[12],
           x13 = in[13], x14 = in[14], x15 = in[15];
  for (int r = 0; r < 10; ++r) {
    TH_QR(x0, x4, x8, x12) TH_QR(x1, x5, x9, x13) TH_QR(x2, x6, x10, x14) TH_QR(x3, x7, x11, x15)
    TH_QR(x0, x5, x10, x15) TH_QR(x1, x6, x11, x12) TH_QR(x2, x7, x8, x13) TH_QR(x3, x4, x9, x14)
  }
  const uint32_t o[16] = {x0, x1, x2, x3, x4, x5, x6, x7, x8, x9, x10, x11, x12, x13, x14, x15};
  for (int i = 0; i < 16; ++i) buf_[i] = o[i] + in[i];
  ++counter_;
  pos_ = 0;
}
#undef TH_QR

uint32_t ChaChaStream::u32() {
  if (pos_ == 16) next_block();
  return buf_[pos_++];
}

uint64_t ChaChaStream::u64() {
  uint64_t lo = u32();
  return lo | ((uint64_t)u32() << 32);
}

uint32_t ChaChaStream::below_u32(uint32_t max) {
  const uint32_t reject_below = (uint32_t)((0x100000000ULL) % max);
  for (;;) {
    uint32_t r = u32();
    if (r >= reject_below) return r % max;
  }
}

uint64_t ChaChaStream::below_u64(uint64_t max) {
  const uint64_t reject_below = (uint64_t)(((u128)1 << 64) % max);
  for (;;) {
    uint64_t r = u64();
    if (r >= reject_below) return r % max;
  }
}

double ChaChaStream::unit_open() { return ((double)(u64() >> 11) + 0.5) / 9007199254740992.0; }

double ChaChaStream::normal(double sigma) {
  double a = unit_open();
  double b = unit_open();
  return sqrt(-2.0 * log(a)) * cos(2.0 * kPi * b) * sigma;
}

void draw_ternary(ChaChaStream& s, size_t n, uint8_t* out) {
  static const uint8_t map[3] = {2, 0, 1};
  for (size_t i = 0; i < n; ++i) out[i] = map[s.below_u32(3)];
}

static inline int64_t round_sat(double x) {
  double r = round(x);
  if (r != r) return 0;
  if (r >= 9223372036854775808.0) return INT64_MAX;
  if (r < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)r;
}

void draw_gaussian(ChaChaStream& s, size_t n, int64_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = round_sat(s.normal(ERROR_SIGMA));
}

// ---------------------------------------------------------------- encoder
// The reference evaluates `angle.cos()` and `angle.sin()` of one angle back
// to back; LLVM lowers that pair to glibc sincos on GNU targets, which rounds
// differently from separate cos/sin calls for ~0.1% of angles. The tables are
// therefore built with sincos explicitly.
void Encoder::init(uint32_t nn) {
  n = nn;
  logn = (uint32_t)__builtin_ctz(nn);
  twist_re.resize(n);
  twist_im.resize(n);
  for (uint32_t j = 0; j < n; ++j) {
    double angle = kPi * (double)j / (double)n;  // encoding.rs:45-49
    sincos(angle, &twist_im[j], &twist_re[j]);
  }
  stage_re.assign(n, 0.0);
  stage_im.assign(n, 0.0);
  for (uint32_t s = 0; s < logn; ++s) {
    uint32_t half = 1u << s;
    for (uint32_t k = 0; k < half; ++k) {
      double angle = -2.0 * kPi * (double)k / (double)(2 * half);  // encoding.rs:70-74
      sincos(angle, &stage_im[half - 1 + k], &stage_re[half - 1 + k]);
    }
  }
}

}  // namespace th

namespace th {

void segment_weights(uint32_t n, uint32_t d, uint32_t cols, double* out) {
  const uint32_t S = n / 2;
  const long double pi = 3.141592653589793238462643383279502884L;
  // angle pi * m / N for an integer m, reduced modulo 2N exactly
  auto ang = [&](uint64_t m) { return pi * (long double)(m % (2ull * n)) / (long double)n; };
  for (uint32_t c = 0; c < cols; ++c) {
    const uint64_t k0 = (uint64_t)c * d, k1 = std::min<uint64_t>((uint64_t)(c + 1) * d, S);
    double* w = out + (size_t)c * n;
    for (uint32_t j = 0; j < n; ++j) {
      if (k1 <= k0) {
        w[j] = 0.0;
      } else if (j == 0) {
        w[j] = (double)(k1 - k0);
      } else {
        const long double num = cosl(ang((uint64_t)j * (k0 + k1))) * sinl(ang((uint64_t)j * (k1 - k0)));
        w[j] = (double)(num / sinl(ang(j)));
      }
    }
  }
}

void segment_weight_pairs(uint32_t n, uint32_t d, double* out) {
  const long double pi = 3.141592653589793238462643383279502884L;
  auto ang = [&](uint64_t m) { return pi * (long double)(m % (2ull * n)) / (long double)n; };
  out[0] = (double)d;
  out[1] = 2.0;
  for (uint32_t j = 1; j < n; ++j) {
    const long double phi = ang((uint64_t)j * d);
    out[2 * j] = (double)(sinl(phi) * cosl(phi) / sinl(ang(j)));
    out[2 * j + 1] = (double)(2.0L * cosl(ang(2ull * j * d)));
  }
}

}  // namespace th
