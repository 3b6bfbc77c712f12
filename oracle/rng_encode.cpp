// Oracle: ChaCha20 RNG, samplers and the f64 canonical-embedding encoder.
// Restates tensafe-he-core/src/rng.rs, sampling.rs and encoding.rs. Test
// infrastructure only (see oracle.h). Built with -ffp-contract=off.
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include <math.h>

#include <cmath>
#include <cstdio>
#include <stdexcept>

#include "oracle.h"

namespace oracle {

static const double PI = 3.14159265358979323846264338327950288;  // std::f64::consts::PI

static inline uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

// rng.rs:190-206
static inline void quarter_round(uint32_t* s, int a, int b, int c, int d) {
  s[a] += s[b]; s[d] ^= s[a]; s[d] = rotl32(s[d], 16);
  s[c] += s[d]; s[b] ^= s[c]; s[b] = rotl32(s[b], 12);
  s[a] += s[b]; s[d] ^= s[a]; s[d] = rotl32(s[d], 8);
  s[c] += s[d]; s[b] ^= s[c]; s[b] = rotl32(s[b], 7);
}

// rng.rs:163-186 — 10 double rounds, then add the input state.
void chacha20_block(const uint32_t state[16], uint32_t out[16]) {
  uint32_t w[16];
  for (int i = 0; i < 16; ++i) w[i] = state[i];
  for (int r = 0; r < 10; ++r) {
    quarter_round(w, 0, 4, 8, 12);
    quarter_round(w, 1, 5, 9, 13);
    quarter_round(w, 2, 6, 10, 14);
    quarter_round(w, 3, 7, 11, 15);
    quarter_round(w, 0, 5, 10, 15);
    quarter_round(w, 1, 6, 11, 12);
    quarter_round(w, 2, 7, 8, 13);
    quarter_round(w, 3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = w[i] + state[i];
}

// rng.rs:38-68 — key words (lo, hi) x4, counter = nonce = 0, block 0 generated now.
TenSafeRng TenSafeRng::from_seed(uint64_t seed) {
  TenSafeRng r;
  uint32_t lo = (uint32_t)seed, hi = (uint32_t)(seed >> 32);
  r.state_[0] = 0x61707865u;
  r.state_[1] = 0x3320646eu;
  r.state_[2] = 0x79622d32u;
  r.state_[3] = 0x6b206574u;
  for (int i = 0; i < 4; ++i) {
    r.state_[4 + i * 2] = lo;
    r.state_[5 + i * 2] = hi;
  }
  r.state_[12] = r.state_[13] = r.state_[14] = r.state_[15] = 0;
  for (int i = 0; i < 16; ++i) r.buffer_[i] = 0;
  r.index_ = 16;
  r.refill();
  return r;
}

// rng.rs:73-76, 210-221
TenSafeRng TenSafeRng::from_entropy() {
  uint64_t seed = 0;
  FILE* f = std::fopen("/dev/urandom", "rb");
  bool ok = false;
  if (f) {
    ok = std::fread(&seed, 1, 8, f) == 8;
    std::fclose(f);
  }
  if (!ok) seed = (uint64_t)(uintptr_t)&seed ^ 0xdeadbeefcafebabeULL;
  return from_seed(seed);
}

// rng.rs:79-84
void TenSafeRng::refill() {
  chacha20_block(state_, buffer_);
  index_ = 0;
  state_[12] += 1;
}

// rng.rs:88-95
uint32_t TenSafeRng::next_u32() {
  if (index_ >= 16) refill();
  return buffer_[index_++];
}

// rng.rs:99-103
uint64_t TenSafeRng::next_u64() {
  uint64_t lo = next_u32();
  uint64_t hi = next_u32();
  return (hi << 32) | lo;
}

// rng.rs:109-120 — reject r < (2^32 - max) % max.
uint32_t TenSafeRng::range_u32(uint32_t max) {
  uint32_t threshold = (0xFFFFFFFFu - max + 1) % max;
  for (;;) {
    uint32_t r = next_u32();
    if (r >= threshold) return r % max;
  }
}

// rng.rs:124-133
uint64_t TenSafeRng::range_u64(uint64_t max) {
  uint64_t threshold = (~0ULL - max + 1) % max;
  for (;;) {
    uint64_t r = next_u64();
    if (r >= threshold) return r % max;
  }
}

// rng.rs:139-144
double TenSafeRng::next_f64() {
  uint64_t bits = next_u64() >> 11;
  return ((double)bits + 0.5) / (double)(1ULL << 53);
}

// rng.rs:152-157 — Box-Muller, cosine branch only.
double TenSafeRng::gaussian(double sigma) {
  double u1 = next_f64();
  double u2 = next_f64();
  double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * PI * u2);
  return z * sigma;
}

// Rust `f as i64`: saturating, NaN -> 0.
static inline int64_t f64_to_i64_sat(double x) {
  if (std::isnan(x)) return 0;
  if (x >= 9223372036854775808.0) return INT64_MAX;
  if (x < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)x;
}

// sampling.rs:17-29 — r=0 -> q-1, r=1 -> 0, r=2 -> 1.
std::vector<uint64_t> sample_ternary(TenSafeRng& rng, size_t n, uint64_t q) {
  std::vector<uint64_t> out(n);
  for (size_t i = 0; i < n; ++i) {
    uint32_t r = rng.range_u32(3);
    out[i] = r == 0 ? q - 1 : (r == 1 ? 0 : 1);
  }
  return out;
}

// sampling.rs:34-47
std::vector<uint64_t> sample_gaussian(TenSafeRng& rng, size_t n, uint64_t q, double sigma) {
  std::vector<uint64_t> out(n);
  for (size_t i = 0; i < n; ++i) {
    int64_t r = f64_to_i64_sat(std::round(rng.gaussian(sigma)));
    out[i] = r >= 0 ? (uint64_t)r % q : q - ((uint64_t)(-r) % q);
  }
  return out;
}

// sampling.rs:51-58
std::vector<int64_t> sample_gaussian_signed(TenSafeRng& rng, size_t n, double sigma) {
  std::vector<int64_t> out(n);
  for (size_t i = 0; i < n; ++i) out[i] = f64_to_i64_sat(std::round(rng.gaussian(sigma)));
  return out;
}

// sampling.rs:62-64
std::vector<uint64_t> sample_uniform(TenSafeRng& rng, size_t n, uint64_t q) {
  std::vector<uint64_t> out(n);
  for (size_t i = 0; i < n; ++i) out[i] = rng.range_u64(q);
  return out;
}

// ciphertext.rs:255-273 — the draws encrypt_pk makes, in order: u via
// sample_ternary(rng, n, 3) (values {2,0,1} for r = {0,1,2}), then e0, then e1.
EncryptPkRandomness sample_encrypt_pk_randomness(TenSafeRng& rng, size_t n) {
  EncryptPkRandomness r;
  std::vector<uint64_t> t = sample_ternary(rng, n, 3);
  r.u.resize(n);
  for (size_t i = 0; i < n; ++i) r.u[i] = (uint32_t)t[i];
  r.e0 = sample_gaussian_signed(rng, n, ERROR_STD_DEV);
  r.e1 = sample_gaussian_signed(rng, n, ERROR_STD_DEV);
  return r;
}

// cos and sin of one angle. The reference computes `angle.cos()` and
// `angle.sin()` back to back (encoding.rs:47-48, :72-73); LLVM lowers such a
// pair of libm calls on one operand to glibc `sincos` on GNU targets, whose
// results differ from separate cos/sin calls in the last bit for ~0.1% of
// angles. Calling sincos explicitly keeps that choice independent of the C++
// compiler's own fusion heuristics. (No reference test pins these values.)
static inline void sincos_pair(double angle, double* c, double* s) { ::sincos(angle, s, c); }

// encoding.rs:39-80
FftTables FftTables::make(size_t n) {
  FftTables t;
  t.n = n;
  size_t log_n = (size_t)__builtin_ctzll((uint64_t)n);
  t.twist_re.assign(n, 0.0);
  t.twist_im.assign(n, 0.0);
  for (size_t j = 0; j < n; ++j) {
    double angle = PI * (double)j / (double)n;
    sincos_pair(angle, &t.twist_re[j], &t.twist_im[j]);
  }
  t.bit_rev.assign(n, 0);
  for (size_t i = 0; i < n; ++i) {
    size_t rev = 0, val = i;
    for (size_t k = 0; k < log_n; ++k) {
      rev = (rev << 1) | (val & 1);
      val >>= 1;
    }
    t.bit_rev[i] = rev;
  }
  for (size_t s = 0; s < log_n; ++s) {
    size_t half_len = (size_t)1 << s;
    std::vector<double> tre, tim;
    tre.reserve(half_len);
    tim.reserve(half_len);
    for (size_t k = 0; k < half_len; ++k) {
      double angle = -2.0 * PI * (double)k / (double)(2 * half_len);
      double c, si;
      sincos_pair(angle, &c, &si);
      tre.push_back(c);
      tim.push_back(si);
    }
    t.twiddle_re.push_back(std::move(tre));
    t.twiddle_im.push_back(std::move(tim));
  }
  return t;
}

// encoding.rs:83-120 — bit-reversal permutation, then radix-2 DIT stages.
void FftTables::fft(double* re, double* im) const {
  for (size_t i = 0; i < n; ++i) {
    size_t j = bit_rev[i];
    if (i < j) {
      double tr = re[i]; re[i] = re[j]; re[j] = tr;
      double ti = im[i]; im[i] = im[j]; im[j] = ti;
    }
  }
  for (size_t s = 0; s < twiddle_re.size(); ++s) {
    size_t half_len = (size_t)1 << s;
    size_t full_len = half_len << 1;
    for (size_t g = 0; g < n; g += full_len) {
      for (size_t k = 0; k < half_len; ++k) {
        double w_re = twiddle_re[s][k];
        double w_im = twiddle_im[s][k];
        size_t i0 = g + k, i1 = i0 + half_len;
        double v_re = w_re * re[i1] - w_im * im[i1];
        double v_im = w_re * im[i1] + w_im * re[i1];
        double u_re = re[i0], u_im = im[i0];
        re[i0] = u_re + v_re;
        im[i0] = u_im + v_im;
        re[i1] = u_re - v_re;
        im[i1] = u_im - v_im;
      }
    }
  }
}

// encoding.rs:152-162
CkksEncoder CkksEncoder::make(const CkksParams& p) {
  CkksEncoder e;
  e.n = p.poly_degree;
  e.num_slots = p.num_slots;
  e.fft = FftTables::make(p.poly_degree);
  return e;
}

// encoding.rs:173-207 — pad, sigma^{-1}, round(coeff * 2^40), signed -> per-limb residue.
RnsPoly CkksEncoder::encode(const double* z, size_t len, const CkksParams& p) const {
  if (len > num_slots) throw std::invalid_argument("Input length exceeds slot count");
  std::vector<double> z_full(num_slots, 0.0);
  for (size_t i = 0; i < len; ++i) z_full[i] = z[i];
  std::vector<double> coeffs = inverse_canonical_embedding(z_full);
  RnsPoly r = RnsPoly::zero(n, p.num_limbs);
  for (size_t l = 0; l < p.num_limbs; ++l) {
    uint64_t q = p.moduli[l].value;
    for (size_t i = 0; i < n; ++i) {
      double scaled = coeffs[i] * SCALE;
      int64_t rounded = f64_to_i64_sat(std::round(scaled));
      r.limbs[l][i] = rounded >= 0 ? (uint64_t)rounded % q : q - ((uint64_t)(-rounded) % q);
    }
  }
  return r;
}

// encoding.rs:219-239 — center limb 0 against q0/2, divide by scale, embed.
std::vector<double> CkksEncoder::decode(const RnsPoly& poly, const CkksParams& p,
                                        double scale) const {
  uint64_t q = p.moduli[0].value;
  uint64_t half_q = q / 2;
  std::vector<double> c(n);
  for (size_t i = 0; i < n; ++i) {
    uint64_t v = poly.limbs[0][i];
    double s = v > half_q ? -((double)(q - v)) : (double)v;
    c[i] = s / scale;
  }
  return canonical_embedding(c);
}

// encoding.rs:250-278
std::vector<double> CkksEncoder::inverse_canonical_embedding(const std::vector<double>& z) const {
  if (z.size() != num_slots) throw std::invalid_argument("slot count mismatch");
  std::vector<double> re(n, 0.0), im(n, 0.0);
  for (size_t k = 0; k < num_slots; ++k) {
    re[k] = z[k];
    re[n - 1 - k] = z[k];
  }
  fft.fft(re.data(), im.data());
  double inv_n = 1.0 / (double)n;
  std::vector<double> coeffs(n);
  for (size_t j = 0; j < n; ++j) {
    double a_re = re[j] * inv_n;
    double a_im = im[j] * inv_n;
    coeffs[j] = a_re * fft.twist_re[j] + a_im * fft.twist_im[j];
  }
  return coeffs;
}

// encoding.rs:282-284
std::vector<double> CkksEncoder::decode_coefficients(const std::vector<double>& c) const {
  return canonical_embedding(c);
}

// encoding.rs:295-315 — b = c * conj(twist), FFT, real parts of the first N/2.
std::vector<double> CkksEncoder::canonical_embedding(const std::vector<double>& c) const {
  if (c.size() != n) throw std::invalid_argument("coefficient count mismatch");
  std::vector<double> re(n), im(n);
  for (size_t j = 0; j < n; ++j) {
    re[j] = c[j] * fft.twist_re[j];
    im[j] = -c[j] * fft.twist_im[j];
  }
  fft.fft(re.data(), im.data());
  re.resize(num_slots);
  return re;
}

}  // namespace oracle
