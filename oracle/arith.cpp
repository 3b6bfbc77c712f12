// Oracle: parameters, RNS arithmetic and NTT.
// Restates tensafe-he-core/src/params.rs, rns.rs and ntt.rs. Test
// infrastructure only (see oracle.h).
#include <stdexcept>
#include <string>

#include "oracle.h"

namespace oracle {

// params.rs:31-43 — Barrett constant floor((2^128-1)/q) split into hi/lo.
Modulus Modulus::make(uint64_t value, uint32_t bits) {
  u128 full = (~(u128)0) / (u128)value;
  Modulus m;
  m.value = value;
  m.bits = bits;
  m.barrett_hi = (uint64_t)(full >> 64);
  m.barrett_lo = (uint64_t)full;
  return m;
}

static CkksParams make_params(size_t n, uint32_t log_n, std::vector<Modulus> moduli) {
  CkksParams p;
  p.poly_degree = n;
  p.num_slots = n / 2;
  p.log_n = log_n;
  p.num_limbs = moduli.size();
  p.moduli = std::move(moduli);
  p.scale_bits = SCALE_BITS;
  return p;
}

// params.rs:66-83
CkksParams CkksParams::n8192() {
  return make_params(8192, 13,
                     {Modulus::make(1152921504606830593ULL, 60), Modulus::make(1099511480321ULL, 40),
                      Modulus::make(1099510890497ULL, 40), Modulus::make(1152921504606601217ULL, 60)});
}

// params.rs:88-105
CkksParams CkksParams::n16384() {
  return make_params(16384, 14,
                     {Modulus::make(1152921504606748673ULL, 60), Modulus::make(1099510054913ULL, 40),
                      Modulus::make(1099508121601ULL, 40), Modulus::make(1152921504606683137ULL, 60)});
}

// params.rs:109-126
CkksParams CkksParams::n32768() {
  return make_params(32768, 15,
                     {Modulus::make(1152921504606584833ULL, 60), Modulus::make(1099507695617ULL, 40),
                      Modulus::make(1099506515969ULL, 40), Modulus::make(1152921504598720513ULL, 60)});
}

// params.rs:129-136
CkksParams CkksParams::for_degree(size_t n) {
  switch (n) {
    case 8192: return n8192();
    case 16384: return n16384();
    case 32768: return n32768();
    default:
      throw std::invalid_argument("Unsupported polynomial degree " + std::to_string(n) +
                                  ". Use 8192, 16384, or 32768.");
  }
}

static uint32_t trailing_zeros(uint64_t x) { return (uint32_t)__builtin_ctzll(x); }

// params.rs:142-162
CkksParams CkksParams::custom(size_t poly_degree, const std::vector<uint32_t>& bits,
                              uint32_t scale_bits) {
  if (poly_degree == 0 || (poly_degree & (poly_degree - 1)) != 0)
    throw std::invalid_argument("poly_degree must be a power of 2");
  uint64_t two_n = 2 * (uint64_t)poly_degree;
  std::vector<Modulus> moduli;
  for (uint32_t b : bits) moduli.push_back(Modulus::make(find_ntt_friendly_prime(b, two_n), b));
  CkksParams p = make_params(poly_degree, trailing_zeros(poly_degree), std::move(moduli));
  p.scale_bits = scale_bits;
  return p;
}

CkksParams CkksParams::from_moduli(size_t poly_degree, const std::vector<uint64_t>& q,
                                   uint32_t scale_bits) {
  if (poly_degree == 0 || (poly_degree & (poly_degree - 1)) != 0)
    throw std::invalid_argument("poly_degree must be a power of 2");
  std::vector<Modulus> moduli;
  for (uint64_t v : q) moduli.push_back(Modulus::make(v, 64 - (uint32_t)__builtin_clzll(v)));
  CkksParams p = make_params(poly_degree, trailing_zeros(poly_degree), std::move(moduli));
  p.scale_bits = scale_bits;
  return p;
}

// params.rs:169-193
uint64_t find_ntt_friendly_prime(uint32_t bits, uint64_t two_n) {
  uint64_t upper = bits >= 64 ? ~0ULL : ((1ULL << bits) - 1);
  uint64_t lower = 1ULL << (bits - 1);
  uint64_t candidate = upper - (upper % two_n) + 1;
  if (candidate > upper) candidate -= two_n;
  while (candidate >= lower) {
    if (is_prime_u64(candidate)) return candidate;
    candidate = candidate - two_n;  // wrapping_sub
    if (candidate < lower) break;
  }
  throw std::runtime_error("No " + std::to_string(bits) + "-bit NTT-friendly prime found");
}

// params.rs:308-326 (trial division; i.saturating_mul(i) <= n)
bool is_prime_u64(uint64_t n) {
  if (n < 2) return false;
  if (n == 2 || n == 3) return true;
  if (n % 2 == 0 || n % 3 == 0) return false;
  uint64_t i = 5;
  for (;;) {
    u128 sq = (u128)i * i;
    uint64_t sat = sq > (u128)~0ULL ? ~0ULL : (uint64_t)sq;
    if (sat > n) break;
    if (n % i == 0 || n % (i + 2) == 0) return false;
    i += 6;
  }
  return true;
}

// rns.rs:10-18
uint64_t mod_add(uint64_t a, uint64_t b, uint64_t q) {
  uint64_t sum = a + b;
  return sum >= q ? sum - q : sum;
}

// rns.rs:22-29
uint64_t mod_sub(uint64_t a, uint64_t b, uint64_t q) { return a >= b ? a - b : q - b + a; }

// rns.rs:33-36
uint64_t mod_mul(uint64_t a, uint64_t b, uint64_t q) { return (uint64_t)(((u128)a * b) % q); }

// rns.rs:45-87 — partial 128x128 product (lo*lo term dropped), two corrections.
uint64_t barrett_reduce(u128 a, const Modulus& m) {
  uint64_t q = m.value;
  uint64_t a_lo = (uint64_t)a;
  uint64_t a_hi = (uint64_t)(a >> 64);
  if (a_hi == 0) return a_lo % q;
  u128 p_hh = (u128)a_hi * m.barrett_hi;
  u128 p_hl = (u128)a_hi * m.barrett_lo;
  u128 p_lh = (u128)a_lo * m.barrett_hi;
  u128 mid_sum = (p_hl >> 64) + (p_lh >> 64);
  u128 mid_lo_sum = (u128)(uint64_t)p_hl + (u128)(uint64_t)p_lh;
  u128 mid_carry = mid_lo_sum >> 64;
  uint64_t approx_quot = (uint64_t)(p_hh + mid_sum + mid_carry);
  uint64_t r = a_lo - approx_quot * q;  // wrapping
  if (r >= q) r -= q;
  if (r >= q) r -= q;
  return r;
}

// rns.rs:91-95
uint64_t mod_mul_barrett(uint64_t a, uint64_t b, const Modulus& m) {
  return barrett_reduce((u128)a * b, m);
}

// rns.rs:99-110
uint64_t mod_pow(uint64_t base, uint64_t exp, uint64_t q) {
  uint64_t result = 1;
  base %= q;
  while (exp > 0) {
    if (exp & 1) result = mod_mul(result, base, q);
    exp >>= 1;
    base = mod_mul(base, base, q);
  }
  return result;
}

// rns.rs:114-117
uint64_t mod_inv(uint64_t a, uint64_t q) {
  if (a == 0) throw std::invalid_argument("Cannot invert zero");
  return mod_pow(a, q - 2, q);
}

// rns.rs:124-154 — first g in 2..10000 with psi=g^((q-1)/2N) > 1 and psi^N = q-1.
uint64_t find_primitive_root(size_t n, uint64_t q) {
  uint64_t two_n = 2 * (uint64_t)n;
  if (q % two_n != 1) throw std::invalid_argument("q is not NTT-friendly");
  uint64_t exponent = (q - 1) / two_n;
  for (uint64_t g = 2; g < 10000; ++g) {
    if (g >= q) break;
    uint64_t psi = mod_pow(g, exponent, q);
    if (psi <= 1) continue;
    if (mod_pow(psi, (uint64_t)n, q) == q - 1) return psi;
  }
  throw std::runtime_error("No primitive 2N-th root of unity found");
}

static uint32_t log2_exact(size_t n) { return (uint32_t)__builtin_ctzll((uint64_t)n); }

// rns.rs:161-171 — tw[bit_reverse(i)] = psi^i
std::vector<uint64_t> compute_twiddle_factors(size_t n, uint64_t psi, uint64_t q) {
  std::vector<uint64_t> tw(n, 0);
  uint32_t log_n = log2_exact(n);
  for (size_t i = 0; i < n; ++i) tw[bit_reverse((uint32_t)i, log_n)] = mod_pow(psi, i, q);
  return tw;
}

// rns.rs:175-185 — inv_tw[bit_reverse(i)] = psi^{-i}
std::vector<uint64_t> compute_inv_twiddle_factors(size_t n, uint64_t psi, uint64_t q) {
  uint64_t psi_inv = mod_inv(psi, q);
  std::vector<uint64_t> tw(n, 0);
  uint32_t log_n = log2_exact(n);
  for (size_t i = 0; i < n; ++i) tw[bit_reverse((uint32_t)i, log_n)] = mod_pow(psi_inv, i, q);
  return tw;
}

// rns.rs:188-196
uint32_t bit_reverse(uint32_t x, uint32_t bits) {
  uint32_t r = 0;
  for (uint32_t k = 0; k < bits; ++k) {
    r = (r << 1) | (x & 1);
    x >>= 1;
  }
  return r;
}

// rns.rs:209-214
RnsPoly RnsPoly::zero(size_t n, size_t num_limbs) {
  RnsPoly p;
  p.n = n;
  p.limbs.assign(num_limbs, std::vector<uint64_t>(n, 0));
  return p;
}

// rns.rs:217-227
RnsPoly RnsPoly::add(const RnsPoly& o, const std::vector<Modulus>& moduli) const {
  if (n != o.n) throw std::invalid_argument("RnsPoly::add size mismatch");
  // o.limbs[l] for every l of self: Rust panics (index out of bounds) when o has fewer limbs
  if (o.limbs.size() < limbs.size()) throw std::invalid_argument("RnsPoly::add: index out of bounds");
  RnsPoly r = zero(n, limbs.size());
  for (size_t l = 0; l < limbs.size(); ++l) {
    uint64_t q = moduli[l].value;
    for (size_t i = 0; i < n; ++i) r.limbs[l][i] = mod_add(limbs[l][i], o.limbs[l][i], q);
  }
  return r;
}

// rns.rs:230-240
RnsPoly RnsPoly::sub(const RnsPoly& o, const std::vector<Modulus>& moduli) const {
  if (n != o.n) throw std::invalid_argument("RnsPoly::sub size mismatch");
  // o.limbs[l] for every l of self: Rust panics (index out of bounds) when o has fewer limbs
  if (o.limbs.size() < limbs.size()) throw std::invalid_argument("RnsPoly::sub: index out of bounds");
  RnsPoly r = zero(n, limbs.size());
  for (size_t l = 0; l < limbs.size(); ++l) {
    uint64_t q = moduli[l].value;
    for (size_t i = 0; i < n; ++i) r.limbs[l][i] = mod_sub(limbs[l][i], o.limbs[l][i], q);
  }
  return r;
}

// rns.rs:243-253 — iterates over self's limbs (other may have more limbs).
RnsPoly RnsPoly::hadamard_mul(const RnsPoly& o, const std::vector<Modulus>& moduli) const {
  if (n != o.n) throw std::invalid_argument("RnsPoly::hadamard_mul size mismatch");
  // o.limbs[l] for every l of self: Rust panics (index out of bounds) when o has fewer limbs
  if (o.limbs.size() < limbs.size()) throw std::invalid_argument("RnsPoly::hadamard_mul: index out of bounds");
  RnsPoly r = zero(n, limbs.size());
  for (size_t l = 0; l < limbs.size(); ++l) {
    const Modulus& m = moduli[l];
    for (size_t i = 0; i < n; ++i) r.limbs[l][i] = mod_mul_barrett(limbs[l][i], o.limbs[l][i], m);
  }
  return r;
}

// rns.rs:256-269
RnsPoly RnsPoly::negate(const std::vector<Modulus>& moduli) const {
  RnsPoly r = zero(n, limbs.size());
  for (size_t l = 0; l < limbs.size(); ++l) {
    uint64_t q = moduli[l].value;
    for (size_t i = 0; i < n; ++i) r.limbs[l][i] = limbs[l][i] == 0 ? 0 : q - limbs[l][i];
  }
  return r;
}

// ntt.rs:38-65
NttTables NttTables::make(size_t n, uint64_t q) {
  if (n == 0 || (n & (n - 1)) != 0) throw std::invalid_argument("N must be a power of 2");
  NttTables t;
  t.log_n = log2_exact(n);
  t.psi = find_primitive_root(n, q);
  t.psi_inv = mod_inv(t.psi, q);
  t.forward_twiddles = compute_twiddle_factors(n, t.psi, q);
  t.inverse_twiddles = compute_inv_twiddle_factors(n, t.psi, q);
  t.n_inv = mod_inv((uint64_t)n, q);
  t.modulus = Modulus::make(q, 64 - (uint32_t)__builtin_clzll(q));
  t.q = q;
  t.n = n;
  return t;
}

// ntt.rs:79-102 — Cooley-Tukey, ascending m, twiddle forward_twiddles[m+i].
void negacyclic_ntt_forward(uint64_t* a, const NttTables& tb) {
  const size_t n = tb.n;
  const uint64_t q = tb.q;
  size_t t = n >> 1, m = 1;
  for (uint32_t s = 0; s < tb.log_n; ++s) {
    for (size_t i = 0; i < m; ++i) {
      uint64_t w = tb.forward_twiddles[m + i];
      size_t j1 = 2 * i * t;
      for (size_t j = j1; j < j1 + t; ++j) {
        uint64_t u = a[j];
        uint64_t v = mod_mul_barrett(a[j + t], w, tb.modulus);
        a[j] = mod_add(u, v, q);
        a[j + t] = mod_sub(u, v, q);
      }
    }
    t >>= 1;
    m <<= 1;
  }
}

// ntt.rs:113-141 — Gentleman-Sande, descending m, twiddle inverse_twiddles[m+i],
// then a separate multiply by N^{-1}.
void negacyclic_ntt_inverse(uint64_t* a, const NttTables& tb) {
  const size_t n = tb.n;
  const uint64_t q = tb.q;
  size_t t = 1, m = n >> 1;
  for (uint32_t s = 0; s < tb.log_n; ++s) {
    for (size_t i = 0; i < m; ++i) {
      uint64_t w = tb.inverse_twiddles[m + i];
      size_t j1 = 2 * i * t;
      for (size_t j = j1; j < j1 + t; ++j) {
        uint64_t u = a[j];
        uint64_t v = a[j + t];
        a[j] = mod_add(u, v, q);
        a[j + t] = mod_mul_barrett(mod_sub(u, v, q), w, tb.modulus);
      }
    }
    t <<= 1;
    m >>= 1;
  }
  for (size_t i = 0; i < n; ++i) a[i] = mod_mul_barrett(a[i], tb.n_inv, tb.modulus);
}

}  // namespace oracle
