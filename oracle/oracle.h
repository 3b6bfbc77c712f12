// CPU oracle: a C++ restatement of the reference CPU CKKS backend
// (tensafe-he/crates/tensafe-he-core/src/*.rs).
//
// TEST INFRASTRUCTURE ONLY. This library gives the results the tests of the
// HIP engine in provenloop_amd/ compare against, and the timed host-CPU
// baseline of bench.py. It is never
// linked into, loaded by, or called from the product path.
//
// Every function follows the reference line by line (same algorithm, same
// evaluation order, same RNG consumption order). Each definition cites the
// reference file:line it restates. Floating-point code is compiled with
// -ffp-contract=off and no fast-math, and calls glibc cos/sin/log like Rust std
// does on Linux, so the f64 steps (encode FFT, Box-Muller, decode) evaluate the
// same IEEE operations in the same order as the reference.
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

namespace oracle {

typedef unsigned __int128 u128;

// params.rs:9-12
constexpr uint32_t SCALE_BITS = 40;
constexpr double SCALE = (double)(1ULL << SCALE_BITS);

// params.rs:15-44
struct Modulus {
  uint64_t value;
  uint32_t bits;
  uint64_t barrett_hi;
  uint64_t barrett_lo;
  static Modulus make(uint64_t value, uint32_t bits);
};

// params.rs:47-61
struct CkksParams {
  size_t poly_degree;
  size_t num_slots;
  uint32_t log_n;
  std::vector<Modulus> moduli;
  size_t num_limbs;
  uint32_t scale_bits;

  static CkksParams n8192();
  static CkksParams n16384();
  static CkksParams n32768();
  static CkksParams for_degree(size_t n);  // throws on unsupported N
  static CkksParams custom(size_t poly_degree, const std::vector<uint32_t>& bits,
                           uint32_t scale_bits);
  // Not in the reference: an explicit chain of distinct primes (used for the
  // 8-limb N=32768 saturation workload, which the reference has no chain for).
  static CkksParams from_moduli(size_t poly_degree, const std::vector<uint64_t>& q,
                                uint32_t scale_bits);
};

uint64_t find_ntt_friendly_prime(uint32_t bits, uint64_t two_n);
bool is_prime_u64(uint64_t n);

// rns.rs
uint64_t mod_add(uint64_t a, uint64_t b, uint64_t q);
uint64_t mod_sub(uint64_t a, uint64_t b, uint64_t q);
uint64_t mod_mul(uint64_t a, uint64_t b, uint64_t q);
uint64_t barrett_reduce(u128 a, const Modulus& m);
uint64_t mod_mul_barrett(uint64_t a, uint64_t b, const Modulus& m);
uint64_t mod_pow(uint64_t base, uint64_t exp, uint64_t q);
uint64_t mod_inv(uint64_t a, uint64_t q);
uint64_t find_primitive_root(size_t n, uint64_t q);
std::vector<uint64_t> compute_twiddle_factors(size_t n, uint64_t psi, uint64_t q);
std::vector<uint64_t> compute_inv_twiddle_factors(size_t n, uint64_t psi, uint64_t q);
uint32_t bit_reverse(uint32_t x, uint32_t bits);

// rns.rs:199-270
struct RnsPoly {
  std::vector<std::vector<uint64_t>> limbs;
  size_t n = 0;
  static RnsPoly zero(size_t n, size_t num_limbs);
  RnsPoly add(const RnsPoly& o, const std::vector<Modulus>& moduli) const;
  RnsPoly sub(const RnsPoly& o, const std::vector<Modulus>& moduli) const;
  RnsPoly hadamard_mul(const RnsPoly& o, const std::vector<Modulus>& moduli) const;
  RnsPoly negate(const std::vector<Modulus>& moduli) const;
};

// ntt.rs:13-66
struct NttTables {
  std::vector<uint64_t> forward_twiddles;
  std::vector<uint64_t> inverse_twiddles;
  uint64_t psi, psi_inv, n_inv, q;
  Modulus modulus;
  uint32_t log_n;
  size_t n;
  static NttTables make(size_t n, uint64_t q);
};
void negacyclic_ntt_forward(uint64_t* a, const NttTables& t);
void negacyclic_ntt_inverse(uint64_t* a, const NttTables& t);

// rng.rs:16-221
void chacha20_block(const uint32_t state[16], uint32_t out[16]);
class TenSafeRng {
 public:
  static TenSafeRng from_seed(uint64_t seed);
  static TenSafeRng from_entropy();
  uint32_t next_u32();
  uint64_t next_u64();
  uint32_t range_u32(uint32_t max);
  uint64_t range_u64(uint64_t max);
  double next_f64();
  double gaussian(double sigma);

 private:
  void refill();
  uint32_t state_[16];
  uint32_t buffer_[16];
  size_t index_;
};

// sampling.rs
constexpr double ERROR_STD_DEV = 3.19;
std::vector<uint64_t> sample_ternary(TenSafeRng& rng, size_t n, uint64_t q);
std::vector<uint64_t> sample_gaussian(TenSafeRng& rng, size_t n, uint64_t q, double sigma);
std::vector<int64_t> sample_gaussian_signed(TenSafeRng& rng, size_t n, double sigma);
std::vector<uint64_t> sample_uniform(TenSafeRng& rng, size_t n, uint64_t q);

// encoding.rs:24-137
struct FftTables {
  size_t n;
  std::vector<double> twist_re, twist_im;
  std::vector<size_t> bit_rev;
  std::vector<std::vector<double>> twiddle_re, twiddle_im;
  static FftTables make(size_t n);
  void fft(double* re, double* im) const;
};

// encoding.rs:140-316
struct CkksEncoder {
  size_t n, num_slots;
  FftTables fft;
  static CkksEncoder make(const CkksParams& p);
  RnsPoly encode(const double* z, size_t len, const CkksParams& p) const;
  std::vector<double> decode(const RnsPoly& poly, const CkksParams& p, double scale) const;
  std::vector<double> inverse_canonical_embedding(const std::vector<double>& z) const;
  std::vector<double> decode_coefficients(const std::vector<double>& c) const;
  std::vector<double> canonical_embedding(const std::vector<double>& c) const;
};

// ciphertext.rs:18-46
struct Ciphertext {
  RnsPoly c0, c1;
  double scale;
};
struct SecretKey {
  RnsPoly s_ntt;
};
struct PublicKey {
  RnsPoly b, a;
};

// Randomness consumed by encrypt_pk, in draw order (ciphertext.rs:255-273):
// u holds the values sample_ternary(rng, n, 3) returns, v in {0,1,2} (mapped
// v=0 -> -1, 1 -> 0, 2 -> +1 per limb), e0/e1 the rounded Gaussian samples.
struct EncryptPkRandomness {
  std::vector<uint32_t> u;
  std::vector<int64_t> e0, e1;
};
EncryptPkRandomness sample_encrypt_pk_randomness(TenSafeRng& rng, size_t n);

// ciphertext.rs:49-546
struct CkksContext {
  CkksParams params;
  std::vector<NttTables> ntt_tables;
  CkksEncoder encoder;

  static CkksContext make(const CkksParams& p);
  SecretKey keygen(TenSafeRng& rng) const;
  PublicKey keygen_public(const SecretKey& sk, TenSafeRng& rng) const;
  Ciphertext encrypt(const double* z, size_t len, const SecretKey& sk, TenSafeRng& rng) const;
  Ciphertext encrypt_pk(const double* z, size_t len, const PublicKey& pk, TenSafeRng& rng) const;
  // encrypt_pk with the randomness supplied by the caller; identical to
  // encrypt_pk after the sampling calls.
  Ciphertext encrypt_pk_with(const double* z, size_t len, const PublicKey& pk,
                             const EncryptPkRandomness& r) const;
  std::vector<double> decrypt(const Ciphertext& ct, const SecretKey& sk) const;
  Ciphertext ct_pt_mul(const Ciphertext& ct, const double* pt, size_t len) const;
  Ciphertext ct_pt_mul_ntt(const Ciphertext& ct, const RnsPoly& pt_ntt) const;
  Ciphertext ct_add(const Ciphertext& a, const Ciphertext& b) const;
  Ciphertext ct_sub(const Ciphertext& a, const Ciphertext& b) const;
  Ciphertext rescale(const Ciphertext& ct) const;
  RnsPoly encode_to_ntt(const double* z, size_t len) const;
};

// serialize.rs
std::vector<uint8_t> rns_poly_to_bytes(const RnsPoly& p);
RnsPoly rns_poly_from_bytes(const uint8_t* b, size_t len, size_t n, size_t num_limbs);
std::vector<uint8_t> pk_to_bytes(const PublicKey& pk);
PublicKey pk_from_bytes(const uint8_t* b, size_t len, size_t n, size_t num_limbs);
std::vector<uint8_t> ct_to_bytes(const Ciphertext& ct);
Ciphertext ct_from_bytes(const uint8_t* b, size_t len, size_t n, size_t num_limbs);

}  // namespace oracle
