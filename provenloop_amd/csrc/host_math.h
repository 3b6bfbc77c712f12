// Host-side arithmetic of the engine: parameter tables, the seeded ChaCha20
// stream and samplers (key generation, secret-key encryption, the host
// sampler option) and the f64 FFT tables of the encoder.
//
// These follow the reference's definitions exactly (they decide ciphertext
// bits), but are this library's own implementation.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <vector>

namespace th {

typedef unsigned __int128 u128;

// Default RNS chains (tensafe-he-core/src/params.rs:66-126).
bool default_chain(uint32_t n, std::vector<uint64_t>& q);
bool is_prime(uint64_t n);
uint64_t powmod(uint64_t b, uint64_t e, uint64_t q);
uint64_t invmod(uint64_t a, uint64_t q);  // q prime, a != 0
// First g = 2, 3, ... whose g^((q-1)/2N) is a primitive 2N-th root (rns.rs:124-155).
uint64_t primitive_2n_root(uint32_t n, uint64_t q);

// Deterministic ChaCha20 stream with the reference's seed expansion and
// draw helpers (tensafe-he-core/src/rng.rs:31-157).
// A seed from the OS (/dev/urandom): TenSafeRng::from_entropy's seed
// (rng.rs:73-76, :210-221), for streams drawn on the device.
uint64_t os_entropy_seed();

class ChaChaStream {
 public:
  explicit ChaChaStream(uint64_t seed);
  static ChaChaStream from_os_entropy();
  uint32_t u32();
  uint64_t u64();
  uint32_t below_u32(uint32_t max);  // rejection sampling, rng.rs:109-120
  uint64_t below_u64(uint64_t max);  // rng.rs:124-133
  double unit_open();                // ((u64 >> 11) + 0.5) / 2^53
  double normal(double sigma);       // Box-Muller cosine branch

 private:
  void next_block();
  uint32_t key_[8];
  uint32_t counter_;
  uint32_t buf_[16];
  int pos_;
};

constexpr double ERROR_SIGMA = 3.19;  // sampling.rs:10

// Ternary draws as sample_ternary(rng, n, 3) stores them: r -> {2, 0, 1}[r].
void draw_ternary(ChaChaStream& s, size_t n, uint8_t* out);
// round(gaussian) as i64, half away from zero, saturating (sampling.rs:51-58).
void draw_gaussian(ChaChaStream& s, size_t n, int64_t* out);

// f64 tables of the canonical-embedding FFT (tensafe-he-core/src/encoding.rs:39-80),
// uploaded once per context for the GPU encoder and decoder.
// Weights of the ZeRo-MOAI segment sums taken straight from decrypted
// coefficients. Decoding (encoding.rs:219-239, :282-315) maps coefficient
// values v_j (centred, divided by the scale) to slots
//   z_k = Re(sum_j v_j e^{-i pi j / N} e^{-2 pi i j k / N}),  k < N/2,
// so the sum of slots [k0, k1) is sum_j v_j W[j] with
//   W[j] = sum_{k0 <= k < k1} cos(pi j (2k + 1) / N)
//        = cos(t (k0 + k1)) sin(t (k1 - k0)) / sin t,   t = pi j / N  (W[0] = k1 - k0).
// out[c * N + j] for segment c = slots [c d, min((c + 1) d, N/2)); long
// double evaluation with exact integer reduction of the angles.
void segment_weights(uint32_t n, uint32_t d, uint32_t cols, double* out);
// The same weights in recurrence form: with phi = pi j d / N, segment c's
// weight is W_c[j] = A_j cos((2c + 1) phi), A_j = sin(phi) / sin(pi j / N),
// so W_{c+1} = 2 cos(2 phi) W_c - W_{c-1} with W_{-1} = W_0. out[2j] = W_0[j],
// out[2j + 1] = 2 cos(2 phi) (j = 0: d and 2). Long double, exact angle
// reduction; n pairs.
void segment_weight_pairs(uint32_t n, uint32_t d, double* out);

struct Encoder {
  uint32_t n = 0, logn = 0;
  std::vector<double> twist_re, twist_im;   // cos/sin(pi j / N)
  std::vector<double> stage_re, stage_im;   // per-stage DIT twiddles, stage s at offset 2^s - 1
  void init(uint32_t n);
};

}  // namespace th
