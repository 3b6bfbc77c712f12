// Driver for the sanitizer build of host_math.cpp (make -C provenloop_amd/csrc
// sanitize): exercises every host-side routine the engine uses and prints
// what it produced, one "name value..." line each (doubles as the hex of
// their bits), so a test can compare the values with the CPU oracle while
// AddressSanitizer and UndefinedBehaviorSanitizer watch the code.
#include <inttypes.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "band.h"
#include "host_math.h"

using namespace th;

static void put_u64(const char* name, const uint64_t* v, size_t n) {
  printf("%s", name);
  for (size_t i = 0; i < n; ++i) printf(" %" PRIu64, v[i]);
  printf("\n");
}

static void put_i64(const char* name, const int64_t* v, size_t n) {
  printf("%s", name);
  for (size_t i = 0; i < n; ++i) printf(" %" PRId64, v[i]);
  printf("\n");
}

static void put_f64(const char* name, const double* v, size_t n) {
  printf("%s", name);
  for (size_t i = 0; i < n; ++i) {
    uint64_t b;
    memcpy(&b, &v[i], 8);
    printf(" %016" PRIx64, b);
  }
  printf("\n");
}

int main() {
  for (uint32_t n : {8192u, 16384u, 32768u}) {
    std::vector<uint64_t> q;
    if (!default_chain(n, q)) return 1;
    char name[64];
    snprintf(name, sizeof name, "chain_%u", n);
    put_u64(name, q.data(), q.size());
    std::vector<uint64_t> roots, inv3, prime;
    for (uint64_t p : q) {
      roots.push_back(primitive_2n_root(n, p));
      inv3.push_back(invmod(3, p));
      prime.push_back(is_prime(p) ? 1 : 0);
    }
    snprintf(name, sizeof name, "psi_%u", n);
    put_u64(name, roots.data(), roots.size());
    snprintf(name, sizeof name, "inv3_%u", n);
    put_u64(name, inv3.data(), inv3.size());
    snprintf(name, sizeof name, "isprime_%u", n);
    put_u64(name, prime.data(), prime.size());
  }
  // composites: a product of two chain-sized primes, Carmichael numbers, a prime square
  const uint64_t comp[] = {1099510054913ULL * 3ULL, 561ULL, 41041ULL, 3215031751ULL, 1000000016000000063ULL,
                           4294967291ULL * 4294967291ULL};
  std::vector<uint64_t> cp;
  for (uint64_t c : comp) cp.push_back(is_prime(c) ? 1 : 0);
  put_u64("isprime_composites", cp.data(), cp.size());
  uint64_t pw[] = {powmod(3, 1000000, 1152921504606748673ULL), powmod(2, 64, 1099510054913ULL)};
  put_u64("powmod", pw, 2);

  {
    ChaChaStream s(42);
    std::vector<uint64_t> w(64);
    for (auto& x : w) x = s.u32();
    put_u64("chacha_u32_42", w.data(), w.size());
  }
  {
    ChaChaStream s(9);
    std::vector<uint64_t> r(256);
    for (auto& x : r) x = s.below_u64(1152921504606748673ULL);
    put_u64("below_u64_9", r.data(), r.size());
  }
  {
    ChaChaStream s(11);
    std::vector<double> g(256);
    for (auto& x : g) x = s.normal(ERROR_SIGMA);
    put_f64("normal_11", g.data(), g.size());
  }
  {
    // encrypt_pk's draws: u, then e0, then e1 (ciphertext.rs:255-273)
    const size_t n = 1024;
    ChaChaStream s(7);
    std::vector<uint8_t> u(n);
    std::vector<int64_t> e0(n), e1(n);
    draw_ternary(s, n, u.data());
    draw_gaussian(s, n, e0.data());
    draw_gaussian(s, n, e1.data());
    std::vector<int64_t> ui(u.begin(), u.end());
    put_i64("pk_u_7", ui.data(), n);
    put_i64("pk_e0_7", e0.data(), n);
    put_i64("pk_e1_7", e1.data(), n);
  }
  {
    Encoder e;
    e.init(1024);
    put_f64("twist_re_1024", e.twist_re.data(), e.twist_re.size());
    put_f64("twist_im_1024", e.twist_im.data(), e.twist_im.size());
    put_f64("stage_re_1024", e.stage_re.data(), e.stage_re.size());
    put_f64("stage_im_1024", e.stage_im.data(), e.stage_im.size());
  }
  {
    const uint32_t n = 1024, d = 100, cols = 5;
    std::vector<double> w((size_t)cols * n), p((size_t)2 * n);
    segment_weights(n, d, cols, w.data());
    segment_weight_pairs(n, d, p.data());
    put_f64("segw_1024_100_5", w.data(), w.size());
    put_f64("segp_1024_100", p.data(), p.size());
  }
  {
    // the sampler's band test on values next to rounding boundaries, far from
    // them, at the exactness limit 2^52 and not finite (each value, then the
    // flags for bands 2^-36 and 2^-40)
    const double h = 0x1p-36;
    const double t[] = {0.5, 2.5 + 0x1p-40, 2.5 - 0x1p-40, 2.5 + 0x1p-37, 2.5 - 0x1p-37, 2.5 + h, 2.5 - h,
                        2.5 + 0x1p-35, -3.5 + 0x1p-38, -3.5 - 0x1p-34, 7.25, -0.75, 0.0, 27.5 + 0x1p-45,
                        0x1p51 + 0.5, 0x1p52, -0x1p52, 1.0 / 0.0, -1.0 / 0.0, 0.0 / 0.0};
    const size_t n = sizeof(t) / sizeof(t[0]);
    std::vector<uint64_t> f36, f40;
    for (double v : t) {
      f36.push_back(near_rounding_boundary(v, 0x1p-36) ? 1 : 0);
      f40.push_back(near_rounding_boundary(v, 0x1p-40) ? 1 : 0);
    }
    put_f64("band_t", t, n);
    put_u64("band_flag_36", f36.data(), n);
    put_u64("band_flag_40", f40.data(), n);
  }
  return 0;
}
