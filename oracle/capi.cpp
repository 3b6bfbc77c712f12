// Flat C interface of the CPU oracle, for ctypes (oracle/oracle.py).
// Test infrastructure only (see oracle.h): called by tests/, the smoke check
// and bench.py's CPU-baseline leg, never by the product path.
#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>

#include "oracle.h"

using namespace oracle;

namespace {
thread_local std::string g_err;

template <class F>
int guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  } catch (...) {
    g_err = "unknown error";
    return -1;
  }
}

std::mutex g_tab_mu;
std::map<std::pair<size_t, uint64_t>, std::shared_ptr<NttTables>> g_tabs;

std::shared_ptr<NttTables> tables_for(size_t n, uint64_t q) {
  std::lock_guard<std::mutex> lk(g_tab_mu);
  auto key = std::make_pair(n, q);
  auto it = g_tabs.find(key);
  if (it != g_tabs.end()) return it->second;
  auto t = std::make_shared<NttTables>(NttTables::make(n, q));
  g_tabs[key] = t;
  return t;
}

void copy_poly_out(const RnsPoly& p, uint64_t* out) {
  size_t off = 0;
  for (const auto& limb : p.limbs) {
    std::memcpy(out + off, limb.data(), p.n * 8);
    off += p.n;
  }
}

RnsPoly poly_in(const uint64_t* in, size_t n, size_t limbs) {
  RnsPoly p = RnsPoly::zero(n, limbs);
  for (size_t l = 0; l < limbs; ++l) std::memcpy(p.limbs[l].data(), in + l * n, n * 8);
  return p;
}
}  // namespace

extern "C" {

const char* orc_last_error() { return g_err.c_str(); }

// ---- parameters -----------------------------------------------------------
int orc_default_chain(size_t n, uint64_t* moduli_out, size_t* L_out) {
  return guard([&] {
    CkksParams p = CkksParams::for_degree(n);
    for (size_t l = 0; l < p.num_limbs; ++l) moduli_out[l] = p.moduli[l].value;
    *L_out = p.num_limbs;
  });
}

int orc_custom_chain(size_t n, const uint32_t* bits, size_t nb, uint64_t* moduli_out) {
  return guard([&] {
    CkksParams p = CkksParams::custom(n, std::vector<uint32_t>(bits, bits + nb), 40);
    for (size_t l = 0; l < nb; ++l) moduli_out[l] = p.moduli[l].value;
  });
}

int orc_modulus(uint64_t q, uint64_t* barrett_hi, uint64_t* barrett_lo) {
  return guard([&] {
    Modulus m = Modulus::make(q, 64 - (uint32_t)__builtin_clzll(q));
    *barrett_hi = m.barrett_hi;
    *barrett_lo = m.barrett_lo;
  });
}

int orc_is_prime(uint64_t n) { return is_prime_u64(n) ? 1 : 0; }

// ---- RNS arithmetic -------------------------------------------------------
uint64_t orc_mod_add(uint64_t a, uint64_t b, uint64_t q) { return mod_add(a, b, q); }
uint64_t orc_mod_sub(uint64_t a, uint64_t b, uint64_t q) { return mod_sub(a, b, q); }
uint64_t orc_mod_mul(uint64_t a, uint64_t b, uint64_t q) { return mod_mul(a, b, q); }
uint64_t orc_mod_pow(uint64_t a, uint64_t e, uint64_t q) { return mod_pow(a, e, q); }
int orc_mod_inv(uint64_t a, uint64_t q, uint64_t* out) {
  return guard([&] { *out = mod_inv(a, q); });
}
uint32_t orc_bit_reverse(uint32_t x, uint32_t bits) { return bit_reverse(x, bits); }
int orc_find_primitive_root(size_t n, uint64_t q, uint64_t* out) {
  return guard([&] { *out = find_primitive_root(n, q); });
}
// Barrett-reduce a batch of 128-bit values (lo/hi word arrays) modulo q.
int orc_barrett_reduce(const uint64_t* lo, const uint64_t* hi, size_t count, uint64_t q,
                       uint64_t* out) {
  return guard([&] {
    Modulus m = Modulus::make(q, 64 - (uint32_t)__builtin_clzll(q));
    for (size_t i = 0; i < count; ++i) out[i] = barrett_reduce(((u128)hi[i] << 64) | lo[i], m);
  });
}
int orc_mod_mul_barrett(const uint64_t* a, const uint64_t* b, size_t count, uint64_t q,
                        uint64_t* out) {
  return guard([&] {
    Modulus m = Modulus::make(q, 64 - (uint32_t)__builtin_clzll(q));
    for (size_t i = 0; i < count; ++i) out[i] = mod_mul_barrett(a[i], b[i], m);
  });
}

// ---- NTT ------------------------------------------------------------------
int orc_ntt_tables(size_t n, uint64_t q, uint64_t* fwd, uint64_t* inv, uint64_t* psi,
                   uint64_t* psi_inv, uint64_t* n_inv) {
  return guard([&] {
    auto t = tables_for(n, q);
    if (fwd) std::memcpy(fwd, t->forward_twiddles.data(), n * 8);
    if (inv) std::memcpy(inv, t->inverse_twiddles.data(), n * 8);
    if (psi) *psi = t->psi;
    if (psi_inv) *psi_inv = t->psi_inv;
    if (n_inv) *n_inv = t->n_inv;
  });
}

// In-place transforms of `count` consecutive polynomials of length n mod q.
int orc_ntt_forward(uint64_t* a, size_t count, size_t n, uint64_t q) {
  return guard([&] {
    auto t = tables_for(n, q);
    for (size_t c = 0; c < count; ++c) negacyclic_ntt_forward(a + c * n, *t);
  });
}
int orc_ntt_inverse(uint64_t* a, size_t count, size_t n, uint64_t q) {
  return guard([&] {
    auto t = tables_for(n, q);
    for (size_t c = 0; c < count; ++c) negacyclic_ntt_inverse(a + c * n, *t);
  });
}

// ---- RNG and sampling -----------------------------------------------------
void orc_chacha20_block(const uint32_t* state, uint32_t* out) { chacha20_block(state, out); }

int orc_rng_u32(uint64_t seed, size_t count, uint32_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    for (size_t i = 0; i < count; ++i) out[i] = r.next_u32();
  });
}
int orc_rng_u64(uint64_t seed, size_t count, uint64_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    for (size_t i = 0; i < count; ++i) out[i] = r.next_u64();
  });
}
int orc_rng_range_u32(uint64_t seed, uint32_t max, size_t count, uint32_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    for (size_t i = 0; i < count; ++i) out[i] = r.range_u32(max);
  });
}
int orc_rng_range_u64(uint64_t seed, uint64_t max, size_t count, uint64_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    for (size_t i = 0; i < count; ++i) out[i] = r.range_u64(max);
  });
}
int orc_rng_f64(uint64_t seed, size_t count, double* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    for (size_t i = 0; i < count; ++i) out[i] = r.next_f64();
  });
}
int orc_rng_gaussian(uint64_t seed, double sigma, size_t count, double* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    for (size_t i = 0; i < count; ++i) out[i] = r.gaussian(sigma);
  });
}
int orc_rng_entropy_u64(size_t count, uint64_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_entropy();
    for (size_t i = 0; i < count; ++i) out[i] = r.next_u64();
  });
}
int orc_sample_ternary(uint64_t seed, size_t n, uint64_t q, uint64_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    auto v = sample_ternary(r, n, q);
    std::memcpy(out, v.data(), n * 8);
  });
}
int orc_sample_gaussian(uint64_t seed, size_t n, uint64_t q, double sigma, uint64_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    auto v = sample_gaussian(r, n, q, sigma);
    std::memcpy(out, v.data(), n * 8);
  });
}
int orc_sample_gaussian_signed(uint64_t seed, size_t n, double sigma, int64_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    auto v = sample_gaussian_signed(r, n, sigma);
    std::memcpy(out, v.data(), n * 8);
  });
}
int orc_sample_uniform(uint64_t seed, size_t n, uint64_t q, uint64_t* out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    auto v = sample_uniform(r, n, q);
    std::memcpy(out, v.data(), n * 8);
  });
}
// The (u, e0, e1) draws of encrypt_pk for a fresh TenSafeRng::from_seed(seed).
int orc_encrypt_pk_randomness(uint64_t seed, size_t n, uint8_t* u, int64_t* e0, int64_t* e1) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    EncryptPkRandomness x = sample_encrypt_pk_randomness(r, n);
    for (size_t i = 0; i < n; ++i) u[i] = (uint8_t)x.u[i];
    std::memcpy(e0, x.e0.data(), n * 8);
    std::memcpy(e1, x.e1.data(), n * 8);
  });
}

// ---- context and handles ---------------------------------------------------
// moduli == NULL selects CkksParams::for_degree(n).
int orc_ctx_new(size_t n, const uint64_t* moduli, size_t L, void** out) {
  return guard([&] {
    CkksParams p = moduli ? CkksParams::from_moduli(n, std::vector<uint64_t>(moduli, moduli + L), 40)
                          : CkksParams::for_degree(n);
    *out = new CkksContext(CkksContext::make(p));
  });
}
void orc_ctx_free(void* c) { delete (CkksContext*)c; }
void orc_sk_free(void* p) { delete (SecretKey*)p; }
void orc_pk_free(void* p) { delete (PublicKey*)p; }
void orc_ct_free(void* p) { delete (Ciphertext*)p; }
void orc_poly_free(void* p) { delete (RnsPoly*)p; }

int orc_fft_tables(void* c, double* twist_re, double* twist_im, double* stage_re, double* stage_im) {
  return guard([&] {
    const FftTables& f = ((CkksContext*)c)->encoder.fft;
    std::memcpy(twist_re, f.twist_re.data(), f.n * 8);
    std::memcpy(twist_im, f.twist_im.data(), f.n * 8);
    size_t off = 0;
    for (size_t s = 0; s < f.twiddle_re.size(); ++s) {
      std::memcpy(stage_re + off, f.twiddle_re[s].data(), f.twiddle_re[s].size() * 8);
      std::memcpy(stage_im + off, f.twiddle_im[s].data(), f.twiddle_im[s].size() * 8);
      off += f.twiddle_re[s].size();
    }
  });
}

int orc_encode(void* c, const double* z, size_t len, uint64_t* out) {
  return guard([&] {
    CkksContext* ctx = (CkksContext*)c;
    copy_poly_out(ctx->encoder.encode(z, len, ctx->params), out);
  });
}
int orc_decode(void* c, const uint64_t* poly, size_t limbs, double scale, double* out) {
  return guard([&] {
    CkksContext* ctx = (CkksContext*)c;
    auto v = ctx->encoder.decode(poly_in(poly, ctx->params.poly_degree, limbs), ctx->params, scale);
    std::memcpy(out, v.data(), v.size() * 8);
  });
}
int orc_decode_coefficients(void* c, const double* coeffs, double* out) {
  return guard([&] {
    CkksContext* ctx = (CkksContext*)c;
    std::vector<double> in(coeffs, coeffs + ctx->params.poly_degree);
    auto v = ctx->encoder.decode_coefficients(in);
    std::memcpy(out, v.data(), v.size() * 8);
  });
}

int orc_keygen(void* c, uint64_t seed, void** out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    *out = new SecretKey(((CkksContext*)c)->keygen(r));
  });
}
int orc_sk_data(void* sk, uint64_t* out) {
  return guard([&] { copy_poly_out(((SecretKey*)sk)->s_ntt, out); });
}
int orc_keygen_public(void* c, void* sk, uint64_t seed, void** out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    *out = new PublicKey(((CkksContext*)c)->keygen_public(*(SecretKey*)sk, r));
  });
}
int orc_pk_data(void* pk, uint64_t* b, uint64_t* a) {
  return guard([&] {
    copy_poly_out(((PublicKey*)pk)->b, b);
    copy_poly_out(((PublicKey*)pk)->a, a);
  });
}

int orc_encrypt(void* c, const double* z, size_t len, void* sk, uint64_t seed, void** out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    *out = new Ciphertext(((CkksContext*)c)->encrypt(z, len, *(SecretKey*)sk, r));
  });
}
// tensafe-he-python/src/lib.rs:230-258 (batch_encrypt): ONE TenSafeRng for the
// whole batch; input i (z + i*stride, lens[i] values) is zero-padded or
// truncated to the slot count (:251-253) and encrypted with ctx.encrypt in
// order, so each encryption continues the stream where the previous stopped.
int orc_batch_encrypt(void* c, const double* z, const size_t* lens, size_t stride, size_t count, void* sk,
                      uint64_t seed, void** outs) {
  return guard([&] {
    CkksContext* ctx = (CkksContext*)c;
    const size_t slots = ctx->params.poly_degree / 2;
    TenSafeRng r = TenSafeRng::from_seed(seed);
    std::vector<Ciphertext*> made;
    try {
      for (size_t i = 0; i < count; ++i) {
        std::vector<double> padded(slots, 0.0);
        const size_t n = std::min(lens[i], slots);
        std::copy(z + i * stride, z + i * stride + n, padded.begin());
        made.push_back(new Ciphertext(ctx->encrypt(padded.data(), slots, *(SecretKey*)sk, r)));
      }
    } catch (...) {
      for (Ciphertext* x : made) delete x;
      throw;
    }
    for (size_t i = 0; i < count; ++i) outs[i] = made[i];
  });
}

int orc_encrypt_pk(void* c, const double* z, size_t len, void* pk, uint64_t seed, void** out) {
  return guard([&] {
    TenSafeRng r = TenSafeRng::from_seed(seed);
    *out = new Ciphertext(((CkksContext*)c)->encrypt_pk(z, len, *(PublicKey*)pk, r));
  });
}
int orc_encrypt_pk_with(void* c, const double* z, size_t len, void* pk, const uint8_t* u,
                        const int64_t* e0, const int64_t* e1, void** out) {
  return guard([&] {
    CkksContext* ctx = (CkksContext*)c;
    size_t n = ctx->params.poly_degree;
    EncryptPkRandomness x;
    x.u.assign(u, u + n);
    x.e0.assign(e0, e0 + n);
    x.e1.assign(e1, e1 + n);
    *out = new Ciphertext(ctx->encrypt_pk_with(z, len, *(PublicKey*)pk, x));
  });
}

int orc_ct_info(void* ct, size_t* limbs, double* scale) {
  return guard([&] {
    *limbs = ((Ciphertext*)ct)->c0.limbs.size();
    *scale = ((Ciphertext*)ct)->scale;
  });
}
int orc_ct_data(void* ct, uint64_t* c0, uint64_t* c1) {
  return guard([&] {
    copy_poly_out(((Ciphertext*)ct)->c0, c0);
    copy_poly_out(((Ciphertext*)ct)->c1, c1);
  });
}
int orc_ct_from_data(void* c, const uint64_t* c0, const uint64_t* c1, size_t limbs, double scale,
                     void** out) {
  return guard([&] {
    size_t n = ((CkksContext*)c)->params.poly_degree;
    *out = new Ciphertext{poly_in(c0, n, limbs), poly_in(c1, n, limbs), scale};
  });
}
int orc_decrypt(void* c, void* ct, void* sk, double* out) {
  return guard([&] {
    auto v = ((CkksContext*)c)->decrypt(*(Ciphertext*)ct, *(SecretKey*)sk);
    std::memcpy(out, v.data(), v.size() * 8);
  });
}
int orc_ct_pt_mul(void* c, void* ct, const double* pt, size_t len, void** out) {
  return guard([&] { *out = new Ciphertext(((CkksContext*)c)->ct_pt_mul(*(Ciphertext*)ct, pt, len)); });
}
int orc_encode_to_ntt(void* c, const double* z, size_t len, void** out) {
  return guard([&] { *out = new RnsPoly(((CkksContext*)c)->encode_to_ntt(z, len)); });
}
int orc_poly_data(void* p, uint64_t* out) {
  return guard([&] { copy_poly_out(*(RnsPoly*)p, out); });
}
int orc_ct_pt_mul_ntt(void* c, void* ct, void* pt, void** out) {
  return guard([&] {
    *out = new Ciphertext(((CkksContext*)c)->ct_pt_mul_ntt(*(Ciphertext*)ct, *(RnsPoly*)pt));
  });
}
int orc_ct_add(void* c, void* a, void* b, void** out) {
  return guard([&] { *out = new Ciphertext(((CkksContext*)c)->ct_add(*(Ciphertext*)a, *(Ciphertext*)b)); });
}
int orc_ct_sub(void* c, void* a, void* b, void** out) {
  return guard([&] { *out = new Ciphertext(((CkksContext*)c)->ct_sub(*(Ciphertext*)a, *(Ciphertext*)b)); });
}
int orc_rescale(void* c, void* ct, void** out) {
  return guard([&] { *out = new Ciphertext(((CkksContext*)c)->rescale(*(Ciphertext*)ct)); });
}

// ---- serialization --------------------------------------------------------
int orc_ct_to_bytes(void* ct, uint8_t* buf, size_t cap, size_t* len) {
  return guard([&] {
    auto v = ct_to_bytes(*(Ciphertext*)ct);
    *len = v.size();
    if (buf) {
      if (cap < v.size()) throw std::invalid_argument("buffer too small");
      std::memcpy(buf, v.data(), v.size());
    }
  });
}
int orc_ct_from_bytes(const uint8_t* b, size_t len, size_t n, size_t limbs, void** out) {
  return guard([&] { *out = new Ciphertext(ct_from_bytes(b, len, n, limbs)); });
}
int orc_pk_to_bytes(void* pk, uint8_t* buf, size_t cap, size_t* len) {
  return guard([&] {
    auto v = pk_to_bytes(*(PublicKey*)pk);
    *len = v.size();
    if (buf) {
      if (cap < v.size()) throw std::invalid_argument("buffer too small");
      std::memcpy(buf, v.data(), v.size());
    }
  });
}
int orc_pk_from_bytes(const uint8_t* b, size_t len, size_t n, size_t limbs, void** out) {
  return guard([&] { *out = new PublicKey(pk_from_bytes(b, len, n, limbs)); });
}

}  // extern "C"
