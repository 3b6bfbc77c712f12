// Oracle: CKKS context, key generation, encryption, ct ops, rescale, decrypt
// and serialization. Restates tensafe-he-core/src/ciphertext.rs and
// serialize.rs. Test infrastructure only (see oracle.h).
#include <cmath>
#include <cstring>
#include <stdexcept>

#include "oracle.h"

namespace oracle {

// ciphertext.rs:61-74
CkksContext CkksContext::make(const CkksParams& p) {
  CkksContext c;
  c.params = p;
  for (const Modulus& m : p.moduli) c.ntt_tables.push_back(NttTables::make(p.poly_degree, m.value));
  c.encoder = CkksEncoder::make(p);
  return c;
}

static inline uint64_t ternary_to_residue(uint64_t r, uint64_t q) {
  // ciphertext.rs:91-96 / :261-266 — 0 -> q-1, 1 -> 0, 2 -> 1
  return r == 0 ? q - 1 : (r == 1 ? 0 : 1);
}

static inline uint64_t signed_to_residue(int64_t e, uint64_t q) {
  // ciphertext.rs:132-136 / :279-285
  return e >= 0 ? (uint64_t)e % q : q - ((uint64_t)(-e) % q);
}

// ciphertext.rs:77-103
SecretKey CkksContext::keygen(TenSafeRng& rng) const {
  size_t n = params.poly_degree, L = params.num_limbs;
  RnsPoly s = RnsPoly::zero(n, L);
  std::vector<uint64_t> t = sample_ternary(rng, n, 3);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    for (size_t i = 0; i < n; ++i) s.limbs[l][i] = ternary_to_residue(t[i], q);
    negacyclic_ntt_forward(s.limbs[l].data(), ntt_tables[l]);
  }
  return SecretKey{std::move(s)};
}

// ciphertext.rs:114-154 — a per limb, then e, then b = -a*s + e.
PublicKey CkksContext::keygen_public(const SecretKey& sk, TenSafeRng& rng) const {
  size_t n = params.poly_degree, L = params.num_limbs;
  RnsPoly a = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    a.limbs[l] = sample_uniform(rng, n, params.moduli[l].value);
    negacyclic_ntt_forward(a.limbs[l].data(), ntt_tables[l]);
  }
  std::vector<int64_t> e_signed = sample_gaussian_signed(rng, n, ERROR_STD_DEV);
  RnsPoly e = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    for (size_t i = 0; i < n; ++i) e.limbs[l][i] = signed_to_residue(e_signed[i], q);
    negacyclic_ntt_forward(e.limbs[l].data(), ntt_tables[l]);
  }
  RnsPoly b = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    const Modulus& m = params.moduli[l];
    for (size_t i = 0; i < n; ++i) {
      uint64_t as = mod_mul_barrett(a.limbs[l][i], sk.s_ntt.limbs[l][i], m);
      uint64_t neg_as = as == 0 ? 0 : q - as;
      b.limbs[l][i] = mod_add(neg_as, e.limbs[l][i], q);
    }
  }
  return PublicKey{std::move(b), std::move(a)};
}

// ciphertext.rs:167-229 — encode+NTT, a per limb (+NTT), e (+NTT), c0 = -a*s + (m + e), c1 = a.
Ciphertext CkksContext::encrypt(const double* z, size_t len, const SecretKey& sk,
                                TenSafeRng& rng) const {
  size_t n = params.poly_degree, L = params.num_limbs;
  RnsPoly m = encoder.encode(z, len, params);
  for (size_t l = 0; l < L; ++l) negacyclic_ntt_forward(m.limbs[l].data(), ntt_tables[l]);
  RnsPoly a = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    a.limbs[l] = sample_uniform(rng, n, params.moduli[l].value);
    negacyclic_ntt_forward(a.limbs[l].data(), ntt_tables[l]);
  }
  std::vector<int64_t> e_signed = sample_gaussian_signed(rng, n, ERROR_STD_DEV);
  RnsPoly e = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    for (size_t i = 0; i < n; ++i) e.limbs[l][i] = signed_to_residue(e_signed[i], q);
    negacyclic_ntt_forward(e.limbs[l].data(), ntt_tables[l]);
  }
  RnsPoly c0 = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    const Modulus& mod = params.moduli[l];
    for (size_t i = 0; i < n; ++i) {
      uint64_t neg_as = mod_sub(0, mod_mul_barrett(a.limbs[l][i], sk.s_ntt.limbs[l][i], mod), q);
      c0.limbs[l][i] = mod_add(neg_as, mod_add(m.limbs[l][i], e.limbs[l][i], q), q);
    }
  }
  return Ciphertext{std::move(c0), std::move(a), SCALE};
}

// ciphertext.rs:240-319
Ciphertext CkksContext::encrypt_pk(const double* z, size_t len, const PublicKey& pk,
                                   TenSafeRng& rng) const {
  // Encoding consumes no randomness, so sampling first and encoding second
  // leaves the RNG draw order of ciphertext.rs:250-273 unchanged.
  if (len > params.num_slots) throw std::invalid_argument("Input length exceeds slot count");
  EncryptPkRandomness r = sample_encrypt_pk_randomness(rng, params.poly_degree);
  return encrypt_pk_with(z, len, pk, r);
}

Ciphertext CkksContext::encrypt_pk_with(const double* z, size_t len, const PublicKey& pk,
                                        const EncryptPkRandomness& r) const {
  size_t n = params.poly_degree, L = params.num_limbs;
  if (r.u.size() != n || r.e0.size() != n || r.e1.size() != n)
    throw std::invalid_argument("randomness length mismatch");
  RnsPoly m = encoder.encode(z, len, params);
  for (size_t l = 0; l < L; ++l) negacyclic_ntt_forward(m.limbs[l].data(), ntt_tables[l]);
  RnsPoly u = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    for (size_t i = 0; i < n; ++i) u.limbs[l][i] = ternary_to_residue(r.u[i], q);
    negacyclic_ntt_forward(u.limbs[l].data(), ntt_tables[l]);
  }
  RnsPoly e0 = RnsPoly::zero(n, L), e1 = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    for (size_t i = 0; i < n; ++i) e0.limbs[l][i] = signed_to_residue(r.e0[i], q);
    negacyclic_ntt_forward(e0.limbs[l].data(), ntt_tables[l]);
    for (size_t i = 0; i < n; ++i) e1.limbs[l][i] = signed_to_residue(r.e1[i], q);
    negacyclic_ntt_forward(e1.limbs[l].data(), ntt_tables[l]);
  }
  RnsPoly c0 = RnsPoly::zero(n, L), c1 = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    const Modulus& mod = params.moduli[l];
    for (size_t i = 0; i < n; ++i) {
      uint64_t bu = mod_mul_barrett(pk.b.limbs[l][i], u.limbs[l][i], mod);
      c0.limbs[l][i] = mod_add(bu, mod_add(e0.limbs[l][i], m.limbs[l][i], q), q);
      uint64_t au = mod_mul_barrett(pk.a.limbs[l][i], u.limbs[l][i], mod);
      c1.limbs[l][i] = mod_add(au, e1.limbs[l][i], q);
    }
  }
  return Ciphertext{std::move(c0), std::move(c1), SCALE};
}

// ciphertext.rs:327-400 — m = c0 + c1*s on ct's limbs, iNTT all of them, then
// either the 2-limb CRT branch (scale > 1.5*2^40 and >= 2 limbs) or limb-0 decode.
std::vector<double> CkksContext::decrypt(const Ciphertext& ct, const SecretKey& sk) const {
  size_t n = params.poly_degree;
  size_t L = ct.c0.limbs.size();
  RnsPoly m = RnsPoly::zero(n, L);
  for (size_t l = 0; l < L; ++l) {
    uint64_t q = params.moduli[l].value;
    const Modulus& mod = params.moduli[l];
    for (size_t i = 0; i < n; ++i) {
      uint64_t c1s = mod_mul_barrett(ct.c1.limbs[l][i], sk.s_ntt.limbs[l][i], mod);
      m.limbs[l][i] = mod_add(ct.c0.limbs[l][i], c1s, q);
    }
  }
  for (size_t l = 0; l < L; ++l) negacyclic_ntt_inverse(m.limbs[l].data(), ntt_tables[l]);

  if (ct.scale > SCALE * 1.5 && L >= 2) {
    uint64_t q0 = params.moduli[0].value, q1 = params.moduli[1].value;
    uint64_t q0_inv_mod_q1 = mod_inv(q0 % q1, q1);
    u128 q_product = (u128)q0 * q1;
    u128 half_product = q_product / 2;
    std::vector<double> coeffs(n, 0.0);
    for (size_t i = 0; i < n; ++i) {
      uint64_t m0 = m.limbs[0][i], m1 = m.limbs[1][i];
      uint64_t m0_mod_q1 = (uint64_t)((u128)m0 % q1);
      uint64_t diff = m1 >= m0_mod_q1 ? m1 - m0_mod_q1 : q1 - m0_mod_q1 + m1;
      uint64_t k = (uint64_t)(((u128)diff * q0_inv_mod_q1) % q1);
      u128 mu = (u128)m0 + (u128)k * q0;
      if (mu >= q_product) mu = mu % q_product;
      double sv = mu > half_product ? -((double)(q_product - mu)) : (double)mu;
      coeffs[i] = sv / ct.scale;
    }
    return encoder.decode_coefficients(coeffs);
  }
  return encoder.decode(m, params, ct.scale);
}

// ciphertext.rs:408-418
Ciphertext CkksContext::ct_pt_mul(const Ciphertext& ct, const double* pt, size_t len) const {
  RnsPoly p = encoder.encode(pt, len, params);
  for (size_t l = 0; l < params.num_limbs; ++l)
    negacyclic_ntt_forward(p.limbs[l].data(), ntt_tables[l]);
  return ct_pt_mul_ntt(ct, p);
}

// ciphertext.rs:422-429 — Hadamard on ct's limbs, scale <- scale^2.
Ciphertext CkksContext::ct_pt_mul_ntt(const Ciphertext& ct, const RnsPoly& pt_ntt) const {
  return Ciphertext{ct.c0.hadamard_mul(pt_ntt, params.moduli),
                    ct.c1.hadamard_mul(pt_ntt, params.moduli), ct.scale * ct.scale};
}

// ciphertext.rs:435-448
Ciphertext CkksContext::ct_add(const Ciphertext& a, const Ciphertext& b) const {
  if (!(std::fabs(a.scale - b.scale) < 1.0)) throw std::invalid_argument("Scale mismatch in ct_add");
  return Ciphertext{a.c0.add(b.c0, params.moduli), a.c1.add(b.c1, params.moduli), a.scale};
}

// ciphertext.rs:453-466
Ciphertext CkksContext::ct_sub(const Ciphertext& a, const Ciphertext& b) const {
  if (!(std::fabs(a.scale - b.scale) < 1.0)) throw std::invalid_argument("Scale mismatch in ct_sub");
  return Ciphertext{a.c0.sub(b.c0, params.moduli), a.c1.sub(b.c1, params.moduli), a.scale};
}

// ciphertext.rs:476-535 — floor rescale by the last prime, coefficient domain.
Ciphertext CkksContext::rescale(const Ciphertext& ct) const {
  size_t n = params.poly_degree;
  size_t L = ct.c0.limbs.size();
  if (L < 2) throw std::invalid_argument("Cannot rescale: only 1 limb left");
  size_t last = L - 1;
  uint64_t last_q = params.moduli[last].value;
  std::vector<uint64_t> c0_last = ct.c0.limbs[last], c1_last = ct.c1.limbs[last];
  negacyclic_ntt_inverse(c0_last.data(), ntt_tables[last]);
  negacyclic_ntt_inverse(c1_last.data(), ntt_tables[last]);
  RnsPoly c0n = RnsPoly::zero(n, L - 1), c1n = RnsPoly::zero(n, L - 1);
  for (size_t l = 0; l < L - 1; ++l) {
    uint64_t ql = params.moduli[l].value;
    uint64_t inv = mod_inv(last_q % ql, ql);
    std::vector<uint64_t> c0l = ct.c0.limbs[l], c1l = ct.c1.limbs[l];
    negacyclic_ntt_inverse(c0l.data(), ntt_tables[l]);
    negacyclic_ntt_inverse(c1l.data(), ntt_tables[l]);
    for (size_t i = 0; i < n; ++i) {
      uint64_t a = c0_last[i] % ql;
      uint64_t d0 = c0l[i] >= a ? c0l[i] - a : ql - a + c0l[i];
      c0n.limbs[l][i] = mod_mul_barrett(d0, inv, params.moduli[l]);
      uint64_t b = c1_last[i] % ql;
      uint64_t d1 = c1l[i] >= b ? c1l[i] - b : ql - b + c1l[i];
      c1n.limbs[l][i] = mod_mul_barrett(d1, inv, params.moduli[l]);
    }
    negacyclic_ntt_forward(c0n.limbs[l].data(), ntt_tables[l]);
    negacyclic_ntt_forward(c1n.limbs[l].data(), ntt_tables[l]);
  }
  return Ciphertext{std::move(c0n), std::move(c1n), ct.scale / (double)last_q};
}

// ciphertext.rs:539-545
RnsPoly CkksContext::encode_to_ntt(const double* z, size_t len) const {
  RnsPoly p = encoder.encode(z, len, params);
  for (size_t l = 0; l < params.num_limbs; ++l)
    negacyclic_ntt_forward(p.limbs[l].data(), ntt_tables[l]);
  return p;
}

// serialize.rs:14-24
std::vector<uint8_t> rns_poly_to_bytes(const RnsPoly& p) {
  std::vector<uint8_t> out(p.limbs.size() * p.n * 8);
  size_t off = 0;
  for (const auto& limb : p.limbs)
    for (size_t i = 0; i < p.n; ++i, off += 8) std::memcpy(&out[off], &limb[i], 8);
  return out;
}

// serialize.rs:27-44
RnsPoly rns_poly_from_bytes(const uint8_t* b, size_t len, size_t n, size_t num_limbs) {
  if (len != num_limbs * n * 8) throw std::invalid_argument("RnsPoly byte length mismatch");
  RnsPoly p = RnsPoly::zero(n, num_limbs);
  size_t off = 0;
  for (size_t l = 0; l < num_limbs; ++l)
    for (size_t i = 0; i < n; ++i, off += 8) std::memcpy(&p.limbs[l][i], b + off, 8);
  return p;
}

// serialize.rs:48-52
std::vector<uint8_t> pk_to_bytes(const PublicKey& pk) {
  std::vector<uint8_t> out = rns_poly_to_bytes(pk.b);
  std::vector<uint8_t> a = rns_poly_to_bytes(pk.a);
  out.insert(out.end(), a.begin(), a.end());
  return out;
}

// serialize.rs:55-67
PublicKey pk_from_bytes(const uint8_t* b, size_t len, size_t n, size_t num_limbs) {
  size_t ps = num_limbs * n * 8;
  if (len != 2 * ps) throw std::invalid_argument("PublicKey byte length mismatch");
  return PublicKey{rns_poly_from_bytes(b, ps, n, num_limbs),
                   rns_poly_from_bytes(b + ps, ps, n, num_limbs)};
}

// serialize.rs:71-77 — [scale f64 LE | c0 | c1]
std::vector<uint8_t> ct_to_bytes(const Ciphertext& ct) {
  std::vector<uint8_t> out(8);
  std::memcpy(out.data(), &ct.scale, 8);
  std::vector<uint8_t> c0 = rns_poly_to_bytes(ct.c0), c1 = rns_poly_to_bytes(ct.c1);
  out.insert(out.end(), c0.begin(), c0.end());
  out.insert(out.end(), c1.begin(), c1.end());
  return out;
}

// serialize.rs:80-93
Ciphertext ct_from_bytes(const uint8_t* b, size_t len, size_t n, size_t num_limbs) {
  size_t ps = num_limbs * n * 8;
  if (len != 8 + 2 * ps) throw std::invalid_argument("Ciphertext byte length mismatch");
  Ciphertext ct;
  std::memcpy(&ct.scale, b, 8);
  ct.c0 = rns_poly_from_bytes(b + 8, ps, n, num_limbs);
  ct.c1 = rns_poly_from_bytes(b + 8 + ps, ps, n, num_limbs);
  return ct;
}

}  // namespace oracle
