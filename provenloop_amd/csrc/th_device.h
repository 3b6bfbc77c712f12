// Device-side definitions shared by the HIP kernels of the CKKS engine.
//
// Residues live in HBM as canonical u64 values in [0, q), limb-major:
// a limb-polynomial is N consecutive u64, a ciphertext is [c0 | c1] with each
// component L limb-polynomials back to back (the reference's RnsPoly layout,
// tensafe-he-core/src/rns.rs:199-206, made contiguous).
//
// Two exact modular-multiply paths are used, chosen per prime:
//  * "int":  64-bit Shoup multiply with a precomputed floor(w*2^64/q) and
//            Harvey-style lazy reduction; any q < 2^61.
//  * "fp64": for q < 2^41 the product w*x is split exactly into hi + lo with
//            one FMA and the quotient comes from x*(w/q) rounded to nearest;
//            the remainder is exact (all intermediate integers < 2^53). Six
//            full-rate FP64 instructions per multiply.
// Both produce the unique canonical residue, so results are bit-identical to
// the reference's u128 Barrett multiply (tensafe-he-core/src/rns.rs:45-95).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace th {

// Largest prime that takes the fp64 multiply path.
constexpr uint64_t FP64_PRIME_LIMIT = 1ULL << 41;

struct ShoupTw {
  uint64_t w, ws;  // twiddle and floor(w * 2^64 / q)
};
struct Fp64Tw {
  double w, wq;  // twiddle and w / q (correctly rounded)
};

// Per-limb constants; one array per context in device memory.
struct LimbConst {
  uint64_t q, two_q;
  uint64_t n_inv, n_inv_s;    // N^{-1} and its Shoup companion
  uint64_t last_w, last_ws;   // inv_tw[1] * N^{-1}: last inverse stage with the scaling folded in
  double qd, qinv;            // q and 1/q as doubles (fp64 path)
  double n_inv_d, n_inv_dq;
  double last_wd, last_wdq;
  const void* fwd;            // N twiddle pairs (ShoupTw or Fp64Tw), fwd[brv(i)] = psi^i
  const void* inv;            // N twiddle pairs, inv[brv(i)] = psi^-i
  const void* fwd_row;        // fwd and inv entries of the split row passes' lane-bit stages
  const void* inv_row;        //   in the order their lanes read them (row_table_index)
  uint32_t fp64;              // 1 if this limb uses the fp64 path
  uint32_t pad_;
};

// ---------------------------------------------------------------- int path
__device__ __forceinline__ uint64_t shoup_lazy(uint64_t x, uint64_t w, uint64_t ws, uint64_t q) {
  // x * w mod q in [0, 2q) for any x < 2^64 (w < q).
  uint64_t qh = __umul64hi(x, ws);
  return x * w - qh * q;
}

__device__ __forceinline__ uint64_t csub(uint64_t x, uint64_t m) { return x >= m ? x - m : x; }

// The same with nm = 2^64 - m supplied: x + nm is one 64-bit add (no borrow
// chain through VCC), and the compare selects between x and the sum.
__device__ __forceinline__ uint64_t csub_n(uint64_t x, uint64_t m, uint64_t nm) {
  const uint64_t t = x + nm;
  return x >= m ? t : x;
}

// v unchanged, but hidden from the optimiser (an empty asm that claims to
// modify it), so that 2^64 - m stays an addend instead of being folded back
// into a subtraction of m.
__device__ __forceinline__ uint64_t opaque_u64(uint64_t v) {
  asm("" : "+v"(v));
  return v;
}

// Pointers known to address global memory (address space 1). Pointers read
// from job descriptors or constant tables are generic to the compiler, and
// generic (flat) loads and stores also count against the LDS wait counter,
// which serialises them with every LDS exchange; accesses through these
// pointers are global_* instructions instead.
template <class T>
using GPtr = const __attribute__((address_space(1))) T*;
template <class T>
using GMut = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ GPtr<T> gld(const T* p) {
  return (GPtr<T>)p;
}
template <class T>
__device__ __forceinline__ GMut<T> gst(T* p) {
  return (GMut<T>)p;
}
// Element i of a global array of 16-byte records (twiddle pairs), loaded as one
// 16-byte vector.
template <class T>
__device__ __forceinline__ T ld16(GPtr<T> p, uint32_t i) {
  static_assert(sizeof(T) == 16, "16-byte records only");
  using V = uint64_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(T, ((GPtr<V>)p)[i]);
}
// The same through the constant address space, for an index that is the same
// on every lane of the wavefront: a scalar load, which leaves the CU's
// vector-memory path to the per-lane accesses (only for tables that no kernel
// writes while it runs).
template <class T>
__device__ __forceinline__ T ld16_uniform(GPtr<T> p, uint32_t i) {
  static_assert(sizeof(T) == 16, "16-byte records only");
  using V = uint64_t __attribute__((ext_vector_type(2)));
  using CPtr = const __attribute__((address_space(4))) V*;
  return __builtin_bit_cast(T, ((CPtr)(const void*)p)[__builtin_amdgcn_readfirstlane(i)]);
}

// floor(x * s / 2^64) - e with e in {0, 1, 2}: x1*s1 + hi(x1*s0) + hi(x0*s1)
// for 32-bit halves; the low halves of the two cross products and hi(x0*s0)
// are dropped, each below 2^32, so at most 2 is lost after the shift. The sum
// stays below 2^64. The last term goes in as a 32-bit add with carry (two
// 32-bit instructions): left to the compiler it becomes a zero-extending move
// and a 64-bit add.
__device__ __forceinline__ uint64_t mulhi_approx(uint64_t x, uint64_t s) {
  const uint32_t x0 = (uint32_t)x, x1 = (uint32_t)(x >> 32), s0 = (uint32_t)s, s1 = (uint32_t)(s >> 32);
  const uint64_t r = (uint64_t)x1 * s1 + __umulhi(x1, s0);
  uint32_t rl = (uint32_t)r, rh = (uint32_t)(r >> 32);
  asm("v_add_co_u32 %0, vcc, %0, %2\n\tv_addc_co_u32 %1, vcc, %1, 0, vcc" : "+v"(rl), "+v"(rh) : "v"(__umulhi(x0, s1))
      : "vcc");
  return ((uint64_t)rh << 32) | rl;
}

// v unchanged, hidden from the optimiser (see opaque_u64).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// x * w mod q in [0, 4q) for any 64-bit x (w < q, ws = floor(w * 2^64 / q)):
// the exact Shoup remainder is below 2q and the quotient estimate is at most
// 2 short.
// The remainder is formed as x*w + qhat*(2^64 - q) mod 2^64 from 32-bit
// partial products, so that the second low product accumulates onto the first
// (one multiply-add) instead of being subtracted as a separate 64-bit word.
__device__ __forceinline__ uint64_t shoup_approx(uint64_t x, uint64_t w, uint64_t ws, uint64_t q) {
  const uint64_t qh = mulhi_approx(x, ws);
  const uint64_t nq = 0 - q;
  const uint32_t x0 = (uint32_t)x, x1 = (uint32_t)(x >> 32), w0 = (uint32_t)w, w1 = (uint32_t)(w >> 32);
  const uint32_t h0 = (uint32_t)qh, h1 = (uint32_t)(qh >> 32), n0 = (uint32_t)nq, n1 = (uint32_t)(nq >> 32);
  const uint64_t lo = (uint64_t)x0 * w0 + (uint64_t)h0 * n0;
  // the high word as one 32-bit sum (the cross products pair up as multiply-
  // adds); kept opaque so that the compiler does not turn the word assembly
  // back into a 64-bit add of the shifted cross terms
  const uint32_t hi = opaque_u32((uint32_t)(lo >> 32) + (x0 * w1 + x1 * w0) + (h0 * n1 + h1 * n0));
  return ((uint64_t)hi << 32) | (uint32_t)lo;
}

// Exact a*b mod q for a, b < q < 2^63 (operands without a precomputed
// companion): 128-bit product, quotient from the high word scaled by a
// per-prime reciprocal, then at most two corrections.
struct BarrettConst {
  uint64_t q;
  uint64_t r_hi, r_lo;  // floor((2^128 - 1) / q) as two words
  uint64_t mq;          // -q^{-1} mod 2^64 (Montgomery products)
  uint64_t r64;         // 2^64 mod q (into Montgomery form)
  uint64_t r64_s;       // floor(r64 2^64 / q): its Shoup companion
};

__device__ __forceinline__ uint64_t mulmod_barrett(uint64_t a, uint64_t b, const BarrettConst& m) {
  uint64_t lo = a * b;
  uint64_t hi = __umul64hi(a, b);
  // quotient estimate = floor((hi*2^64 + lo) * (r_hi*2^64 + r_lo) / 2^128), lo*r_lo term dropped
  uint64_t t1_lo = lo * m.r_hi, t1_hi = __umul64hi(lo, m.r_hi);
  uint64_t t2_lo = hi * m.r_lo, t2_hi = __umul64hi(hi, m.r_lo);
  uint64_t mid = t1_lo + t2_lo;
  uint64_t carry = mid < t1_lo ? 1 : 0;
  uint64_t quot = hi * m.r_hi + t1_hi + t2_hi + carry;
  uint64_t r = lo - quot * m.q;
  r = csub(r, m.q);
  r = csub(r, m.q);
  return r;
}

__device__ __forceinline__ uint64_t addmod(uint64_t a, uint64_t b, uint64_t q) { return csub(a + b, q); }

// Montgomery product a * b * 2^-64 mod q in [0, 2q) for any 64-bit a and
// b < q: with T = a b and m = T mod 2^64 * (-q^{-1}) mod 2^64, T + m q is a
// multiple of 2^64, its low words cancel (a carry exactly when T mod 2^64 is
// nonzero), and (T + m q) / 2^64 < 2q. With b = w 2^64 mod q (w in Montgomery
// form) this is a * w mod q, in about half the multiplies of a Barrett product.
__device__ __forceinline__ uint64_t mont_mul(uint64_t a, uint64_t b, const BarrettConst& m) {
  const uint64_t t_lo = a * b, t_hi = __umul64hi(a, b);
  const uint64_t k = t_lo * m.mq;
  return t_hi + __umul64hi(k, m.q) + (t_lo != 0 ? 1 : 0);
}

// e >= 0 ? e mod q : q - (|e| mod q) (ciphertext.rs:132-136, :275-287; encoding.rs:198-202)
__device__ __forceinline__ uint64_t signed_residue_dev(int64_t e, const BarrettConst& m) {
  const uint64_t a = e >= 0 ? (uint64_t)e : (uint64_t)0 - (uint64_t)e;
  const uint64_t r = a < m.q ? a : mulmod_barrett(a, 1, m);
  return e >= 0 ? r : m.q - r;
}

__device__ __forceinline__ uint64_t submod(uint64_t a, uint64_t b, uint64_t q) {
  return a >= b ? a - b : a + q - b;
}

// Rescale constants of one output limb l (ciphertext.rs:497-522).
struct RescaleConst {
  uint64_t q, inv, inv_s;  // q_l, (q_last mod q_l)^{-1} and its Shoup companion
  BarrettConst b;          // remainder of a 64-bit value modulo q_l
  double qd, qinv;         // q_l and 1/q_l as doubles (limbs below 2^41)
  double inv_d, inv_dq;    // inv and inv / q_l as doubles (limbs below 2^41)
  double k32, k32q;        // 2^32 mod q_l and that / q_l as doubles (limbs below 2^41)
};

// ---------------------------------------------------------------- fp64 path
// x*w mod q as an exact integer in about (-q/2, q/2); requires |x| < 2^46, w < q < 2^41.
__device__ __forceinline__ double mulmod_f64(double x, double w, double wq, double q) {
  double hi = x * w;
  double lo = __fma_rn(x, w, -hi);
  double quot = __builtin_rint(x * wq);
  double r = __fma_rn(-quot, q, hi);
  return r + lo;
}

// c mod q_l for any c < 2^61 on a limb below 2^41, as an exact double in
// [0, q_l): with c = ch 2^32 + cl (ch < 2^29), c = ch (2^32 mod q_l) + cl
// (mod q_l), the first term an exact FP64 product in (-q_l, q_l) and cl < q_l.
__device__ __forceinline__ double reduce_u64_f64(uint64_t c, const RescaleConst& rc) {
  const double ch = (double)(uint32_t)(c >> 32), cl = (double)(uint32_t)c;
  double r = mulmod_f64(ch, rc.k32, rc.k32q, rc.qd) + cl;  // (-q_l, 2 q_l)
  r = r < 0.0 ? r + rc.qd : r;
  return r >= rc.qd ? r - rc.qd : r;
}

// a*b mod q in [0, q) for integers 0 <= a, b < q < 2^41 held exactly in
// doubles, without a precomputed companion: hi + lo = a*b exactly (one FMA),
// and quot = rint(hi / q) through qinv = 1/q is within 0.5 + 2^-10 of a*b/q
// (a*b/q < 2^41, relative error below 2^-51), so r = a*b - quot*q, formed
// exactly, lies in (-q, q).
__device__ __forceinline__ double mulmod_f64_any(double a, double b, double q, double qinv) {
  const double hi = a * b;
  const double lo = __fma_rn(a, b, -hi);
  const double quot = __builtin_rint(hi * qinv);
  const double r = __fma_rn(-quot, q, hi) + lo;
  return r < 0.0 ? r + q : r;
}

// x mod q into [0, q) for an exact integer |x| < 2^50.
__device__ __forceinline__ double reduce_f64(double x, double q, double qinv) {
  double quot = __builtin_rint(x * qinv);
  double r = __fma_rn(-quot, q, x);
  return r < 0.0 ? r + q : r;
}

// x mod q into about (-q/2, q/2) (no sign fix) for an exact integer |x| < 2^50.
__device__ __forceinline__ double reduce_f64_signed(double x, double q, double qinv) {
  double quot = __builtin_rint(x * qinv);
  return __fma_rn(-quot, q, x);
}

__device__ __forceinline__ double u64_to_f64(uint64_t x) { return (double)x; }  // exact for x < 2^53
__device__ __forceinline__ uint64_t f64_to_u64(double x) { return (uint64_t)x; }  // x integral, 0 <= x < 2^53

}  // namespace th
