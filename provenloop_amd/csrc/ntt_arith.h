// Butterfly arithmetic and load-side operations shared by the NTT kernels.
//
// Two exact modular-multiply policies (chosen per limb prime):
//  IntArith  - 64-bit Shoup products with an approximate quotient (at most
//              2 short) and lazy ranges [0, 8q) forward, [0, 4q) inverse;
//              q < 2^61 so that 8q fits in 64 bits.
//  Fp64Arith - q < 2^41: exact products from one FMA split and a quotient
//              rounded from x * (w / q); values are exact integers in doubles.
// Both end on the canonical residue, so transforms are bit-identical to the
// reference's u128 Barrett NTT (tensafe-he-core/src/ntt.rs:79-141).
// raw()/unraw() carry a policy's intermediate values through global memory
// between the two kernels of a split transform (u64 lazy residues, or the
// bit pattern of the double).
#pragma once
#include <type_traits>

#include "th_internal.h"

namespace th {

// ------------------------------------------------------------------ arithmetic policies
struct IntArith {
  using V = uint64_t;
  using Tw = ShoupTw;
  uint64_t q, two_q, four_q;
  __device__ IntArith(const LimbConst& c) : q(c.q), two_q(c.two_q), four_q(2 * c.two_q) {}
  // 2^64 - 4q, the forward butterfly's csub_n addend (the same value at every
  // call, so the compiler keeps one copy)
  __device__ __forceinline__ uint64_t n4q() const { return opaque_u64(0 - four_q); }
  __device__ __forceinline__ V load(uint64_t x) const { return x; }
  // forward CT butterfly, inputs/outputs in [0, 8q): X < 4q, T < 4q
  __device__ __forceinline__ void fwd(V& a, V& b, const Tw& t) const {
    const uint64_t X = csub_n(a, four_q, n4q());
    const uint64_t T = shoup_approx(b, t.w, t.ws, q);
    a = X + T;
    b = X + four_q - T;
  }
  // inverse GS butterfly, inputs/outputs in [0, 4q)
  __device__ __forceinline__ void inv(V& a, V& b, const Tw& t) const {
    const uint64_t X = a, Y = b;
    a = csub_n(X + Y, four_q, n4q());
    b = shoup_approx(X + four_q - Y, t.w, t.ws, q);
  }
  // last inverse stage with N^{-1} folded in; canonical outputs
  __device__ __forceinline__ void inv_last(V& a, V& b, const LimbConst& c) const {
    const uint64_t X = a, Y = b;
    a = csub(csub(shoup_approx(X + Y, c.n_inv, c.n_inv_s, q), two_q), q);
    b = csub(csub(shoup_approx(X + four_q - Y, c.last_w, c.last_ws, q), two_q), q);
  }
  __device__ __forceinline__ void inv_pass_end(V&) const {}
  __device__ __forceinline__ uint64_t fwd_store(V x) const { return csub(csub(csub_n(x, four_q, n4q()), two_q), q); }
  __device__ __forceinline__ uint64_t inv_store(V x) const { return x; }
  __device__ __forceinline__ uint64_t raw(V x) const { return x; }
  __device__ __forceinline__ V unraw(uint64_t x) const { return x; }
};

struct Fp64Arith {
  using V = double;
  using Tw = Fp64Tw;
  double q, qinv;
  __device__ Fp64Arith(const LimbConst& c) : q(c.qd), qinv(c.qinv) {}
  __device__ __forceinline__ V load(uint64_t x) const { return u64_to_f64(x); }
  // values grow by at most 0.51 q per stage; no reduction needed inside the transform
  __device__ __forceinline__ void fwd(V& a, V& b, const Tw& t) const {
    double X = a;
    double T = mulmod_f64(b, t.w, t.wq, q);
    a = X + T;
    b = X - T;
  }
  // the sum doubles per stage: reduced at the end of every register pass
  __device__ __forceinline__ void inv(V& a, V& b, const Tw& t) const {
    double X = a, Y = b;
    a = X + Y;
    b = mulmod_f64(X - Y, t.w, t.wq, q);
  }
  __device__ __forceinline__ void inv_last(V& a, V& b, const LimbConst& c) const {
    double X = a, Y = b;
    double r0 = mulmod_f64(X + Y, c.n_inv_d, c.n_inv_dq, q);
    double r1 = mulmod_f64(X - Y, c.last_wd, c.last_wdq, q);
    a = r0 < 0.0 ? r0 + q : r0;
    b = r1 < 0.0 ? r1 + q : r1;
  }
  __device__ __forceinline__ void inv_pass_end(V& x) const { x = reduce_f64_signed(x, q, qinv); }
  __device__ __forceinline__ uint64_t fwd_store(V x) const { return f64_to_u64(reduce_f64(x, q, qinv)); }
  __device__ __forceinline__ uint64_t inv_store(V x) const { return f64_to_u64(x); }
  __device__ __forceinline__ uint64_t raw(V x) const { return __builtin_bit_cast(uint64_t, x); }
  __device__ __forceinline__ V unraw(uint64_t x) const { return __builtin_bit_cast(double, x); }
};

// The operation fused into the coefficient load (NttLoad), fixed at compile
// time so that each kernel carries only its own operation; `i` indexes the
// limb-polynomial, so src, aux and key are read at the same position.
template <uint32_t LD>
struct LoadOp {
  const uint64_t* aux;
  const uint64_t* key;  // secret-key limb-poly (DOT)
  BarrettConst bc;
  RescaleConst rc;
  uint32_t sub;         // ENC variant (uniform over the job)
  double qd, qinv;      // q and 1/q as doubles (ENC)
  // signed_residue_dev with |e| in [q, 2^53) reduced by one exact FP64 step:
  // quot = rint(|e| / q) is within one of the true quotient, and the remainder
  // fma(-quot, q, |e|) is an exact integer in (-q, q)
  __device__ __forceinline__ uint64_t enc_residue(int64_t e) const {
    const uint64_t a = e >= 0 ? (uint64_t)e : (uint64_t)0 - (uint64_t)e;
    uint64_t r = a;
    if (a >= bc.q) {
      if (a < (1ULL << 53)) {
        const double ad = u64_to_f64(a);
        double t = __fma_rn(-__builtin_rint(ad * qinv), qd, ad);
        t = t < 0.0 ? t + qd : t;
        r = f64_to_u64(t >= qd ? t - qd : t);
      } else {
        r = mulmod_barrett(a, 1, bc);
      }
    }
    return e >= 0 ? r : bc.q - r;
  }
  // MULM and ENC in two steps, so that a pass issues all 16 of a thread's
  // operand loads before any arithmetic (the per-element branches of the
  // residue forms would otherwise hold each load until the previous
  // element's result): fetch16 reads the operands of positions idx(0..15),
  // finish forms one position's value. MULM reads (ct, pt); ENC, by the
  // job's variant, the ternary byte (2), m or e1 (1), or m and e0 (0).
  static constexpr uint32_t kind = LD;
  struct Raw {
    uint64_t x, a;
  };
  __device__ __forceinline__ Raw fetch(const uint64_t* src, uint32_t i) const {
    static_assert(LD == NTT_LOAD_MULM || LD == NTT_LOAD_ENC, "two-step loads are for MULM and ENC");
    if constexpr (LD == NTT_LOAD_ENC) {
      if (sub == 2) return Raw{gld(reinterpret_cast<const uint8_t*>(src))[i], 0};
      return Raw{gld(src)[i], sub == 0 ? gld(aux)[i] : 0};
    } else {
      return Raw{gld(src)[i], gld(aux)[i]};
    }
  }
  // the variant test outside the element loop, so the 16 requests issue together
  template <class Idx>
  __device__ __forceinline__ void fetch16(const uint64_t* src, const Idx& idx, Raw (&r)[16]) const {
    static_assert(LD == NTT_LOAD_MULM || LD == NTT_LOAD_ENC, "two-step loads are for MULM and ENC");
    const GPtr<uint64_t> s = gld(src);
    if constexpr (LD == NTT_LOAD_ENC) {
      if (sub == 2) {
        const GPtr<uint8_t> u = gld(reinterpret_cast<const uint8_t*>(src));
#pragma unroll
        for (int k = 0; k < 16; ++k) r[k] = Raw{u[idx(k)], 0};
      } else if (sub == 0) {
        const GPtr<uint64_t> e = gld(aux);
#pragma unroll
        for (int k = 0; k < 16; ++k) r[k] = Raw{s[idx(k)], e[idx(k)]};
      } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) r[k] = Raw{s[idx(k)], 0};
      }
    } else {
      const GPtr<uint64_t> a = gld(aux);
#pragma unroll
      for (int k = 0; k < 16; ++k) r[k] = Raw{s[idx(k)], a[idx(k)]};
    }
  }
  __device__ __forceinline__ uint64_t finish(const Raw& r) const {
    if constexpr (LD == NTT_LOAD_ENC) {
      if (sub == 2) return r.x == 0 ? bc.q - 1 : (r.x == 1 ? 0 : 1);
      const uint64_t v = enc_residue((int64_t)r.x);
      return sub == 0 ? csub(v + enc_residue((int64_t)r.a), bc.q) : v;
    } else {
      return mont_mul(r.x, r.a, bc);
    }
  }
  __device__ __forceinline__ uint64_t operator()(const uint64_t* src, uint32_t i) const {
    if constexpr (LD == NTT_LOAD_ENC || LD == NTT_LOAD_MULM) return finish(fetch(src, i));
    const uint64_t x = gld(src)[i];
    if constexpr (LD == NTT_LOAD_DOTM) return x + mont_mul(gld(aux)[i], gld(key)[i], bc);
    if constexpr (LD == NTT_LOAD_MUL) return mulmod_barrett(x, gld(aux)[i], bc);
    if constexpr (LD == NTT_LOAD_REDUCE) return x < rc.q ? x : mulmod_barrett(x, 1, rc.b);
    if constexpr (LD == NTT_LOAD_DOT) return addmod(x, mulmod_barrett(gld(aux)[i], gld(key)[i], bc), bc.q);
    return x;
  }
};

// The operation fused into a forward transform's final store (NttStore), or,
// for SEGSUM, the inverse transform's segment-sum epilogue's operands.
template <uint32_t ST>
struct StoreOp {
  static constexpr uint32_t kind = ST;
  const uint64_t* aux;
  const uint64_t* aux2;
  BarrettConst bc;
  RescaleConst rc;
  const double* segw;  // SEGSUM
  double* seg;
  double scale;
  uint32_t cols;
  // Operands the store reads at position i (ct x pt factors, or the value the
  // rescale subtracts from); loaded apart from the arithmetic so that a pass
  // can issue these loads early and hide their latency behind its butterflies.
  static constexpr int NAUX = ST == NTT_STORE_MUL_RESCALE ? 2 : ST == NTT_STORE_RESCALE ? 1 : 0;
  // Store of transform output x at position i of dst (MONT: its Montgomery
  // form, and the plain residue to aux when aux is set).
  template <class A>
  __device__ __forceinline__ void store(const A& ar, typename A::V x, GMut<uint64_t> dst, uint32_t i,
                                        uint64_t cp) const {
    if constexpr (ST == NTT_STORE_MONT) {
      const uint64_t y = ar.fwd_store(x);
      dst[i] = csub(shoup_lazy(y, bc.r64, bc.r64_s, bc.q), bc.q);  // y 2^64 mod q
      if (aux) gst(const_cast<uint64_t*>(aux))[i] = y;
    } else {
      dst[i] = apply_prep(ar, x, cp);
    }
  }
  struct Aux {
    uint64_t a, b;
  };
  __device__ __forceinline__ Aux load_aux(uint32_t i) const {
    Aux v{0, 0};
    if constexpr (NAUX >= 1) v.a = gld(aux)[i];
    if constexpr (NAUX >= 2) v.b = gld(aux2)[i];
    return v;
  }
  // The value the rescale subtracts from (ct x pt product, or the single
  // operand), reduced modulo q, from the operands v: a double's bit pattern
  // on limbs below 2^41 (Fp64Arith), else the residue.
  template <class A>
  __device__ __forceinline__ uint64_t prep(const A&, const Aux& v) const {
    if constexpr (NAUX == 0) {
      return 0;
    } else if constexpr (std::is_same_v<A, Fp64Arith>) {
      double c;
      if constexpr (ST == NTT_STORE_MUL_RESCALE)
        c = mulmod_f64_any(u64_to_f64(v.a), u64_to_f64(v.b), rc.qd, rc.qinv);
      else
        c = u64_to_f64(v.a);
      return __builtin_bit_cast(uint64_t, c);
    } else {
      if constexpr (ST == NTT_STORE_MUL_RESCALE)
        return mulmod_barrett(v.a, v.b, bc);
      else
        return v.a;
    }
  }
  // The stored word for transform output x (the arithmetic's representation)
  // with the prepared value c of its position (prep). Limbs below 2^41
  // (Fp64Arith) do the rescale in doubles: exact products without
  // precomputed companions instead of 64-bit Barrett.
  template <class A>
  __device__ __forceinline__ uint64_t apply_prep(const A& ar, typename A::V x, uint64_t cp) const {
    if constexpr (std::is_same_v<A, Fp64Arith> && NAUX > 0) {
      const double y = reduce_f64(x, rc.qd, rc.qinv);  // canonical transform output
      const double c = __builtin_bit_cast(double, cp);
      const double r = mulmod_f64(c - y, rc.inv_d, rc.inv_dq, rc.qd);  // (c - y) * inv, |c - y| < q
      return f64_to_u64(r < 0.0 ? r + rc.qd : r);
    } else {
      const uint64_t y = ar.fwd_store(x);
      if constexpr (NAUX == 0)
        return y;
      else
        return csub(shoup_lazy(submod(cp, y, rc.q), rc.inv, rc.inv_s, rc.q), rc.q);
    }
  }
};

// Load and store operations of job `jb` in launch `a` for limb `limb`.
template <uint32_t LD, uint32_t ST>
__device__ __forceinline__ void job_ops(const NttArgs& a, const NttJob& jb, uint32_t limb, uint32_t n,
                                        LoadOp<LD>& op, StoreOp<ST>& so) {
  op.aux = jb.aux;
  if constexpr (LD == NTT_LOAD_MUL || LD == NTT_LOAD_DOT || LD == NTT_LOAD_ENC || LD == NTT_LOAD_MULM ||
                LD == NTT_LOAD_DOTM)
    op.bc = a.bc[limb];
  if constexpr (LD == NTT_LOAD_ENC) {
    op.sub = jb.sub;
    op.qd = a.lc[limb].qd;
    op.qinv = a.lc[limb].qinv;
  }
  if constexpr (LD == NTT_LOAD_DOT || LD == NTT_LOAD_DOTM) op.key = a.key + (uint64_t)limb * n;
  if constexpr (LD == NTT_LOAD_REDUCE) op.rc = a.rc[limb];
  so.aux = jb.aux;
  so.aux2 = jb.aux2;
  if constexpr (ST == NTT_STORE_RESCALE || ST == NTT_STORE_MUL_RESCALE) so.rc = a.rc[limb];
  if constexpr (ST == NTT_STORE_MUL_RESCALE || ST == NTT_STORE_MONT) so.bc = a.bc[limb];
  if constexpr (ST == NTT_STORE_SEGSUM) {
    so.segw = a.segw;
    so.seg = reinterpret_cast<double*>(jb.dst);
    so.scale = jb.scale;
    so.cols = a.cols;
  }
}

// Calls f.template operator()<LD, ST>() for the (load, store) pair of a launch.
// Only the pairs the engine issues are instantiated: forward (NONE | ENC,
// NONE), (REDUCE, RESCALE), (REDUCE, MUL_RESCALE), (NONE, MONT); inverse
// (NONE | MUL | MULM | DOT | DOTM, NONE), (DOT | DOTM, SEGSUM).
template <bool INV, class F>
__host__ hipError_t with_ops(uint32_t load, uint32_t store, F&& f) {
  if constexpr (!INV) {
    if (load == NTT_LOAD_NONE && store == NTT_STORE_NONE) return f.template operator()<NTT_LOAD_NONE, NTT_STORE_NONE>();
    if (load == NTT_LOAD_ENC && store == NTT_STORE_NONE) return f.template operator()<NTT_LOAD_ENC, NTT_STORE_NONE>();
    if (load == NTT_LOAD_REDUCE && store == NTT_STORE_RESCALE)
      return f.template operator()<NTT_LOAD_REDUCE, NTT_STORE_RESCALE>();
    if (load == NTT_LOAD_REDUCE && store == NTT_STORE_MUL_RESCALE)
      return f.template operator()<NTT_LOAD_REDUCE, NTT_STORE_MUL_RESCALE>();
    if (load == NTT_LOAD_NONE && store == NTT_STORE_MONT) return f.template operator()<NTT_LOAD_NONE, NTT_STORE_MONT>();
    return hipErrorInvalidValue;
  } else {
    if (load == NTT_LOAD_DOT && store == NTT_STORE_SEGSUM)
      return f.template operator()<NTT_LOAD_DOT, NTT_STORE_SEGSUM>();
    if (load == NTT_LOAD_DOTM && store == NTT_STORE_SEGSUM)
      return f.template operator()<NTT_LOAD_DOTM, NTT_STORE_SEGSUM>();
    if (store != NTT_STORE_NONE) return hipErrorInvalidValue;
    if (load == NTT_LOAD_NONE) return f.template operator()<NTT_LOAD_NONE, NTT_STORE_NONE>();
    if (load == NTT_LOAD_MUL) return f.template operator()<NTT_LOAD_MUL, NTT_STORE_NONE>();
    if (load == NTT_LOAD_MULM) return f.template operator()<NTT_LOAD_MULM, NTT_STORE_NONE>();
    if (load == NTT_LOAD_DOT) return f.template operator()<NTT_LOAD_DOT, NTT_STORE_NONE>();
    if (load == NTT_LOAD_DOTM) return f.template operator()<NTT_LOAD_DOTM, NTT_STORE_NONE>();
    return hipErrorInvalidValue;
  }
}

}  // namespace th
