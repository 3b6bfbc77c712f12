// Batched negacyclic NTT for gfx950: one workgroup transforms one
// limb-polynomial entirely on chip.
//
// Semantics (bit-exact with tensafe-he-core/src/ntt.rs):
//  forward (ntt.rs:79-102): Cooley-Tukey, stage s pairs j and j + N/2^(s+1)
//    with twiddle fwd[2^s + (j >> (log N - s))]; output in bit-reversed
//    evaluation order.
//  inverse (ntt.rs:113-141): Gentleman-Sande with inv[...] in the mirrored
//    order, then a multiply by N^{-1} (folded into the last stage here).
// Writing b for the bit a butterfly pairs (b = log N - 1 - s forward), both
// directions read twiddle (N + j) >> (b + 1) for the lower element j.
//
// Work split: T = N/E threads, each holding E = 16 (32 for N = 32768)
// coefficients in registers. A register pass performs log2(E) butterfly
// stages on the register-resident bits; between passes the coefficients are
// exchanged through LDS (one padding slot per 16 u64 to spread the strided
// pass patterns over the banks). N = 16384 needs 136 KiB of LDS (one
// workgroup per CU); N = 32768 exchanges in two rounds of half the
// coefficients through the same 136 KiB. Global loads and stores are
// lane-contiguous (lane t touches element t + k*T), except the N = 32768
// inverse load / forward store (see run_ntt).
#include "th_internal.h"

namespace th {

template <int LOGN>
struct Shape {
  static constexpr int N = 1 << LOGN;
  static constexpr int LE = LOGN >= 15 ? 5 : 4;
  static constexpr int E = 1 << LE;
  static constexpr int T = N / E;
  static constexpr int HALVES = LOGN >= 15 ? 2 : 1;
  static constexpr int LDS_ELEMS = (N / HALVES) + ((N / HALVES) >> 4);
  static constexpr int COAL_LO = LOGN - LE;  // register bits on top: lane-contiguous global access
};

size_t ntt_lds_bytes(int logn) {
  switch (logn) {
    case 10: return Shape<10>::LDS_ELEMS * 8;
    case 11: return Shape<11>::LDS_ELEMS * 8;
    case 12: return Shape<12>::LDS_ELEMS * 8;
    case 13: return Shape<13>::LDS_ELEMS * 8;
    case 14: return Shape<14>::LDS_ELEMS * 8;
    case 15: return Shape<15>::LDS_ELEMS * 8;
    default: return 0;
  }
}

// Element index held by thread `tid` in register k, for the layout whose
// register bits are [LO, LO + LE).
template <int LE, int LO>
__device__ __forceinline__ uint32_t elem(uint32_t tid, uint32_t k) {
  return (tid & ((1u << LO) - 1)) | ((tid >> LO) << (LO + LE)) | (k << LO);
}

constexpr int tid_bit(int c, int lo, int le) { return c < lo ? c : c - le; }

// Split bit of a two-round exchange: an element bit that is the SAME thread
// bit in both layouts, so every thread takes part in exactly one round as
// writer and reader (a thread must not overwrite its registers with new
// values while it still has old ones to write). -1 if there is none.
constexpr int split_bit(int logn, int le, int lo_s, int lo_d) {
  for (int c = logn - 1; c >= 0; --c) {
    bool ts = c < lo_s || c >= lo_s + le;
    bool td = c < lo_d || c >= lo_d + le;
    if (ts && td && tid_bit(c, lo_s, le) == tid_bit(c, lo_d, le)) return c;
  }
  return -1;
}

template <int HALVES, int C>
__device__ __forceinline__ uint32_t phys(uint32_t j) {
  if constexpr (HALVES == 2) j = (j & ((1u << C) - 1)) | ((j >> (C + 1)) << C);
  return j + (j >> 4);
}

// Re-distribute the coefficients from layout LO_S to layout LO_D through LDS.
template <int LOGN, int LO_S, int LO_D, class V>
__device__ __forceinline__ void exchange(V (&x)[Shape<LOGN>::E], V* lds, uint32_t tid) {
  using S = Shape<LOGN>;
  constexpr int C = split_bit(LOGN, S::LE, LO_S, LO_D);
  static_assert(S::HALVES == 1 || C >= 0, "no split bit with the same thread bit in both layouts");
#pragma unroll
  for (int h = 0; h < S::HALVES; ++h) {
    if (S::HALVES == 1 || ((tid >> tid_bit(C, LO_S, S::LE)) & 1) == (uint32_t)h) {
#pragma unroll
      for (int k = 0; k < S::E; ++k) lds[phys<S::HALVES, C>(elem<S::LE, LO_S>(tid, k))] = x[k];
    }
    __syncthreads();
    if (S::HALVES == 1 || ((tid >> tid_bit(C, LO_D, S::LE)) & 1) == (uint32_t)h) {
#pragma unroll
      for (int k = 0; k < S::E; ++k) x[k] = lds[phys<S::HALVES, C>(elem<S::LE, LO_D>(tid, k))];
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ arithmetic policies
struct IntArith {
  using V = uint64_t;
  using Tw = ShoupTw;
  uint64_t q, two_q;
  __device__ IntArith(const LimbConst& c) : q(c.q), two_q(c.two_q) {}
  __device__ __forceinline__ V load(uint64_t x) const { return x; }
  // forward CT butterfly, inputs/outputs in [0, 4q)
  __device__ __forceinline__ void fwd(V& a, V& b, const Tw& t) const {
    uint64_t X = csub(a, two_q);
    uint64_t T = shoup_lazy(b, t.w, t.ws, q);
    a = X + T;
    b = X + two_q - T;
  }
  // inverse GS butterfly, inputs/outputs in [0, 2q)
  __device__ __forceinline__ void inv(V& a, V& b, const Tw& t) const {
    uint64_t X = a, Y = b;
    a = csub(X + Y, two_q);
    b = shoup_lazy(X + two_q - Y, t.w, t.ws, q);
  }
  __device__ __forceinline__ void inv_last(V& a, V& b, const LimbConst& c) const {
    uint64_t X = a, Y = b;
    a = csub(shoup_lazy(X + Y, c.n_inv, c.n_inv_s, q), q);
    b = csub(shoup_lazy(X + two_q - Y, c.last_w, c.last_ws, q), q);
  }
  __device__ __forceinline__ void inv_pass_end(V&) const {}
  __device__ __forceinline__ uint64_t fwd_store(V x) const { return csub(csub(x, two_q), q); }
  __device__ __forceinline__ uint64_t inv_store(V x) const { return x; }
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
};

// ------------------------------------------------------------------ register passes
// Forward stages for bits BHI down to BLO on the layout with register bits [LO, LO+LE).
template <int LOGN, int LO, int BHI, int BLO, bool FIRST, class A>
__device__ __forceinline__ void fwd_pass(typename A::V (&x)[Shape<LOGN>::E], uint32_t tid,
                                         const typename A::Tw* __restrict__ tw, const A& ar) {
  using S = Shape<LOGN>;
  // thread's element bits above the register window (zero for the first pass)
  const uint32_t jhi = FIRST ? 0u : ((tid >> LO) << (LO + S::LE));
#pragma unroll
  for (int b = BHI; b >= BLO; --b) {
    const int rb = b - LO;
    const uint32_t base = ((uint32_t)S::N | jhi) >> (b + 1);
#pragma unroll
    for (int k = 0; k < S::E; ++k) {
      if (k & (1 << rb)) continue;
      const int k2 = k | (1 << rb);
      const typename A::Tw t = tw[base | (uint32_t)(k >> (rb + 1))];
      ar.fwd(x[k], x[k2], t);
    }
  }
}

template <int LOGN, int LO, int BLO, int BHI, class A>
__device__ __forceinline__ void inv_pass(typename A::V (&x)[Shape<LOGN>::E], uint32_t tid,
                                         const typename A::Tw* __restrict__ tw, const A& ar,
                                         const LimbConst& lc) {
  using S = Shape<LOGN>;
  const uint32_t jhi = (tid >> LO) << (LO + S::LE);
#pragma unroll
  for (int b = BLO; b <= BHI; ++b) {
    const int rb = b - LO;
    const uint32_t base = ((uint32_t)S::N | jhi) >> (b + 1);
#pragma unroll
    for (int k = 0; k < S::E; ++k) {
      if (k & (1 << rb)) continue;
      const int k2 = k | (1 << rb);
      if (b == LOGN - 1) {
        ar.inv_last(x[k], x[k2], lc);
      } else {
        const typename A::Tw t = tw[base | (uint32_t)(k >> (rb + 1))];
        ar.inv(x[k], x[k2], t);
      }
    }
  }
  if (BHI != LOGN - 1) {
#pragma unroll
    for (int k = 0; k < S::E; ++k) ar.inv_pass_end(x[k]);
  }
}

// Remaining forward passes: bits [TOP-1 .. 0] still to do, registers in layout CUR_LO.
template <int LOGN, int TOP, int CUR_LO, bool FIRST, class A>
__device__ __forceinline__ void fwd_passes(typename A::V (&x)[Shape<LOGN>::E], typename A::V* lds,
                                           uint32_t tid, const typename A::Tw* tw, const A& ar) {
  using S = Shape<LOGN>;
  if constexpr (TOP > 0) {
    constexpr int LO = TOP - S::LE > 0 ? TOP - S::LE : 0;
    if constexpr (LO != CUR_LO) exchange<LOGN, CUR_LO, LO>(x, lds, tid);
    fwd_pass<LOGN, LO, TOP - 1, LO, FIRST, A>(x, tid, tw, ar);
    fwd_passes<LOGN, LO, LO, false, A>(x, lds, tid, tw, ar);
  } else {
    // single-round LDS: restage to the lane-contiguous layout for the store
    if constexpr (S::HALVES == 1 && CUR_LO != S::COAL_LO) exchange<LOGN, CUR_LO, S::COAL_LO>(x, lds, tid);
  }
}

// Remaining inverse passes: bits [BOT .. LOGN-1] still to do.
template <int LOGN, int BOT, int CUR_LO, class A>
__device__ __forceinline__ void inv_passes(typename A::V (&x)[Shape<LOGN>::E], typename A::V* lds,
                                           uint32_t tid, const typename A::Tw* tw, const A& ar,
                                           const LimbConst& lc) {
  using S = Shape<LOGN>;
  if constexpr (BOT < LOGN) {
    constexpr int LO = BOT < S::COAL_LO ? BOT : S::COAL_LO;
    constexpr int HI = LO + S::LE - 1;
    if constexpr (LO != CUR_LO) exchange<LOGN, CUR_LO, LO>(x, lds, tid);
    inv_pass<LOGN, LO, BOT, HI, A>(x, tid, tw, ar, lc);
    inv_passes<LOGN, HI + 1, LO, A>(x, lds, tid, tw, ar, lc);
  }
}

// The operation fused into the coefficient load (NttLoad); `i` indexes the
// limb-polynomial, so src, aux and key are read at the same position.
struct LoadOp {
  uint32_t kind;
  const uint64_t* aux;
  const uint64_t* key;  // secret-key limb-poly (DOT)
  BarrettConst bc;
  RescaleConst rc;
  __device__ __forceinline__ uint64_t operator()(const uint64_t* __restrict__ src, uint32_t i) const {
    const uint64_t x = src[i];
    switch (kind) {
      case NTT_LOAD_MUL: return mulmod_barrett(x, aux[i], bc);
      case NTT_LOAD_RESCALE: return rescale_coeff(x, aux[i], rc);
      case NTT_LOAD_DOT: return addmod(x, mulmod_barrett(aux[i], key[i], bc), bc.q);
      default: return x;
    }
  }
};

// Global access: lane-contiguous (element t + k*T) whenever LDS can restage
// the whole polynomial in one round. With the two-round exchange (N = 32768)
// the layout-0 <-> lane-contiguous restaging has no valid split bit, so the
// first inverse load and the last forward store use the layout-0 registers
// directly (each lane owns E consecutive words).
template <int LOGN, bool INV, class A>
__device__ __forceinline__ void run_ntt(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                        const LimbConst& lc, const LoadOp& op, void* lds_raw) {
  using S = Shape<LOGN>;
  const uint32_t tid = threadIdx.x;
  const A ar(lc);
  typename A::V x[S::E];
  typename A::V* lds = reinterpret_cast<typename A::V*>(lds_raw);
  if constexpr (!INV) {
#pragma unroll
    for (int k = 0; k < S::E; ++k) x[k] = ar.load(op(src, tid + k * S::T));
    const typename A::Tw* tw = reinterpret_cast<const typename A::Tw*>(lc.fwd);
    fwd_passes<LOGN, LOGN, S::COAL_LO, true, A>(x, lds, tid, tw, ar);
    constexpr int OUT_LO = S::HALVES == 1 ? S::COAL_LO : 0;
#pragma unroll
    for (int k = 0; k < S::E; ++k) dst[elem<S::LE, OUT_LO>(tid, k)] = ar.fwd_store(x[k]);
  } else {
    constexpr int IN_LO = S::HALVES == 1 ? S::COAL_LO : 0;
#pragma unroll
    for (int k = 0; k < S::E; ++k) x[k] = ar.load(op(src, elem<S::LE, IN_LO>(tid, k)));
    const typename A::Tw* tw = reinterpret_cast<const typename A::Tw*>(lc.inv);
    inv_passes<LOGN, 0, IN_LO, A>(x, lds, tid, tw, ar, lc);
#pragma unroll
    for (int k = 0; k < S::E; ++k) dst[tid + k * S::T] = ar.inv_store(x[k]);
  }
}

template <int LOGN, bool INV>
__global__ __launch_bounds__(Shape<LOGN>::T) void ntt_kernel(NttArgs a) {
  extern __shared__ uint64_t lds[];
  const uint32_t job = blockIdx.x;
  const uint64_t* src;
  uint64_t* dst;
  uint32_t limb;
  LoadOp op{};
  if (a.jobs) {
    const NttJob jb = a.jobs[job];
    src = jb.src;
    dst = jb.dst;
    limb = jb.limb;
    op.kind = a.load;
    op.aux = jb.aux;
    if (a.load == NTT_LOAD_MUL || a.load == NTT_LOAD_DOT) op.bc = a.bc[limb];
    if (a.load == NTT_LOAD_DOT) op.key = a.key + (uint64_t)limb * Shape<LOGN>::N;
    if (a.load == NTT_LOAD_RESCALE) op.rc = a.rc[limb];
  } else {
    src = a.src + (uint64_t)job * a.stride;
    dst = a.dst + (uint64_t)job * a.stride;
    limb = a.limb_base + job % a.limb_mod;
    op.kind = NTT_LOAD_NONE;
  }
  const LimbConst& lc = a.lc[limb];
  if (lc.fp64)
    run_ntt<LOGN, INV, Fp64Arith>(src, dst, lc, op, lds);
  else
    run_ntt<LOGN, INV, IntArith>(src, dst, lc, op, lds);
}

template <int LOGN, bool INV>
static hipError_t launch_one(const NttArgs& a, uint32_t njobs, hipStream_t s) {
  using S = Shape<LOGN>;
  static bool attr_set = false;
  const size_t lds = (size_t)S::LDS_ELEMS * 8;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)ntt_kernel<LOGN, INV>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((ntt_kernel<LOGN, INV>), dim3(njobs), dim3(S::T), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_ntt(int logn, bool inverse, const NttArgs& a, uint32_t njobs, hipStream_t s) {
  if (njobs == 0) return hipSuccess;
#define TH_NTT_CASE(L) \
  case L: return inverse ? launch_one<L, true>(a, njobs, s) : launch_one<L, false>(a, njobs, s);
  switch (logn) {
    TH_NTT_CASE(10)
    TH_NTT_CASE(11)
    TH_NTT_CASE(12)
    TH_NTT_CASE(13)
    TH_NTT_CASE(14)
    TH_NTT_CASE(15)
    default: return hipErrorInvalidValue;
  }
#undef TH_NTT_CASE
}

}  // namespace th
