// Batched negacyclic NTT for gfx950 (bit-exact with tensafe-he-core/src/ntt.rs):
//  forward (ntt.rs:79-102): Cooley-Tukey, stage s pairs j and j + N/2^(s+1)
//    with twiddle fwd[2^s + (j >> (log N - s))]; output in bit-reversed
//    evaluation order.
//  inverse (ntt.rs:113-141): Gentleman-Sande with inv[...] in the mirrored
//    order, then a multiply by N^{-1} (folded into the last stage here).
// Writing b for the bit a butterfly pairs (b = log N - 1 - s forward), both
// directions read twiddle (N + j) >> (b + 1) for the lower element j.
//
// Two kernel families. Here: one workgroup transforms one limb-polynomial
// on chip (N <= 16384). In ntt_split.hip: a column pass plus a row pass of
// single-wavefront workgroups (N >= 8192). The whole-polynomial kernel moves
// each coefficient through HBM once but, at N = 16384, fills a CU's LDS, so
// a CU cannot overlap one polynomial's loads with another's arithmetic; the
// split kernels move the data twice but keep many wavefronts per CU. The
// whole-polynomial kernel's time grows in steps of one round of workgroups
// (one per CU) and a round takes a transform's time however few workgroups
// it holds, while the split kernels spread every transform over 16
// workgroups. Measured on MI355X at N = 16384 (forward, 4-limb chain): 4
// transforms 23.8 us whole against 11.0 us split, 64: 25.2 against 19.5,
// 128: 26.5 against 32.6, 256: 29.2 against 35.9; from 384 transforms on the
// split kernels win again (1792: 197 us against 256 us). So batches of
// NTT_WHOLE_MIN_JOBS = 96 to NTT_WHOLE_MAX_JOBS = 256 (the CU count) use the
// first, the others the second (the segment-sum epilogue exists in the first
// only).
//
// Whole-polynomial kernel: T = N/16 threads hold 16 coefficients each in
// registers; a register pass performs up to 4 butterfly stages on the
// register-resident bits, and between passes the coefficients are exchanged
// through LDS (one padding slot per 16 u64 spreads the strided patterns over
// the banks). Only one exchange per transform spans the workgroup: in every
// layout whose register window starts at or below bit 6, wavefront w holds
// the 1024 elements whose bits >= 10 equal w, so the exchanges among those
// layouts stay inside a wavefront (its own LDS slice, no barrier) and the
// wavefronts drift apart, overlapping one another's twiddle loads, arithmetic
// and stores. Forward: bits 13..10 in the lane-contiguous load layout, the
// workgroup exchange, then bits 9..0 in wavefront-local passes, stored from
// the wavefront-contiguous layout. Inverse: the mirror image. Passes whose
// twiddle indices are uniform across a wavefront read them with scalar loads.
// Every other global access goes through address-space-1 pointers, so it is a
// global_* instruction: generic (flat) accesses would also count against the
// LDS wait counter and hold up every exchange. The fused load/store
// operations are template parameters, so each kernel carries only its own.
#include "ntt_arith.h"

namespace th {

constexpr int NTT_WHOLE_MAX_LOGN = 14;
#ifndef NTT_WHOLE_MAX_JOBS
#define NTT_WHOLE_MAX_JOBS 256
#endif
#ifndef NTT_WHOLE_MIN_JOBS
#define NTT_WHOLE_MIN_JOBS 96
#endif
hipError_t launch_ntt_split(int logn, bool inverse, const NttArgs& a, uint32_t njobs, hipStream_t s);
hipError_t launch_rescale_split(int logn, const NttArgs& inv, uint32_t ninv, const NttArgs& fwd, uint32_t nf,
                                hipStream_t s);
hipError_t launch_encrypt_split(int logn, const NttArgs& a, uint32_t ninputs, uint32_t L, uint32_t limb_mask,
                                const EncDot& dot, const uint64_t* pkp, uint64_t* cts, hipStream_t s);

template <int LOGN>
struct Shape {
  static constexpr int N = 1 << LOGN;
  static constexpr int LE = 4;
  static constexpr int E = 1 << LE;
  static constexpr int T = N / E;
  static constexpr int LDS_ELEMS = N + (N >> 4);
  static constexpr int COAL_LO = LOGN - LE;  // register bits on top: lane-contiguous global access
  static constexpr int WAVE_LO = 6;          // lane-contiguous inside each wavefront's 1024 elements
};

// Element index held by thread `tid` in register k, for the layout whose
// register bits are [LO, LO + LE). In every layout with LO <= 6, wavefront
// w = tid >> 6 holds exactly the 1024 elements whose bits >= 10 equal w
// (tid bits [LO, 6) land on element bits [LO + 4, 10), tid bits >= 6 on
// bits >= 10), so an exchange between two such layouts stays inside the
// wavefront and its LDS region, and needs no workgroup barrier.
template <int LE, int LO>
__device__ __forceinline__ uint32_t elem(uint32_t tid, uint32_t k) {
  return (tid & ((1u << LO) - 1)) | ((tid >> LO) << (LO + LE)) | (k << LO);
}

__device__ __forceinline__ uint32_t phys(uint32_t j) { return j + (j >> 4); }

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Re-distribute the coefficients from layout LO_S to layout LO_D through LDS.
template <int LOGN, int LO_S, int LO_D, class V>
__device__ __forceinline__ void exchange(V (&x)[Shape<LOGN>::E], V* lds, uint32_t tid) {
  using S = Shape<LOGN>;
  constexpr bool WAVE = LO_S <= S::WAVE_LO && LO_D <= S::WAVE_LO;
#pragma unroll
  for (int k = 0; k < S::E; ++k) lds[phys(elem<S::LE, LO_S>(tid, k))] = x[k];
  if constexpr (WAVE) wave_sync(); else __syncthreads();
#pragma unroll
  for (int k = 0; k < S::E; ++k) x[k] = lds[phys(elem<S::LE, LO_D>(tid, k))];
  if constexpr (WAVE) wave_sync(); else __syncthreads();
}

// Element bits above the register window of layout LO for this thread; the
// same for a whole wavefront when LO >= 6 (then read through readfirstlane so
// that the pass's twiddle loads are scalar).
template <int LOGN, int LO>
__device__ __forceinline__ uint32_t jhi_of(uint32_t tid) {
  uint32_t h = tid >> LO;
  if constexpr (LO >= Shape<LOGN>::WAVE_LO) h = __builtin_amdgcn_readfirstlane(h);
  return h << (LO + Shape<LOGN>::LE);
}

// ------------------------------------------------------------------ register passes
// Forward stages for bits BHI down to BLO on the layout with register bits [LO, LO+LE).
template <int LOGN, int LO, int BHI, int BLO, class A>
__device__ __forceinline__ void fwd_pass(typename A::V (&x)[Shape<LOGN>::E], uint32_t tid,
                                         GPtr<typename A::Tw> tw, const A& ar) {
  using S = Shape<LOGN>;
  const uint32_t jhi = jhi_of<LOGN, LO>(tid);
#pragma unroll
  for (int b = BHI; b >= BLO; --b) {
    const int rb = b - LO;
    const uint32_t base = ((uint32_t)S::N | jhi) >> (b + 1);
#pragma unroll
    for (int k = 0; k < S::E; ++k) {
      if (k & (1 << rb)) continue;
      const int k2 = k | (1 << rb);
      const typename A::Tw t = ld16(tw, base | (uint32_t)(k >> (rb + 1)));
      ar.fwd(x[k], x[k2], t);
    }
  }
}

// Inverse stages for bits BLO up to BHI.
template <int LOGN, int LO, int BLO, int BHI, class A>
__device__ __forceinline__ void inv_pass(typename A::V (&x)[Shape<LOGN>::E], uint32_t tid,
                                         GPtr<typename A::Tw> tw, const A& ar, const LimbConst& lc) {
  using S = Shape<LOGN>;
  const uint32_t jhi = jhi_of<LOGN, LO>(tid);
#pragma unroll
  for (int b = BLO; b <= BHI; ++b) {
    const int rb = b - LO;
    const uint32_t base = ((uint32_t)S::N | jhi) >> (b + 1);
    if (b == LOGN - 1) {
#pragma unroll
      for (int k = 0; k < S::E; ++k)
        if (!(k & (1 << rb))) ar.inv_last(x[k], x[k | (1 << rb)], lc);
    } else {
      // the stage's twiddles (E >> (rb + 1) of them) requested before its
      // first butterfly, so they arrive together (measured faster here; in
      // the forward passes the compiler's own schedule was faster)
      constexpr int NT = S::E >> 1;
      typename A::Tw t[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j)
        if (j < (S::E >> (rb + 1))) t[j] = ld16(tw, base | (uint32_t)j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < S::E; ++k)
        if (!(k & (1 << rb))) ar.inv(x[k], x[k | (1 << rb)], t[k >> (rb + 1)]);
    }
  }
  if (BHI != LOGN - 1) {
#pragma unroll
    for (int k = 0; k < S::E; ++k) ar.inv_pass_end(x[k]);
  }
}

// Remaining forward passes: bits [TOP-1 .. 0] still to do, registers in layout CUR_LO.
// Windows step down from the top; once below bit 10 every exchange is inside a
// wavefront, so after the first exchange the wavefronts run without barriers.
template <int LOGN, int TOP, int CUR_LO, class A>
__device__ __forceinline__ void fwd_passes(typename A::V (&x)[Shape<LOGN>::E], typename A::V* lds,
                                           uint32_t tid, GPtr<typename A::Tw> tw, const A& ar) {
  using S = Shape<LOGN>;
  if constexpr (TOP > 0) {
    constexpr int LO = TOP - S::LE > 0 ? TOP - S::LE : 0;
    if constexpr (LO != CUR_LO) exchange<LOGN, CUR_LO, LO>(x, lds, tid);
    fwd_pass<LOGN, LO, TOP - 1, LO, A>(x, tid, tw, ar);
    fwd_passes<LOGN, LO, LO, A>(x, lds, tid, tw, ar);
  } else {
    // restage inside each wavefront to the wavefront-contiguous layout for the store
    if constexpr (CUR_LO != S::WAVE_LO) exchange<LOGN, CUR_LO, S::WAVE_LO>(x, lds, tid);
  }
}

// Window of the inverse pass that starts at bit BOT: below bit 10 the window
// starts at most at bit 6 (exchanges inside a wavefront), above it the
// lane-contiguous layout is reached with the one workgroup-wide exchange.
template <int LOGN>
constexpr int inv_lo(int bot) {
  return bot < 10 ? (bot < Shape<LOGN>::WAVE_LO ? bot : Shape<LOGN>::WAVE_LO)
                  : (bot < Shape<LOGN>::COAL_LO ? bot : Shape<LOGN>::COAL_LO);
}
template <int LOGN>
constexpr int inv_hi(int bot) {
  return inv_lo<LOGN>(bot) + Shape<LOGN>::LE - 1 < LOGN - 1 ? inv_lo<LOGN>(bot) + Shape<LOGN>::LE - 1 : LOGN - 1;
}
// The layout the inverse passes end in.
template <int LOGN>
constexpr int inv_end_lo() {
  int bot = 0, lo = 0;
  while (bot < LOGN) {
    lo = inv_lo<LOGN>(bot);
    bot = inv_hi<LOGN>(bot) + 1;
  }
  return lo;
}

// Remaining inverse passes: bits [BOT .. LOGN-1] still to do.
template <int LOGN, int BOT, int CUR_LO, class A>
__device__ __forceinline__ void inv_passes(typename A::V (&x)[Shape<LOGN>::E], typename A::V* lds,
                                           uint32_t tid, GPtr<typename A::Tw> tw, const A& ar,
                                           const LimbConst& lc) {
  if constexpr (BOT < LOGN) {
    constexpr int LO = inv_lo<LOGN>(BOT);
    constexpr int HI = inv_hi<LOGN>(BOT);
    if constexpr (LO != CUR_LO) exchange<LOGN, CUR_LO, LO>(x, lds, tid);
    inv_pass<LOGN, LO, BOT, HI, A>(x, tid, tw, ar, lc);
    inv_passes<LOGN, HI + 1, LO, A>(x, lds, tid, tw, ar, lc);
  }
}

// Segment-sum epilogue of an inverse transform on limb 0 (NTT_STORE_SEGSUM):
// the thread's canonical coefficients m (element k at j = elem(tid, k) of
// layout END) are centred against q / 2 and accumulated as v_j W_c[j] for
// every segment c; a fixed shuffle tree sums each wavefront and the
// wavefronts' sums are added in order, so the result does not depend on
// scheduling. RESCALED: m is first taken to (m - (xl[j] mod q)) * inv mod q
// with the rescale constants *rc (the coefficient-domain end of a rescaled
// decryption, rescale_decrypt_kernel).
template <int LOGN, int END, bool RESCALED, class A>
__device__ __forceinline__ void segsum_store(const typename A::V (&x)[Shape<LOGN>::E], const A& ar, uint64_t q,
                                             uint32_t tid, const double* segw, uint32_t cols, double* seg,
                                             double scale, const uint64_t* xl, const RescaleConst* rcp,
                                             void* lds_raw) {
  using S = Shape<LOGN>;
  constexpr int MAXC = NTT_SEGSUM_FUSED_MAX_COLS;
  const uint64_t half = q >> 1;
  using D2 = double __attribute__((ext_vector_type(2)));
  const GPtr<D2> W = gld(reinterpret_cast<const D2*>(segw));
  double acc[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) acc[c] = 0.0;
  // the weights (and subtrahends) of element k + PF are requested while
  // element k is summed
  constexpr int PF = S::E < 4 ? S::E : 4;
  D2 wq[PF];
  uint64_t xq[PF];
  RescaleConst rc{};
  if constexpr (RESCALED) rc = *rcp;
  __builtin_amdgcn_sched_barrier(0);  // keep the requests after the last pass (register peak)
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    wq[k] = W[elem<S::LE, END>(tid, k)];
    if constexpr (RESCALED) xq[k] = gld(xl)[elem<S::LE, END>(tid, k)];
  }
#pragma unroll
  for (int k = 0; k < S::E; ++k) {
    uint64_t m = ar.inv_store(x[k]);
    if constexpr (RESCALED) {
      const uint64_t xv = xq[k % PF];
      if (k + PF < S::E) xq[k % PF] = gld(xl)[elem<S::LE, END>(tid, k + PF)];
      const uint64_t xr = xv < rc.q ? xv : mulmod_barrett(xv, 1, rc.b);
      m = csub(shoup_lazy(submod(m, xr, q), rc.inv, rc.inv_s, q), q);
    }
    const double v = m > half ? -(double)(q - m) : (double)m;
    const D2 p = wq[k % PF];  // W_0[j], 2 cos(2 phi_j) at j = elem(tid, k)
    if (k + PF < S::E) wq[k % PF] = W[elem<S::LE, END>(tid, k + PF)];
    double wp = p.x, wc = p.x;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      if (c >= (int)cols) break;
      acc[c] += v * wc;
      const double wn = p.y * wc - wp;
      wp = wc;
      wc = wn;
    }
  }
  double* red = reinterpret_cast<double*>(lds_raw);
  const uint32_t lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    if (c >= (int)cols) break;
    double a = acc[c];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) a += __shfl_xor(a, off);
    if (lane == 0) red[wave * MAXC + c] = a;
  }
  __syncthreads();
  if (tid < cols) {
    double t = 0.0;
    for (uint32_t w = 0; w < S::T / 64; ++w) t += red[w * MAXC + tid];
    gst(seg)[tid] = t / scale;
  }
}

template <int LOGN, bool INV, class A, class LOp, class SOp>
__device__ __forceinline__ void run_ntt(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                        const LimbConst& lc, const LOp& op, const SOp& so, void* lds_raw) {
  using S = Shape<LOGN>;
  const uint32_t tid = threadIdx.x;
  const A ar(lc);
  const GMut<uint64_t> gdst = gst(dst);
  typename A::V x[S::E];
  typename A::V* lds = reinterpret_cast<typename A::V*>(lds_raw);
  if constexpr (!INV) {
#pragma unroll
    for (int k = 0; k < S::E; ++k) x[k] = ar.load(op(src, elem<S::LE, S::COAL_LO>(tid, k)));
    const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.fwd));
    fwd_passes<LOGN, LOGN, S::COAL_LO, A>(x, lds, tid, tw, ar);
#pragma unroll
    for (int k = 0; k < S::E; ++k) {
      const uint32_t i = elem<S::LE, S::WAVE_LO>(tid, k);
      so.store(ar, x[k], gdst, i, so.prep(ar, so.load_aux(i)));
    }
  } else {
    const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.inv));
#pragma unroll
    for (int k = 0; k < S::E; ++k) x[k] = ar.load(op(src, elem<S::LE, S::WAVE_LO>(tid, k)));
    inv_passes<LOGN, 0, S::WAVE_LO, A>(x, lds, tid, tw, ar, lc);
    constexpr int END = inv_end_lo<LOGN>();
    if constexpr (SOp::kind == NTT_STORE_SEGSUM) {
      segsum_store<LOGN, END, false>(x, ar, lc.q, tid, so.segw, so.cols, so.seg, so.scale, nullptr, nullptr, lds_raw);
    } else {
#pragma unroll
      for (int k = 0; k < S::E; ++k) gdst[elem<S::LE, END>(tid, k)] = ar.inv_store(x[k]);
    }
  }
}

template <int LOGN, bool INV, uint32_t LD, uint32_t ST>
__global__ __launch_bounds__(Shape<LOGN>::T) void ntt_kernel(NttArgs a) {
  extern __shared__ uint64_t lds[];
  const uint32_t job = blockIdx.x;
  const uint64_t* src;
  uint64_t* dst;
  uint32_t limb;
  LoadOp<LD> op{};
  StoreOp<ST> so{};
  if (a.jobs) {
    const NttJob jb = a.jobs[job];
    src = jb.src;
    dst = jb.dst;
    limb = jb.limb;
    job_ops(a, jb, limb, Shape<LOGN>::N, op, so);
  } else {
    src = a.src + (uint64_t)job * a.stride;
    dst = a.dst + (uint64_t)job * a.stride;
    limb = a.limb_base + job % a.limb_mod;
  }
  const LimbConst& lc = a.lc[limb];
  if (lc.fp64)
    run_ntt<LOGN, INV, Fp64Arith>(src, dst, lc, op, so, lds);
  else
    run_ntt<LOGN, INV, IntArith>(src, dst, lc, op, so, lds);
}

// One rescaled product's decryption on limb 0, with its segment sums
// (RescaleDecryptJob). The rescale (ciphertext.rs:476-535) takes each
// component c_i of ct x pt to (c_i - NTT(r_i)) inv on limb 0, where r_i is the
// last limb's coefficients reduced mod q and inv = q_last^{-1} mod q, and the
// decryption (ciphertext.rs:327-346) forms c'_0 + c'_1 s and transforms it
// back. With c_i = ct_i pt and D = ct_0 + ct_1 s, and the NTT linear mod q,
//   INTT(c'_0 + c'_1 s) = (INTT(D pt - NTT(r_1) s) - r_0) inv  (mod q),
// the same residues. So one workgroup runs the forward transform of r_1 (the
// loads reduce the last limb's coefficients Y mod q), forms D pt - NTT(r_1) s
// in registers at the forward's output positions (the inverse's input
// positions), runs the inverse transform, and subtracts r_0 (from X) and
// scales in the segment-sum epilogue. Two transforms per product, where the
// rescaled ciphertext and its decryption take three, and nothing but the
// segment sums is written.
template <int LOGN, class A>
__device__ __forceinline__ void run_rescale_decrypt(const RescaleDecryptArgs& a, const RescaleDecryptJob& jb,
                                                    const LimbConst& lc, void* lds_raw) {
  using S = Shape<LOGN>;
  const uint32_t tid = threadIdx.x;
  const A ar(lc);
  const RescaleConst* rcp = a.rc;
  const BarrettConst bc = *a.bc;
  typename A::V x[S::E];
  typename A::V* lds = reinterpret_cast<typename A::V*>(lds_raw);
  {
    const GPtr<uint64_t> y = gld(jb.y);
    const uint64_t q = rcp->q;
#pragma unroll
    for (int k = 0; k < S::E; ++k) {
      const uint64_t v = y[elem<S::LE, S::COAL_LO>(tid, k)];
      x[k] = ar.load(v < q ? v : mulmod_barrett(v, 1, rcp->b));
    }
  }
  fwd_passes<LOGN, LOGN, S::COAL_LO, A>(x, lds, tid, gld(reinterpret_cast<const typename A::Tw*>(lc.fwd)), ar);
  {
    // D pt - NTT(r_1) s: Montgomery products with pt and s in Montgomery
    // form, each in [0, 2q), so the difference plus 2q is in (0, 4q): the
    // integer inverse's input range; the FP64 inverse gets it canonical
    const GPtr<uint64_t> d = gld(jb.d), p = gld(jb.ptm), sk = gld(a.skm);
    const uint64_t q = lc.q, two_q = 2 * lc.q;
#pragma unroll
    for (int k = 0; k < S::E; ++k) {
      const uint32_t i = elem<S::LE, S::WAVE_LO>(tid, k);
      const uint64_t u = mont_mul(d[i], p[i], bc);
      const uint64_t t = mont_mul(ar.fwd_store(x[k]), sk[i], bc);
      uint64_t e = u + two_q - t;
      if constexpr (std::is_same_v<A, Fp64Arith>) e = csub(csub(e, two_q), q);
      x[k] = ar.load(e);
    }
  }
  inv_passes<LOGN, 0, S::WAVE_LO, A>(x, lds, tid, gld(reinterpret_cast<const typename A::Tw*>(lc.inv)), ar, lc);
  segsum_store<LOGN, inv_end_lo<LOGN>(), true>(x, ar, lc.q, tid, a.segw, a.cols, jb.seg, jb.scale, jb.x, rcp,
                                               lds_raw);
}

template <int LOGN>
__global__ __launch_bounds__(Shape<LOGN>::T) void rescale_decrypt_kernel(RescaleDecryptArgs a) {
  extern __shared__ uint64_t lds[];
  const RescaleDecryptJob jb = a.jobs[blockIdx.x];
  const LimbConst& lc = a.lc[0];
  if (lc.fp64)
    run_rescale_decrypt<LOGN, Fp64Arith>(a, jb, lc, lds);
  else
    run_rescale_decrypt<LOGN, IntArith>(a, jb, lc, lds);
}

template <int LOGN>
static hipError_t launch_rescale_decrypt_t(const RescaleDecryptArgs& a, uint32_t njobs, hipStream_t s) {
  const hipError_t e = allow_full_lds<rescale_decrypt_kernel<LOGN>>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((rescale_decrypt_kernel<LOGN>), dim3(njobs), dim3(Shape<LOGN>::T),
                     (size_t)Shape<LOGN>::LDS_ELEMS * 8, s, a);
  return hipGetLastError();
}

hipError_t launch_rescale_decrypt(int logn, const RescaleDecryptArgs& a, uint32_t njobs, hipStream_t s) {
  if (njobs == 0) return hipSuccess;
  if (a.cols < 1 || a.cols > NTT_SEGSUM_FUSED_MAX_COLS) return hipErrorInvalidValue;
  switch (logn) {
    case 10: return launch_rescale_decrypt_t<10>(a, njobs, s);
    case 11: return launch_rescale_decrypt_t<11>(a, njobs, s);
    case 12: return launch_rescale_decrypt_t<12>(a, njobs, s);
    case 13: return launch_rescale_decrypt_t<13>(a, njobs, s);
    case 14: return launch_rescale_decrypt_t<14>(a, njobs, s);
    default: return hipErrorInvalidValue;
  }
}

template <int LOGN, bool INV>
static hipError_t launch_one(const NttArgs& a, uint32_t njobs, hipStream_t s) {
  using S = Shape<LOGN>;
  const size_t lds = (size_t)S::LDS_ELEMS * 8;
  return with_ops<INV>(a.jobs ? a.load : NTT_LOAD_NONE, a.jobs ? a.store : NTT_STORE_NONE,
                  [&]<uint32_t LD, uint32_t ST>() -> hipError_t {
                    const hipError_t e = allow_full_lds<ntt_kernel<LOGN, INV, LD, ST>>();
                    if (e != hipSuccess) return e;
                    hipLaunchKernelGGL((ntt_kernel<LOGN, INV, LD, ST>), dim3(njobs), dim3(S::T), lds, s, a);
                    return hipGetLastError();
                  });
}

// Sizes and batches the whole-polynomial kernel cannot serve.
static bool whole_unavailable(int logn, uint32_t njobs) {
  return logn >= NTT_SPLIT_MIN_LOGN && (logn > NTT_WHOLE_MAX_LOGN || njobs > NTT_WHOLE_MAX_JOBS);
}
static bool use_split(int logn, uint32_t njobs) {
  return whole_unavailable(logn, njobs) || (logn >= NTT_SPLIT_MIN_LOGN && njobs < NTT_WHOLE_MIN_JOBS);
}

hipError_t launch_rescale(int logn, const NttArgs& inv, uint32_t ninv, const NttArgs& fwd, uint32_t nfwd,
                          hipStream_t s) {
  if (ninv == 0) return hipSuccess;
  if (use_split(logn, nfwd) && inv.jobs && fwd.jobs && nfwd % ninv == 0 && inv.store == NTT_STORE_NONE &&
      fwd.load == NTT_LOAD_REDUCE)
    return launch_rescale_split(logn, inv, ninv, fwd, nfwd / ninv, s);
  hipError_t e = launch_ntt(logn, true, inv, ninv, s);
  if (e != hipSuccess) return e;
  return launch_ntt(logn, false, fwd, nfwd, s);
}

bool encrypt_limbs_supported(int logn) { return logn >= NTT_SPLIT_MIN_LOGN && logn <= NTT_MAX_LOGN; }

hipError_t launch_encrypt(int logn, const NttArgs& a, uint32_t ninputs, uint32_t L, uint32_t limb_mask,
                          const EncDot& dot, const uint64_t* pkp, uint64_t* cts, bool* combined, hipStream_t s) {
  *combined = false;
  if (ninputs == 0) return hipSuccess;
  const uint32_t nl = (uint32_t)__builtin_popcount(limb_mask);
  if (nl == 0 || limb_mask >> L || (dot.mask & ~limb_mask)) return hipErrorInvalidValue;
  // the split kernels also serve limb subsets and D (k_encrypt_combine forms every limb of c0 and c1)
  const bool split = use_split(logn, ninputs * 3 * nl) || ((nl != L || dot.mask) && encrypt_limbs_supported(logn));
  if (split && a.jobs && a.load == NTT_LOAD_ENC && a.store == NTT_STORE_NONE) {
    *combined = true;
    return launch_encrypt_split(logn, a, ninputs, L, limb_mask, dot, pkp, cts, s);
  }
  if (nl != L || dot.mask) return hipErrorInvalidValue;  // k_encrypt_combine forms every limb, no D
  return launch_ntt(logn, false, a, ninputs * 3 * L, s);
}

hipError_t launch_ntt(int logn, bool inverse, const NttArgs& a, uint32_t njobs, hipStream_t s) {
  if (njobs == 0) return hipSuccess;
  const bool segsum = a.jobs && a.store == NTT_STORE_SEGSUM;
  if (segsum && (!inverse || whole_unavailable(logn, njobs) || logn > NTT_WHOLE_MAX_LOGN || a.cols < 1 ||
                 a.cols > NTT_SEGSUM_FUSED_MAX_COLS))
    return hipErrorInvalidValue;  // the segment-sum epilogue exists in the whole-polynomial inverse only
  if (!segsum && use_split(logn, njobs)) return launch_ntt_split(logn, inverse, a, njobs, s);
#define TH_NTT_CASE(L) \
  case L: return inverse ? launch_one<L, true>(a, njobs, s) : launch_one<L, false>(a, njobs, s);
  switch (logn) {
    TH_NTT_CASE(10)
    TH_NTT_CASE(11)
    TH_NTT_CASE(12)
    TH_NTT_CASE(13)
    TH_NTT_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef TH_NTT_CASE
}

}  // namespace th
