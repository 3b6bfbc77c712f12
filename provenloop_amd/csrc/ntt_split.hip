// Split negacyclic NTT for N = 2^13 .. 2^15: a column pass and a row pass,
// each one launch of single-wavefront workgroups.
//
// The coefficient index j = (row << CB) | col splits into CB low "column"
// bits and RB = log N - CB high "row" bits. Every butterfly pairs two
// indices that differ in one bit b, and its twiddle is (N + j) >> (b + 1)
// for the lower index j (tensafe-he-core/src/ntt.rs:79-141, SEAL-style
// tables). Stages on row bits only mix coefficients of one column; stages on
// column bits only mix coefficients of one row. So
//   forward = column pass (row bits, high to low) then row pass (column bits),
//   inverse = row pass (column bits, low to high) then column pass (row bits,
//             ending with the stage that folds in N^{-1}),
// with no extra twiddle factors between the passes.
//
// Each wavefront owns 1024 coefficients of one limb-polynomial (16 per
// lane), runs two register passes of up to four butterfly stages, and
// re-distributes its coefficients between them through a private 8.5 KiB
// LDS slice (no workgroup barrier beyond its own wavefront). Small LDS and
// register footprints let many wavefronts share a CU, so global loads,
// stores and arithmetic of different wavefronts overlap. The first pass
// writes its intermediate values in the arithmetic's own representation
// (lazy u64 residues, or f64 bit patterns) to the destination, where the
// second pass reads them back, in the natural coefficient order. Every
// workgroup reads and writes exactly the same set of positions in each pass
// (its columns, or its rows), so a transform may run in place and no
// workgroup can overwrite data another one has still to read.
//
// Wavefront layouts (l = lane, k = register, e = index within the
// wavefront's 1024 coefficients):
//   column pass, CW = 2^(10-RB) adjacent columns x all 2^RB rows:
//     Q1: col = l mod CW, row = (l / CW) | (k << (RB-4))     registers = row bits [RB-4, RB)
//     Q2: col = l mod CW, row = k | ((l / CW) << 4)           registers = row bits [0, 4)
//   row pass, 2^(10-CB) adjacent rows x 2^CB columns:
//     P1: col = (l mod 2^(CB-4)) | (k << (CB-4))              registers = col bits [CB-4, CB)
//     P2: col = k | ((l mod 2^(CB-4)) << 4)                   registers = col bits [0, 4)
//     G:  e = l + 64 k                                        (lane-contiguous global access)
// Column-pass wavefronts 2m and 2m+1 share the 128-byte lines of the
// natural layout; they are given workgroup ids that the dispatcher sends to
// the same XCD (ids are dealt round-robin over the 8 XCDs), so the second
// half of each line is served by that XCD's L2.
#include "ntt_arith.h"

namespace th {

template <int LOGN>
struct Split {
  static constexpr int N = 1 << LOGN;
  static constexpr int CB = split_column_bits(LOGN);  // column bits
  static constexpr int RB = LOGN - CB;           // row bits
  static constexpr int E = 16;
  static constexpr int PARTS = N >> 10;          // wavefronts per limb-polynomial
  static constexpr int CW = 1 << (10 - RB);      // columns per column-pass wavefront
  static constexpr int LDS = 1024 + 64;          // one padding word per 16
  // twiddle entries of stages CB-1 .. CB-3 of a forward row-pass wavefront's
  // first register pass (2^(9-b) entries of stage b over its 2^(10-CB) rows;
  // the staged ones, RowStage)
  static constexpr int TW1S = 7 << (10 - CB);
  // and of an inverse row-pass wavefront's second register pass (stages 4 ..
  // CB-1)
  static constexpr int TWI = ((1 << (CB - 4)) - 1) << (10 - CB);
  static_assert(CB >= 4 && RB >= 4 && RB <= 10 && CB <= 10, "unsupported split");
};

__device__ __forceinline__ uint32_t pad16(uint32_t e) { return e + (e >> 4); }

// Forward stages BHI down to BLO on registers that hold index bits
// [EB, EB + 4); f = index of register 0 (its register bits are zero). With
// BATCH, each stage's twiddles (16 >> (rb + 1) of them) are all requested
// before its first butterfly, for kernels whose register pressure otherwise
// leads the scheduler to wait on each twiddle in turn. Measured per caller:
// batched are the row passes with a fused store, the encrypt row kernel and
// the rescale column kernel's forward passes (and every inverse pass, in
// inv_stages); the plain forward column and row passes keep the compiler's
// schedule, which measured faster there (N=32768 forward row pass 35.0
// against 36.1 us).
// The twiddles come from get(b, base, s): entry base | s of stage b's table
// (s = the slot of the register pair among the stage's twiddles of the lane).
template <int LOGN, int EB, int BHI, int BLO, class A, bool BATCH, class Get>
__device__ __forceinline__ void fwd_stages_get(typename A::V (&x)[16], uint32_t f, const Get& get, const A& ar) {
#pragma unroll
  for (int b = BHI; b >= BLO; --b) {
    const int rb = b - EB;
    const uint32_t base = ((1u << LOGN) | f) >> (b + 1);
    if constexpr (BATCH) {
      constexpr int NT = 16 >> 1;
      typename A::Tw t[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j)
        if (j < (16 >> (rb + 1))) t[j] = get(b, base, (uint32_t)j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (k & (1 << rb)) continue;
        ar.fwd(x[k], x[k | (1 << rb)], t[k >> (rb + 1)]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (k & (1 << rb)) continue;
        const typename A::Tw t = get(b, base, (uint32_t)(k >> (rb + 1)));
        ar.fwd(x[k], x[k | (1 << rb)], t);
      }
    }
  }
}
template <int LOGN, int EB, int BHI, int BLO, class A, bool BATCH = true>
__device__ __forceinline__ void fwd_stages(typename A::V (&x)[16], uint32_t f, GPtr<typename A::Tw> tw,
                                           const A& ar) {
  fwd_stages_get<LOGN, EB, BHI, BLO, A, BATCH>(x, f, [&](int, uint32_t base, uint32_t s) { return ld16(tw, base | s); },
                                               ar);
}

// Inverse stages BLO up to BHI; the stage on bit LOGN-1 folds in N^{-1}.
// With BATCH, as in fwd_stages, each stage's twiddles are requested before
// its first butterfly.
// The twiddles come from get(b, base, s), as in fwd_stages_get.
template <int LOGN, int EB, int BLO, int BHI, class A, bool BATCH, class Get>
__device__ __forceinline__ void inv_stages_get(typename A::V (&x)[16], uint32_t f, const Get& get, const A& ar,
                                               const LimbConst& lc) {
#pragma unroll
  for (int b = BLO; b <= BHI; ++b) {
    const int rb = b - EB;
    const uint32_t base = ((1u << LOGN) | f) >> (b + 1);
    if (b == LOGN - 1) {
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (!(k & (1 << rb))) ar.inv_last(x[k], x[k | (1 << rb)], lc);
    } else if constexpr (BATCH) {
      constexpr int NT = 16 >> 1;
      typename A::Tw t[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j)
        if (j < (16 >> (rb + 1))) t[j] = get(b, base, (uint32_t)j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (!(k & (1 << rb))) ar.inv(x[k], x[k | (1 << rb)], t[k >> (rb + 1)]);
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (k & (1 << rb)) continue;
        const typename A::Tw t = get(b, base, (uint32_t)(k >> (rb + 1)));
        ar.inv(x[k], x[k | (1 << rb)], t);
      }
    }
  }
  if (BHI != LOGN - 1) {
#pragma unroll
    for (int k = 0; k < 16; ++k) ar.inv_pass_end(x[k]);
  }
}
template <int LOGN, int EB, int BLO, int BHI, class A, bool BATCH = true>
__device__ __forceinline__ void inv_stages(typename A::V (&x)[16], uint32_t f, GPtr<typename A::Tw> tw,
                                           const A& ar, const LimbConst& lc) {
  inv_stages_get<LOGN, EB, BLO, BHI, A, BATCH>(x, f, [&](int, uint32_t base, uint32_t s) { return ld16(tw, base | s); },
                                               ar, lc);
}

// Re-distribute the wavefront's 16 x 64 coefficients from layout `from` to
// layout `to` (functions of the register index giving the index e in
// [0, 1024)) through its LDS slice.
// The slice is the wavefront's own, so a wavefront-level barrier orders it.
__device__ __forceinline__ void slice_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <class V, class From, class To>
__device__ __forceinline__ void wave_exchange(V (&x)[16], V* lds, From from, To to) {
#pragma unroll
  for (int k = 0; k < 16; ++k) lds[pad16(from(k))] = x[k];
  slice_sync();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = lds[pad16(to(k))];
  slice_sync();
}

// The same exchange through half the LDS (1024 + 64 32-bit words): the
// coefficients' low words first, then their high words. A register's low
// word is free once written, so it takes its new value at once and no
// register holds both layouts' words.
template <class V, class From, class To>
__device__ __forceinline__ void wave_exchange_half(V (&x)[16], uint32_t* lds, From from, To to) {
  uint32_t lo[16], hi[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint64_t v = __builtin_bit_cast(uint64_t, x[k]);
    lo[k] = (uint32_t)v;
    hi[k] = (uint32_t)(v >> 32);
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) lds[pad16(from(k))] = lo[k];
  slice_sync();
#pragma unroll
  for (int k = 0; k < 16; ++k) lo[k] = lds[pad16(to(k))];
  slice_sync();
#pragma unroll
  for (int k = 0; k < 16; ++k) lds[pad16(from(k))] = hi[k];
  slice_sync();
#pragma unroll
  for (int k = 0; k < 16; ++k) hi[k] = lds[pad16(to(k))];
  slice_sync();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = __builtin_bit_cast(V, ((uint64_t)hi[k] << 32) | lo[k]);
}

template <bool HALF, class V, class From, class To>
__device__ __forceinline__ void exchange_in(V (&x)[16], uint64_t* lds_raw, From from, To to) {
  if constexpr (HALF)
    wave_exchange_half(x, reinterpret_cast<uint32_t*>(lds_raw), from, to);
  else
    wave_exchange(x, reinterpret_cast<V*>(lds_raw), from, to);
}

// ------------------------------------------------------------------ column pass
// Column geometry of wavefront `part`: CW adjacent columns, all 2^RB rows.
template <int LOGN>
struct ColumnMap {
  using S = Split<LOGN>;
  static constexpr int RB = S::RB, CB = S::CB, CW = S::CW, WL = 10 - RB;  // WL = log2(CW)
  uint32_t lcol, lrow, col;
  __device__ explicit ColumnMap(uint32_t part) {
    const uint32_t l = threadIdx.x;
    lcol = l & (CW - 1);
    lrow = l >> WL;
    col = part * CW + lcol;
  }
  // Q1 and Q2 element maps: local e = (row << WL) | lcol, global j = (row << CB) | col
  __device__ uint32_t row1(uint32_t k) const { return lrow | (k << (RB - 4)); }
  __device__ uint32_t row2(uint32_t k) const { return k | (lrow << 4); }
  __device__ uint32_t e1(uint32_t k) const { return (row1(k) << WL) | lcol; }
  __device__ uint32_t e2(uint32_t k) const { return (row2(k) << WL) | lcol; }
  __device__ uint32_t j1(uint32_t k) const { return (row1(k) << CB) | col; }
  __device__ uint32_t j2(uint32_t k) const { return (row2(k) << CB) | col; }
};

// Forward column pass on coefficients already in registers (Q1 layout, the
// arithmetic's representation); writes the intermediate to dst (Q2). HALF:
// the exchange goes through half the LDS (wave_exchange_half).
template <int LOGN, class A, bool BATCH = false, bool HALF = false>
__device__ __forceinline__ void column_fwd_regs(typename A::V (&x)[16], uint64_t* dst, const LimbConst& lc,
                                                const ColumnMap<LOGN>& m, const A& ar, uint64_t* lds_raw) {
  constexpr int CB = Split<LOGN>::CB;
  const GMut<uint64_t> gdst = gst(dst);
  const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.fwd));
  // stages on bits >= LOGN - 4 (the Q1 registers): every lane's element
  // bits above the stage are zero, so the twiddle index is uniform (f = 0)
  fwd_stages_get<LOGN, LOGN - 4, LOGN - 1, LOGN - 4, A, BATCH>(
      x, 0u, [&](int, uint32_t base, uint32_t s) { return ld16_uniform(tw, base | s); }, ar);
  exchange_in<HALF>(x, lds_raw, [&](uint32_t k) { return m.e1(k); }, [&](uint32_t k) { return m.e2(k); });
  fwd_stages<LOGN, CB, LOGN - 5, CB, A, BATCH>(x, m.j2(0), tw, ar);
#pragma unroll
  for (int k = 0; k < 16; ++k) gdst[m.j2(k)] = ar.raw(x[k]);
}

// Inverse column pass from the row pass's intermediate in buf (Q2); leaves
// the transform's final values in registers (Q1 layout).
template <int LOGN, class A>
__device__ __forceinline__ void column_inv_regs(typename A::V (&x)[16], const uint64_t* buf, const LimbConst& lc,
                                                const ColumnMap<LOGN>& m, const A& ar, uint64_t* lds_raw) {
  constexpr int CB = Split<LOGN>::CB;
  const GPtr<uint64_t> gbuf = gld(buf);
  typename A::V* lds = reinterpret_cast<typename A::V*>(lds_raw);
  const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.inv));
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = ar.unraw(gbuf[m.j2(k)]);
  inv_stages<LOGN, CB, CB, CB + 3>(x, m.j2(0), tw, ar, lc);
  wave_exchange(x, lds, [&](uint32_t k) { return m.e2(k); }, [&](uint32_t k) { return m.e1(k); });
  // stages CB + 4 .. LOGN - 1 on the Q1 registers (bits LOGN - 4 ..): uniform
  // twiddle indices, as in column_fwd_regs
  static_assert(CB + 4 >= LOGN - 4, "the second inverse column pass must lie in the Q1 register bits");
  inv_stages_get<LOGN, LOGN - 4, CB + 4, LOGN - 1, A, true>(
      x, 0u, [&](int, uint32_t base, uint32_t s) { return ld16_uniform(tw, base | s); }, ar, lc);
}

template <int LOGN, bool INV, class A, class LOp>
__device__ __forceinline__ void column_pass(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                            const LimbConst& lc, const LOp& op, uint32_t part, uint64_t* lds_raw) {
  const ColumnMap<LOGN> m(part);
  const A ar(lc);
  typename A::V x[16];
  if constexpr (!INV) {
    if constexpr (LOp::kind == NTT_LOAD_ENC) {
      // every operand load in flight before the first residue
      typename LOp::Raw r[16];
      op.fetch16(src, [&](int k) { return m.j1(k); }, r);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = ar.load(op.finish(r[k]));
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = ar.load(op(src, m.j1(k)));
    }
    column_fwd_regs<LOGN, A, false, true>(x, dst, lc, m, ar, lds_raw);
  } else {
    column_inv_regs<LOGN>(x, dst, lc, m, ar, lds_raw);
    const GMut<uint64_t> gdst = gst(dst);
#pragma unroll
    for (int k = 0; k < 16; ++k) gdst[m.j1(k)] = ar.inv_store(x[k]);
  }
}

// ------------------------------------------------------------------ row pass
// The twiddles of a row-pass register pass on the P1 bits (stages CB - 1 down
// to CB - 4, or the inverse pass's 4 .. CB - 1) are shared by the 2^(CB-4)
// lanes of a row: a workgroup can load each of them once into LDS and let
// the lanes read them there. Entry e holds stage b = CB - 1 - s, with
// s = log2(e / 2^(10-CB) + 1); stage b's entries of part jbase / 1024 are
// those of index base | j in the twiddle table, base >= nj >> (b + 1).
template <int LOGN, class Tw>
struct RowStage {
  static constexpr int CB = Split<LOGN>::CB;
  Tw* tl;
  uint32_t nj;
  __device__ RowStage(Tw* t, uint32_t jbase) : tl(t), nj((1u << LOGN) | jbase) {}
  // entries t, t + STRIDE, ... below COUNT, by thread t of STRIDE
  template <int COUNT, int STRIDE>
  __device__ void fill(const GPtr<Tw>& tw, uint32_t t) const {
#pragma unroll
    for (int r = 0; r < (COUNT + STRIDE - 1) / STRIDE; ++r) {
      const uint32_t e = t + (uint32_t)STRIDE * r;
      if (e < (uint32_t)COUNT) {
        const uint32_t s = 31u - (uint32_t)__builtin_clz((e >> (10 - CB)) + 1);
        const uint32_t b = CB - 1 - s;
        tl[e] = ld16(tw, (nj >> (b + 1)) + e - (((1u << s) - 1) << (10 - CB)));
      }
    }
  }
  __device__ Tw operator()(int b, uint32_t base, uint32_t j) const {
    const int s = CB - 1 - b;
    return tl[(((1u << s) - 1) << (10 - CB)) + (base | j) - (nj >> (b + 1))];
  }
};

// Forward row pass of part `part` from the column pass's intermediate in buf;
// leaves the transform's outputs (the arithmetic's representation) in
// registers in the lane-contiguous layout G: x[k] is element part * 1024 +
// lane + 64 k.
template <int LOGN, class A>
__device__ __forceinline__ void row_fwd_regs(typename A::V (&x)[16], const uint64_t* buf, const LimbConst& lc,
                                             const A& ar, uint32_t part, uint64_t* lds_raw) {
  constexpr int CB = Split<LOGN>::CB, M = (1 << (CB - 4)) - 1;
  const uint32_t l = threadIdx.x & 63;
  const uint32_t jbase = part << 10;
  const uint32_t rowbits = (l >> (CB - 4)) << CB;
  auto p1 = [&](uint32_t k) { return (l & M) | (k << (CB - 4)) | rowbits; };
  auto p2 = [&](uint32_t k) { return k | ((l & M) << 4) | rowbits; };
  auto g = [&](uint32_t k) { return l + 64 * k; };
  typename A::V* lds = reinterpret_cast<typename A::V*>(lds_raw);
  const GPtr<uint64_t> gbuf = gld(buf);
  const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.fwd));
  const GPtr<typename A::Tw> tr = gld(reinterpret_cast<const typename A::Tw*>(lc.fwd_row));
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = ar.unraw(gbuf[jbase + p1(k)]);
  fwd_stages<LOGN, CB - 4, CB - 1, CB - 4>(x, jbase + p1(0), tw, ar);
  wave_exchange(x, lds, p1, p2);
  // the stages on the P2 register bits read the row table (one load of
  // consecutive entries per slot)
  fwd_stages_get<LOGN, 0, CB - 5, 0, A, true>(
      x, jbase + p2(0),
      [&](int b, uint32_t, uint32_t s) { return ld16(tr, row_table_index(Split<LOGN>::N, b, part, s, l)); }, ar);
  wave_exchange(x, lds, p2, g);
}

template <int LOGN, bool INV, class A, class LOp, class SOp>
__device__ __forceinline__ void row_pass(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                         const LimbConst& lc, const LOp& op, const SOp& so, uint32_t part,
                                         uint64_t* lds_raw) {
  using S = Split<LOGN>;
  constexpr int CB = S::CB, M = (1 << (CB - 4)) - 1;
  const uint32_t l = threadIdx.x;
  const uint32_t jbase = part << 10;
  const uint32_t rowbits = (l >> (CB - 4)) << CB;
  auto p1 = [&](uint32_t k) { return (l & M) | (k << (CB - 4)) | rowbits; };
  auto p2 = [&](uint32_t k) { return k | ((l & M) << 4) | rowbits; };
  auto g = [&](uint32_t k) { return l + 64 * k; };
  const A ar(lc);
  const GMut<uint64_t> gdst = gst(dst);
  typename A::V x[16];
  typename A::V* lds = reinterpret_cast<typename A::V*>(lds_raw);
  // the stages on the P2 register bits (bits 0..3, every lane its own
  // twiddles) read the row table, one load of consecutive entries per slot
  auto row_get = [&](const void* table) {
    const GPtr<typename A::Tw> tr = gld(reinterpret_cast<const typename A::Tw*>(table));
    return [=](int b, uint32_t, uint32_t s) { return ld16(tr, row_table_index(S::N, b, part, s, l)); };
  };
  if constexpr (!INV) {
    const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.fwd));
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = ar.unraw(gdst[jbase + p1(k)]);
    if constexpr (SOp::NAUX > 0) {
      // The store's operands and outputs in pairs of adjacent positions per
      // lane: register k is position h(k) = 2 lane + (k & 1) + 128 (k >> 1)
      // of the part, so they move as 16-byte accesses, half the memory
      // instructions of the lane-contiguous layout (this pass is bound by
      // the CUs' vector-memory address processing more than by its
      // arithmetic). The operands are requested after the first register
      // pass and combined after the exchange that follows it: held from the
      // start, they cost the kernel a wavefront per SIMD (156 VGPRs against
      // 127), which measured slower (106.3 against 104.1 us per token).
      auto h = [&](uint32_t k) { return (l << 1) + (k & 1) + ((k >> 1) << 7); };
      using U2 = uint64_t __attribute__((ext_vector_type(2)));
      typename SOp::Aux v[16];
      uint64_t c[16];
      // the first register pass's twiddles of stages CB - 1 .. CB - 3 staged
      // once per wavefront in LDS (those of stage CB - 4 are read from the
      // table: staging them too would cost a workgroup per CU)
      const RowStage<LOGN, typename A::Tw> st(reinterpret_cast<typename A::Tw*>(lds_raw + S::LDS), jbase);
      st.template fill<S::TW1S, 64>(tw, l);
      slice_sync();
      fwd_stages_get<LOGN, CB - 4, CB - 1, CB - 4, A, true>(
          x, jbase + p1(0),
          [&](int b, uint32_t base, uint32_t j) { return b >= CB - 3 ? st(b, base, j) : ld16(tw, base | j); }, ar);
#pragma unroll
      for (int k = 0; k < 16; k += 2) {
        const U2 a = ((GPtr<U2>)gld(so.aux))[(jbase + h(k)) >> 1];
        v[k].a = a.x;
        v[k + 1].a = a.y;
        if constexpr (SOp::NAUX >= 2) {
          const U2 b = ((GPtr<U2>)gld(so.aux2))[(jbase + h(k)) >> 1];
          v[k].b = b.x;
          v[k + 1].b = b.y;
        }
      }
      wave_exchange(x, lds, p1, p2);
#pragma unroll
      for (int k = 0; k < 16; ++k) c[k] = so.prep(ar, v[k]);
      fwd_stages_get<LOGN, 0, CB - 5, 0, A, true>(x, jbase + p2(0), row_get(lc.fwd_row), ar);
      wave_exchange(x, lds, p2, h);
      const GMut<U2> d2 = (GMut<U2>)gdst;
#pragma unroll
      for (int k = 0; k < 16; k += 2) {
        U2 o;
        o.x = so.apply_prep(ar, x[k], c[k]);
        o.y = so.apply_prep(ar, x[k + 1], c[k + 1]);
        d2[(jbase + h(k)) >> 1] = o;
      }
    } else {
      fwd_stages<LOGN, CB - 4, CB - 1, CB - 4, A, false>(x, jbase + p1(0), tw, ar);
      wave_exchange(x, lds, p1, p2);
      fwd_stages_get<LOGN, 0, CB - 5, 0, A, false>(x, jbase + p2(0), row_get(lc.fwd_row), ar);
      wave_exchange(x, lds, p2, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) so.store(ar, x[k], gdst, jbase + g(k), 0);
    }
  } else {
    const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.inv));
    if constexpr (LOp::kind == NTT_LOAD_MULM) {
      // The product's operands in pairs of adjacent positions per lane (the
      // layout h of the forward pass with a fused store: 16-byte loads, half
      // the memory instructions), all in flight before the first product.
      auto h = [&](uint32_t k) { return (l << 1) + (k & 1) + ((k >> 1) << 7); };
      using U2 = uint64_t __attribute__((ext_vector_type(2)));
      const GPtr<U2> s2 = (const GPtr<U2>)gld(src), a2 = (const GPtr<U2>)gld(op.aux);
      typename LOp::Raw r[16];
#pragma unroll
      for (int k = 0; k < 16; k += 2) {
        const U2 s = s2[(jbase + h(k)) >> 1], a = a2[(jbase + h(k)) >> 1];
        r[k] = typename LOp::Raw{s.x, a.x};
        r[k + 1] = typename LOp::Raw{s.y, a.y};
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = ar.load(op.finish(r[k]));
      // the second register pass's twiddles (stages 4 .. CB - 1) staged once
      // per wavefront in LDS; the exchanges' barriers order the staging
      const RowStage<LOGN, typename A::Tw> st(reinterpret_cast<typename A::Tw*>(lds_raw + S::LDS), jbase);
      st.template fill<S::TWI, 64>(tw, l);
      wave_exchange(x, lds, h, p2);
      inv_stages_get<LOGN, 0, 0, 3, A, true>(x, jbase + p2(0), row_get(lc.inv_row), ar, lc);
      wave_exchange(x, lds, p2, p1);
      inv_stages_get<LOGN, CB - 4, 4, CB - 1, A, true>(x, jbase + p1(0), st, ar, lc);
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = ar.load(op(src, jbase + g(k)));
      wave_exchange(x, lds, g, p2);
      inv_stages_get<LOGN, 0, 0, 3, A, true>(x, jbase + p2(0), row_get(lc.inv_row), ar, lc);
      wave_exchange(x, lds, p2, p1);
      inv_stages<LOGN, CB - 4, 4, CB - 1>(x, jbase + p1(0), tw, ar, lc);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) gdst[jbase + p1(k)] = ar.raw(x[k]);
  }
}

// ------------------------------------------------------------------ kernels
// Column-pass part of workgroup part id p: 8-column parts share 128-byte lines
// in pairs; ids i and i + 8 run on one XCD (ids are dealt round-robin over the
// 8 XCDs), so they get the column parts 2m and 2m + 1.
template <int LOGN>
__device__ __forceinline__ uint32_t column_part(uint32_t p) {
  using S = Split<LOGN>;
  if constexpr (S::CW < 16) {
    static_assert(S::CW == 8 && S::PARTS % 16 == 0, "column-part pairing needs 8 columns and 16 | PARTS");
    return (p & ~15u) | ((p & 7u) << 1) | ((p >> 3) & 1u);
  } else {
    return p;
  }
}

// Workgroup b works on part b % PARTS of job b / PARTS. The pass that reads
// the transform's input applies the fused load operation and the forward
// row pass the fused store operation; otherwise passes read and write the
// destination only.
template <int LOGN, bool INV, bool COLUMN, uint32_t LD, uint32_t ST>
__global__ __launch_bounds__(64) void ntt_split_kernel(NttArgs a) {
  using S = Split<LOGN>;
  // the forward row pass with a fused rescale store, and the inverse row pass
  // with the product in its loads, also hold one register pass's twiddles
  // (16-byte entries); the forward column passes exchange through half the
  // LDS (their occupancy is then set by their registers: 20 or 24 wavefronts
  // per CU instead of 18)
  __shared__ uint64_t lds[!INV && COLUMN ? S::LDS / 2
                          : S::LDS + (!INV && StoreOp<ST>::NAUX > 0 ? 2 * S::TW1S
                                      : INV && LD == NTT_LOAD_MULM  ? 2 * S::TWI
                                                                    : 0)];
  const uint32_t job = blockIdx.x / S::PARTS;
  uint32_t part = blockIdx.x % S::PARTS;
  if constexpr (COLUMN) part = column_part<LOGN>(part);
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
    job_ops(a, jb, limb, S::N, op, so);
  } else {
    src = a.src + (uint64_t)job * a.stride;
    dst = a.dst + (uint64_t)job * a.stride;
    limb = a.limb_base + job % a.limb_mod;
  }
  const LimbConst& lc = a.lc[limb];
  if constexpr (COLUMN) {
    if (lc.fp64)
      column_pass<LOGN, INV, Fp64Arith>(src, dst, lc, op, part, lds);
    else
      column_pass<LOGN, INV, IntArith>(src, dst, lc, op, part, lds);
  } else {
    if (lc.fp64)
      row_pass<LOGN, INV, Fp64Arith>(src, dst, lc, op, so, part, lds);
    else
      row_pass<LOGN, INV, IntArith>(src, dst, lc, op, so, part, lds);
  }
}

// Rescale column kernel: the column pass that ends the inverse transform of a
// product's last limb, fused with the column passes that begin the forward
// transforms of that limb reduced modulo each lower limb (the evaluation-
// domain rescale), so the coefficient-domain last limb stays in registers.
// Inverse job i (its dst holds the inverse row pass's intermediate) owns
// forward jobs i * nf .. i * nf + nf - 1, the order in which the rescale lists
// them; each forward job's dst receives its column-pass intermediate, where
// the forward row pass continues (with the rescale's store operation).
// With fan (batches too small to fill the GPU), nf workgroups per inverse
// job and part each repeat the inverse column pass and run one of the
// forward passes (workgroup b: part b % PARTS of forward job b / PARTS), so
// the launch takes one inverse and one forward pass instead of the inverse
// and nf forward passes in turn.
template <int LOGN>
__global__ __launch_bounds__(64) void rescale_column_kernel(NttArgs inv, NttArgs fwd, uint32_t nf, uint32_t fan) {
  using S = Split<LOGN>;
  __shared__ uint64_t lds[S::LDS];
  const uint32_t unit = blockIdx.x / S::PARTS;  // inverse job, or forward job with fan
  const uint32_t job = fan ? unit / nf : unit;
  const uint32_t f0 = fan ? unit % nf : 0, f1 = fan ? f0 + 1 : nf;
  const ColumnMap<LOGN> m(column_part<LOGN>(blockIdx.x % S::PARTS));
  const NttJob ij = inv.jobs[job];
  const LimbConst& lci = inv.lc[ij.limb];
  uint64_t c[16];  // canonical last-limb coefficients of this wavefront's columns (Q1)
  if (lci.fp64) {
    const Fp64Arith ar(lci);
    Fp64Arith::V x[16];
    column_inv_regs<LOGN>(x, ij.dst, lci, m, ar, lds);
#pragma unroll
    for (int k = 0; k < 16; ++k) c[k] = ar.inv_store(x[k]);
  } else {
    const IntArith ar(lci);
    IntArith::V x[16];
    column_inv_regs<LOGN>(x, ij.dst, lci, m, ar, lds);
#pragma unroll
    for (int k = 0; k < 16; ++k) c[k] = ar.inv_store(x[k]);
  }
  // c mod q_l: FP64 on limbs below 2^41, else Barrett when c >= q_l
  for (uint32_t f = f0; f < f1; ++f) {
    const NttJob fj = fwd.jobs[(uint64_t)job * nf + f];
    const LimbConst& lcf = fwd.lc[fj.limb];
    const RescaleConst rc = fwd.rc[fj.limb];
    // c is the same at every iteration; hiding that keeps the compiler from
    // hoisting per-coefficient terms out of the loop into extra registers
#pragma unroll
    for (int k = 0; k < 16; ++k) c[k] = opaque_u64(c[k]);
    if (lcf.fp64) {
      const Fp64Arith ar(lcf);
      Fp64Arith::V x[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = reduce_u64_f64(c[k], rc);
      column_fwd_regs<LOGN, Fp64Arith, true>(x, fj.dst, lcf, m, ar, lds);
    } else {
      const IntArith ar(lcf);
      IntArith::V x[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = c[k] < rc.q ? c[k] : mulmod_barrett(c[k], 1, rc.b);
      column_fwd_regs<LOGN, IntArith, true>(x, fj.dst, lcf, m, ar, lds);
    }
  }
}

// Largest fanned-out rescale column launch: one round of that kernel's
// wavefronts (3 per SIMD at its registers, 1024 SIMDs).
constexpr uint32_t RESCALE_FAN_MAX_WAVES = 3072;

template <int LOGN>
static hipError_t launch_rescale_t(const NttArgs& inv, uint32_t ninv, const NttArgs& fwd, uint32_t nf, hipStream_t s) {
  using S = Split<LOGN>;
  const dim3 block(64);
  const hipError_t e = with_ops<true>(inv.load, inv.store, [&]<uint32_t LD, uint32_t ST>() -> hipError_t {
    if constexpr (ST != NTT_STORE_NONE) return hipErrorInvalidValue;  // segment sums: whole kernel only
    hipLaunchKernelGGL((ntt_split_kernel<LOGN, true, false, LD, NTT_STORE_NONE>), dim3(ninv * S::PARTS), block, 0, s,
                       inv);
    return hipGetLastError();
  });
  if (e != hipSuccess) return e;
  // a batch whose nf passes per inverse job would leave most SIMDs idle
  // fans them out (RESCALE_FAN_MAX_WAVES)
  const uint32_t fan = ninv * nf * S::PARTS <= RESCALE_FAN_MAX_WAVES ? 1u : 0u;
  hipLaunchKernelGGL((rescale_column_kernel<LOGN>), dim3(ninv * S::PARTS * (fan ? nf : 1)), block, 0, s, inv, fwd, nf,
                     fan);
  const hipError_t e2 = hipGetLastError();
  if (e2 != hipSuccess) return e2;
  return with_ops<false>(fwd.load, fwd.store, [&]<uint32_t LD, uint32_t ST>() -> hipError_t {
    hipLaunchKernelGGL((ntt_split_kernel<LOGN, false, false, NTT_LOAD_NONE, ST>), dim3(ninv * nf * S::PARTS), block, 0,
                       s, fwd);
    return hipGetLastError();
  });
}

hipError_t launch_rescale_split(int logn, const NttArgs& inv, uint32_t ninv, const NttArgs& fwd, uint32_t nf,
                                hipStream_t s) {
  switch (logn) {
    case 13: return launch_rescale_t<13>(inv, ninv, fwd, nf, s);
    case 14: return launch_rescale_t<14>(inv, ninv, fwd, nf, s);
    case 15: return launch_rescale_t<15>(inv, ninv, fwd, nf, s);
    default: return hipErrorInvalidValue;
  }
}

// Encrypt row kernel: the forward row passes of one input's M_l, U_l and E1_l
// (their column passes, with the residues formed in the loads, have left the
// intermediates in the jobs' dst), combined as they are stored into
//   c0_l = b_l * U_l + M_l,  c1_l = a_l * U_l + E1_l   (ciphertext.rs:298-312)
// so the three transforms are never written out. Workgroup w works on part
// w % PARTS of input / limb w / PARTS with three wavefronts, one per
// transform (0: M, 1: U, 2: E1), each with its own LDS slice; U's wavefront
// hands its canonical outputs to the other two through LDS, which form and
// store c0 and c1. The limbs are those in mask (n of them); jobs: 3n per
// input (M, E1 and U of each of those limbs in increasing order);
// pkp = [b (L) | a (L)] as prepared pairs (w, companion), so each product is
// one Shoup or FP64 step; input i's ciphertext at cts + i 2 L N. On the limbs
// in dot.mask the kernel stores D = c0 + c1 s instead (EncDot): M's and E1's
// wavefronts each hand the other half of their outputs over through LDS and
// form D on their own half.
template <int LOGN>
__global__ __launch_bounds__(192) void encrypt_row_kernel(NttArgs a, const uint64_t* pkp, uint64_t* cts, uint32_t L,
                                                          uint32_t mask, EncDot dot) {
  using S = Split<LOGN>;
  __shared__ uint64_t lds[3][S::LDS];
  const uint32_t nl = (uint32_t)__builtin_popcount(mask);
  const uint32_t part = blockIdx.x % S::PARTS, il = blockIdx.x / S::PARTS;
  const uint32_t i = il / nl, kl = il % nl;
  uint32_t rest = mask;  // the kl-th set bit of mask is the limb
  for (uint32_t j = 0; j < kl; ++j) rest &= rest - 1;
  const uint32_t l = (uint32_t)__builtin_ctz(rest);
  const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const NttJob* jb = a.jobs + (size_t)i * 3 * nl;
  const uint32_t job = wv == 0 ? kl : (wv == 1 ? 2 * nl + kl : nl + kl);
  const LimbConst& lc = a.lc[l];
  const BarrettConst bc = a.bc[l];
  const size_t off = (size_t)l * S::N + ((size_t)part << 10) + lane;
  uint64_t* shared_u = lds[1];
  const bool form_d = (dot.mask >> l) & 1;  // uniform over the workgroup
  auto run = [&]<class A>() {
    const A ar(lc);
    typename A::V x[16];
    row_fwd_regs<LOGN>(x, jb[job].dst, lc, ar, part, lds[wv]);
    // the key pairs are requested before the barrier, so their latency
    // overlaps U's hand-over
    ShoupTw kp[16];
    if (wv != 1) {
      const GPtr<ShoupTw> key = gld(reinterpret_cast<const ShoupTw*>(pkp) + (wv == 0 ? 0 : (size_t)L * S::N) + off);
#pragma unroll
      for (int k = 0; k < 16; ++k) kp[k] = ld16(key, 64 * k);
    }
    if (wv == 1) {
#pragma unroll
      for (int k = 0; k < 16; ++k) shared_u[lane + 64 * k] = ar.fwd_store(x[k]);
    }
    __syncthreads();
    uint64_t c[16];  // M's and E1's wavefronts keep c0, c1 where D is formed
    if (wv != 1) {
      const GMut<uint64_t> out = gst(cts + (size_t)i * 2 * L * S::N + (wv == 0 ? 0 : (size_t)L * S::N)) + off;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const uint64_t u = shared_u[lane + 64 * k], m = ar.fwd_store(x[k]);
        const ShoupTw p = kp[k];
        uint64_t r;
        if constexpr (std::is_same_v<A, Fp64Arith>) {
          // (-q/2, q/2) + [0, q)
          double t = mulmod_f64(u64_to_f64(u), u64_to_f64(p.w), __builtin_bit_cast(double, p.ws), lc.qd) +
                     u64_to_f64(m);
          t = t < 0.0 ? t + lc.qd : t;
          r = f64_to_u64(t >= lc.qd ? t - lc.qd : t);
        } else {
          r = shoup_approx(u, p.w, p.ws, bc.q) + m;  // [0, 5q)
          r = csub(csub(csub(r, 4 * bc.q), 2 * bc.q), bc.q);
        }
        if (!form_d) {
          out[64 * k] = r;
        } else {
          // M's wavefront forms D on elements 0..7 and hands c0 of 8..15 to
          // E1's, which forms D on 8..15 (its own slice, free once its passes
          // are done, holds the exchange)
          c[k] = r;
          if ((wv == 0) == (k >= 8)) lds[2][lane + 64 * k] = r;
        }
      }
    }
    if (form_d) {
      // D = c0 + c1 s in [0, 3q) (the key in Montgomery form), at input i's
      // slot for this limb: the position of l among dot.mask's limbs
      const uint32_t kd = (uint32_t)__builtin_popcount(dot.mask & ((1u << l) - 1));
      const uint32_t nd = (uint32_t)__builtin_popcount(dot.mask);
      const GPtr<uint64_t> key = gld(dot.skm) + off;
      const GMut<uint64_t> dst = gst(dot.out) + ((size_t)i * nd + kd) * S::N + ((size_t)part << 10) + lane;
      uint64_t sv[8];
      const int k0 = wv == 0 ? 0 : 8;
      if (wv != 1) {
#pragma unroll
        for (int k = 0; k < 8; ++k) sv[k] = key[64 * (k0 + k)];
      }
      __syncthreads();
      if (wv == 0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) dst[64 * k] = c[k] + mont_mul(lds[2][lane + 64 * k], sv[k], bc);
      } else if (wv == 2) {
#pragma unroll
        for (int k = 0; k < 8; ++k) dst[64 * (8 + k)] = lds[2][lane + 64 * (8 + k)] + mont_mul(c[8 + k], sv[k], bc);
      }
    }
  };
  if (lc.fp64)
    run.template operator()<Fp64Arith>();
  else
    run.template operator()<IntArith>();
}

template <int LOGN>
static hipError_t launch_encrypt_t(const NttArgs& a, uint32_t ninputs, uint32_t L, uint32_t mask, const EncDot& dot,
                                   const uint64_t* pkp, uint64_t* cts, hipStream_t s) {
  using S = Split<LOGN>;
  const uint32_t nl = (uint32_t)__builtin_popcount(mask);
  hipLaunchKernelGGL((ntt_split_kernel<LOGN, false, true, NTT_LOAD_ENC, NTT_STORE_NONE>),
                     dim3(ninputs * 3 * nl * S::PARTS), dim3(64), 0, s, a);
  hipLaunchKernelGGL((encrypt_row_kernel<LOGN>), dim3(ninputs * nl * S::PARTS), dim3(192), 0, s, a, pkp, cts, L,
                     mask, dot);
  return hipGetLastError();
}

hipError_t launch_encrypt_split(int logn, const NttArgs& a, uint32_t ninputs, uint32_t L, uint32_t limb_mask,
                                const EncDot& dot, const uint64_t* pkp, uint64_t* cts, hipStream_t s) {
  switch (logn) {
    case 13: return launch_encrypt_t<13>(a, ninputs, L, limb_mask, dot, pkp, cts, s);
    case 14: return launch_encrypt_t<14>(a, ninputs, L, limb_mask, dot, pkp, cts, s);
    case 15: return launch_encrypt_t<15>(a, ninputs, L, limb_mask, dot, pkp, cts, s);
    default: return hipErrorInvalidValue;
  }
}

// The pass that reads the transform's input (column pass forward, row pass
// inverse) carries the load operation, the forward row pass the store
// operation; the other pass is instantiated with none.
template <int LOGN, bool INV>
static hipError_t launch_split_t(const NttArgs& a, uint32_t njobs, hipStream_t s) {
  using S = Split<LOGN>;
  const dim3 grid(njobs * S::PARTS), block(64);
  return with_ops<INV>(a.jobs ? a.load : NTT_LOAD_NONE, a.jobs ? a.store : NTT_STORE_NONE,
                       [&]<uint32_t LD, uint32_t ST>() -> hipError_t {
                         if constexpr (ST == NTT_STORE_SEGSUM) return hipErrorInvalidValue;  // whole kernel only
                         if constexpr (!INV) {
                           hipLaunchKernelGGL((ntt_split_kernel<LOGN, false, true, LD, NTT_STORE_NONE>), grid, block,
                                              0, s, a);
                           hipLaunchKernelGGL((ntt_split_kernel<LOGN, false, false, NTT_LOAD_NONE, ST>), grid, block,
                                              0, s, a);
                         } else {
                           hipLaunchKernelGGL((ntt_split_kernel<LOGN, true, false, LD, NTT_STORE_NONE>), grid, block,
                                              0, s, a);
                           hipLaunchKernelGGL((ntt_split_kernel<LOGN, true, true, NTT_LOAD_NONE, NTT_STORE_NONE>), grid,
                                              block, 0, s, a);
                         }
                         return hipGetLastError();
                       });
}

hipError_t launch_ntt_split(int logn, bool inverse, const NttArgs& a, uint32_t njobs, hipStream_t s) {
  switch (logn) {
    case 13: return inverse ? launch_split_t<13, true>(a, njobs, s) : launch_split_t<13, false>(a, njobs, s);
    case 14: return inverse ? launch_split_t<14, true>(a, njobs, s) : launch_split_t<14, false>(a, njobs, s);
    case 15: return inverse ? launch_split_t<15, true>(a, njobs, s) : launch_split_t<15, false>(a, njobs, s);
    default: return hipErrorInvalidValue;
  }
}

// ------------------------------------------------------------------ rescale-decrypt, split sizes
// The rescale and decryption of a LoRA set's products on limb 0 (the
// algebra of rescale_decrypt_kernel, ntt.hip) in four launches of
// single-wavefront workgroups, for sizes and batch counts the
// whole-polynomial kernel does not serve. Per batch, with X, Y the last limb
// of c0 pt, c1 pt:
//   1. inverse row passes of X and Y with ct x pt in the loads
//      (ntt_split_kernel, NTT_LOAD_MULM);
//   2. rd_column_kernel: inverse column passes; X's canonical coefficients
//      are reduced mod q0 (r0) and written in place, Y's reduced mod q0 and
//      carried through the forward column pass at q0;
//   3. rd_row_kernel: forward row pass of r1, D pt - NTT(r1) s in
//      registers, inverse row pass (the same 1024 coefficients of a row);
//   4. rd_column_sums_kernel: inverse column pass, (m - r0) inv mod q0,
//      centred, and each lane's partial segment sums;
//   5. rd_sums_final_kernel: the partial sums of each batch added up.
// Lane l of column part p holds coefficients t + k 2^(LOGN-4), k = 0..15,
// with t = (row << CB) | col (ColumnMap, Q1), the elements thread t holds
// in the whole-polynomial kernel's epilogue at N = 16384; its partial sums
// run over k in the same order, and step 5 adds them as that epilogue does
// (a butterfly tree over 64 consecutive t, then the trees in order), so the
// sums are bit-identical to rescale_decrypt_kernel's.

// Step 2. Workgroup w: part w % PARTS of inverse job w / PARTS (jobs 2b, 2b+1
// = X, Y of batch b; their dst holds step 1's intermediate).
template <int LOGN>
__global__ __launch_bounds__(64) void rd_column_kernel(NttArgs inv, const RescaleConst* __restrict__ rc0,
                                                       const LimbConst* __restrict__ lc0p) {
  using S = Split<LOGN>;
  __shared__ uint64_t lds[S::LDS];
  const uint32_t job = blockIdx.x / S::PARTS;
  const ColumnMap<LOGN> m(column_part<LOGN>(blockIdx.x % S::PARTS));
  const NttJob ij = inv.jobs[job];
  const LimbConst& lci = inv.lc[ij.limb];
  const RescaleConst rc = *rc0;
  uint64_t c[16];  // the last limb's canonical coefficients, then reduced mod q0
  if (lci.fp64) {
    const Fp64Arith ar(lci);
    Fp64Arith::V x[16];
    column_inv_regs<LOGN>(x, ij.dst, lci, m, ar, lds);
#pragma unroll
    for (int k = 0; k < 16; ++k) c[k] = ar.inv_store(x[k]);
  } else {
    const IntArith ar(lci);
    IntArith::V x[16];
    column_inv_regs<LOGN>(x, ij.dst, lci, m, ar, lds);
#pragma unroll
    for (int k = 0; k < 16; ++k) c[k] = ar.inv_store(x[k]);
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) c[k] = c[k] < rc.q ? c[k] : mulmod_barrett(c[k], 1, rc.b);
  if ((job & 1) == 0) {
    const GMut<uint64_t> out = gst(ij.dst);
#pragma unroll
    for (int k = 0; k < 16; ++k) out[m.j1(k)] = c[k];  // r0, natural order
    return;
  }
  const LimbConst& lc0 = *lc0p;
  if (lc0.fp64) {
    const Fp64Arith ar(lc0);
    Fp64Arith::V x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = ar.load(c[k]);
    column_fwd_regs<LOGN, Fp64Arith, true>(x, ij.dst, lc0, m, ar, lds);
  } else {
    const IntArith ar(lc0);
    IntArith::V x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = ar.load(c[k]);
    column_fwd_regs<LOGN, IntArith, true>(x, ij.dst, lc0, m, ar, lds);
  }
}

// Step 3. Workgroup w: part w % PARTS of batch w / PARTS (RescaleDecryptJob:
// y holds step 2's forward column intermediate; rewritten in place with the
// inverse row pass's intermediate of D pt - NTT(r1) s).
template <int LOGN>
__global__ __launch_bounds__(64) void rd_row_kernel(RescaleDecryptArgs a) {
  using S = Split<LOGN>;
  constexpr int CB = S::CB, M = (1 << (CB - 4)) - 1;
  __shared__ uint64_t lds_raw[S::LDS];
  const RescaleDecryptJob jb = a.jobs[blockIdx.x / S::PARTS];
  const uint32_t part = blockIdx.x % S::PARTS;
  const LimbConst& lc = a.lc[0];
  const BarrettConst bc = *a.bc;
  const uint32_t l = threadIdx.x;
  const uint32_t jbase = part << 10;
  const uint32_t rowbits = (l >> (CB - 4)) << CB;
  auto p1 = [&](uint32_t k) { return (l & M) | (k << (CB - 4)) | rowbits; };
  auto p2 = [&](uint32_t k) { return k | ((l & M) << 4) | rowbits; };
  auto g = [&](uint32_t k) { return l + 64 * k; };
  auto run = [&]<class A>() {
    const A ar(lc);
    typename A::V x[16];
    typename A::V* lds = reinterpret_cast<typename A::V*>(lds_raw);
    row_fwd_regs<LOGN>(x, jb.y, lc, ar, part, lds_raw);
    {
      // D pt - NTT(r1) s at positions jbase + g(k): Montgomery products, each
      // in [0, 2q), so the difference plus 2q is in (0, 4q), the integer
      // inverse's input range; the FP64 inverse gets it canonical
      const GPtr<uint64_t> d = gld(jb.d), p = gld(jb.ptm), sk = gld(a.skm);
      const uint64_t q = lc.q, two_q = 2 * lc.q;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const uint32_t i = jbase + g(k);
        const uint64_t u = mont_mul(d[i], p[i], bc);
        const uint64_t t = mont_mul(ar.fwd_store(x[k]), sk[i], bc);
        uint64_t e = u + two_q - t;
        if constexpr (std::is_same_v<A, Fp64Arith>) e = csub(csub(e, two_q), q);
        x[k] = ar.load(e);
      }
    }
    const GPtr<typename A::Tw> tw = gld(reinterpret_cast<const typename A::Tw*>(lc.inv));
    const GPtr<typename A::Tw> tr = gld(reinterpret_cast<const typename A::Tw*>(lc.inv_row));
    wave_exchange(x, lds, g, p2);
    inv_stages_get<LOGN, 0, 0, 3, A, true>(
        x, jbase + p2(0), [&](int b, uint32_t, uint32_t s) { return ld16(tr, row_table_index(S::N, b, part, s, l)); },
        ar, lc);
    wave_exchange(x, lds, p2, p1);
    inv_stages<LOGN, CB - 4, 4, CB - 1>(x, jbase + p1(0), tw, ar, lc);
    const GMut<uint64_t> out = gst(const_cast<uint64_t*>(jb.y));
#pragma unroll
    for (int k = 0; k < 16; ++k) out[jbase + p1(k)] = ar.raw(x[k]);
  };
  if (lc.fp64)
    run.template operator()<Fp64Arith>();
  else
    run.template operator()<IntArith>();
}

// Step 4. Workgroup w: column part w % PARTS of batch w / PARTS; writes
// lane t's sums for segments c < cols at partials + (b cols + c) T + t,
// T = 2^(LOGN-4). Without RESCALED (a plain decryption, launch_decrypt_sums_split)
// the decrypted coefficient is the transform's output itself.
template <int LOGN, bool RESCALED = true>
__global__ __launch_bounds__(64) void rd_column_sums_kernel(RescaleDecryptArgs a, double* __restrict__ partials) {
  using S = Split<LOGN>;
  constexpr int MAXC = NTT_SEGSUM_FUSED_MAX_COLS;
  constexpr uint32_t T = 1u << (LOGN - 4);
  __shared__ uint64_t lds[S::LDS];
  const uint32_t b = blockIdx.x / S::PARTS;
  const RescaleDecryptJob jb = a.jobs[b];
  const ColumnMap<LOGN> m(column_part<LOGN>(blockIdx.x % S::PARTS));
  const LimbConst& lc = a.lc[0];
  const RescaleConst rc = RESCALED ? *a.rc : RescaleConst{};
  const uint64_t q = lc.q, half = q >> 1;
  uint64_t mv[16];
  if (lc.fp64) {
    const Fp64Arith ar(lc);
    Fp64Arith::V x[16];
    column_inv_regs<LOGN>(x, jb.y, lc, m, ar, lds);
#pragma unroll
    for (int k = 0; k < 16; ++k) mv[k] = ar.inv_store(x[k]);
  } else {
    const IntArith ar(lc);
    IntArith::V x[16];
    column_inv_regs<LOGN>(x, jb.y, lc, m, ar, lds);
#pragma unroll
    for (int k = 0; k < 16; ++k) mv[k] = ar.inv_store(x[k]);
  }
  using D2 = double __attribute__((ext_vector_type(2)));
  const GPtr<D2> W = gld(reinterpret_cast<const D2*>(a.segw));
  const GPtr<uint64_t> r0 = gld(RESCALED ? jb.x : jb.y);
  double acc[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) acc[c] = 0.0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t j = m.j1(k);
    const uint64_t v0 = RESCALED ? csub(shoup_lazy(submod(mv[k], r0[j], q), rc.inv, rc.inv_s, q), q) : mv[k];
    const double v = v0 > half ? -(double)(q - v0) : (double)v0;
    const D2 p = W[j];  // W_0[j], 2 cos(2 phi_j)
    double wp = p.x, wc = p.x;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      if (c >= (int)a.cols) break;
      acc[c] += v * wc;
      const double wn = p.y * wc - wp;
      wp = wc;
      wc = wn;
    }
  }
  const uint32_t t = m.j1(0);  // < T
  const GMut<double> out = gst(partials) + (size_t)b * a.cols * T + t;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    if (c >= (int)a.cols) break;
    out[(size_t)c * T] = acc[c];
  }
}

// Step 5. One wavefront per batch and segment: the sum over groups of 64
// consecutive lanes t by a butterfly tree, the groups added in order (every
// group's values requested first, the trees independent of one another).
template <int LOGN>
__global__ __launch_bounds__(64) void rd_sums_final_kernel(RescaleDecryptArgs a, const double* __restrict__ partials) {
  constexpr uint32_t T = 1u << (LOGN - 4), G = T / 64;
  const uint32_t b = blockIdx.x / a.cols, c = blockIdx.x % a.cols, lane = threadIdx.x;
  const RescaleDecryptJob jb = a.jobs[b];
  const GPtr<double> in = gld(partials) + ((size_t)b * a.cols + c) * T + lane;
  double v[G];
#pragma unroll
  for (uint32_t w = 0; w < G; ++w) v[w] = in[w * 64];
#pragma unroll
  for (uint32_t w = 0; w < G; ++w)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v[w] += __shfl_xor(v[w], off);
  double t = 0.0;
#pragma unroll
  for (uint32_t w = 0; w < G; ++w) t += v[w];
  if (lane == 0) gst(jb.seg)[c] = t / jb.scale;
}

template <int LOGN>
static hipError_t launch_rd_split_t(const NttArgs& inv, const RescaleDecryptArgs& a, uint32_t nb, double* partials,
                                    hipStream_t s) {
  using S = Split<LOGN>;
  const dim3 block(64);
  hipLaunchKernelGGL((ntt_split_kernel<LOGN, true, false, NTT_LOAD_MULM, NTT_STORE_NONE>), dim3(2 * nb * S::PARTS),
                     block, 0, s, inv);
  hipLaunchKernelGGL((rd_column_kernel<LOGN>), dim3(2 * nb * S::PARTS), block, 0, s, inv, a.rc, a.lc);
  hipLaunchKernelGGL((rd_row_kernel<LOGN>), dim3(nb * S::PARTS), block, 0, s, a);
  hipLaunchKernelGGL((rd_column_sums_kernel<LOGN>), dim3(nb * S::PARTS), block, 0, s, a, partials);
  hipLaunchKernelGGL((rd_sums_final_kernel<LOGN>), dim3(nb * a.cols), block, 0, s, a, (const double*)partials);
  return hipGetLastError();
}

// A plain batched decryption with segment sums on the split kernels: the
// inverse row pass of c0 + c1 s (row: NTT_LOAD_DOTM jobs on limb 0, one per
// batch, dst = the batch's y), then steps 4 and 5 without the rescale.
template <int LOGN>
static hipError_t launch_dec_split_t(const NttArgs& row, const RescaleDecryptArgs& a, uint32_t nb, double* partials,
                                     hipStream_t s) {
  using S = Split<LOGN>;
  const dim3 block(64);
  hipLaunchKernelGGL((ntt_split_kernel<LOGN, true, false, NTT_LOAD_DOTM, NTT_STORE_NONE>), dim3(nb * S::PARTS), block,
                     0, s, row);
  hipLaunchKernelGGL((rd_column_sums_kernel<LOGN, false>), dim3(nb * S::PARTS), block, 0, s, a, partials);
  hipLaunchKernelGGL((rd_sums_final_kernel<LOGN>), dim3(nb * a.cols), block, 0, s, a, (const double*)partials);
  return hipGetLastError();
}

hipError_t launch_decrypt_sums_split(int logn, const NttArgs& row, const RescaleDecryptArgs& a, uint32_t nb,
                                     double* partials, hipStream_t s) {
  if (nb == 0) return hipSuccess;
  if (!row.jobs || row.load != NTT_LOAD_DOTM || a.cols < 1 || a.cols > NTT_SEGSUM_FUSED_MAX_COLS)
    return hipErrorInvalidValue;
  switch (logn) {
    case 13: return launch_dec_split_t<13>(row, a, nb, partials, s);
    case 14: return launch_dec_split_t<14>(row, a, nb, partials, s);
    case 15: return launch_dec_split_t<15>(row, a, nb, partials, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rescale_decrypt_split(int logn, const NttArgs& inv, const RescaleDecryptArgs& a, uint32_t nb,
                                        double* partials, hipStream_t s) {
  if (nb == 0) return hipSuccess;
  if (!inv.jobs || inv.load != NTT_LOAD_MULM || a.cols < 1 || a.cols > NTT_SEGSUM_FUSED_MAX_COLS)
    return hipErrorInvalidValue;
  switch (logn) {
    case 13: return launch_rd_split_t<13>(inv, a, nb, partials, s);
    case 14: return launch_rd_split_t<14>(inv, a, nb, partials, s);
    case 15: return launch_rd_split_t<15>(inv, a, nb, partials, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace th
