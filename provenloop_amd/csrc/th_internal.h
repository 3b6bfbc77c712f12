// Host-side declarations shared between the host runtime (runtime.h and its
// translation units) and the kernel translation units. Not part of the public
// C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <atomic>
#include <stdint.h>

#include "th_device.h"

namespace th {

// Operation applied to every coefficient as an NTT loads it (fused producer
// of the transform's input; the result is what gets transformed):
//   NONE     x = src[i]
//   MUL      x = src[i] * aux[i] mod q                    (ct x pt, ciphertext.rs:422-429)
//   REDUCE   x = src[i] mod q for any src[i] < 2^61       (a last-limb coefficient
//                                                         taken to limb q: rescale)
//   DOT      x = src[i] + aux[i] * key[i] mod q, src = c0, aux = c1, key = s
//                                                         (decrypt, ciphertext.rs:332-341)
//   ENC      the encrypt_pk inputs' residues (ciphertext.rs:256-296), by the job's sub:
//            0: x = (m + e0) mod q, src = m, aux = e0 (i64 coefficients)
//            1: x = e1 mod q, src = e1 (i64)
//            2: x = u mapped 0 -> q-1, 1 -> 0, 2 -> 1, src = u (u8)
//   MULM     MUL with aux in Montgomery form (launch_to_montgomery); x in [0, 2q)
//   DOTM     DOT with the key in Montgomery form; x in [0, 3q)
enum NttLoad : uint32_t {
  NTT_LOAD_NONE = 0,
  NTT_LOAD_MUL = 1,
  NTT_LOAD_REDUCE = 2,
  NTT_LOAD_DOT = 3,
  NTT_LOAD_ENC = 4,
  NTT_LOAD_MULM = 5,
  NTT_LOAD_DOTM = 6
};

// Operation applied to every output of a FORWARD transform before it is
// stored (fused consumer), y = the transformed value in [0, q):
//   NONE         dst[i] = y
//   RESCALE      dst[i] = (aux[i] - y) * q_last^{-1} mod q
//   MUL_RESCALE  dst[i] = (aux[i] * aux2[i] - y) * q_last^{-1} mod q
//   MONT         dst[i] = y 2^64 mod q (Montgomery form), and aux[i] = y when the
//                job's aux is not null (aux is then written, not read)
// With y = NTT_q(c_last mod q) the rescale forms are the rescale of
// ciphertext.rs:476-535 in the evaluation domain: the NTT is linear mod q, so
//   NTT_q((c_q - (c_last mod q)) * inv) = (C_q - NTT_q(c_last mod q)) * inv
// for the limb's evaluation-domain input C_q (aux, or the product aux * aux2).
enum NttStore : uint32_t {
  NTT_STORE_NONE = 0,
  NTT_STORE_RESCALE = 1,
  NTT_STORE_MUL_RESCALE = 2,
  NTT_STORE_SEGSUM = 3,
  NTT_STORE_MONT = 4
};
// NTT_STORE_SEGSUM (inverse, whole-polynomial kernel, limb 0 only): instead of
// storing the decrypted coefficients m, the transform writes the ZeRo-MOAI
// segment sums seg[c] = (sum_j v_j W_c[j]) / scale, v_j = m_j centred against
// q0 / 2 (encoding.rs:221-233), with the segment weights W_c generated from
// NttArgs::segw (N pairs W_0[j], 2 cos(2 phi_j); segment_weight_pairs) by
// W_{c+1} = 2 cos(2 phi_j) W_c - W_{c-1}, W_{-1} = W_0; seg = (double*) job
// dst, scale = job scale.
constexpr uint32_t NTT_SEGSUM_MAX_COLS = 16;       // standalone segment-sum kernels
constexpr uint32_t NTT_SEGSUM_FUSED_MAX_COLS = 8;  // NTT_STORE_SEGSUM epilogue (register budget)

// One limb-polynomial transform. In strided mode job i reads src + i*stride,
// writes dst + i*stride and uses limb limb_base + i % limb_mod.
struct NttJob {
  const uint64_t* src;
  uint64_t* dst;
  const uint64_t* aux;   // operand of the load or store operation
  const uint64_t* aux2;  // second store operand (MUL_RESCALE)
  uint32_t limb;
  uint32_t sub;          // variant of the load operation (ENC)
  double scale;          // ciphertext scale (SEGSUM)
};

struct NttArgs {
  const LimbConst* lc;
  const NttJob* jobs;  // non-null: explicit job list
  const uint64_t* src;
  uint64_t* dst;
  uint64_t stride;
  uint32_t limb_mod;
  uint32_t limb_base;
  uint32_t load;              // NttLoad (explicit job lists only)
  uint32_t store;             // NttStore (explicit job lists, forward transforms only)
  const BarrettConst* bc;     // per limb (MUL, DOT)
  const RescaleConst* rc;     // per limb at the input's level (REDUCE, RESCALE stores)
  const uint64_t* key;        // secret key, L x N (DOT)
  const double* segw;         // segment weight pairs, N x 2 (SEGSUM)
  uint32_t cols;              // segments per job (SEGSUM)
  uint32_t pad_;
};

// One product ct x pt of a LoRA set, rescaled and decrypted on limb 0 into
// its segment sums (rescale_decrypt_kernel): X, Y = the last limb of c0 pt
// and c1 pt as coefficients (inverse transforms, canonical mod q_last).
struct RescaleDecryptJob {
  const uint64_t* y;
  const uint64_t* x;
  const uint64_t* d;    // c0 + c1 s of the product's input on limb 0, in [0, 3q) (k_key_dot)
  const uint64_t* ptm;  // the plaintext's limb 0 in Montgomery form
  double* seg;          // cols segment sums
  double scale;         // the rescaled ciphertext's scale
};
struct RescaleDecryptArgs {
  const LimbConst* lc;          // limb 0 is lc[0]
  const BarrettConst* bc;       // limb 0
  const RescaleConst* rc;       // limb 0 at the products' level
  const uint64_t* skm;          // the secret key's limb 0 in Montgomery form
  const double* segw;           // segment weight pairs, N x 2 (NTT_STORE_SEGSUM)
  const RescaleDecryptJob* jobs;
  uint32_t cols;                // segments per job, at most NTT_SEGSUM_FUSED_MAX_COLS
  uint32_t pad_;
};

// Compute units of the current device (256 on MI355X), queried once per
// device; a launch heuristic only, so a failed query falls back to 256.
inline uint32_t device_cu_count() {
  static std::atomic<uint32_t> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  uint32_t v = cache[dev].load(std::memory_order_relaxed);
  if (!v) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    v = (uint32_t)n;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Lets kernel K use up to the whole 160 KiB of a CU's LDS as dynamic shared
// memory. Set once per kernel (the first call's result is kept), so launches
// on the per-token path do not repeat the driver call.
template <auto K>
hipError_t allow_full_lds() {
  static const hipError_t e =
      hipFuncSetAttribute((const void*)K, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

// Launch njobs forward (inverse=false) or inverse negacyclic NTTs of size 2^logn.
hipError_t launch_ntt(int logn, bool inverse, const NttArgs& a, uint32_t njobs, hipStream_t s);
// The decryption's D = c0 + c1 s (in [0, 3q)), formed by the encrypt row
// passes on the limbs in mask instead of storing c0 and c1 there: input i's D
// on the k-th limb of mask at out + (i n + k) N for n limbs in mask; skm =
// the secret key (L x N) in Montgomery form.
struct EncDot {
  uint32_t mask;
  const uint64_t* skm;
  uint64_t* out;
};

// The forward transforms of ninputs encrypt_pk inputs on the limbs in
// limb_mask (bit l: limb l; n of them): a is the NTT_LOAD_ENC job list (3n
// jobs per input, M, E1 and U of each of those limbs in increasing order). At
// split sizes the row passes also combine them with the public key, given as
// prepared pairs pkp of [b | a] (launch_prepare_pairs), into those limbs of
// the ciphertexts at cts + i 2 L N (*combined = true, k_encrypt_combine not
// needed); otherwise (all L limbs only) the transforms are written to the
// jobs' dst and *combined = false. Limb subsets and dot (limbs of limb_mask
// whose D is formed in place of the ciphertext) take the split kernels, which
// exist for the sizes encrypt_limbs_supported accepts (other sizes: all
// limbs and no D only).
hipError_t launch_encrypt(int logn, const NttArgs& a, uint32_t ninputs, uint32_t L, uint32_t limb_mask,
                          const EncDot& dot, const uint64_t* pkp, uint64_t* cts, bool* combined, hipStream_t s);
// Whether launch_encrypt takes limb subsets at transform size 2^logn.
bool encrypt_limbs_supported(int logn);
// The two transform launches of an evaluation-domain rescale: ninv inverse
// transforms (inv, store NONE) of the products' last limbs, then nfwd forward
// transforms (fwd, load REDUCE) of each last limb reduced modulo the lower
// limbs, inverse job i owning forward jobs i * (nfwd / ninv) .. on. Where the
// split kernels run, the inverse column pass and the forward column passes
// are one kernel (the last limb's coefficients stay in registers).
hipError_t launch_rescale(int logn, const NttArgs& inv, uint32_t ninv, const NttArgs& fwd, uint32_t nfwd,
                          hipStream_t s);
// njobs rescale_decrypt_kernel workgroups (whole-polynomial sizes, N <= 16384).
hipError_t launch_rescale_decrypt(int logn, const RescaleDecryptArgs& a, uint32_t njobs, hipStream_t s);
// The same for nb batches on the split kernels (N = 8192 .. 32768), from the
// products' last limbs: inv = the 2 nb inverse jobs (X, Y of batch b at 2b,
// 2b+1; src = ct's last limb, aux = pt's last limb in Montgomery form, load
// NTT_LOAD_MULM, dst = the batch's x, y work areas); partials: scratch of
// nb x cols x N/16 doubles. The segment sums equal launch_rescale_decrypt's
// bit for bit at N = 16384.
hipError_t launch_rescale_decrypt_split(int logn, const NttArgs& inv, const RescaleDecryptArgs& a, uint32_t nb,
                                        double* partials, hipStream_t s);
// A plain batched decryption with segment sums on the split kernels (N =
// 8192 .. 32768) for nb batches: row = the nb inverse jobs of c0 + c1 s on
// limb 0 (src = c0, aux = c1, load NTT_LOAD_DOTM with row.key the secret key
// in Montgomery form, dst = the batch's work area, which a.jobs[b].y names
// too); a.jobs[b].seg and .scale as for the rescale-decrypt; partials: nb x
// cols x N/16 doubles. At N = 16384 the sums equal, bit for bit, those of the
// whole-polynomial decrypt's segment-sum epilogue (NTT_STORE_SEGSUM).
hipError_t launch_decrypt_sums_split(int logn, const NttArgs& row, const RescaleDecryptArgs& a, uint32_t nb,
                                     double* partials, hipStream_t s);
// Supported transform sizes.
constexpr int NTT_MIN_LOGN = 10;
constexpr int NTT_MAX_LOGN = 15;
// Transform sizes of the split kernels, and their column bits CB: the index
// j = (row << CB) | col of a coefficient, column passes over the row bits and
// row passes over the column bits (1024 coefficients per wavefront).
constexpr int NTT_SPLIT_MIN_LOGN = 13;
__host__ __device__ constexpr int split_column_bits(int logn) { return logn >= 15 ? 8 : 7; }
// Row-pass twiddle tables (LimbConst::fwd_row, inv_row): the row passes' stages
// on bits b = 0..3, where each lane holds its own elements, read entry
// ((N | j) >> (b + 1)) of the table for slot s = 0 .. (16 >> (b + 1)) - 1 of
// lane l in wavefront part p, with j = p 1024 + (s << (b + 1)) + ((l mod 2^(CB-4))
// << 4) + ((l >> (CB - 4)) << CB). The row table holds those entries stage by
// stage (stage b from N - (N >> b), N >> (b + 1) entries) in the order
// (p, s, l), so that a load instruction of the 64 lanes reads 1 KiB of
// consecutive entries: 15 N / 16 entries per direction.
__host__ __device__ constexpr uint32_t row_table_index(uint32_t n, int b, uint32_t part, uint32_t s, uint32_t lane) {
  return n - (n >> b) + ((part * (16u >> (b + 1)) + s) << 6) + lane;
}
__host__ __device__ constexpr uint32_t row_table_source(uint32_t n, int logn, int b, uint32_t part, uint32_t s,
                                                        uint32_t lane) {
  const int cb = split_column_bits(logn);
  const uint32_t j = (part << 10) + (s << (b + 1)) + ((lane & ((1u << (cb - 4)) - 1)) << 4) +
                     ((lane >> (cb - 4)) << cb);
  return (n | j) >> (b + 1);
}

}  // namespace th
