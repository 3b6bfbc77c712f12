// Job descriptors and launchers of the element-wise and decode kernels.
#pragma once
#include "th_internal.h"

namespace th {

struct CtPtJob {
  const uint64_t* ct0;  // component c0 (limbs x N)
  const uint64_t* ct1;  // component c1
  const uint64_t* pt;   // plaintext, NTT domain (>= limbs x N)
  uint64_t* out;        // [c0 | c1], limbs x N each
  uint32_t limbs;
  uint32_t pad_;
};

// out = a +- b on a's limbs; the operands' c0 and c1 are addressed apart so
// that b may hold more limbs than a.
struct AddJob {
  const uint64_t* a0;
  const uint64_t* a1;
  const uint64_t* b0;
  const uint64_t* b1;
  uint64_t* out;  // [c0 | c1], limbs each
  uint32_t limbs;
  uint32_t sub;
};

struct EncCombineJob {
  const uint64_t* prep;  // NTT of [M | E1 | U]
  const uint64_t* pk_b;
  const uint64_t* pk_a;
  uint64_t* out;         // [c0 | c1]
};

struct DecodeConst {
  uint64_t q0, q1, half_q0;
  uint64_t q0_inv_q1, q0_inv_q1_s;  // (q0 mod q1)^{-1} mod q1, Shoup companion
  BarrettConst b1;                  // remainder modulo q1
  uint64_t Q_lo, Q_hi, halfQ_lo, halfQ_hi;
};

struct DecodeJob {
  const uint64_t* m;  // limb 0 (and limb 1 at m + N for the CRT branch), coefficient domain
  double* parts;      // P parts x (re, im) x N/P doubles
  double* out;        // N/2 decoded slots (may be null)
  double* seg;        // cols segment sums (may be null)
  double scale;
  uint32_t crt;
  uint32_t pad_;
};

// delta = B @ intermediate for one LoRA projection. Rows of the LoRA-A side
// are numbered so that row r's segment sum sits at sums[first_row * cols + r]
// (batches of one projection are consecutive), which is the ZeRo-MOAI
// extraction order (inference_engine.py:1379-1386).
struct LoraBJob {
  const double* b;     // B (d_out x rank) stored rank-major: element (i, r) at r * d_out + i
  uint32_t d_out;
  uint32_t rank;
  uint32_t first_row;  // first plaintext batch of the projection
  uint32_t input;      // the input the projection reads (its band flag)
  uint64_t out_off;    // offset of the projection's deltas in the output
};

hipError_t launch_lora_b(const LoraBJob* jobs, uint32_t njobs, uint32_t max_d_out, const double* sums, double* out,
                         uint32_t cols, hipStream_t s, const uint32_t* flags = nullptr, uint32_t gen = 0);

// One plaintext batch of a mixture LoRA set: its projection and how many of
// its slots hold A rows (rows x d).
struct MoeBatch {
  uint32_t proj;
  uint32_t n_valid;
};
// One projection's B in a mixture set: offset of its mixed B (count doubles,
// rank-major) in the mixed buffer; its k experts' B sit at off * k + x * count.
struct MoeProj {
  uint64_t off;
  uint32_t count;
  uint32_t pad_;
};
// bmix = sum_x g_x B_x per projection (k_moe_mix_b).
hipError_t launch_moe_mix_b(const double* bexp, const MoeProj* projs, const double* gates, uint32_t n_proj, uint32_t k,
                            uint32_t max_count, double* bmix, hipStream_t s);

hipError_t launch_ct_pt_mul(const CtPtJob* jobs, uint32_t njobs, uint32_t max_limbs, const BarrettConst* bc,
                            uint32_t n, hipStream_t s);
hipError_t launch_ct_addsub(const AddJob* jobs, uint32_t njobs, uint32_t max_limbs, const uint64_t* q,
                            uint32_t n, hipStream_t s);
// pk (optional): the public key [b | a] for every job instead of the jobs' fields.
// D = c0 + c1 s (lazy, [0, 3q)) on limbs 0..nl-1 of count ciphertexts, key in Montgomery form (k_key_dot).
hipError_t launch_key_dot(const uint64_t* cts, uint64_t ct_stride, const uint64_t* skm, uint64_t* out,
                          const BarrettConst* bc, uint32_t n, uint32_t L, uint32_t nl, uint32_t count, hipStream_t s);
// count x L x n residues -> Montgomery form, w 2^64 mod q (k_to_montgomery).
hipError_t launch_to_montgomery(const uint64_t* src, uint64_t* dst, const BarrettConst* bc, uint32_t n, uint32_t L,
                                uint32_t count, hipStream_t s);
// count x L x n residues -> the same as (w, companion) pairs (k_prepare_pairs).
hipError_t launch_prepare_pairs(const uint64_t* src, uint64_t* dst, const BarrettConst* bc, const LimbConst* lc,
                                uint32_t n, uint32_t L, uint32_t count, hipStream_t s);
hipError_t launch_encrypt_combine(const EncCombineJob* jobs, uint32_t njobs, const BarrettConst* bc,
                                  uint32_t n, uint32_t L, hipStream_t s, const uint64_t* pk = nullptr);
hipError_t launch_signed_to_rns(const int64_t* x, uint64_t* dst, const BarrettConst* bc, uint32_t n, uint32_t L,
                               hipStream_t s);
hipError_t launch_sub_product(const uint64_t* x, const uint64_t* a, const uint64_t* sk, uint64_t* out,
                              const BarrettConst* bc, uint32_t n, uint32_t L, hipStream_t s);
// Decode (encoding.rs:219-239, :282-315) of njobs decrypted polynomials:
// centring / CRT, twist, radix-2 DIT FFT and the real parts of the first N/2
// outputs, optionally followed by sums over `cols` segments of d slots.
hipError_t launch_decode(const DecodeJob* jobs, uint32_t njobs, const DecodeConst* dc, const double* twist_re,
                         const double* twist_im, const double* stage_re, const double* stage_im, uint32_t logn,
                         uint32_t d, uint32_t cols, hipStream_t s);
size_t decode_parts_doubles(uint32_t logn);  // scratch doubles per job
size_t segsum_parts_doubles(uint32_t cols);  // scratch doubles per job of launch_segsum
// Segment sums of the decoded slots taken straight from the decrypted
// coefficients with segment weights W (cols x N, segment_weights()); each
// job's `seg` receives cols sums, within rounding of decode-then-sum. Uses
// the first 16 * cols doubles of each job's `parts` as scratch.
constexpr uint32_t SEGSUM_MAX_COLS = NTT_SEGSUM_MAX_COLS;
hipError_t launch_segsum(const DecodeJob* jobs, uint32_t njobs, const DecodeConst* dc, const double* W,
                         uint32_t logn, uint32_t cols, hipStream_t s);

}  // namespace th
