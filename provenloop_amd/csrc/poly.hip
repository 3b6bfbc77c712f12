// Element-wise RNS kernels: fused across limbs, ciphertext components and
// batch entries. Every launch covers a list of jobs; each job is a run of
// limb-polynomials with a common layout, and blockIdx.y selects the job.
// These kernels are HBM-bound (two or three u64 streams per output word).
#include <algorithm>

#include "poly_kernels.h"

namespace th {

// tensafe-he-core/src/ciphertext.rs:132-136: e >= 0 ? e % q : q - (|e| % q).
// |e| < 2^63 < q^2 for every prime used, so the Barrett remainder is exact.
__device__ __forceinline__ uint64_t signed_residue(int64_t e, const BarrettConst& m) {
  const uint64_t a = e >= 0 ? (uint64_t)e : (uint64_t)0 - (uint64_t)e;
  const uint64_t r = a < m.q ? a : mulmod_barrett(a, 1, m);
  return e >= 0 ? r : m.q - r;
}

// out[c][l][i] = ct[c][l][i] * pt[l][i] for c in {0,1}, l < limbs
// (ciphertext.rs:422-429 / rns.rs:243-253), all jobs in one launch.
__global__ void k_ct_pt_mul(const CtPtJob* __restrict__ jobs, const BarrettConst* __restrict__ bc,
                            uint32_t n) {
  const CtPtJob jb = jobs[blockIdx.y];
  const uint32_t per_comp = jb.limbs * n;
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < 2 * per_comp; e += gridDim.x * blockDim.x) {
    const uint32_t w = e < per_comp ? e : e - per_comp;
    const uint32_t l = w / n;
    const uint64_t c = gld(e < per_comp ? jb.ct0 : jb.ct1)[w];
    gst(jb.out)[e] = mulmod_barrett(c, gld(jb.pt)[w], bc[l]);
  }
}

// out = a +/- b over 2 * limbs limb-polynomials (ciphertext.rs:435-466).
__global__ void k_ct_addsub(const AddJob* __restrict__ jobs, const uint64_t* __restrict__ q, uint32_t n) {
  const AddJob jb = jobs[blockIdx.y];
  const uint32_t half = jb.limbs * n, total = 2 * half;
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const bool c1 = e >= half;
    const uint32_t r = c1 ? e - half : e;
    const uint64_t m = q[r / n];
    const uint64_t a = gld(c1 ? jb.a1 : jb.a0)[r], b = gld(c1 ? jb.b1 : jb.b0)[r];
    gst(jb.out)[e] = jb.sub ? submod(a, b, m) : addmod(a, b, m);
  }
}

// Operands fixed for many products (keys) prepared as pairs in the twiddle
// tables' formats: (w, floor(w 2^64 / q)) on the integer limbs, (w, w / q as
// a double) on limbs below 2^41, so a product by w is one Shoup or one FP64
// step instead of a 64-bit Barrett reduction. src: count x L x n residues;
// dst: the same as 16-byte pairs.
__device__ __forceinline__ uint64_t shoup_companion(uint64_t w, const BarrettConst& b) {
  // w 2^64 r / 2^128 with r = floor((2^128 - 1) / q) is at most 1 short of
  // floor(w 2^64 / q); the remainder w 2^64 - est q (< 2q) is exact mod 2^64
  uint64_t est = w * b.r_hi + __umul64hi(w, b.r_lo);
  uint64_t rem = (uint64_t)0 - est * b.q;
  while (rem >= b.q) {
    ++est;
    rem -= b.q;
  }
  return est;
}

__global__ void k_prepare_pairs(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                const BarrettConst* __restrict__ bc, const LimbConst* __restrict__ lc, uint32_t n,
                                uint32_t L, uint64_t total) {
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t l = (uint32_t)((e / n) % L);
    const uint64_t w = src[e];
    uint64_t c;
    if (lc[l].fp64)
      c = __builtin_bit_cast(uint64_t, (double)w / lc[l].qd);  // correctly rounded: both exact below 2^53
    else
      c = shoup_companion(w, bc[l]);
    dst[2 * e] = w;
    dst[2 * e + 1] = c;
  }
}

// count x L x n residues into Montgomery form, w 2^64 mod q (mont_mul).
__global__ void k_to_montgomery(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                const BarrettConst* __restrict__ bc, uint32_t n, uint32_t L, uint64_t total) {
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (uint64_t)gridDim.x * blockDim.x) {
    const BarrettConst& m = bc[(e / n) % L];
    dst[e] = csub(shoup_lazy(src[e], m.r64, m.r64_s, m.q), m.q);
  }
}

// dst[l][i] = x[i] mod q_l for signed integer coefficients (encoding.rs:193-204).
__global__ void k_signed_to_rns(const int64_t* __restrict__ x, uint64_t* __restrict__ dst,
                                const BarrettConst* __restrict__ bc, uint32_t n, uint32_t L) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const int64_t v = x[i];
    for (uint32_t l = 0; l < L; ++l) dst[(uint64_t)l * n + i] = signed_residue(v, bc[l]);
  }
}

// out = x - a*s over L x N (keygen_public b = -a*s + e, ciphertext.rs:141-151;
// secret-key encrypt c0 = -a*s + (m + e), ciphertext.rs:209-222).
__global__ void k_sub_product(const uint64_t* __restrict__ x, const uint64_t* __restrict__ a,
                              const uint64_t* __restrict__ s, uint64_t* __restrict__ out,
                              const BarrettConst* __restrict__ bc, uint32_t n, uint32_t L) {
  const uint32_t total = L * n;
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const BarrettConst m = bc[e / n];
    out[e] = submod(x[e], mulmod_barrett(a[e], s[e], m), m.q);
  }
}

// D = c0 + c1 s on limbs 0..nl-1 of count ciphertexts at cts + i ct_stride
// ([c0 | c1], L limbs each), with the secret key in Montgomery form: the
// decryption's c0 + c1 s (ciphertext.rs:332-341), lazily in [0, 3q). For a
// product ciphertext (c0 pt, c1 pt) the decryption is pt (c0 + c1 s), so one
// D per input serves every plaintext it is multiplied by.
__global__ void k_key_dot(const uint64_t* __restrict__ cts, uint64_t ct_stride, const uint64_t* __restrict__ skm,
                          uint64_t* __restrict__ out, const BarrettConst* __restrict__ bc, uint32_t n, uint32_t L,
                          uint32_t nl, uint64_t total) {
  const uint64_t per = (uint64_t)nl * n;
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t i = e / per, r = e - i * per;
    const uint32_t l = (uint32_t)(r / n);
    const uint64_t* c = cts + i * ct_stride;
    out[e] = c[r] + mont_mul(c[(uint64_t)L * n + r], skm[r], bc[l]);
  }
}

// c0 = b*U + M, c1 = a*U + E1 in the NTT domain (ciphertext.rs:298-312).
__global__ void k_encrypt_combine(const EncCombineJob* __restrict__ jobs, const BarrettConst* __restrict__ bc,
                                  uint32_t n, uint32_t L, const uint64_t* __restrict__ pk) {
  EncCombineJob jb = jobs[blockIdx.y];
  if (pk) {
    jb.pk_b = pk;
    jb.pk_a = pk + (size_t)L * n;
  }
  const uint32_t total = L * n;
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const uint32_t l = e / n;
    const BarrettConst m = bc[l];
    const GPtr<uint64_t> prep = gld(jb.prep);
    const uint64_t U = prep[2 * total + e];
    const uint64_t bu = mulmod_barrett(gld(jb.pk_b)[e], U, m);
    const uint64_t au = mulmod_barrett(gld(jb.pk_a)[e], U, m);
    gst(jb.out)[e] = addmod(bu, prep[e], m.q);
    gst(jb.out)[total + e] = addmod(au, prep[total + e], m.q);
  }
}

static dim3 grid_for(uint32_t elems, uint32_t jobs) {
  uint32_t bx = (elems + 255) / 256;
  if (bx > 64) bx = 64;
  return dim3(bx, jobs);
}

hipError_t launch_ct_pt_mul(const CtPtJob* jobs, uint32_t njobs, uint32_t max_limbs, const BarrettConst* bc,
                            uint32_t n, hipStream_t s) {
  if (!njobs) return hipSuccess;
  hipLaunchKernelGGL(k_ct_pt_mul, grid_for(2 * max_limbs * n, njobs), dim3(256), 0, s, jobs, bc, n);
  return hipGetLastError();
}

hipError_t launch_ct_addsub(const AddJob* jobs, uint32_t njobs, uint32_t max_limbs, const uint64_t* q,
                            uint32_t n, hipStream_t s) {
  if (!njobs) return hipSuccess;
  hipLaunchKernelGGL(k_ct_addsub, grid_for(2 * max_limbs * n, njobs), dim3(256), 0, s, jobs, q, n);
  return hipGetLastError();
}

hipError_t launch_prepare_pairs(const uint64_t* src, uint64_t* dst, const BarrettConst* bc, const LimbConst* lc,
                                uint32_t n, uint32_t L, uint32_t count, hipStream_t s) {
  const uint64_t total = (uint64_t)count * L * n;
  if (!total) return hipSuccess;
  const uint32_t blocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(k_prepare_pairs, dim3(blocks), dim3(256), 0, s, src, dst, bc, lc, n, L, total);
  return hipGetLastError();
}

hipError_t launch_to_montgomery(const uint64_t* src, uint64_t* dst, const BarrettConst* bc, uint32_t n, uint32_t L,
                                uint32_t count, hipStream_t s) {
  const uint64_t total = (uint64_t)count * L * n;
  if (!total) return hipSuccess;
  const uint32_t blocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(k_to_montgomery, dim3(blocks), dim3(256), 0, s, src, dst, bc, n, L, total);
  return hipGetLastError();
}

hipError_t launch_key_dot(const uint64_t* cts, uint64_t ct_stride, const uint64_t* skm, uint64_t* out,
                          const BarrettConst* bc, uint32_t n, uint32_t L, uint32_t nl, uint32_t count, hipStream_t s) {
  const uint64_t total = (uint64_t)count * nl * n;
  if (!total) return hipSuccess;
  const uint32_t blocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(k_key_dot, dim3(blocks), dim3(256), 0, s, cts, ct_stride, skm, out, bc, n, L, nl, total);
  return hipGetLastError();
}

hipError_t launch_encrypt_combine(const EncCombineJob* jobs, uint32_t njobs, const BarrettConst* bc,
                                  uint32_t n, uint32_t L, hipStream_t s, const uint64_t* pk) {
  if (!njobs) return hipSuccess;
  hipLaunchKernelGGL(k_encrypt_combine, grid_for(L * n, njobs), dim3(256), 0, s, jobs, bc, n, L, pk);
  return hipGetLastError();
}

hipError_t launch_signed_to_rns(const int64_t* x, uint64_t* dst, const BarrettConst* bc, uint32_t n, uint32_t L,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_signed_to_rns, grid_for(n, 1), dim3(256), 0, s, x, dst, bc, n, L);
  return hipGetLastError();
}

hipError_t launch_sub_product(const uint64_t* x, const uint64_t* a, const uint64_t* sk, uint64_t* out,
                              const BarrettConst* bc, uint32_t n, uint32_t L, hipStream_t s) {
  hipLaunchKernelGGL(k_sub_product, grid_for(L * n, 1), dim3(256), 0, s, x, a, sk, out, bc, n, L);
  return hipGetLastError();
}

}  // namespace th
