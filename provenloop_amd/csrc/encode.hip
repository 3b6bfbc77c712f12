// GPU CKKS encode fused with the RNS preparation of encrypt_pk
// (tensafe-he-core/src/encoding.rs:173-207, :250-278; ciphertext.rs:250-296).
//
//   z~_re[k] = z~_re[N-1-k] = z[k] (k < N/2), z~_im = 0
//   a = FFT(z~)                      radix-2 DIT, the reference's order
//   coeff_j = (a_re_j / N) * cos(pi j/N) + (a_im_j / N) * sin(pi j/N)
//   m_j = round(coeff_j * 2^40) as i64 (half away from zero, saturating)
// then per limb l:  M_l = (m + e0) mod q_l,  E1_l = e1 mod q_l,  U_l = u mod q_l
// which the forward NTT and the combine kernel turn into the ciphertext.
// All f64 steps round exactly as on the host (-ffp-contract=off, host
// twiddles), so m is bit-identical to the reference encoder's.
#include "encode_sample.h"
#include "fft_device.h"

namespace th {

constexpr int ENC_THREADS = 1024;

template <int LP>
__global__ __launch_bounds__(ENC_THREADS) void k_encode_parts(const EncodeJob* __restrict__ jobs,
                                                              const double* __restrict__ stage_re,
                                                              const double* __restrict__ stage_im, uint32_t logn,
                                                              const double* __restrict__ z_base) {
  extern __shared__ double sh[];
  const uint32_t n = 1u << logn, S = n / 2;
  const uint32_t M = n >> LP;
  const uint32_t part = blockIdx.x;
  const EncodeJob jb = jobs[blockIdx.y];
  const GPtr<double> z = gld(z_base ? z_base + (size_t)blockIdx.y * (jb.rep_d ? jb.rep_d : S) : jb.z);
  double* re = sh;
  double* im = sh + M;
  const uint32_t r = brv_bits(part, LP);
  const uint32_t lb = logn - LP;
  for (uint32_t jj = threadIdx.x; jj < M; jj += blockDim.x) {
    const uint32_t j = (jj << LP) | r;  // element at bit-reversed position part*M + pos
    const uint32_t pos = brv_bits(jj, lb);
    const uint32_t slot = j < S ? j : n - 1 - j;
    double v;
    if (jb.rep_d)  // inference_engine.py:1266-1269: [h | h | ... | 0]
      v = slot < jb.rep_cols * jb.rep_d ? z[slot % jb.rep_d] : 0.0;
    else
      v = z[slot];
    re[pos] = v;
    im[pos] = 0.0;
  }
  __syncthreads();
  dit_stages_reg(re, im, lb, stage_re, stage_im);
  const GMut<double> out = gst(jb.parts) + (size_t)part * 2 * M;
  for (uint32_t i = threadIdx.x; i < M; i += blockDim.x) {
    out[i] = re[i];
    out[M + i] = im[i];
  }
}

// Rust `f64::round() as i64`: half away from zero, saturating, NaN -> 0.
__device__ __forceinline__ int64_t round_sat_i64(double x) {
  const double r = round(x);
  if (r != r) return 0;
  if (r >= 9223372036854775808.0) return INT64_MAX;
  if (r < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)r;
}

__device__ __forceinline__ uint64_t signed_residue_dev(int64_t e, const BarrettConst& m) {
  const uint64_t a = e >= 0 ? (uint64_t)e : (uint64_t)0 - (uint64_t)e;
  const uint64_t r = a < m.q ? a : mulmod_barrett(a, 1, m);
  return e >= 0 ? r : m.q - r;
}

__device__ __forceinline__ void emit_coefficient(const EncodeJob& jb, const BarrettConst* __restrict__ bc,
                                                 const double* __restrict__ twist_re,
                                                 const double* __restrict__ twist_im, uint32_t j, Cx a,
                                                 double inv_n, uint32_t n, uint32_t L) {
  const double a_re = a.re * inv_n;
  const double a_im = a.im * inv_n;
  const double coeff = a_re * twist_re[j] + a_im * twist_im[j];
  const int64_t m = round_sat_i64(coeff * 1099511627776.0);  // * 2^40 (params.rs:12)
  const int64_t e0 = jb.e0 ? gld(jb.e0)[j] : 0;
  const int64_t e1 = jb.e1 ? gld(jb.e1)[j] : 0;
  const uint8_t u = jb.u ? gld(jb.u)[j] : 1;  // ciphertext.rs:261-266: 0 -> q-1, 1 -> 0, 2 -> 1
  const GMut<uint64_t> dst = gst(jb.dst);
  for (uint32_t l = 0; l < L; ++l) {
    const BarrettConst c = bc[l];
    const uint64_t mm = signed_residue_dev(m, c);
    dst[(size_t)l * n + j] = jb.e0 ? csub(mm + signed_residue_dev(e0, c), c.q) : mm;
    if (jb.e1) dst[(size_t)(L + l) * n + j] = signed_residue_dev(e1, c);
    if (jb.u) dst[(size_t)(2 * L + l) * n + j] = u == 0 ? c.q - 1 : (u == 1 ? 0 : 1);
  }
}

template <int LP>
__global__ __launch_bounds__(256) void k_encode_final(const EncodeJob* __restrict__ jobs,
                                                      const BarrettConst* __restrict__ bc,
                                                      const double* __restrict__ twist_re,
                                                      const double* __restrict__ twist_im,
                                                      const double* __restrict__ stage_re,
                                                      const double* __restrict__ stage_im, uint32_t logn,
                                                      uint32_t L) {
  const uint32_t n = 1u << logn;
  const uint32_t M = n >> LP;
  const EncodeJob jb = jobs[blockIdx.y];
  const GPtr<double> P = gld(jb.parts);
  const double inv_n = 1.0 / (double)n;
  auto at = [&](uint32_t part, uint32_t i) { return Cx{P[(size_t)part * 2 * M + i], P[(size_t)part * 2 * M + M + i]}; };
  for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < M; k += gridDim.x * blockDim.x) {
    if constexpr (LP == 0) {
      emit_coefficient(jb, bc, twist_re, twist_im, k, at(0, k), inv_n, n, L);
    } else if constexpr (LP == 1) {
      const uint32_t S = n / 2;
      Cx t, b;
      dit(at(0, k), at(1, k), stage_re[S - 1 + k], stage_im[S - 1 + k], t, b);
      emit_coefficient(jb, bc, twist_re, twist_im, k, t, inv_n, n, L);
      emit_coefficient(jb, bc, twist_re, twist_im, k + S, b, inv_n, n, L);
    } else {  // LP == 2
      const uint32_t S = n / 2, Q4 = n / 4;
      Cx y0, y1, y2, y3, o0, o1, o2, o3;
      dit(at(0, k), at(1, k), stage_re[Q4 - 1 + k], stage_im[Q4 - 1 + k], y0, y1);
      dit(at(2, k), at(3, k), stage_re[Q4 - 1 + k], stage_im[Q4 - 1 + k], y2, y3);
      dit(y0, y2, stage_re[S - 1 + k], stage_im[S - 1 + k], o0, o2);
      dit(y1, y3, stage_re[S - 1 + k + Q4], stage_im[S - 1 + k + Q4], o1, o3);
      emit_coefficient(jb, bc, twist_re, twist_im, k, o0, inv_n, n, L);
      emit_coefficient(jb, bc, twist_re, twist_im, k + Q4, o1, inv_n, n, L);
      emit_coefficient(jb, bc, twist_re, twist_im, k + S, o2, inv_n, n, L);
      emit_coefficient(jb, bc, twist_re, twist_im, k + S + Q4, o3, inv_n, n, L);
    }
  }
}

size_t encode_parts_doubles(uint32_t logn) { return (size_t)2 << logn; }

hipError_t launch_encode(const EncodeJob* jobs, uint32_t njobs, const BarrettConst* bc, const double* twist_re,
                         const double* twist_im, const double* stage_re, const double* stage_im, uint32_t logn,
                         uint32_t L, hipStream_t s, const double* z_base) {
  if (!njobs) return hipSuccess;
  // at least one part per LDS budget; more parts (up to 4) while the batch
  // would leave most CUs idle (the parts are independent workgroups and the
  // result is the same for any split)
  uint32_t lp = fft_parts_log(logn);
  while (lp < 2 && logn - lp > 10 && njobs * (1u << lp) < 256) ++lp;
  const uint32_t M = (1u << logn) >> lp;
  const size_t lds = (size_t)2 * M * sizeof(double);
  const uint32_t gx = (M + 255) / 256 < 32 ? (M + 255) / 256 : 32;
  hipError_t e;
#define TH_ENC(LP)                                                                                         \
  case LP:                                                                                                 \
    e = hipFuncSetAttribute((const void*)k_encode_parts<LP>, hipFuncAttributeMaxDynamicSharedMemorySize,   \
                            (int)lds);                                                                     \
    if (e != hipSuccess) return e;                                                                         \
    hipLaunchKernelGGL(k_encode_parts<LP>, dim3(1u << LP, njobs), dim3(ENC_THREADS), lds, s, jobs,         \
                       stage_re, stage_im, logn, z_base);                                                  \
    hipLaunchKernelGGL(k_encode_final<LP>, dim3(gx, njobs), dim3(256), 0, s, jobs, bc, twist_re, twist_im, \
                       stage_re, stage_im, logn, L);                                                       \
    return hipGetLastError();
  switch (lp) {
    TH_ENC(0)
    TH_ENC(1)
    TH_ENC(2)
    default: return hipErrorInvalidValue;
  }
#undef TH_ENC
}

}  // namespace th
