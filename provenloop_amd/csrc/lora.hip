// LoRA-B application on the device: delta_j = B_j @ intermediate_j
// (demonstrator/server/inference_engine.py:1392), where intermediate_j is
// gathered from the ZeRo-MOAI segment sums of projection j's plaintext
// batches (:1379-1386): row r of the LoRA-A side is segment r % cols of
// batch first_row + r / cols.
#include "poly_kernels.h"

namespace th {

// A projection whose input has its sampler band flag set (flags: the token's
// band flags in device memory, one generation per input, written by the
// sampler earlier on the stream; the input is flagged when it holds this
// token's generation gen; null for none) gets NaN deltas: its randomness is
// drawn again on the host and the token queued again, which overwrites them,
// so work ordered after the token on the stream never reads an unverified
// finite delta. (The host-visible copy of the flags would cost a read across
// PCIe per workgroup: about 30 us per token.)
__global__ __launch_bounds__(256) void k_lora_b(const LoraBJob* __restrict__ jobs, const double* __restrict__ sums,
                                                double* __restrict__ out, uint32_t cols, const uint32_t* flags,
                                                uint32_t gen) {
  const LoraBJob jb = jobs[blockIdx.y];
  const double* seg = sums + (size_t)jb.first_row * cols;  // batch-major: seg[b * cols + c]
  const bool flagged = flags && flags[jb.input] == gen;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < jb.d_out; i += gridDim.x * blockDim.x) {
    const double* bcol = jb.b + i;  // rank-major: consecutive lanes read consecutive doubles
    double acc = 0.0;
#pragma unroll 8
    for (uint32_t r = 0; r < jb.rank; ++r) acc = __fma_rn(bcol[(size_t)r * jb.d_out], seg[r], acc);
    out[jb.out_off + i] = flagged ? __builtin_nan("") : acc;
  }
}

hipError_t launch_lora_b(const LoraBJob* jobs, uint32_t njobs, uint32_t max_d_out, const double* sums, double* out,
                         uint32_t cols, hipStream_t s, const uint32_t* flags, uint32_t gen) {
  if (!njobs) return hipSuccess;
  uint32_t bx = (max_d_out + 255) / 256;
  if (bx > 64) bx = 64;
  hipLaunchKernelGGL(k_lora_b, dim3(bx, njobs), dim3(256), 0, s, jobs, sums, out, cols, flags, gen);
  return hipGetLastError();
}

// B of each projection mixed over its experts, sum_x g_x B_x, accumulated
// from 0.0 in expert order as separate multiplies and adds (rank-major, as the
// experts' B are stored).
__global__ __launch_bounds__(256) void k_moe_mix_b(const double* __restrict__ bexp, const MoeProj* __restrict__ projs,
                                                   const double* __restrict__ gates, uint32_t k,
                                                   double* __restrict__ bmix) {
  const MoeProj mp = projs[blockIdx.y];
  const double* g = gates + (size_t)blockIdx.y * k;
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < mp.count; t += gridDim.x * blockDim.x) {
    double acc = 0.0;
    for (uint32_t x = 0; x < k; ++x) {
      const double p = g[x] * bexp[mp.off * k + (size_t)x * mp.count + t];
      acc = acc + p;
    }
    bmix[mp.off + t] = acc;
  }
}

hipError_t launch_moe_mix_b(const double* bexp, const MoeProj* projs, const double* gates, uint32_t n_proj, uint32_t k,
                            uint32_t max_count, double* bmix, hipStream_t s) {
  if (!n_proj) return hipSuccess;
  uint32_t bx = (max_count + 255) / 256;
  if (bx > 64) bx = 64;
  hipLaunchKernelGGL(k_moe_mix_b, dim3(bx, n_proj), dim3(256), 0, s, bexp, projs, gates, k, bmix);
  return hipGetLastError();
}

}  // namespace th
