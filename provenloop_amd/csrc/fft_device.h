// Radix-2 DIT complex FFT in f64 shared by the GPU encode and decode, with
// the reference's evaluation order (tensafe-he-core/src/encoding.rs:83-120):
//   v = w * x[i1]  (v_re = w_re*x_re - w_im*x_im, v_im = w_re*x_im + w_im*x_re)
//   x[i0] = u + v, x[i1] = u - v.
// Compiled with -ffp-contract=off, so every product and sum rounds exactly as
// on the host. Twiddles of stage s live at offset 2^s - 1 of the stage tables.
//
// A transform of N values after the bit-reversal permutation is split into
// 2^LP parts of M = N >> LP consecutive positions: stages 0 .. logN-LP-1 act
// inside a part (one workgroup, in LDS); the last LP stages combine the parts
// element-wise.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace th {

__device__ __forceinline__ uint32_t brv_bits(uint32_t x, uint32_t bits) {
  return bits ? (__brev(x) >> (32 - bits)) : 0;
}

struct Cx {
  double re, im;
};

// (u + w*x, u - w*x) in the reference's order.
__device__ __forceinline__ void dit(Cx u, Cx x, double w_re, double w_im, Cx& top, Cx& bot) {
  const double v_re = w_re * x.re - w_im * x.im;
  const double v_im = w_re * x.im + w_im * x.re;
  top.re = u.re + v_re;
  top.im = u.im + v_im;
  bot.re = u.re - v_re;
  bot.im = u.im - v_im;
}

// Stages 0 .. lb-1 on M = 2^lb values held in LDS (re[], im[]), whole block.
__device__ __forceinline__ void dit_stages_lds(double* re, double* im, uint32_t lb,
                                               const double* __restrict__ stage_re,
                                               const double* __restrict__ stage_im) {
  const uint32_t M = 1u << lb;
  for (uint32_t s = 0; s < lb; ++s) {
    const uint32_t half = 1u << s;
    const double* wr = stage_re + (half - 1);
    const double* wi = stage_im + (half - 1);
    for (uint32_t b = threadIdx.x; b < M / 2; b += blockDim.x) {
      const uint32_t k = b & (half - 1);
      const uint32_t i0 = ((b >> s) << (s + 1)) | k;
      const uint32_t i1 = i0 + half;
      Cx t, u;
      dit(Cx{re[i0], im[i0]}, Cx{re[i1], im[i1]}, wr[k], wi[k], t, u);
      re[i0] = t.re;
      im[i0] = t.im;
      re[i1] = u.re;
      im[i1] = u.im;
    }
    __syncthreads();
  }
}

// The same stages 0 .. lb-1, up to three at a time in registers: for a pass
// on bits [s0, s0 + R) each thread loads the 2^R values whose positions
// differ only in those bits, runs the R stages on them and writes them back,
// so LDS is read and written once per pass instead of once per stage. Every
// butterfly sees the same operands and twiddle as in dit_stages_lds, so the
// result is bit-identical. Needs blockDim.x * 8 >= M. With PAD, value i
// lives at re/im[i + i / 8] (fft_pad): one spare slot per 8 values puts the
// lanes of the first two passes (8 consecutive values per lane, and groups of
// 8 lanes 64 values apart) on different LDS banks.
__host__ __device__ constexpr uint32_t fft_pad(uint32_t i) { return i + (i >> 3); }

template <bool PAD = false>
__device__ __forceinline__ void dit_stages_reg(double* re, double* im, uint32_t lb,
                                               const double* __restrict__ stage_re,
                                               const double* __restrict__ stage_im) {
  auto P = [](uint32_t i) { return PAD ? fft_pad(i) : i; };
  const uint32_t M = 1u << lb;
  for (uint32_t s0 = 0; s0 < lb; s0 += 3) {
    const uint32_t R = lb - s0 < 3 ? lb - s0 : 3;
    const uint32_t groups = M >> R;
    for (uint32_t t = threadIdx.x; t < groups; t += blockDim.x) {
      const uint32_t lo = t & ((1u << s0) - 1), hi = t >> s0;
      const uint32_t base = lo | (hi << (s0 + R));
      Cx x[8];
#pragma unroll
      for (uint32_t r = 0; r < 8; ++r)
        if (r < (1u << R)) x[r] = Cx{re[P(base | (r << s0))], im[P(base | (r << s0))]};
      // The twiddle of x[r]'s pair at stage s0 + rb is selected by its
      // position's bits below s0 + rb: lo + (g << s0), g = r mod 2^rb (base
      // has no bits in [s0, s0 + R)). So the group needs 2^rb twiddles per
      // stage, 7 in all, requested together before the first butterfly.
      double twr[7], twi[7];  // stage rb's twiddle g at (1 << rb) - 1 + g
#pragma unroll
      for (uint32_t rb = 0; rb < 3; ++rb) {
        if (rb >= R) break;
#pragma unroll
        for (uint32_t g = 0; g < (1u << rb); ++g) {
          const uint32_t w = (1u << (s0 + rb)) - 1 + lo + (g << s0);
          twr[(1u << rb) - 1 + g] = stage_re[w];
          twi[(1u << rb) - 1 + g] = stage_im[w];
        }
      }
#pragma unroll
      for (uint32_t rb = 0; rb < 3; ++rb) {
        if (rb >= R) break;
#pragma unroll
        for (uint32_t r = 0; r < 8; ++r) {
          if (r >= (1u << R) || (r & (1u << rb))) continue;
          const uint32_t ti = (1u << rb) - 1 + (r & ((1u << rb) - 1));
          Cx t0, t1;
          dit(x[r], x[r | (1u << rb)], twr[ti], twi[ti], t0, t1);
          x[r] = t0;
          x[r | (1u << rb)] = t1;
        }
      }
#pragma unroll
      for (uint32_t r = 0; r < 8; ++r)
        if (r < (1u << R)) {
          re[P(base | (r << s0))] = x[r].re;
          im[P(base | (r << s0))] = x[r].im;
        }
    }
    __syncthreads();
  }
}

// Parts per transform: one part fits LDS (2^13 complex = 128 KiB).
__host__ __device__ constexpr uint32_t fft_parts_log(uint32_t logn) { return logn <= 13 ? 0 : logn - 13; }

}  // namespace th
