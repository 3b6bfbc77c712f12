// GPU-resident decode of decrypted polynomials (tensafe-he-core/src/encoding.rs
// :219-239 and :282-315, ciphertext.rs:351-399).
//
// Evaluation order and rounding follow the reference exactly (this file is
// compiled with -ffp-contract=off, twiddles are the host's glibc values), so
// the decoded slots are bit-identical to the reference CPU decode:
//   coefficient: centre against q0/2 (or the 2-limb CRT value against
//                q0*q1/2), convert to f64 (round to nearest even), / scale
//   twist:       b = c * (cos(pi j/N), -sin(pi j/N))
//   FFT:         bit-reversal permutation, radix-2 DIT stages with
//                v = w*x[i1]; x[i0] = u + v; x[i1] = u - v
//   output:      real parts of the first N/2 values.
//
// The N complex values (256 KiB at N = 16384) exceed LDS, so the transform is
// split: after the bit-reversal, stages 0 .. logN-p-1 act inside 2^p
// independent parts of N/2^p values (one workgroup each, in LDS); the last p
// stages combine the parts element-wise in a second kernel, which also forms
// the ZeRo-MOAI segment sums.
#include "fft_device.h"
#include "poly_kernels.h"

namespace th {

// Rust `u128 as f64`: round to nearest, ties to even.
__device__ __forceinline__ double u128_to_f64(uint64_t hi, uint64_t lo) {
  if (hi == 0) return (double)lo;
  const int lz = __clzll(hi);
  const uint64_t h = lz ? ((hi << lz) | (lo >> (64 - lz))) : hi;
  const uint64_t l = lo << lz;
  uint64_t mant = h >> 11;
  const uint64_t rem = h & 0x7FFu;
  if (rem > 0x400u || (rem == 0x400u && (l != 0 || (mant & 1)))) ++mant;
  return ldexp((double)mant, 75 - lz);
}

// Decrypted coefficient j, centred (or CRT-combined and centred), as f64.
__device__ __forceinline__ double coeff_centred(const DecodeJob& jb, const DecodeConst& dc, uint32_t j, uint32_t n) {
  if (!jb.crt) {
    const uint64_t c = gld(jb.m)[j];
    return c > dc.half_q0 ? -((double)(dc.q0 - c)) : (double)c;
  }
  // ciphertext.rs:360-392
  const uint64_t m0 = gld(jb.m)[j], m1 = gld(jb.m)[n + j];
  const uint64_t m0q1 = m0 < dc.q1 ? m0 : mulmod_barrett(m0, 1, dc.b1);
  const uint64_t diff = m1 >= m0q1 ? m1 - m0q1 : dc.q1 - m0q1 + m1;
  const uint64_t k = csub(shoup_lazy(diff, dc.q0_inv_q1, dc.q0_inv_q1_s, dc.q1), dc.q1);
  // M = m0 + k * q0 (128-bit)
  uint64_t lo = k * dc.q0;
  uint64_t hi = __umul64hi(k, dc.q0);
  lo += m0;
  hi += lo < m0 ? 1 : 0;
  if (hi > dc.Q_hi || (hi == dc.Q_hi && lo >= dc.Q_lo)) {  // M >= Q (unreachable for canonical inputs)
    const uint64_t nlo = lo - dc.Q_lo;
    hi = hi - dc.Q_hi - (lo < dc.Q_lo ? 1 : 0);
    lo = nlo;
  }
  if (hi > dc.halfQ_hi || (hi == dc.halfQ_hi && lo > dc.halfQ_lo)) {
    const uint64_t dlo = dc.Q_lo - lo;
    const uint64_t dhi = dc.Q_hi - hi - (dc.Q_lo < lo ? 1 : 0);
    return -u128_to_f64(dhi, dlo);
  }
  return u128_to_f64(hi, lo);
}

// The reference's f64 coefficient value before the twist (encoding.rs:221-233,
// ciphertext.rs:360-392): centred value / scale.
__device__ __forceinline__ double coeff_value(const DecodeJob& jb, const DecodeConst& dc, uint32_t j, uint32_t n) {
  return coeff_centred(jb, dc, j, n) / jb.scale;
}

constexpr int DEC_THREADS = 1024;

template <int LP>
__global__ __launch_bounds__(DEC_THREADS) void k_decode_parts(const DecodeJob* __restrict__ jobs, const DecodeConst* dcp,
                                                              const double* __restrict__ twist_re,
                                                              const double* __restrict__ twist_im,
                                                              const double* __restrict__ stage_re,
                                                              const double* __restrict__ stage_im, uint32_t logn) {
  extern __shared__ double sh[];
  const DecodeConst dc = *dcp;
  const uint32_t n = 1u << logn;
  const uint32_t M = n >> LP;
  const uint32_t part = blockIdx.x;
  const DecodeJob jb = jobs[blockIdx.y];
  double* re = sh;
  double* im = sh + M;
  const uint32_t r = brv_bits(part, LP);
  const uint32_t lb = logn - LP;
  for (uint32_t jj = threadIdx.x; jj < M; jj += blockDim.x) {
    const uint32_t j = (jj << LP) | r;
    const double c = coeff_value(jb, dc, j, n);
    const uint32_t pos = brv_bits(jj, lb);
    re[pos] = c * twist_re[j];
    im[pos] = -c * twist_im[j];
  }
  __syncthreads();
  dit_stages_reg(re, im, lb, stage_re, stage_im);
  const GMut<double> out = gst(jb.parts) + (size_t)part * 2 * M;
  for (uint32_t i = threadIdx.x; i < M; i += blockDim.x) {
    out[i] = re[i];
    out[M + i] = im[i];
  }
}

template <int LP>
__global__ __launch_bounds__(DEC_THREADS) void k_decode_final(const DecodeJob* __restrict__ jobs,
                                                              const double* __restrict__ stage_re,
                                                              const double* __restrict__ stage_im, uint32_t logn,
                                                              uint32_t d, uint32_t cols) {
  extern __shared__ double dec[];
  const uint32_t n = 1u << logn;
  const uint32_t S = n / 2;
  const uint32_t M = n >> LP;
  const DecodeJob jb = jobs[blockIdx.x];
  const GPtr<double> P = gld(jb.parts);
  auto at = [&](uint32_t part, uint32_t i) { return Cx{P[(size_t)part * 2 * M + i], P[(size_t)part * 2 * M + M + i]}; };
  if constexpr (LP == 0) {
    for (uint32_t k = threadIdx.x; k < S; k += blockDim.x) dec[k] = P[k];
  } else if constexpr (LP == 1) {
    const double* wr = stage_re + (S - 1);
    const double* wi = stage_im + (S - 1);
    for (uint32_t k = threadIdx.x; k < S; k += blockDim.x) {
      const Cx u = at(0, k), x = at(1, k);
      const double v_re = wr[k] * x.re - wi[k] * x.im;
      dec[k] = u.re + v_re;
    }
  } else {  // LP == 2
    const uint32_t Q4 = n / 4;
    const double* w1r = stage_re + (Q4 - 1);
    const double* w1i = stage_im + (Q4 - 1);
    const double* w2r = stage_re + (S - 1);
    const double* w2i = stage_im + (S - 1);
    for (uint32_t k = threadIdx.x; k < Q4; k += blockDim.x) {
      Cx y0, y1, y2, y3;
      dit(at(0, k), at(1, k), w1r[k], w1i[k], y0, y1);  // positions k, k + N/4
      dit(at(2, k), at(3, k), w1r[k], w1i[k], y2, y3);  // positions N/2 + k, 3N/4 + k
      dec[k] = y0.re + (w2r[k] * y2.re - w2i[k] * y2.im);
      dec[k + Q4] = y1.re + (w2r[k + Q4] * y3.re - w2i[k + Q4] * y3.im);
    }
  }
  __syncthreads();
  if (jb.out)
    for (uint32_t k = threadIdx.x; k < S; k += blockDim.x) gst(jb.out)[k] = dec[k];
  if (jb.seg) {
    // one wavefront per segment; lane-strided partial sums, then a fixed butterfly tree
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nwaves = blockDim.x >> 6;
    for (uint32_t sg = wave; sg < cols; sg += nwaves) {
      double acc = 0.0;
      const uint32_t base = sg * d;
      for (uint32_t i = lane; i < d; i += 64)
        if (base + i < S) acc += dec[base + i];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
      if (lane == 0) gst(jb.seg)[sg] = acc;
    }
  }
}

size_t decode_parts_doubles(uint32_t logn) { return (size_t)2 << logn; }

// ZeRo-MOAI segment sums straight from the decrypted coefficients:
// seg[c] = (sum_j m_j W[c][j]) / scale with m_j the decode's centred (or
// CRT-combined) coefficient and W the host-computed segment weights. Equal to
// decoding and summing the slots up to rounding (the slots themselves are
// never formed). Each job is cut into SEGSUM_CHUNKS chunks of coefficients,
// one workgroup each, whose partial sums go to the job's scratch (parts);
// a second kernel adds them in chunk order, so results are deterministic.
constexpr uint32_t SEGSUM_CHUNKS = 16;

template <int MAXC>
__global__ __launch_bounds__(256) void k_segsum_partial(const DecodeJob* __restrict__ jobs,
                                                        const DecodeConst* __restrict__ dcp,
                                                        const double* __restrict__ W, uint32_t n, uint32_t cols) {
  __shared__ double part[4][MAXC];
  const DecodeConst dc = *dcp;
  const DecodeJob jb = jobs[blockIdx.y];
  const uint32_t len = n / SEGSUM_CHUNKS, base = blockIdx.x * len;
  double acc[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) acc[c] = 0.0;
  for (uint32_t j = base + threadIdx.x; j < base + len; j += blockDim.x) {
    const double v = coeff_centred(jb, dc, j, n);
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
      if (c < (int)cols) acc[c] += v * W[(size_t)c * n + j];
  }
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    double a = acc[c];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) a += __shfl_xor(a, off);
    if (lane == 0) part[wave][c] = a;
  }
  __syncthreads();
  if (threadIdx.x < cols) {
    const int c = threadIdx.x;
    gst(jb.parts)[blockIdx.x * cols + c] = (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
  }
}

__global__ void k_segsum_final(const DecodeJob* __restrict__ jobs, uint32_t njobs, uint32_t cols) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= njobs * cols) return;
  const DecodeJob jb = jobs[t / cols];
  const uint32_t c = t % cols;
  double s = 0.0;
  for (uint32_t k = 0; k < SEGSUM_CHUNKS; ++k) s += gld(jb.parts)[k * cols + c];
  gst(jb.seg)[c] = s / jb.scale;
}

size_t segsum_parts_doubles(uint32_t cols) { return (size_t)SEGSUM_CHUNKS * cols; }

hipError_t launch_segsum(const DecodeJob* jobs, uint32_t njobs, const DecodeConst* dc, const double* W,
                         uint32_t logn, uint32_t cols, hipStream_t s) {
  if (!njobs) return hipSuccess;
  if (cols < 1 || cols > SEGSUM_MAX_COLS) return hipErrorInvalidValue;
  const uint32_t n = 1u << logn;
  const dim3 grid(SEGSUM_CHUNKS, njobs);
  if (cols <= 8)
    hipLaunchKernelGGL(k_segsum_partial<8>, grid, dim3(256), 0, s, jobs, dc, W, n, cols);
  else
    hipLaunchKernelGGL(k_segsum_partial<SEGSUM_MAX_COLS>, grid, dim3(256), 0, s, jobs, dc, W, n, cols);
  hipLaunchKernelGGL(k_segsum_final, dim3((njobs * cols + 255) / 256), dim3(256), 0, s, jobs, njobs, cols);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeJob* jobs, uint32_t njobs, const DecodeConst* dc, const double* twist_re,
                         const double* twist_im, const double* stage_re, const double* stage_im, uint32_t logn,
                         uint32_t d, uint32_t cols, hipStream_t s) {
  if (!njobs) return hipSuccess;
  const uint32_t lp = fft_parts_log(logn);
  const uint32_t M = (1u << logn) >> lp;
  const size_t lds_a = (size_t)2 * M * sizeof(double);
  const size_t lds_b = (size_t)(1u << logn) / 2 * sizeof(double);
  hipError_t e;
#define TH_DEC(LP)                                                                                         \
  case LP:                                                                                                 \
    e = allow_full_lds<k_decode_parts<LP>>();                                                              \
    if (e != hipSuccess) return e;                                                                         \
    e = allow_full_lds<k_decode_final<LP>>();                                                              \
    if (e != hipSuccess) return e;                                                                         \
    hipLaunchKernelGGL(k_decode_parts<LP>, dim3(1u << LP, njobs), dim3(DEC_THREADS), lds_a, s, jobs, dc,   \
                       twist_re, twist_im, stage_re, stage_im, logn);                                      \
    hipLaunchKernelGGL(k_decode_final<LP>, dim3(njobs), dim3(DEC_THREADS), lds_b, s, jobs, stage_re,       \
                       stage_im, logn, d, cols);                                                           \
    return hipGetLastError();
  switch (lp) {
    TH_DEC(0)
    TH_DEC(1)
    TH_DEC(2)
    default: return hipErrorInvalidValue;
  }
#undef TH_DEC
}

}  // namespace th
