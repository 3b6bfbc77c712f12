// GPU CKKS encode fused with the RNS preparation of encrypt_pk
// (tensafe-he-core/src/encoding.rs:173-207, :250-278; ciphertext.rs:250-296).
//
//   z~_re[k] = z~_re[N-1-k] = z[k] (k < N/2), z~_im = 0
//   a = FFT(z~)                      radix-2 DIT, the reference's order
//   coeff_j = (a_re_j / N) * cos(pi j/N) + (a_im_j / N) * sin(pi j/N)
//   m_j = round(coeff_j * 2^40) as i64 (half away from zero, saturating)
// then per limb l:  M_l = (m + e0) mod q_l,  E1_l = e1 mod q_l,  U_l = u mod q_l
// which the forward NTT and the combine kernel turn into the ciphertext. A
// job with mvals set writes m itself instead (the LoRA set's token pass: its
// encrypt transforms form the residues as they load, NTT_LOAD_ENC).
// All f64 steps round exactly as on the host (-ffp-contract=off, host
// twiddles), so m is bit-identical to the reference encoder's.
#include "fft_device.h"
#include "sample_device.h"

namespace th {

constexpr int ENC_THREADS = 1024;

// Part `part` of encode job `job`: the first lb = logn - LP stages of the
// N-point transform over the elements whose bit-reversed position lies in the
// part, in LDS (sh), written to the job's parts scratch. Any block size works:
// every loop strides by blockDim.x.
template <int LP>
__device__ __forceinline__ void encode_part(const EncodeJob* __restrict__ jobs, const double* __restrict__ stage_re,
                                            const double* __restrict__ stage_im, uint32_t logn,
                                            const double* __restrict__ z_base, uint32_t part, uint32_t job,
                                            double* sh) {
  const uint32_t n = 1u << logn, S = n / 2;
  const uint32_t M = n >> LP;
  const EncodeJob jb = jobs[job];
  const GPtr<double> z = gld(z_base ? z_base + (size_t)job * (jb.rep_d ? jb.rep_d : S) : jb.z);
  const uint32_t MP = fft_pad(M);  // padded length of re and im
  double* re = sh;
  double* im = sh + MP;
  const uint32_t r = brv_bits(part, LP);
  const uint32_t lb = logn - LP;
  // With 8 or more parts the in-part stages' twiddles (entries 0 .. M-2 of
  // the stage tables) are staged in LDS beside the values, read in the same
  // coalesced phase as the input instead of once per register pass.
  constexpr bool TWL = LP >= 3;
  const double* twr = stage_re;
  const double* twi = stage_im;
  // 8 entries of each table per thread per round (one round with
  // blockDim.x = M / 8), all loads issued before the first LDS store
  constexpr int FV = 8;
  if constexpr (TWL) {
    double* tr = sh + 2 * MP;
    double* ti = sh + 2 * MP + M;
    for (uint32_t i0 = threadIdx.x; i0 + 1 < M; i0 += FV * blockDim.x) {
      double a[FV], b[FV];
#pragma unroll
      for (int e = 0; e < FV; ++e) {
        const uint32_t i = i0 + e * blockDim.x;
        const uint32_t ic = i + 1 < M ? i : 0;
        a[e] = gld(stage_re)[ic];
        b[e] = gld(stage_im)[ic];
      }
#pragma unroll
      for (int e = 0; e < FV; ++e) {
        const uint32_t i = i0 + e * blockDim.x;
        if (i + 1 < M) {
          tr[i] = a[e];
          ti[i] = b[e];
        }
      }
    }
    twr = tr;
    twi = ti;
  }
  // input gather, 8 values per thread per round: all loads issued before the
  // first LDS store
  const double g = jb.gate ? *gld(jb.gate) : 1.0;
  for (uint32_t j0 = threadIdx.x; j0 < M; j0 += FV * blockDim.x) {
    double v[FV];
#pragma unroll
    for (int e = 0; e < FV; ++e) {
      const uint32_t jj = j0 + e * blockDim.x;
      const bool in = jj < M;
      const uint32_t j = ((in ? jj : 0) << LP) | r;  // element at bit-reversed position part*M + brv(jj)
      const uint32_t slot = j < S ? j : n - 1 - j;
      bool keep = in;
      uint32_t idx = slot;
      if (jb.rep_d) {  // inference_engine.py:1266-1269: [h | h | ... | 0]
        keep = keep && slot < jb.rep_cols * jb.rep_d;
        idx = keep ? slot % jb.rep_d : 0;
      }
      double t = z[idx];  // unconditional (index 0 when unused), so the loads issue together
      if (jb.gate) t = slot < jb.n_valid ? g * t : 0.0;  // the same f64 products as gating on the host
      v[e] = keep ? t : 0.0;
    }
#pragma unroll
    for (int e = 0; e < FV; ++e) {
      const uint32_t jj = j0 + e * blockDim.x;
      if (jj < M) {
        const uint32_t pos = fft_pad(brv_bits(jj, lb));
        re[pos] = v[e];
        im[pos] = 0.0;
      }
    }
  }
  __syncthreads();
  dit_stages_reg<true>(re, im, lb, twr, twi);
  const GMut<double> out = gst(jb.parts) + (size_t)part * 2 * M;
  for (uint32_t i0 = threadIdx.x; i0 < M; i0 += FV * blockDim.x) {
    double a[FV], b[FV];
#pragma unroll
    for (int e = 0; e < FV; ++e) {
      const uint32_t i = i0 + e * blockDim.x;
      const uint32_t ic = fft_pad(i < M ? i : 0);
      a[e] = re[ic];
      b[e] = im[ic];
    }
#pragma unroll
    for (int e = 0; e < FV; ++e) {
      const uint32_t i = i0 + e * blockDim.x;
      if (i < M) {
        out[i] = a[e];
        out[M + i] = b[e];
      }
    }
  }
}

template <int LP>
__global__ __launch_bounds__(ENC_THREADS) void k_encode_parts(const EncodeJob* __restrict__ jobs,
                                                              const double* __restrict__ stage_re,
                                                              const double* __restrict__ stage_im, uint32_t logn,
                                                              const double* __restrict__ z_base) {
  extern __shared__ double sh[];
  encode_part<LP>(jobs, stage_re, stage_im, logn, z_base, blockIdx.x, blockIdx.y, sh);
}

// k_encode_parts with the sampler's blocks of the same jobs (sample[y] for
// encode job y) as further workgroups: x < 2^LP encodes part x, every later
// workgroup draws SPT * SAMPLE_ENC_THREADS ChaCha20 blocks of job y's stream,
// one per thread per step (k_sample_blocks' work). The sampler's VALU-bound
// workgroups and the encoder's latency-bound ones share the CUs instead of
// running one launch after the other.
constexpr uint32_t SAMPLE_ENC_THREADS = 256;
template <int LP, int SPT>
__global__ __launch_bounds__(SAMPLE_ENC_THREADS) void k_sample_encode_parts(
    const EncodeJob* __restrict__ jobs, const double* __restrict__ stage_re, const double* __restrict__ stage_im,
    uint32_t logn, const double* __restrict__ z_base, const SampleJob* __restrict__ sample, SeedBlock sb, int use_sb,
    BandArgs band) {
  extern __shared__ double sh[];
  constexpr uint32_t P = 1u << LP;
  if (blockIdx.x < P) {
    encode_part<LP>(jobs, stage_re, stage_im, logn, z_base, blockIdx.x, blockIdx.y, sh);
    return;
  }
  const SampleJob jb = sample[blockIdx.y];
  const uint64_t seed = job_seed(jb, sb, use_sb, blockIdx.y);
  const FlagOut flag = flag_of(band, blockIdx.y);
  const uint32_t b0 = (blockIdx.x - P) * SPT * SAMPLE_ENC_THREADS + threadIdx.x;
#pragma unroll 1
  for (int k = 0; k < SPT; ++k) sample_block(jb, seed, 1u << logn, b0 + k * SAMPLE_ENC_THREADS, band.band, flag);
}

// Rust `f64::round() as i64`: half away from zero, saturating, NaN -> 0.
__device__ __forceinline__ int64_t round_sat_i64(double x) {
  const double r = round(x);
  if (r != r) return 0;
  if (r >= 9223372036854775808.0) return INT64_MAX;
  if (r < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)r;
}

// m_j from FFT output a at position j (encoding.rs:186-204).
__device__ __forceinline__ int64_t encoded_m(Cx a, uint32_t j, double inv_n, const double* __restrict__ twist_re,
                                             const double* __restrict__ twist_im) {
  const double a_re = a.re * inv_n;
  const double a_im = a.im * inv_n;
  const double coeff = a_re * twist_re[j] + a_im * twist_im[j];
  return round_sat_i64(coeff * 1099511627776.0);  // * 2^40 (params.rs:12)
}

__device__ __forceinline__ void emit_coefficient(const EncodeJob& jb, const BarrettConst* __restrict__ bc,
                                                 const double* __restrict__ twist_re,
                                                 const double* __restrict__ twist_im, uint32_t j, Cx a,
                                                 double inv_n, uint32_t n, uint32_t L) {
  const int64_t m = encoded_m(a, j, inv_n, twist_re, twist_im);
  if (jb.mvals) {
    gst(jb.mvals)[j] = m;
    return;
  }
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

// The FFT outputs at positions p*M + k of all P parts (x[p]), from the parts' stage-lb values.
template <int LP>
__device__ __forceinline__ void combine_parts(GPtr<double> Pd, uint32_t k, uint32_t M, GPtr<double> wr,
                                              GPtr<double> wi, Cx (&x)[1 << LP]) {
  constexpr int P = 1 << LP;
#pragma unroll
  for (int p = 0; p < P; ++p) x[p] = Cx{Pd[(size_t)p * 2 * M + k], Pd[(size_t)p * 2 * M + M + k]};
#pragma unroll
  for (int t = 0; t < LP; ++t) {
    const uint32_t half = M << t;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (p & (1 << t)) continue;
      const uint32_t w = half - 1 + (uint32_t)(p & ((1 << t) - 1)) * M + k;
      dit(x[p], x[p | (1 << t)], wr[w], wi[w], x[p], x[p | (1 << t)]);
    }
  }
}

// The last LP stages combine element k of every part: position p*M + k of
// stage lb + t pairs with the part whose index differs in bit t, and its
// twiddle index is its position modulo the stage's half size, (p mod 2^t)*M + k,
// the same operands and twiddles as dit_stages_lds, so the result is
// bit-identical to one transform of N values. G = 2^LP / 4 threads share a
// position k (thread o of them emits parts s*G + o); each recomputes the
// small combine, which costs far less than the residues it writes.
template <int LP>
__global__ __launch_bounds__(256) void k_encode_final(const EncodeJob* __restrict__ jobs,
                                                      const BarrettConst* __restrict__ bc,
                                                      const double* __restrict__ twist_re,
                                                      const double* __restrict__ twist_im,
                                                      const double* __restrict__ stage_re,
                                                      const double* __restrict__ stage_im, uint32_t logn,
                                                      uint32_t L, const SampleJob* __restrict__ fix, SeedBlock sb,
                                                      int use_sb, int force_serial, BandArgs band) {
  constexpr int P = 1 << LP;
  constexpr int G = P >= 4 ? P / 4 : 1;
  const uint32_t n = 1u << logn, lb = logn - LP;
  // the sampler's blocks of this launch's jobs ran before this kernel: replay
  // a job whose u words held a rejected value (jobs with fix write mvals, so
  // no thread of this kernel reads the randomness being rewritten)
  if (fix && blockIdx.x == 0 && threadIdx.x == 0) {
    const SampleJob sj = fix[blockIdx.y];
    sample_fix_job(sj, job_seed(sj, sb, use_sb, blockIdx.y), n, force_serial, flag_of(band, blockIdx.y), band.band);
  }
  const uint32_t M = n >> LP;
  const EncodeJob jb = jobs[blockIdx.y];
  const GPtr<double> Pd = gld(jb.parts);
  const GPtr<double> wr = gld(stage_re), wi = gld(stage_im);
  const double inv_n = 1.0 / (double)n;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < G * M; i += gridDim.x * blockDim.x) {
    const uint32_t o = i >> lb, k = i & (M - 1);  // o is uniform over a wavefront (M >= 64)
    Cx x[P];
    combine_parts<LP>(Pd, k, M, wr, wi, x);
#pragma unroll
    for (int s = 0; s < P / G; ++s) {
      Cx v = x[s * G];
#pragma unroll
      for (int g = 1; g < G; ++g)
        if (o == (uint32_t)g) v = x[s * G + g];
      emit_coefficient(jb, bc, twist_re, twist_im, (uint32_t)(s * G) * M + o * M + k, v, inv_n, n, L);
    }
  }
}

// k_encode_final for groups of fold consecutive jobs (the experts of one
// mixture batch) summed into one residue polynomial: group b writes, for each
// limb l of limb_mask (at most ENC_FOLD_MAX_LIMBS of them), the sum over its
// jobs x of (m_x mod q_l) mod q_l at jobs[b * fold].dst + l n: the residues
// k_encode_final writes for each job (encoded_m, signed_residue_dev), summed.
template <int LP>
__global__ __launch_bounds__(256) void k_encode_final_fold(const EncodeJob* __restrict__ jobs, uint32_t fold,
                                                           uint32_t limb_mask, const BarrettConst* __restrict__ bc,
                                                           const double* __restrict__ twist_re,
                                                           const double* __restrict__ twist_im,
                                                           const double* __restrict__ stage_re,
                                                           const double* __restrict__ stage_im, uint32_t logn) {
  constexpr int P = 1 << LP;
  constexpr int G = P >= 4 ? P / 4 : 1;
  constexpr int C = P / G;  // coefficients per thread and job
  constexpr int ML = ENC_FOLD_MAX_LIMBS;
  const uint32_t n = 1u << logn, lb = logn - LP;
  const uint32_t M = n >> LP;
  const EncodeJob* grp = jobs + (size_t)blockIdx.y * fold;
  uint32_t limb[ML];
  uint32_t nl = 0;
  for (uint32_t l = 0; l < 32 && nl < (uint32_t)ML; ++l)
    if (limb_mask >> l & 1) limb[nl++] = l;
  const GMut<uint64_t> dst = gst(grp[0].dst);
  const GPtr<double> wr = gld(stage_re), wi = gld(stage_im);
  const double inv_n = 1.0 / (double)n;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < G * M; i += gridDim.x * blockDim.x) {
    const uint32_t o = i >> lb, k = i & (M - 1);  // o is uniform over a wavefront (M >= 64)
    uint64_t acc[C][ML];
#pragma unroll
    for (int s = 0; s < C; ++s)
#pragma unroll
      for (int t = 0; t < ML; ++t) acc[s][t] = 0;
    for (uint32_t e = 0; e < fold; ++e) {
      Cx x[P];
      combine_parts<LP>(gld(grp[e].parts), k, M, wr, wi, x);
#pragma unroll
      for (int s = 0; s < C; ++s) {
        Cx v = x[s * G];
#pragma unroll
        for (int g = 1; g < G; ++g)
          if (o == (uint32_t)g) v = x[s * G + g];
        const uint32_t j = (uint32_t)(s * G) * M + o * M + k;
        const int64_t m = encoded_m(v, j, inv_n, twist_re, twist_im);
#pragma unroll
        for (int t = 0; t < ML; ++t) {
          if (t >= (int)nl) break;
          const BarrettConst c = bc[limb[t]];
          acc[s][t] = addmod(acc[s][t], signed_residue_dev(m, c), c.q);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < C; ++s) {
      const uint32_t j = (uint32_t)(s * G) * M + o * M + k;
#pragma unroll
      for (int t = 0; t < ML; ++t) {
        if (t >= (int)nl) break;
        dst[(size_t)limb[t] * n + j] = acc[s][t];
      }
    }
  }
}

size_t encode_parts_doubles(uint32_t logn) { return (size_t)2 << logn; }

hipError_t launch_encode(const EncodeJob* jobs, uint32_t njobs, const BarrettConst* bc, const double* twist_re,
                         const double* twist_im, const double* stage_re, const double* stage_im, uint32_t logn,
                         uint32_t L, hipStream_t s, const double* z_base, const SampleJob* sample,
                         const uint64_t* seeds, int force_serial, BandArgs band, uint32_t fold, uint32_t fold_limbs) {
  if (!njobs) return hipSuccess;
  const uint32_t n = 1u << logn;
  if (sample && (njobs > SEEDS_PER_LAUNCH || fold || n % 16)) return hipErrorInvalidValue;
  if (fold && (njobs % fold || !fold_limbs || __builtin_popcount(fold_limbs) > (int)ENC_FOLD_MAX_LIMBS ||
               (L < 32 && fold_limbs >> L)))
    return hipErrorInvalidValue;
  SeedBlock sb{};
  if (sample && seeds)
    for (uint32_t i = 0; i < njobs; ++i) sb.v[i] = seeds[i];
  const int use_sb = seeds != nullptr;
  // parts of at most 4096 values (two workgroups' LDS per CU; with 672
  // encodes of N=16384 per CryptoMOE token, the token measured 0.656 ms with
  // 4096-value parts against 0.697 ms with 8192, 0.675 ms with 2048 and
  // 0.727 ms with 1024); more parts (up to 16, of at least 1024 values)
  // while the batch would leave CUs idle: the parts are independent
  // workgroups and the result is the same for any split
  const uint32_t lp_min = fft_parts_log(logn);
  uint32_t lp = logn > 12 && logn - 12 > lp_min ? logn - 12 : lp_min;
  while (lp < 4 && logn - lp > 10 && njobs * (1u << lp) < 512) ++lp;
  const uint32_t M = n >> lp;
  // padded values (+ twiddles with 8 or more parts)
  const size_t lds = ((size_t)2 * fft_pad(M) + (lp >= 3 ? (size_t)2 * M : 0)) * sizeof(double);
  // dit_stages_reg needs 8 values per thread at most
  const uint32_t threads = M / 8 < 64 ? 64 : (M / 8 > ENC_THREADS ? ENC_THREADS : M / 8);
  const uint32_t fin = lp >= 2 ? M << (lp - 2) : M;  // threads of the final kernel per encode
  const uint32_t gx = (fin + 255) / 256 < 32 ? (fin + 255) / 256 : 32;
  // With sample, the sampler's workgroups join the parts kernel while a part
  // leaves LDS for several workgroups per CU (at most 1024 values, 34 KiB:
  // four per CU); each thread draws two blocks where one each would make more
  // workgroups than the CUs hold at once. Per token of 28 encodes at
  // N=16384: 0.2241 ms with two blocks per thread, 0.2249 ms with one,
  // 0.2296 ms with the sampler launched on its own before the encoder.
  // Larger parts keep a sampler launch of their own. Either way the final
  // kernel finishes the rejection handling.
  const bool merge = sample && M <= 1024;
  hipError_t e;
  if (sample && !merge) {
    e = launch_sample_pk(sample, njobs, n, force_serial, s, seeds, true, true, band);
    if (e != hipSuccess) return e;
  }
  const uint32_t sblocks = 9 * (n / 16);  // ChaCha20 blocks per job
  uint32_t spt = 1;
  if (merge) {
    constexpr uint32_t WG_PER_CU_WAVES = 7;  // 28 waves per CU at this kernel's VGPRs
    const uint32_t per_cu = (uint32_t)((160u * 1024) / lds) < WG_PER_CU_WAVES ? (uint32_t)((160u * 1024) / lds)
                                                                              : WG_PER_CU_WAVES;
    if (njobs * ((1u << lp) + (sblocks + SAMPLE_ENC_THREADS - 1) / SAMPLE_ENC_THREADS) > device_cu_count() * per_cu)
      spt = 2;
  }
  const uint32_t sx = (sblocks + spt * SAMPLE_ENC_THREADS - 1) / (spt * SAMPLE_ENC_THREADS);
#define TH_ENC(LP)                                                                                              \
  case LP:                                                                                                      \
    if (merge) {                                                                                                \
      const dim3 grid((1u << LP) + sx, njobs);                                                                  \
      if (spt == 2)                                                                                             \
        hipLaunchKernelGGL((k_sample_encode_parts<LP, 2>), grid, dim3(SAMPLE_ENC_THREADS), lds, s, jobs,        \
                           stage_re, stage_im, logn, z_base, sample, sb, use_sb, band);                         \
      else                                                                                                      \
        hipLaunchKernelGGL((k_sample_encode_parts<LP, 1>), grid, dim3(SAMPLE_ENC_THREADS), lds, s, jobs,        \
                           stage_re, stage_im, logn, z_base, sample, sb, use_sb, band);                         \
    } else {                                                                                                    \
      e = allow_full_lds<k_encode_parts<LP>>();                                                                 \
      if (e != hipSuccess) return e;                                                                            \
      hipLaunchKernelGGL(k_encode_parts<LP>, dim3(1u << LP, njobs), dim3(threads), lds, s, jobs, stage_re,      \
                         stage_im, logn, z_base);                                                               \
    }                                                                                                           \
    if (fold)                                                                                                   \
      hipLaunchKernelGGL(k_encode_final_fold<LP>, dim3(gx, njobs / fold), dim3(256), 0, s, jobs, fold,          \
                         fold_limbs, bc, twist_re, twist_im, stage_re, stage_im, logn);                         \
    else                                                                                                        \
      hipLaunchKernelGGL(k_encode_final<LP>, dim3(gx, njobs), dim3(256), 0, s, jobs, bc, twist_re, twist_im,    \
                         stage_re, stage_im, logn, L, sample, sb, use_sb, force_serial, band);                  \
    return hipGetLastError();
  switch (lp) {
    TH_ENC(0)
    TH_ENC(1)
    TH_ENC(2)
    TH_ENC(3)
    TH_ENC(4)
    default: return hipErrorInvalidValue;
  }
#undef TH_ENC
}

}  // namespace th
