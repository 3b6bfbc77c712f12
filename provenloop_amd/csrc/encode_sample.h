// Job descriptors and launchers of the GPU encoder and randomness sampler.
#pragma once
#include "th_internal.h"

namespace th {

struct EncodeJob {
  const double* z;     // N/2 padded slots, or (rep_d > 0) one d-value vector
  uint32_t rep_d;      // > 0: slots are rep_cols copies of z[0..rep_d) then zeros (ZeRo-MOAI replication)
  uint32_t rep_cols;
  const uint8_t* u;    // sample_ternary values {0,1,2}, or null
  const int64_t* e0;   // rounded Gaussian e0, or null (plain encode)
  const int64_t* e1;   // rounded Gaussian e1, or null
  uint64_t* dst;       // [M (L) | E1 (L) | U (L)] limb-polys; only M when e1/u are null
  int64_t* mvals;      // non-null: write m itself (N i64) instead of dst (the residues are then
                       // formed by the encrypt transforms' loads, NTT_LOAD_ENC)
  double* parts;       // scratch, encode_parts_doubles(logn) doubles
  const double* gate;  // non-null (no replication): slots are gate[0] * z[slot] for slot < n_valid,
                       // 0 beyond (a gated expert's packed rows, inference_engine.py:1300-1308)
  uint32_t n_valid;
};

struct SampleJob;
// Seeds travel with a sampler launch for up to this many jobs.
constexpr uint32_t SEEDS_PER_LAUNCH = 64;

// Band flags of a sampler launch: flags[j] (one byte per job, in host-visible
// memory; null for none) is set to 1 when a Gaussian draw of job j lands
// within `band` of a rounding boundary (near_rounding_boundary), where the
// device's log/cos could round differently from glibc's. The host then
// redraws that job's randomness with glibc. With dflags, dflags[j] (device
// memory) is set to gen as well, for kernels later on the stream that check a
// job's flag without a read across PCIe (a value left by an earlier launch
// holds an older generation, so the array needs no clearing).
struct BandArgs {
  uint8_t* flags;
  double band;
  uint32_t* dflags = nullptr;
  uint32_t gen = 0;
};
// The flags of launch `b` from job `first` on.
inline BandArgs band_from(const BandArgs& b, uint32_t first) {
  return BandArgs{b.flags ? b.flags + first : nullptr, b.band, b.dflags ? b.dflags + first : nullptr, b.gen};
}
// One job's band-flag outputs (FlagOut::raise sets both).
struct FlagOut {
  uint8_t* host;
  uint32_t* dev;
  uint32_t gen;
  __device__ void raise() const {
    if (host) *host = 1;
    if (dev) *dev = gen;
  }
};
__device__ inline FlagOut flag_of(const BandArgs& b, uint32_t j) {
  return FlagOut{b.flags ? b.flags + j : nullptr, b.dflags ? b.dflags + j : nullptr, b.gen};
}
// Default band: 2^-36, about 2^9 times the largest difference between the
// device's and glibc's z * 3.19.
constexpr double SAMPLER_BAND_DEFAULT = 0x1p-36;

// Encode z and write the per-limb residues of m (+ e0), e1 and u. With
// z_base, job i reads its input at z_base + i * (rep_d, or N/2 without
// replication) instead of its z field. With sample (one flagged sampler job
// per encode job, at most SEEDS_PER_LAUNCH of them, seeds as in
// launch_sample_pk; the encode jobs must write mvals), the launch also draws
// those jobs' encrypt_pk randomness, as launch_sample_pk(flagged) would,
// rejection handling and band flags included. With fold
// > 0, every fold consecutive jobs are summed into one residue polynomial
// (the experts of a mixture batch): the group's first job's dst receives, on
// the limbs in fold_limbs (at most ENC_FOLD_MAX_LIMBS), the sum mod q_l of
// the residues each job would write; the jobs' other outputs are unused.
constexpr uint32_t ENC_FOLD_MAX_LIMBS = 4;
hipError_t launch_encode(const EncodeJob* jobs, uint32_t njobs, const BarrettConst* bc, const double* twist_re,
                         const double* twist_im, const double* stage_re, const double* stage_im, uint32_t logn,
                         uint32_t L, hipStream_t s, const double* z_base = nullptr, const SampleJob* sample = nullptr,
                         const uint64_t* seeds = nullptr, int force_serial = 0, BandArgs band = BandArgs{nullptr, 0.0},
                         uint32_t fold = 0, uint32_t fold_limbs = 0);
size_t encode_parts_doubles(uint32_t logn);

struct SampleJob {
  uint64_t seed;     // TenSafeRng::from_seed(seed)
  uint8_t* u;        // n ternary values
  int64_t* e0;       // n rounded Gaussians
  int64_t* e1;       // n rounded Gaussians
  uint32_t* reject;  // zero-initialised flag set when a u word is rejected, or null
};

// encrypt_pk's randomness (ciphertext.rs:255-273) for each job, drawn from the
// job's ChaCha20 stream in the reference's order. force_serial makes every job
// take the serial path that handles range_u32 rejections (for testing). With
// seeds (host array, one per job) the jobs' seed fields are ignored and the
// seeds travel in the launch arguments. Jobs with a reject flag (all or none
// of them) skip the re-derivation pass: the block kernel raises the flag and
// only flagged jobs are replayed; the flag is cleared again. band: the band
// flags of the njobs jobs (BandArgs).
hipError_t launch_sample_pk(const SampleJob* jobs, uint32_t njobs, uint32_t n, int force_serial, hipStream_t s,
                            const uint64_t* seeds, bool flagged, bool fix_later, BandArgs band);

// Key and secret-key-encryption randomness drawn on the device from the
// reference's ChaCha20 stream (rng.rs:31-157, sampling.rs:17-64). A job is
// one stretch of a stream: kind KEY_TERNARY is keygen's N x range_u32(3)
// (ciphertext.rs:86-97), written as the signed values -1, 0, 1 it stands for;
// kind KEY_UNIFORM_GAUSS is a = range_u64(q_l) for N coefficients of every
// limb l = 0..L-1, then N rounded Gaussians e (keygen_public,
// ciphertext.rs:119-127, and the secret-key encrypt, :183-196). Job j's draws
// start at word word0 of the stream of its seed and are drawn in parallel as
// if none of its words were rejected (launch_key_draws): *reject receives the
// lowest index of a job that held a rejected word (range_u32: 0; range_u64:
// r < 2^64 mod q_l), for which launch_key_replay draws that job serially in
// the reference's order and writes the word where its draws ended to *end.
// Gaussian draws near a rounding boundary raise their job's band flag
// (BandArgs), for a redraw with glibc.
enum : uint32_t { KEY_TERNARY = 0, KEY_UNIFORM_GAUSS = 1 };
struct KeyDrawJob {
  uint64_t seed;
  uint64_t word0;
  uint32_t kind;
  uint32_t pad_;
  int64_t* s;   // KEY_TERNARY: N values
  uint64_t* a;  // KEY_UNIFORM_GAUSS: L x N residues, limb-major
  int64_t* e;   // KEY_UNIFORM_GAUSS: N values
};
// Stream words a job of `kind` takes when none is rejected.
__host__ __device__ inline uint64_t key_draw_words(uint32_t kind, uint32_t n, uint32_t L) {
  return kind == KEY_TERNARY ? n : (uint64_t)(2 * L + 4) * n;
}
// reject: a device word that must hold 0xFFFFFFFF before the launch.
hipError_t launch_key_draws(const KeyDrawJob* jobs, uint32_t njobs, uint32_t n, uint32_t L, const BarrettConst* bc,
                            uint32_t* reject, BandArgs band, hipStream_t s);
// Serial draws of one job (device job descriptor); band: the job's own flags.
hipError_t launch_key_replay(const KeyDrawJob* job, uint32_t n, uint32_t L, const BarrettConst* bc, uint64_t* end,
                             BandArgs band, hipStream_t s);

}  // namespace th
