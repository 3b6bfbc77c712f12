/* tensafe_he.h — C ABI of the MI355X (gfx950) CKKS engine for the encrypted
 * LoRA-delta path.
 *
 * This is the drop-in boundary under the reference's Python-facing backend
 * interface (the PyO3 module `tensafe_he`,
 * tensafe-he/crates/tensafe-he-python/src/lib.rs:18-405). Every entry point
 * below names the reference function it replaces. Results are bit-identical
 * to the reference CPU backend (tensafe-he-core) for the same inputs and the
 * same seeded randomness.
 *
 * Conventions
 *  - All functions return 0 on success and a negative TH_E* code on error;
 *    th_last_error() returns a thread-local message for the last failure.
 *    No C++ exception or panic crosses this boundary.
 *  - Handles (th_ctx, th_sk, th_pk, th_ct, th_pt, th_lora) are opaque and
 *    owned by the library; release them with the matching *_free. Ciphertext,
 *    key and plaintext data stay resident in device memory (HBM) for their
 *    lifetime. Keys, ciphertexts, plaintexts and LoRA sets hold a reference
 *    to their context, so they may be freed before or after it (as the
 *    reference's objects outlive its CkksContext): th_ctx_free refuses new
 *    work on the context (TH_ESTATE) and its device memory is released when
 *    the last handle made from it is freed.
 *  - Host input arrays are caller-owned and only read during the call; host
 *    output arrays are caller-owned and fully written before return.
 *  - `has_seed == 0` draws the seed from the OS (the reference's
 *    TenSafeRng::from_entropy); otherwise a fresh ChaCha20 stream seeded with
 *    `seed` is used for that call (lib.rs:93-96, rng.rs:38-68).
 *  - One HIP stream per context: a context is thread-compatible, not
 *    thread-safe. Operations are asynchronous on that stream except those
 *    that return host data, which synchronise it once per call.
 *  - Ciphertext layout: c0 then c1, each `limbs` limb-polynomials of N
 *    little-endian u64 residues in [0, q_l), NTT (evaluation) domain.
 */
#ifndef TENSAFE_HE_H
#define TENSAFE_HE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct th_ctx th_ctx;
typedef struct th_sk th_sk;
typedef struct th_pk th_pk;
typedef struct th_ct th_ct;
typedef struct th_pt th_pt;

enum {
  TH_OK = 0,
  TH_EINVAL = -1,   /* bad argument (reference: PyValueError / assert!) */
  TH_EDEVICE = -2,  /* no usable gfx950 device or a HIP runtime error */
  TH_ENOMEM = -3,   /* device or host allocation failed */
  TH_ESTATE = -4    /* operation not valid for this object (e.g. rescale at 1 limb) */
};

/* Message of the last failing call on this thread (never NULL). */
const char* th_last_error(void);
/* Library version string. */
const char* th_version(void);
/* Number of visible HIP devices. */
int th_device_count(int* count);

/* ---------------------------------------------------------------- context */
/* Replaces CkksContext::new (lib.rs:35-56, ciphertext.rs:61-74).
 * moduli == NULL selects the reference chain for N in {8192, 16384, 32768}
 * (params.rs:66-126); otherwise `L` distinct NTT-friendly primes
 * (q = 1 mod 2N, q < 2^61) define the chain. scale_bits must be 40
 * (params.rs:9). */
int th_ctx_create(uint32_t N, const uint64_t* moduli, uint32_t L, uint32_t scale_bits, int device,
                  th_ctx** out);
int th_ctx_free(th_ctx* ctx);
/* Replaces the num_slots / poly_mod_degree getters (lib.rs:79-88) and
 * get_backend_info's num_limbs (lib.rs:282-294). moduli_out may be NULL. */
int th_ctx_info(const th_ctx* ctx, uint32_t* N, uint32_t* L, uint64_t* moduli_out);
/* Wait for all work queued on the context's stream. */
int th_ctx_sync(th_ctx* ctx);
/* The context's HIP stream (hipStream_t), for callers that order their own work after it. */
int th_ctx_stream(th_ctx* ctx, void** stream);

/* Context options (no counterpart in the reference; defaults shown first).
 * TH_OPT_SAMPLER: where seeded encrypt_pk draws (u, e0, e1):
 *   TH_SAMPLER_DEVICE (default) - ChaCha20 + Box-Muller on the GPU, same
 *     stream positions as the reference; draws whose rounding could depend on
 *     the math library are redrawn on the host (TH_OPT_SAMPLER_BAND);
 *   TH_SAMPLER_HOST - the host draws them exactly as the reference does.
 * TH_OPT_FORCE_SERIAL_SAMPLER: 1 makes the device samplers replay every
 *   stream serially (the path taken after a range_u32 or range_u64
 *   rejection), encrypt_pk's and the key and secret-key-encryption draws
 *   alike; testing only.
 * TH_OPT_SAMPLER_BAND: v in [-40, -1], default -36: the device sampler flags
 *   every Gaussian draw whose z * 3.19 lies within 2^v of a rounding boundary
 *   k + 1/2 (where the device's log/cos could round differently from glibc's;
 *   their difference stays below about 2^-45), and such an input's randomness
 *   is drawn again on the host with glibc, so the device sampler's draws equal
 *   the reference's in every case. Calls that return results check the flags
 *   before returning (th_encrypt_pk and th_encrypt_pk_batch therefore wait for
 *   their work); tokens th_lora_deltas queues without waiting are checked at
 *   the next th_ctx_sync, th_memcpy_h2d, th_memcpy_d2h, th_dev_free,
 *   th_lora_free or synchronising call, which queues a flagged token again
 *   (and, in order, the tokens queued after it) before returning. A wider
 *   band only makes the host redraw more often (tests use it to exercise that
 *   path); bands below 2^-40 would come within 2^5 of the largest
 *   device-glibc difference and are refused.
 * TH_OPT_RESCALE_DECRYPT: which kernels LoRA sets created afterwards use to
 *   rescale and decrypt their products: TH_RD_AUTO (default) - one workgroup
 *   per product from 160 to 256 batches at N <= 16384 (and at every batch
 *   count below N = 8192), the split kernels otherwise; TH_RD_SPLIT - the
 *   split kernels wherever they exist (N >= 8192); TH_RD_WHOLE - one
 *   workgroup per product wherever it serves. The results are the same bit
 *   for bit; testing and measurement only. */
enum {
  TH_OPT_SAMPLER = 1,
  TH_OPT_FORCE_SERIAL_SAMPLER = 2,
  TH_OPT_SAMPLER_BAND = 3,
  TH_OPT_RESCALE_DECRYPT = 4
};
enum { TH_RD_AUTO = 0, TH_RD_SPLIT = 1, TH_RD_WHOLE = 2 };
enum { TH_SAMPLER_DEVICE = 0, TH_SAMPLER_HOST = 1 };
int th_ctx_set_option(th_ctx* ctx, int option, int64_t value);
/* Counters of the context (no counterpart in the reference): the number of
 * encrypt_pk inputs whose randomness the device sampler flagged and the host
 * drew again with glibc (TH_OPT_SAMPLER_BAND). */
int th_ctx_stats(th_ctx* ctx, uint64_t* redrawn_inputs);

/* ---------------------------------------------------------------- keys */
/* Replaces CkksContext.keygen (lib.rs:91-99, ciphertext.rs:77-103). */
int th_keygen(th_ctx* ctx, uint64_t seed, int has_seed, th_sk** out);
/* Replaces CkksContext.keygen_public (lib.rs:102-110, ciphertext.rs:114-154). */
int th_keygen_public(th_ctx* ctx, const th_sk* sk, uint64_t seed, int has_seed, th_pk** out);
int th_sk_free(th_sk* sk);
int th_pk_free(th_pk* pk);
/* Secret key s (NTT domain, L x N) to host; for tests and key escrow. */
int th_sk_download(th_ctx* ctx, const th_sk* sk, uint64_t* out);
/* Public key (b, a), each L x N, to host. */
int th_pk_download(th_ctx* ctx, const th_pk* pk, uint64_t* b, uint64_t* a);

/* ---------------------------------------------------------------- encryption */
/* Replaces CkksContext.encrypt (lib.rs:115-138, ciphertext.rs:167-229).
 * z has n <= N/2 values (zero-padded; longer input is truncated as lib.rs:124-126 does). */
int th_encrypt(th_ctx* ctx, const th_sk* sk, const double* z, size_t n, uint64_t seed, int has_seed,
               th_ct** out);
/* Replaces CkksContext.batch_encrypt (lib.rs:230-258): secret-key encryption
 * of `count` inputs (input i is z + i*stride with lens[i] values) drawing
 * from ONE ChaCha20 stream in order, as the reference's shared RNG does. */
int th_encrypt_batch(th_ctx* ctx, const th_sk* sk, const double* z, const uint64_t* lens, size_t stride,
                     size_t count, uint64_t seed, int has_seed, th_ct** outs);
/* Replaces CkksContext.encrypt_pk (lib.rs:141-164, ciphertext.rs:240-319). */
int th_encrypt_pk(th_ctx* ctx, const th_pk* pk, const double* z, size_t n, uint64_t seed, int has_seed,
                  th_ct** out);
/* encrypt_pk with caller-supplied randomness, for parity runs: u holds the
 * values sample_ternary(rng, N, 3) returns ({0,1,2} meaning -1, 0, +1;
 * sampling.rs:17-29, ciphertext.rs:256-268), e0 and e1 the rounded Gaussian
 * samples (sampling.rs:51-58), N entries each. */
int th_encrypt_pk_explicit(th_ctx* ctx, const th_pk* pk, const double* z, size_t n, const uint8_t* u,
                           const int64_t* e0, const int64_t* e1, th_ct** out);
/* `count` encrypt_pk calls in one batch: input i is z + i*stride (n values),
 * seeded with seeds[i]. Replaces a loop of encrypt_pk (the engine's one
 * encrypt per layer input, inference_engine.py:1272). */
int th_encrypt_pk_batch(th_ctx* ctx, const th_pk* pk, const double* z, size_t n, size_t stride, size_t count,
                        const uint64_t* seeds, th_ct** outs);

/* ---------------------------------------------------------------- plaintexts and products */
/* Replaces CkksContext::encode_to_ntt (ciphertext.rs:539-545): the cached
 * LoRA-A plaintext batches (inference_engine.py:1037-1074). */
int th_encode_to_ntt(th_ctx* ctx, const double* z, size_t n, th_pt** out);
int th_pt_free(th_pt* pt);
int th_pt_download(th_ctx* ctx, const th_pt* pt, uint64_t* out);
/* Replaces CkksContext.ct_pt_mul / TenSafeCiphertext.__mul__
 * (lib.rs:178-195, :336-356; ciphertext.rs:408-418). */
int th_ct_pt_mul(th_ctx* ctx, const th_ct* ct, const double* pt, size_t n, th_ct** out);
/* Replaces CkksContext::ct_pt_mul_ntt (ciphertext.rs:422-429). */
int th_ct_pt_mul_ntt(th_ctx* ctx, const th_ct* ct, const th_pt* pt, th_ct** out);
/* `count` ct_pt_mul_ntt products in one launch: outs[i] = cts[i] x pts[i]
 * (the ZeRo-MOAI column-packed matvec batches, inference_engine.py:1292-1316). */
int th_ct_pt_mul_ntt_batch(th_ctx* ctx, const th_ct* const* cts, const th_pt* const* pts, size_t count,
                           th_ct** outs);
/* Replace CkksContext.ct_add / ct_sub (lib.rs:198-215, ciphertext.rs:435-466).
 * The result has a's limbs and scale; b must have at least as many limbs
 * (RnsPoly::add/sub run over self's limbs, rns.rs:217-240). */
int th_ct_add(th_ctx* ctx, const th_ct* a, const th_ct* b, th_ct** out);
int th_ct_sub(th_ctx* ctx, const th_ct* a, const th_ct* b, th_ct** out);
/* Replaces CkksContext.rescale (lib.rs:218-225, ciphertext.rs:476-535). */
int th_rescale(th_ctx* ctx, const th_ct* ct, th_ct** out);
/* `count` rescales in one batch (all inputs must have the same limb count). */
int th_rescale_batch(th_ctx* ctx, const th_ct* const* cts, size_t count, th_ct** outs);

/* ---------------------------------------------------------------- decryption */
/* Replaces CkksContext.decrypt (lib.rs:167-175, ciphertext.rs:327-400):
 * out receives N/2 doubles. */
int th_decrypt(th_ctx* ctx, const th_ct* ct, const th_sk* sk, double* out);
/* Replaces CkksContext.batch_decrypt (lib.rs:261-273) with a GPU-resident
 * batch: all decrypts and decodes run on the device and the results come
 * back in one device-to-host copy. out receives count x N/2 doubles. */
int th_batch_decrypt(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk, double* out);
/* As th_batch_decrypt, but returns only the ZeRo-MOAI segment sums
 * out[i*cols + c] = sum(dec_i[c*d : (c+1)*d]) (inference_engine.py:1379-1386):
 * one host sync and count x cols doubles per batch. */
int th_batch_decrypt_segsum(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk, uint32_t d,
                            uint32_t cols, double* out);
/* th_batch_decrypt_segsum that allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code that
 * must not call hipMalloc, tight serving loops, allocation-free harnesses).
 * Job lists, segment weights, decrypted coefficients and partial sums live in
 * a static 32 MiB device array per GPU (held until the process ends); host
 * staging uses the context's pinned ring. Results equal
 * th_batch_decrypt_segsum's. A batch whose working set exceeds the 32 MiB
 * (about 60 ciphertexts at N = 16384 on the CRT or full-decode paths, far
 * more on the limb-0 path with at most 8 segments) is refused with TH_EINVAL.
 * Calls on one GPU share its array: this library runs them one at a time
 * (a per-device lock held until the call returns), and each call writes
 * everything it reads in the array before reading it. */
int th_batch_decrypt_segsum_noalloc(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk,
                                    uint32_t d, uint32_t cols, double* out);
/* As th_batch_decrypt, writing count x N/2 doubles to device memory at
 * dev_out (e.g. a ROCm torch tensor; the engine's decrypt_to_gpu,
 * inference_engine.py:190-205). The context stream is synchronised before return. */
int th_batch_decrypt_device(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk,
                            double* dev_out);

/* One encrypted ZeRo-MOAI LoRA-A pass (the encrypted branch of the engine's
 * _he_lora_delta, inference_engine.py:1244-1392, for a whole set of inputs):
 * input i (d values at hidden + i*d) is replicated into cols = (N/2) / d
 * segments (:1258-1269) and encrypted with encrypt_pk seeded by seeds[i];
 * cached plaintext batch j (th_encode_to_ntt of packed LoRA-A rows,
 * :1037-1074) multiplies the ciphertext of input pt_input[j] (:1311); the
 * products are rescaled if do_rescale (ciphertext.rs:476-535), decrypted and
 * decoded on the device, and each d-slot segment is summed (:1379-1386).
 * out receives n_pts x cols doubles after ONE device-to-host copy; no
 * intermediate ciphertext leaves the device. */
int th_lora_a_pass(th_ctx* ctx, const th_pk* pk, const th_sk* sk, const double* hidden, uint32_t n_inputs,
                   uint32_t d, const uint64_t* seeds, const th_pt* const* pts, const uint32_t* pt_input,
                   uint32_t n_pts, int do_rescale, double* out);

/* ---------------------------------------------------------------- LoRA sets */
typedef struct th_lora th_lora;
/* A set of LoRA projections resident on the device: the engine's cached
 * packed plaintexts (_precompute_he_cache, inference_engine.py:1037-1074)
 * plus the LoRA-B matrices applied after decryption (:1392), with the
 * working memory of one token so that th_lora_deltas allocates nothing.
 * Projection j reads input input_of[j] (< n_inputs). Its LoRA-A is a[j]
 * (ranks[j] x d, row-major, PEFT layout :1054-1055) and its LoRA-B is b[j]
 * (d_out[j] x ranks[j], row-major). A rows are packed cols = (N/2)/d per
 * plaintext batch (:1258-1259, :1300-1308); batches are numbered projection
 * by projection. */
int th_lora_create(th_ctx* ctx, uint32_t n_inputs, uint32_t d, uint32_t n_proj, const uint32_t* input_of,
                   const uint32_t* ranks, const uint32_t* d_out, const double* const* a, const double* const* b,
                   th_lora** out);
/* CryptoMOE set: n_experts adapters per projection, combined with gate
 * weights. No counterpart in the reference, which routes each query to one
 * adapter by keyword step-gates (inference_engine.py:1155-1171); the
 * combination rule is this library's. Expert x of projection j has LoRA-A
 * a[j*n_experts + x] (ranks[j] x d), LoRA-B b[j*n_experts + x]
 * (d_out[j] x ranks[j]) and weight gates[j*n_experts + x]. Each expert's
 * gate-scaled A rows g*A are packed and encoded as a plaintext of its own;
 * the batch's ciphertext is the ct_add (ciphertext.rs:435-450) of the
 * experts' ct x pt products (:422-429), bit for bit, so the decrypted
 * intermediate is sum_x g_x A_x h. The B side applies sum_x g_x B_x to it.
 * gates == NULL (allowed only with n_experts == 1) is th_lora_create.
 * Gate weights must be finite; n_experts is at most 64. */
int th_lora_create_moe(th_ctx* ctx, uint32_t n_inputs, uint32_t d, uint32_t n_proj, const uint32_t* input_of,
                       const uint32_t* ranks, const uint32_t* d_out, uint32_t n_experts, const double* gates,
                       const double* const* a, const double* const* b, th_lora** out);
/* Gates of a set made by th_lora_create_moe with gates, replaced (a gate
 * that changes per token; no counterpart in the reference, see
 * th_lora_create_moe). gates: n_proj x n_experts, finite. The experts'
 * plaintexts g*A are encoded, transformed and folded again and B = sum_x
 * g_x B_x is mixed again, all on the device and queued on the context's
 * stream: th_lora_deltas calls made after it use the new gates, bit for bit
 * as a set created with them. Tokens queued without waiting are settled
 * first. TH_ESTATE for a set created without gates. */
int th_lora_set_gates(th_ctx* ctx, th_lora* set, const double* gates);
int th_lora_free(th_lora* set);
/* n_deltas = sum of d_out (length of th_lora_deltas' output), n_batches =
 * number of plaintext batches, cols = segments per batch. Any may be NULL. */
int th_lora_info(const th_lora* set, uint64_t* n_deltas, uint32_t* n_batches, uint32_t* cols);
/* th_lora_deltas mode bits.
 * TH_LORA_RESCALE: rescale each product before decrypting it
 *   (ciphertext.rs:476-535), as the per-token LoRA pass (encrypt, ct x pt,
 *   rescale, decrypt) does.
 * TH_LORA_SK_FUSED: the decryption-fused shortcut. Without it (the default)
 *   the token runs the reference's client/server sequence
 *   (inference_engine.py:1477-1482): encrypt_pk forms every limb of c0 and c1
 *   of each input from the public key alone; ct x pt (fused into the rescale
 *   with TH_LORA_RESCALE) forms every limb of each batch's product or
 *   rescaled product without the secret key; then one batched decrypt reads
 *   only what it decodes (limb 0, or limbs 0 and 1 in the CRT branch) with the
 *   secret key. Those ciphertexts stay in the set's working memory until the
 *   next token (th_lora_ct). With TH_LORA_SK_FUSED the token forms only the
 *   limbs its decryptions read and uses the secret key inside the encryption
 *   (c0 + c1 s on limb 0 replaces c0 and c1 there), so no complete ciphertext
 *   exists at any point: a single-party shortcut with the same deltas bit for
 *   bit, not the reference's architecture (no counterpart in the reference). */
enum { TH_LORA_RESCALE = 1, TH_LORA_SK_FUSED = 2 };
/* One token of the encrypted LoRA path for every projection of the set (the
 * engine's _he_lora_delta, inference_engine.py:1244-1392, for all layers at
 * once), entirely on the device: encrypt_pk of each input replicated into
 * cols segments and seeded with seeds[i] (host array); ct x pt with every
 * cached batch; rescale when mode has TH_LORA_RESCALE (the product is formed
 * inside the rescale's transforms); batched decrypt + decode with segment
 * sums; then delta_j = B_j @ intermediate_j. mode: TH_LORA_* bits above
 * (0 and 1 keep the meaning of the earlier do_rescale flag).
 *   hidden: n_inputs x d doubles, device memory if hidden_on_device, else host.
 *   deltas: n_deltas doubles (projection j at offset sum_{k<j} d_out[k]),
 *           device memory if deltas_on_device, else host.
 *   inter:  NULL, or a host array of n_batches x cols segment sums.
 * With hidden and deltas in device memory and inter == NULL the call only
 * queues the token's kernels on the context stream and returns (no host
 * synchronisation; order later work with th_ctx_stream / th_ctx_sync). The
 * device input, the output buffer and the keys must then stay unchanged (and
 * allocated) until the next th_ctx_sync; th_memcpy_h2d, th_memcpy_d2h and
 * th_dev_free settle queued tokens first. If a Gaussian draw of the token
 * landed in the sampler's band (TH_OPT_SAMPLER_BAND), the token writes NaN
 * for every delta of the projections that read that input, and the settling
 * call queues the token again from glibc draws, which overwrites them: work
 * the caller orders after the token on the stream sees the exact deltas or
 * NaN, never another value; read the deltas after th_ctx_sync to have them
 * exact in every case.
 * Otherwise it returns after one synchronisation of the stream and one
 * device-to-host copy. */
int th_lora_deltas(th_ctx* ctx, th_lora* set, const th_pk* pk, const th_sk* sk, const double* hidden,
                   int hidden_on_device, const uint64_t* seeds, int mode, double* deltas, int deltas_on_device,
                   double* inter);
/* A copy, as a new ciphertext object, of one ciphertext that the set's last
 * token formed (no counterpart in the reference, whose per-token objects are
 * the TenSafeCiphertext values of _he_lora_delta, inference_engine.py:1272,
 * :1311): which = TH_LORA_CT_INPUT, the encrypt_pk output of input `index`
 * (L limbs, scale 2^40); TH_LORA_CT_PRODUCT, batch `index`'s product
 * ct x pt (L limbs, scale 2^80), rescaled (L - 1 limbs) if the token had
 * TH_LORA_RESCALE. Queued tokens are settled first. TH_ESTATE if the set has
 * run no token yet or its last token had TH_LORA_SK_FUSED (which forms no
 * complete ciphertext). */
enum { TH_LORA_CT_INPUT = 0, TH_LORA_CT_PRODUCT = 1 };
int th_lora_ct(th_ctx* ctx, th_lora* set, int which, uint32_t index, th_ct** out);

/* ---------------------------------------------------------------- ciphertext objects */
int th_ct_free(th_ct* ct);
/* Replace TenSafeCiphertext.num_limbs / scale getters (lib.rs:385-394). */
int th_ct_info(const th_ct* ct, uint32_t* limbs, double* scale);
/* c0 and c1 (limbs x N each) to host. */
int th_ct_download(th_ctx* ctx, const th_ct* ct, uint64_t* c0, uint64_t* c1);
/* A ciphertext from host residues (limbs x N each, NTT domain). */
int th_ct_upload(th_ctx* ctx, const uint64_t* c0, const uint64_t* c1, uint32_t limbs, double scale,
                 th_ct** out);
/* Wire format of serialize.rs:71-93: [scale f64 LE | c0 | c1]. With buf ==
 * NULL only *len is set. */
int th_ct_export(th_ctx* ctx, const th_ct* ct, uint8_t* buf, size_t cap, size_t* len);
int th_ct_import(th_ctx* ctx, const uint8_t* buf, size_t len, uint32_t limbs, th_ct** out);
/* Wire format of serialize.rs:48-67: [b | a]. */
int th_pk_export(th_ctx* ctx, const th_pk* pk, uint8_t* buf, size_t cap, size_t* len);
int th_pk_import(th_ctx* ctx, const uint8_t* buf, size_t len, th_pk** out);

/* ---------------------------------------------------------------- raw transforms */
/* In-place forward / inverse negacyclic NTT (ntt.rs:79-141) of `count`
 * polynomials, each `limbs` consecutive limb-polynomials of N u64 using
 * moduli q_0 .. q_{limbs-1}. `polys` is a host pointer (on_device == 0) or a
 * device pointer (on_device == 1; asynchronous on the context stream). */
int th_ntt_forward_batch(th_ctx* ctx, uint64_t* polys, size_t count, uint32_t limbs, int on_device);
int th_ntt_inverse_batch(th_ctx* ctx, uint64_t* polys, size_t count, uint32_t limbs, int on_device);
/* Device-memory helpers for callers without their own allocator. th_dev_free
 * accepts only a pointer from th_dev_alloc that has not been freed yet. */
int th_dev_alloc(th_ctx* ctx, size_t bytes, void** out);
int th_dev_free(th_ctx* ctx, void* p);
int th_memcpy_h2d(th_ctx* ctx, void* dst, const void* src, size_t bytes);
int th_memcpy_d2h(th_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Times `reps` back-to-back launches of the batched transform of
 * th_ntt_*_batch(on_device = 1) with HIP events on the context stream;
 * *avg_ms receives the mean duration of one launch. */
int th_ntt_time(th_ctx* ctx, uint64_t* dev_polys, size_t count, uint32_t limbs, int inverse, int reps,
                float* avg_ms);

#ifdef __cplusplus
}
#endif
#endif /* TENSAFE_HE_H */
