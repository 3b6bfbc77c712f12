// Internal declarations of the host runtime behind the C ABI in
// include/tensafe_he.h (not part of that ABI). The runtime is split by concern:
//   runtime_common.hip  handle lifetime, band flags, NTT dispatch, context
//                       tables and the encode / encrypt / product / rescale /
//                       decrypt pipelines the entry points share;
//   context.hip         contexts, options, device memory helpers, raw NTTs;
//   ops.hip             keys, encryption, plaintexts, ct x pt, add / sub,
//                       rescale, decryption, th_lora_a_pass, serialisation;
//   noalloc.hip         the no-allocation decrypt entry point and its scratch;
//   lora_set.hip        LoRA sets: the per-token pass, CryptoMOE regating and
//                       tokens queued without a host synchronisation.
//
// A context owns: the per-limb NTT twiddle tables and constants in HBM, the
// decode tables, one HIP stream, a size-bucketed device memory pool (buffers
// are recycled in stream order, never returned to HIP until the context is
// freed) and a pinned staging ring for host<->device traffic (job lists and
// input vectors). Every operation is a short fixed pipeline of kernel
// launches on the context stream; only calls that return host data wait.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <map>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "encode_sample.h"
#include "host_math.h"
#include "poly_kernels.h"
#include "tensafe_he.h"

using namespace th;

namespace thrt {

extern thread_local std::string g_err;  // th_last_error's message

struct ThError : std::runtime_error {
  int code;
  ThError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void raise(int code, const std::string& m) { throw ThError(code, m); }

inline void hipchk(hipError_t e, const char* what) {
  if (e != hipSuccess) raise(TH_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPCHK(x) hipchk((x), #x)

constexpr double kScale = 1099511627776.0;  // 2^40, params.rs:9-12

// ---------------------------------------------------------------- memory
class DevicePool {
 public:
  void* get(size_t bytes) {
    bytes = (bytes + 255) & ~(size_t)255;
    std::lock_guard<std::mutex> lk(mu_);
    auto& fl = free_[bytes];
    if (!fl.empty()) return take(fl);
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess || !p) {
      (void)hipGetLastError();
      raise(TH_ENOMEM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    sizes_[p] = bytes;
    return p;
  }
  // Returns a buffer to its free list; false (and nothing changes) for a
  // pointer the pool did not hand out or one that is already free, so a
  // second put can never make two later get() calls share one buffer.
  bool put(void* p) {
    if (!p) return true;
    std::lock_guard<std::mutex> lk(mu_);
    auto it = sizes_.find(p);
    if (it == sizes_.end() || !is_free_.insert(p).second) return false;
    free_[it->second].push_back(p);
    return true;
  }
  void release_all() {
    std::lock_guard<std::mutex> lk(mu_);
    for (auto& kv : sizes_) (void)hipFree(kv.first);
    sizes_.clear();
    free_.clear();
    is_free_.clear();
  }

 private:
  // get() takes a pointer off a free list, so it is no longer free
  void* take(std::vector<void*>& fl) {
    void* p = fl.back();
    fl.pop_back();
    is_free_.erase(p);
    return p;
  }

  std::mutex mu_;
  std::unordered_map<size_t, std::vector<void*>> free_;
  std::unordered_map<void*, size_t> sizes_;
  std::unordered_set<void*> is_free_;
};

// Pinned host staging for host<->device copies. Allocation is a bump pointer;
// when the ring is full the stream is drained first, so a region is never
// rewritten while a queued copy may still read it. Device-side destinations
// come from the pool through an OpScope (below), so nothing a queued kernel
// reads is ever recycled before the kernels of the current call are queued.
class StagingRing {
 public:
  void init(size_t bytes) {
    cap_ = bytes;
    HIPCHK(hipHostMalloc(&host_, cap_, hipHostMallocDefault));
    memset(host_, 0, cap_);  // touched once here rather than by the first copies through each page
    off_ = 0;
  }
  void destroy() {
    if (host_) (void)hipHostFree(host_);
    host_ = nullptr;
  }
  void* reserve(size_t bytes, hipStream_t s) {
    bytes = (bytes + 255) & ~(size_t)255;
    if (bytes > cap_) {
      HIPCHK(hipStreamSynchronize(s));
      destroy();
      init(std::max(bytes, cap_ * 2));
    } else if (off_ + bytes > cap_) {
      HIPCHK(hipStreamSynchronize(s));
      off_ = 0;
    }
    void* h = (char*)host_ + off_;
    off_ += bytes;
    return h;
  }

 private:
  void* host_ = nullptr;
  size_t cap_ = 0, off_ = 0;
};

// Parallel loop over independent host work items (sampling, encoding).
template <class F>
void parallel_for(size_t count, F&& f) {
  size_t nt = std::min<size_t>(count, std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
  if (nt <= 1) {
    for (size_t i = 0; i < count; ++i) f(i);
    return;
  }
  std::vector<std::thread> ts;
  std::vector<std::exception_ptr> errs(nt);
  for (size_t t = 0; t < nt; ++t)
    ts.emplace_back([&, t] {
      try {
        for (size_t i = t; i < count; i += nt) f(i);
      } catch (...) {
        errs[t] = std::current_exception();
      }
    });
  for (auto& th : ts) th.join();
  for (auto& e : errs)
    if (e) std::rethrow_exception(e);
}

}  // namespace thrt

using namespace thrt;

// ---------------------------------------------------------------- handles
struct th_lora;
struct th_pk;
struct th_sk;

// A token of th_lora_deltas queued without a host synchronisation: what it
// takes to queue it again if one of its Gaussian draws turns out to lie in
// the sampler's band (the redo draws that token's randomness with glibc).
struct AsyncToken {
  th_lora* set;
  const th_pk* pk;
  const th_sk* sk;
  const double* hidden;  // device
  std::vector<uint64_t> seeds;
  int mode;              // TH_LORA_* bits
  double* deltas;        // device
  uint32_t flag_off;     // band flags of its inputs
};

struct th_ctx {
  // Lifetime: the context and every handle made from it hold one reference;
  // th_ctx_free drops the context's own and marks it closed (no new work),
  // and the last release frees the device memory, the stream and the object.
  std::atomic<uint32_t> refs{1};
  std::atomic<bool> closed{false};
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t N = 0, logn = 0, L = 0;
  std::vector<uint64_t> q;
  std::vector<LimbConst> h_lc;
  LimbConst* d_lc = nullptr;
  BarrettConst* d_bc = nullptr;
  uint64_t* d_q = nullptr;
  RescaleConst* d_rc = nullptr;  // [level][l], level = input limb count (2..L), row stride L
  DecodeConst* d_dc = nullptr;
  double *d_twist_re = nullptr, *d_twist_im = nullptr, *d_stage_re = nullptr, *d_stage_im = nullptr;
  void* d_tables = nullptr;  // twiddle storage
  Encoder enc;
  int host_sampler = 0;   // TH_OPT_SAMPLER
  int force_serial = 0;   // TH_OPT_FORCE_SERIAL_SAMPLER
  double band = SAMPLER_BAND_DEFAULT;  // TH_OPT_SAMPLER_BAND
  int rd_kernels = TH_RD_AUTO;  // TH_OPT_RESCALE_DECRYPT
  // Band flags of the device sampler (BandArgs): pinned host bytes the
  // kernels write through bflag_dev. A call takes a region of one byte per
  // sampled input (take_flags); asynchronous tokens keep theirs until the
  // next resolve_pending.
  uint8_t* bflag_host = nullptr;
  uint8_t* bflag_dev = nullptr;
  uint32_t bflag_cap = 0, bflag_used = 0;
  // The same flags in device memory as generations (BandArgs::dflags): a
  // token's kernels read them there instead of across PCIe; band_gen numbers
  // the calls that sample.
  uint32_t* bflag_gen = nullptr;
  uint32_t band_gen = 0;
  // launch_key_draws' reject word and launch_key_replay's end word (device)
  uint32_t* key_reject = nullptr;
  uint64_t* key_end = nullptr;
  std::vector<AsyncToken> pending;
  uint64_t redrawn_inputs = 0;  // inputs whose randomness was drawn again on the host (th_ctx_stats)
  std::unordered_set<void*> user_allocs;  // th_dev_alloc buffers not yet freed
  unsigned char* scratch = nullptr;  // this device's copy of the no-allocation scratch
  DevicePool pool;
  StagingRing ring;
  std::map<std::pair<uint32_t, uint32_t>, double*> seg_w;  // segment-sum weights by (d, cols)
  std::map<uint32_t, double*> seg_p;                        // recurrence-form weight pairs by d
  std::mutex mu;
};

struct th_sk {
  th_ctx* ctx;
  uint64_t* d;                     // L x N, NTT domain
  mutable uint64_t* dm = nullptr;  // the same in Montgomery form (launch_to_montgomery), made on first use
};
struct th_pk {
  th_ctx* ctx;
  uint64_t* d;                  // [b | a], L x N each
  mutable uint64_t* dp = nullptr;  // the same as prepared pairs (launch_prepare_pairs), made on first use
};
struct th_ct {
  th_ctx* ctx;
  uint32_t limbs;
  double scale;
  uint64_t* d;  // [c0 | c1], limbs x N each
};
struct th_pt {
  th_ctx* ctx;
  uint32_t limbs;
  uint64_t* d;  // limbs x N
};

// A LoRA set: cached plaintext batches, LoRA-B matrices, one token's working
// memory and the job lists of its launches, all in device memory taken from
// the context pool (returned to it by th_lora_free).
struct th_lora {
  th_ctx* ctx;
  uint32_t n_in = 0, d = 0, n_proj = 0, cols = 0, n_batches = 0, max_d_out = 0;
  uint64_t n_deltas = 0;
  std::vector<void*> owned;
  uint64_t* pts = nullptr;     // n_batches x L x N, NTT domain
  uint64_t* ptm = nullptr;     // the same in Montgomery form (launch_to_montgomery)
  double* hidden = nullptr;    // n_in x d
  uint8_t* u = nullptr;        // n_in x N
  int64_t *e0 = nullptr, *e1 = nullptr;
  int64_t* mvals = nullptr;    // n_in x N encoded messages m (i64)
  uint64_t* prep = nullptr;    // n_in x 3L x N
  uint64_t* cts = nullptr;     // n_in x 2L x N
  uint64_t* work = nullptr;    // n_batches x 2 x N: the last limb of each product as coefficients (inverse transforms)
  uint64_t* res = nullptr;     // n_batches x 2 nl_r x N: the rescaled limbs the decryption reads
  uint64_t* m = nullptr;       // n_batches x 2 x N, decrypted coefficients
  double* sums = nullptr;      // n_batches x cols
  const SampleJob* d_sample = nullptr;
  const EncCombineJob* d_comb = nullptr;
  const EncodeJob* d_enc = nullptr;
  const NttJob *d_inv_mul = nullptr, *d_fwd_rs = nullptr, *d_dot_r = nullptr;
  // encrypt transforms (residues of m + e0, e1, u formed in the loads) of the
  // limbs a token with (r) or without (n) a rescale reads, and those limbs
  const NttJob *d_enc_r = nullptr, *d_enc_n = nullptr;
  uint32_t enc_mask_r = 0, enc_mask_n = 0;
  const NttJob* d_dot_seg = nullptr;  // rescaled decrypts whose transform writes the segment sums
  // rescaled products decrypted on limb 0 straight from the last limb's
  // inverse transforms, one job per batch: rescale_decrypt_kernel, or the
  // split kernels (rd_split, with nb x cols x N/16 doubles of partial sums)
  const RescaleDecryptJob* d_rd = nullptr;
  bool rd_split = false;
  double* rd_partials = nullptr;
  // decrypt without a rescale: D = c0 + c1 s per input (k_key_dot), then per
  // batch the inverse transforms of pt * D (the product's decryption)
  uint64_t* dkey = nullptr;           // n_in x nl x N
  const NttJob* d_inv_nr = nullptr;
  uint32_t inv_nr_jobs = 0, nl_n = 1;
  uint32_t nl_r = 1;  // limbs a rescaled product's decryption reads (1, or 2 for the CRT branch)
  const DecodeJob *d_dec_r = nullptr, *d_dec_n = nullptr;
  // The complete pass (th_lora_deltas without TH_LORA_SK_FUSED): every limb of
  // each input's ciphertext (encrypt jobs of all limbs), every limb of each
  // batch's product or rescaled product in outs, then the batched decrypt of
  // the limbs it reads.
  uint64_t* outs = nullptr;                   // n_batches x 2L x N (rescaled: 2(L-1) limb-polys each)
  const NttJob* d_enc_all = nullptr;          // encrypt transforms of every limb
  const NttJob* d_fwd_all = nullptr;          // rescale forward jobs of limbs 0..L-2 into outs
  const NttJob* d_seg_all = nullptr;          // decrypt + segment sums in one transform (limb-0 branch)
  const NttJob* d_dec_row = nullptr;          // or the same on the split kernels (decrypt_sums_path)
  const RescaleDecryptJob* d_dec_rj = nullptr;
  double* dec_partials = nullptr;
  const NttJob *d_dot_all_r = nullptr, *d_dot_all_n = nullptr;  // decrypt transforms into m
  uint32_t dot_all_r_jobs = 0, dot_all_n_jobs = 0;
  const CtPtJob* d_ctpt = nullptr;            // products without a rescale
  int last_mode = -1;                         // mode of the last token queued (th_lora_ct)
  const LoraBJob* d_bjobs = nullptr;
  uint32_t dot_r_jobs = 0;
  const double* seg_w = nullptr;  // segment weights, or null: decode the slots and sum them
  const double* seg_p = nullptr;  // the same in recurrence form (decrypt transform's epilogue)
  // gated (mixture) sets: k experts per projection, regated by th_lora_set_gates
  uint32_t k = 1;
  const double* apack = nullptr;  // n_batches x k x N/2: the experts' packed A rows, ungated
  const double* bexp = nullptr;   // the experts' B, rank-major (MoeProj)
  double* bmix = nullptr;         // sum_x g_x B_x: what the B jobs read
  const MoeProj* d_moe_p = nullptr;
  uint32_t max_b_count = 0;
  std::vector<MoeBatch> moe_b;     // per batch: projection and rows (host copy)
  double* d_gates = nullptr;       // n_proj x k, the current gates
  uint32_t moe_limbs = 0;          // the plaintext limbs a token reads (bit l: limb l)
  const NttJob* d_moe_ntt = nullptr;  // per batch and such limb: transform in place, Montgomery copy
  uint32_t moe_ntt_jobs = 0;
  // pinned host staging of host-I/O tokens (hidden states in, deltas and
  // segment sums out), the same pages every token; mapped into the device's
  // address space (io_dev), so the token's last kernel writes host deltas
  // there itself instead of a device-to-host copy after it
  void* io_host = nullptr;
  double* io_dev = nullptr;
  size_t io_bytes = 0;
  size_t io_in_off = 0;  // byte offset of the hidden states, past the deltas and sums
  void* alloc(size_t bytes) {
    void* p = ctx->pool.get(bytes);
    owned.push_back(p);
    return p;
  }
};

namespace thrt {

// Device buffers used by one API call (job lists, uploaded inputs, scratch).
// They go back to the pool when the call returns, after all of its kernels
// are queued; the next user of a recycled buffer is ordered after them on
// the same stream.
struct OpScope {
  th_ctx* c;
  std::vector<void*> bufs;
  explicit OpScope(th_ctx* ctx) : c(ctx) {}
  ~OpScope() {
    for (void* p : bufs) c->pool.put(p);
  }
  OpScope(const OpScope&) = delete;
  OpScope& operator=(const OpScope&) = delete;
  void* dev(size_t bytes) {
    void* p = c->pool.get(bytes);
    bufs.push_back(p);
    return p;
  }
  void* upload(const void* src, size_t bytes) {
    void* h = c->ring.reserve(bytes, c->stream);
    memcpy(h, src, bytes);
    void* d = dev(bytes);
    HIPCHK(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, c->stream));
    return d;
  }
  template <class T>
  T* up(const std::vector<T>& v) {
    return (T*)upload(v.data(), v.size() * sizeof(T));
  }
};

template <class F>
int guarded(F&& f) {
  try {
    f();
    return TH_OK;
  } catch (const ThError& e) {
    g_err = e.what();
    return e.code;
  } catch (const std::bad_alloc&) {
    g_err = "host allocation failed";
    return TH_ENOMEM;
  } catch (const std::exception& e) {
    g_err = e.what();
    return TH_EINVAL;
  } catch (...) {
    g_err = "unknown error";
    return TH_EINVAL;
  }
}

inline void need(bool cond, const std::string& msg, int code = TH_EINVAL) {
  if (!cond) raise(code, msg);
}

inline void use_device(th_ctx* c) { HIPCHK(hipSetDevice(c->device)); }
inline size_t poly_bytes(const th_ctx* c) { return (size_t)c->N * 8; }

#define TH_LOCK(c)                                                      \
  need((c) != nullptr, "null context");                                 \
  need(!(c)->closed.load(), "the context has been freed", TH_ESTATE);  \
  std::lock_guard<std::mutex> _lk((c)->mu);                             \
  use_device(c)

inline void ctx_retain(th_ctx* c) { c->refs.fetch_add(1, std::memory_order_relaxed); }

// Fewest batches for which a LoRA set rescales and decrypts with one
// workgroup per product by default (build_lora).
constexpr uint32_t RD_WHOLE_MIN_BATCHES = 160;

// The address of this device's copy of the no-allocation scratch array
// (noalloc.hip); requires `device` to be the current device.
unsigned char* scratch_base(int device);

void ctx_release(th_ctx* c);
void drop(th_ct* x);
void drop(th_pt* x);
void drop(th_sk* x);
void drop(th_pk* x);

// A new handle holds a reference to its context.
template <class H>
H* adopt(H* h) {
  ctx_retain(h->ctx);
  return h;
}

// Drops every handle of a partly built batch of outputs, then rethrows.
template <class H>
[[noreturn]] void drop_all_rethrow(std::vector<H*>& made) {
  for (H* h : made) drop(h);
  made.clear();
  throw;
}

// A ciphertext in device memory: c0 then c1, `limbs` limb-polys each.
struct CtView {
  const uint64_t* d;
  uint32_t limbs;
  double scale;
};


th_ct* new_ct(th_ctx* c, uint32_t limbs, double scale);
void wait_stream(th_ctx* c);
void drain(th_ctx* c);
void settle_before_free(th_ctx* c, const void* key);
uint32_t take_flags(th_ctx* c, uint32_t n);
void release_flags(th_ctx* c, uint32_t off);
bool any_flag(const th_ctx* c, uint32_t off, uint32_t n);
BandArgs band_args(th_ctx* c, uint32_t off);
const uint64_t* pk_pairs(th_ctx* c, const th_pk* pk);
const uint64_t* sk_montgomery(th_ctx* c, const th_sk* sk);
void check_ct(th_ctx* c, const th_ct* ct);
void ntt_strided(th_ctx* c, bool inverse, const uint64_t* src, uint64_t* dst, uint32_t njobs, uint32_t limb_mod,
                 uint32_t limb_base = 0);
void ntt_list(OpScope& sc, bool inverse, const std::vector<NttJob>& jobs, NttLoad load = NTT_LOAD_NONE,
              const RescaleConst* rc = nullptr, const uint64_t* key = nullptr, NttStore store = NTT_STORE_NONE);
void build_tables(th_ctx* c);
void destroy_ctx(th_ctx* c);
void pad_input(const th_ctx* c, const double* z, size_t n, double* out);
void host_key_draws(OpScope& sc, uint64_t seed, size_t count, uint64_t* const* a, int64_t* e);
bool device_key_draws(th_ctx* c, std::vector<KeyDrawJob> jobs);
void queue_encode(OpScope& sc, const double* z, size_t count, const uint8_t* u, const int64_t* e0,
                  const int64_t* e1, uint64_t* dst, size_t dst_stride, uint32_t rep_d = 0, uint32_t rep_cols = 0);
void draw_pk_randomness(uint64_t seed, int has_seed, uint32_t N, uint8_t* u, int64_t* e0, int64_t* e1);
void upload_host_draws(OpScope& sc, const uint64_t* seeds, size_t count, uint8_t* u, int64_t* e0, int64_t* e1);
void queue_encrypt_pk(OpScope& sc, const th_pk* pk, const double* z, size_t count, const uint64_t* seeds,
                      uint32_t rep_d, uint32_t rep_cols, uint64_t* const* out, bool host_draw, BandArgs band);
void queue_encrypt_pk_explicit(OpScope& sc, const th_pk* pk, const double* z, size_t count, const uint8_t* hu,
                               const int64_t* he0, const int64_t* he1, uint64_t* const* out);
std::vector<th_ct*> new_encrypt_outputs(th_ctx* c, size_t count);
void encrypt_pk_explicit_many(th_ctx* c, const th_pk* pk, const double* zh, size_t count, const uint8_t* hu,
                              const int64_t* he0, const int64_t* he1, th_ct** outs);
void encrypt_pk_seeded(th_ctx* c, const th_pk* pk, const double* zh, size_t count, const uint64_t* seeds,
                       th_ct** outs);
std::vector<CtView> views_of(const th_ct* const* cts, size_t count);
const double* seg_weights(th_ctx* c, uint32_t d, uint32_t cols);
const double* seg_pairs(th_ctx* c, uint32_t d);
bool segsum_in_transform(const th_ctx* c, uint32_t jobs, uint32_t cols);
// How a batch of `jobs` limb-0 decryptions with `cols` segment sums runs:
// WHOLE - the whole-polynomial decrypt with the sums in its epilogue
// (launch_dot_segsum, launches of at most 256 jobs); SPLIT - the split
// kernels' decrypt with the sums in the same order (launch_dec_sums_split;
// at N = 16384 the two are equal bit for bit, and at N = 8192 and 32768 the
// split form is the one every limb-0 decryption with sums takes); KERNELS -
// decrypted coefficients, then the segment-sum or decode kernels. Below
// DECRYPT_WHOLE_MIN_JOBS jobs the whole kernel leaves most CUs idle for a
// whole transform's time: one delta's 4 decryptions took 36 us there.
enum class SumsPath { WHOLE, SPLIT, KERNELS };
constexpr uint32_t DECRYPT_WHOLE_MIN_JOBS = 96;
SumsPath decrypt_sums_path(const th_ctx* c, uint32_t jobs, uint32_t cols);
// The SPLIT path for n decryptions: d_row = their NTT_LOAD_DOTM jobs on limb
// 0 (src c0, aux c1, dst the work area named by d_jobs[i].y); partials: n x
// cols x N/16 doubles of scratch.
void launch_dec_sums_split(th_ctx* c, const NttJob* d_row, const RescaleDecryptJob* d_jobs, uint32_t n,
                           const th_sk* sk, const double* W, uint32_t cols, double* partials);
void launch_dot_segsum(th_ctx* c, const NttJob* d_jobs, uint32_t n, const th_sk* sk, const double* W, uint32_t cols);
void queue_decrypt(OpScope& sc, const std::vector<CtView>& cts, const th_sk* sk, double* out_dev, double* seg_dev,
                   uint32_t d, uint32_t cols);
void queue_ct_pt(OpScope& sc, const std::vector<CtView>& in, const uint64_t* const* pts, uint64_t* const* out);
void queue_rescale(OpScope& sc, const std::vector<CtView>& in, uint64_t* const* out,
                   const uint64_t* const* pts = nullptr);
void check_decrypt_args(th_ctx* c, const th_ct* const* cts, size_t count, const th_sk* sk);
void download(th_ctx* c, void* dst, const void* src_dev, size_t bytes);
void rescale_many(th_ctx* c, const th_ct* const* cts, size_t count, th_ct** outs);
th_pt* encode_pt(th_ctx* c, const double* z, size_t n);
void ct_pt_many(th_ctx* c, const th_ct* const* cts, const th_pt* const* pts, size_t count, th_ct** outs);
void add_sub(th_ctx* c, const th_ct* a, const th_ct* b, bool sub, th_ct** out);
void ntt_batch(th_ctx* c, uint64_t* polys, size_t count, uint32_t limbs, int on_device, bool inverse);

// After the stream has drained: queue again, with glibc draws, every
// asynchronous token whose band flags are set (and, in order, the tokens
// queued after it, which may share its outputs), then wait (lora_set.hip).
void resolve_pending(th_ctx* c);

}  // namespace thrt
