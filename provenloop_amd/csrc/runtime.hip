// Host runtime of the CKKS engine and the implementation of the C ABI in
// include/tensafe_he.h.
//
// A context owns: the per-limb NTT twiddle tables and constants in HBM, the
// decode tables, one HIP stream, a size-bucketed device memory pool (buffers
// are recycled in stream order, never returned to HIP until the context is
// freed) and a pinned staging ring for host<->device traffic (job lists and
// input vectors). Every operation is a short fixed pipeline of kernel
// launches on the context stream; only calls that return host data wait.
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

// Device scratch of th_batch_decrypt_segsum_noalloc, one copy per GPU for the
// life of the process. In host code this name is only a stand-in for the
// symbol, not a device address: host code uses the pointer that
// hipGetSymbolAddress returns for each device (scratch_base).
constexpr size_t TH_NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[TH_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err = "";

struct ThError : std::runtime_error {
  int code;
  ThError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void raise(int code, const std::string& m) { throw ThError(code, m); }

void hipchk(hipError_t e, const char* what) {
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

}  // namespace

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

namespace {

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

void need(bool cond, const std::string& msg, int code = TH_EINVAL) {
  if (!cond) raise(code, msg);
}

void use_device(th_ctx* c) { HIPCHK(hipSetDevice(c->device)); }

size_t poly_bytes(const th_ctx* c) { return (size_t)c->N * 8; }

// ---------------------------------------------------------------- no-allocation scratch
// The address of each device's copy of `scratch`, looked up once per device
// (with that device current) and kept; calls of the no-allocation entry point
// on one device hold its mutex, so they use the array one at a time.
constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  hipError_t err = hipSuccess;
  unsigned char* ptr = nullptr;
  std::mutex mu;
};
ScratchSlot g_scratch[kMaxScratchDevices];

// Requires `device` to be the current device.
unsigned char* scratch_base(int device) {
  need(device >= 0 && device < kMaxScratchDevices, "device index out of range for the scratch table", TH_EDEVICE);
  ScratchSlot& sl = g_scratch[device];
  std::call_once(sl.once, [&] { sl.err = hipGetSymbolAddress((void**)&sl.ptr, HIP_SYMBOL(scratch)); });
  if (sl.err != hipSuccess || !sl.ptr)
    raise(TH_EDEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(sl.err));
  return sl.ptr;
}

// ---------------------------------------------------------------- handle lifetime
void destroy_ctx(th_ctx* c);

void ctx_retain(th_ctx* c) { c->refs.fetch_add(1, std::memory_order_relaxed); }

// Drops one reference; the last one destroys the context.
void ctx_release(th_ctx* c) {
  if (c->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) destroy_ctx(c);
}

// A new handle holds a reference to its context.
template <class H>
H* adopt(H* h) {
  ctx_retain(h->ctx);
  return h;
}

void drop(th_ct* x) {
  th_ctx* c = x->ctx;
  c->pool.put(x->d);
  delete x;
  ctx_release(c);
}
void drop(th_pt* x) {
  th_ctx* c = x->ctx;
  c->pool.put(x->d);
  delete x;
  ctx_release(c);
}
void drop(th_sk* x) {
  th_ctx* c = x->ctx;
  if (x->dm) c->pool.put(x->dm);
  c->pool.put(x->d);
  delete x;
  ctx_release(c);
}
void drop(th_pk* x) {
  th_ctx* c = x->ctx;
  if (x->dp) c->pool.put(x->dp);
  c->pool.put(x->d);
  delete x;
  ctx_release(c);
}

th_ct* new_ct(th_ctx* c, uint32_t limbs, double scale) {
  th_ct* ct = adopt(new th_ct{c, limbs, scale, nullptr});
  try {
    ct->d = (uint64_t*)c->pool.get(2 * limbs * poly_bytes(c));
  } catch (...) {
    drop(ct);
    throw;
  }
  return ct;
}

// Drops every handle of a partly built batch of outputs, then rethrows.
template <class H>
[[noreturn]] void drop_all_rethrow(std::vector<H*>& made) {
  for (H* h : made) drop(h);
  made.clear();
  throw;
}

// Wait until everything queued on the context's stream, by this library or
// by a caller through th_ctx_stream, has finished. The stream is polled: no
// marker is queued, and the caller resumes within a microsecond or so of the
// last kernel, which matters when the host synchronises once per token.
void wait_stream(th_ctx* c) {
  hipError_t e;
  while ((e = hipStreamQuery(c->stream)) == hipErrorNotReady) __builtin_ia32_pause();
  HIPCHK(e);
}

// ---------------------------------------------------------------- sampler band flags
// After the stream has drained: queue again, with glibc draws, every
// asynchronous token whose band flags are set (and, in order, the tokens
// queued after it, which may share its outputs), then wait.
void resolve_pending(th_ctx* c);

// Waits for the stream and settles the asynchronous tokens' band flags.
void drain(th_ctx* c) {
  wait_stream(c);
  resolve_pending(c);
}

// Before a key goes away: settle the queued tokens that read it.
void settle_before_free(th_ctx* c, const void* key) {
  std::lock_guard<std::mutex> lk(c->mu);
  for (const AsyncToken& t : c->pending)
    if ((const void*)t.pk == key || (const void*)t.sk == key) {
      use_device(c);
      drain(c);
      return;
    }
}

// A zeroed region of n band flags (one per sampled input) for one call.
uint32_t take_flags(th_ctx* c, uint32_t n) {
  need(n <= c->bflag_cap, "too many sampled inputs in one call", TH_EINVAL);
  if (c->bflag_used + n > c->bflag_cap) drain(c);  // frees every region held by queued tokens
  const uint32_t off = c->bflag_used;
  memset(c->bflag_host + off, 0, n);
  c->bflag_used += n;
  return off;
}

// The region taken last by a call that has checked its flags.
void release_flags(th_ctx* c, uint32_t off) { c->bflag_used = off; }

bool any_flag(const th_ctx* c, uint32_t off, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i)
    if (c->bflag_host[off + i]) return true;
  return false;
}

// The band flags of one sampling call (a new generation for the device copy).
BandArgs band_args(th_ctx* c, uint32_t off) {
  if (++c->band_gen == 0) {  // the generations wrapped: clear the device copy
    HIPCHK(hipMemsetAsync(c->bflag_gen, 0, (size_t)c->bflag_cap * 4, c->stream));
    c->band_gen = 1;
  }
  return BandArgs{c->bflag_dev + off, c->band, c->bflag_gen + off, c->band_gen};
}

// The public key as prepared pairs, made on the context's stream the first
// time it is needed (queued before its first reader).
const uint64_t* pk_pairs(th_ctx* c, const th_pk* pk) {
  if (!pk->dp) {
    uint64_t* p = (uint64_t*)c->pool.get(2 * 2 * (size_t)c->L * c->N * 8);
    HIPCHK(launch_prepare_pairs(pk->d, p, c->d_bc, c->d_lc, c->N, c->L, 2, c->stream));
    pk->dp = p;
  }
  return pk->dp;
}

// The secret key in Montgomery form, made likewise.
const uint64_t* sk_montgomery(th_ctx* c, const th_sk* sk) {
  if (!sk->dm) {
    uint64_t* p = (uint64_t*)c->pool.get((size_t)c->L * c->N * 8);
    HIPCHK(launch_to_montgomery(sk->d, p, c->d_bc, c->N, c->L, 1, c->stream));
    sk->dm = p;
  }
  return sk->dm;
}

void check_ct(th_ctx* c, const th_ct* ct) {
  need(ct != nullptr, "null ciphertext");
  need(ct->ctx == c, "ciphertext belongs to another context");
}

// ---------------------------------------------------------------- NTT dispatch
void ntt_strided(th_ctx* c, bool inverse, const uint64_t* src, uint64_t* dst, uint32_t njobs, uint32_t limb_mod,
                 uint32_t limb_base = 0) {
  NttArgs a{};
  a.lc = c->d_lc;
  a.jobs = nullptr;
  a.src = src;
  a.dst = dst;
  a.stride = c->N;
  a.limb_mod = limb_mod;
  a.limb_base = limb_base;
  HIPCHK(launch_ntt((int)c->logn, inverse, a, njobs, c->stream));
}

// Transforms of an explicit job list, with an optional operation fused into
// the coefficient load (NttLoad): rc is the rescale-constant row of the
// inputs' level (RESCALE), key the secret key (DOT).
void ntt_list(OpScope& sc, bool inverse, const std::vector<NttJob>& jobs, NttLoad load = NTT_LOAD_NONE,
              const RescaleConst* rc = nullptr, const uint64_t* key = nullptr, NttStore store = NTT_STORE_NONE) {
  th_ctx* c = sc.c;
  if (jobs.empty()) return;
  NttArgs a{};
  a.lc = c->d_lc;
  a.jobs = sc.up(jobs);
  a.load = load;
  a.store = store;
  a.bc = c->d_bc;
  a.rc = rc;
  a.key = key;
  HIPCHK(launch_ntt((int)c->logn, inverse, a, (uint32_t)jobs.size(), c->stream));
}

// ---------------------------------------------------------------- context setup
void build_tables(th_ctx* c) {
  const uint32_t N = c->N, L = c->L;
  std::vector<BarrettConst> bc(L);
  c->h_lc.resize(L);
  // twiddles: per limb forward then inverse, N pairs of 16 bytes each
  const size_t tab_bytes = (size_t)L * 2 * N * 16;
  HIPCHK(hipMalloc(&c->d_tables, tab_bytes));
  std::vector<uint64_t> fw(N), iw(N);
  std::vector<unsigned char> host_tab(tab_bytes);
  for (uint32_t l = 0; l < L; ++l) {
    const uint64_t q = c->q[l];
    const uint64_t psi = primitive_2n_root(N, q);
    need(psi != 0, "no primitive 2N-th root of unity for q=" + std::to_string(q));
    const uint64_t psi_inv = invmod(psi, q);
    uint64_t p = 1, pi = 1;
    for (uint32_t i = 0; i < N; ++i) {  // fwd[brv(i)] = psi^i, inv[brv(i)] = psi^-i (rns.rs:161-185)
      const uint32_t r = __builtin_bitreverse32(i) >> (32 - c->logn);
      fw[r] = p;
      iw[r] = pi;
      p = (uint64_t)(((u128)p * psi) % q);
      pi = (uint64_t)(((u128)pi * psi_inv) % q);
    }
    const bool fp = q < FP64_PRIME_LIMIT;
    unsigned char* fdst = host_tab.data() + (size_t)(2 * l) * N * 16;
    unsigned char* idst = host_tab.data() + (size_t)(2 * l + 1) * N * 16;
    for (uint32_t i = 0; i < N; ++i) {
      if (fp) {
        Fp64Tw a{(double)fw[i], (double)fw[i] / (double)q}, b{(double)iw[i], (double)iw[i] / (double)q};
        memcpy(fdst + 16 * (size_t)i, &a, 16);
        memcpy(idst + 16 * (size_t)i, &b, 16);
      } else {
        ShoupTw a{fw[i], (uint64_t)(((u128)fw[i] << 64) / q)}, b{iw[i], (uint64_t)(((u128)iw[i] << 64) / q)};
        memcpy(fdst + 16 * (size_t)i, &a, 16);
        memcpy(idst + 16 * (size_t)i, &b, 16);
      }
    }
    LimbConst& lc = c->h_lc[l];
    memset(&lc, 0, sizeof(lc));
    lc.q = q;
    lc.two_q = 2 * q;
    lc.n_inv = invmod(N % q, q);
    lc.n_inv_s = (uint64_t)(((u128)lc.n_inv << 64) / q);
    lc.last_w = (uint64_t)(((u128)iw[1] * lc.n_inv) % q);
    lc.last_ws = (uint64_t)(((u128)lc.last_w << 64) / q);
    lc.qd = (double)q;
    lc.qinv = 1.0 / (double)q;
    lc.n_inv_d = (double)lc.n_inv;
    lc.n_inv_dq = (double)lc.n_inv / (double)q;
    lc.last_wd = (double)lc.last_w;
    lc.last_wdq = (double)lc.last_w / (double)q;
    lc.fwd = (const char*)c->d_tables + (size_t)(2 * l) * N * 16;
    lc.inv = (const char*)c->d_tables + (size_t)(2 * l + 1) * N * 16;
    lc.fp64 = fp ? 1 : 0;
    const u128 r = (~(u128)0) / q;
    uint64_t qi = 1;  // q^{-1} mod 2^64 by Newton's iteration (each step doubles the correct bits)
    for (int it = 0; it < 6; ++it) qi *= 2 - q * qi;
    const uint64_t r64 = (uint64_t)(((u128)1 << 64) % q);
    bc[l] = BarrettConst{q, (uint64_t)(r >> 64), (uint64_t)r, (uint64_t)0 - qi, r64, (uint64_t)(((u128)r64 << 64) / q)};
  }
  HIPCHK(hipMemcpy(c->d_tables, host_tab.data(), tab_bytes, hipMemcpyHostToDevice));
  HIPCHK(hipMalloc(&c->d_lc, L * sizeof(LimbConst)));
  HIPCHK(hipMemcpy(c->d_lc, c->h_lc.data(), L * sizeof(LimbConst), hipMemcpyHostToDevice));
  HIPCHK(hipMalloc(&c->d_bc, L * sizeof(BarrettConst)));
  HIPCHK(hipMemcpy(c->d_bc, bc.data(), L * sizeof(BarrettConst), hipMemcpyHostToDevice));
  HIPCHK(hipMalloc(&c->d_q, L * 8));
  HIPCHK(hipMemcpy(c->d_q, c->q.data(), L * 8, hipMemcpyHostToDevice));

  // rescale constants (ciphertext.rs:496-497)
  std::vector<RescaleConst> rc((size_t)(L + 1) * L);
  for (uint32_t lev = 2; lev <= L; ++lev) {
    const uint64_t qlast = c->q[lev - 1];
    for (uint32_t l = 0; l + 1 < lev; ++l) {
      const uint64_t q = c->q[l];
      RescaleConst& x = rc[(size_t)lev * L + l];
      x.q = q;
      x.inv = invmod(qlast % q, q);
      x.inv_s = (uint64_t)(((u128)x.inv << 64) / q);
      x.b = bc[l];
      x.qd = (double)q;
      x.qinv = 1.0 / (double)q;
      x.inv_d = (double)x.inv;
      x.inv_dq = (double)x.inv / (double)q;  // correctly rounded: both operands are exact (q < 2^53)
      x.k32 = (double)((1ULL << 32) % q);
      x.k32q = x.k32 / (double)q;
    }
  }
  HIPCHK(hipMalloc(&c->d_rc, rc.size() * sizeof(RescaleConst)));
  HIPCHK(hipMemcpy(c->d_rc, rc.data(), rc.size() * sizeof(RescaleConst), hipMemcpyHostToDevice));

  // decode constants (encoding.rs:221-233, ciphertext.rs:352-390)
  DecodeConst dc;
  memset(&dc, 0, sizeof(dc));
  dc.q0 = c->q[0];
  dc.half_q0 = c->q[0] / 2;
  if (L >= 2) {
    dc.q1 = c->q[1];
    dc.q0_inv_q1 = invmod(c->q[0] % c->q[1], c->q[1]);
    dc.q0_inv_q1_s = (uint64_t)(((u128)dc.q0_inv_q1 << 64) / c->q[1]);
    dc.b1 = bc[1];
    const u128 Q = (u128)c->q[0] * c->q[1], h = Q / 2;
    dc.Q_lo = (uint64_t)Q;
    dc.Q_hi = (uint64_t)(Q >> 64);
    dc.halfQ_lo = (uint64_t)h;
    dc.halfQ_hi = (uint64_t)(h >> 64);
  }
  HIPCHK(hipMalloc(&c->d_dc, sizeof(DecodeConst)));
  HIPCHK(hipMemcpy(c->d_dc, &dc, sizeof(dc), hipMemcpyHostToDevice));

  c->enc.init(N);
  HIPCHK(hipMalloc(&c->d_twist_re, N * 8));
  HIPCHK(hipMalloc(&c->d_twist_im, N * 8));
  HIPCHK(hipMalloc(&c->d_stage_re, N * 8));
  HIPCHK(hipMalloc(&c->d_stage_im, N * 8));
  HIPCHK(hipMemcpy(c->d_twist_re, c->enc.twist_re.data(), N * 8, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d_twist_im, c->enc.twist_im.data(), N * 8, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d_stage_re, c->enc.stage_re.data(), N * 8, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d_stage_im, c->enc.stage_im.data(), N * 8, hipMemcpyHostToDevice));
}

void destroy_ctx(th_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  c->pool.release_all();
  c->ring.destroy();
  void* bufs[] = {c->d_lc, c->d_bc, c->d_q, c->d_rc, c->d_dc, c->d_twist_re, c->d_twist_im,
                  c->d_stage_re, c->d_stage_im, c->d_tables, c->bflag_gen, c->key_end};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  for (auto& kv : c->seg_w) (void)hipFree(kv.second);
  for (auto& kv : c->seg_p) (void)hipFree(kv.second);
  if (c->bflag_host) (void)hipHostFree(c->bflag_host);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

// ---------------------------------------------------------------- host-side inputs
void pad_input(const th_ctx* c, const double* z, size_t n, double* out) {
  // lib.rs:123-126: pad or truncate to N/2 slots
  const size_t S = c->N / 2;
  const size_t m = std::min(n, S);
  if (m) memcpy(out, z, m * 8);
  if (m < S) memset(out + m, 0, (S - m) * 8);
}


void download(th_ctx* c, void* dst, const void* src_dev, size_t bytes);

// The draws of device_key_draws' KEY_UNIFORM_GAUSS jobs made on the host with
// glibc, for calls whose device draws had a Gaussian in the sampler's band:
// `count` stretches of the stream of `seed`, input after input (a for every
// limb, then e; ciphertext.rs:119-127, :183-196), uploaded to a[i] (L x N)
// and e + i N.
void host_key_draws(OpScope& sc, uint64_t seed, size_t count, uint64_t* const* a, int64_t* e) {
  th_ctx* c = sc.c;
  const uint32_t N = c->N, L = c->L;
  ChaChaStream s(seed);
  std::vector<uint64_t> av((size_t)L * N);
  std::vector<int64_t> ev((size_t)count * N);
  for (size_t i = 0; i < count; ++i) {
    for (uint32_t l = 0; l < L; ++l)
      for (uint32_t k = 0; k < N; ++k) av[(size_t)l * N + k] = s.below_u64(c->q[l]);
    draw_gaussian(s, N, ev.data() + i * N);
    HIPCHK(hipMemcpyAsync(a[i], sc.up(av), av.size() * 8, hipMemcpyDeviceToDevice, c->stream));
  }
  HIPCHK(hipMemcpyAsync(e, sc.up(ev), ev.size() * 8, hipMemcpyDeviceToDevice, c->stream));
}

// Key and secret-key-encryption draws (launch_key_draws) for `jobs`,
// consecutive stretches of one stream: job i starts where job i - 1's draws
// end. Every job is drawn in parallel as if no word were rejected; from the
// first job that held a rejected word, that job is drawn serially
// (launch_key_replay) and the jobs after it are drawn again in parallel from
// where it ended, until no rejection is left. Waits for the stream. Returns
// whether a Gaussian draw landed in the sampler's band, in which case the
// caller draws the randomness again on the host with glibc.
bool device_key_draws(th_ctx* c, std::vector<KeyDrawJob> jobs) {
  const uint32_t N = c->N, L = c->L, nj = (uint32_t)jobs.size();
  if (!nj) return false;
  const uint32_t off = take_flags(c, nj);
  const BandArgs band{c->bflag_dev + off, c->band};
  uint64_t word = jobs[0].word0;
  for (uint32_t j = 0; j < nj;) {
    for (uint32_t i = j; i < nj; ++i) {
      jobs[i].word0 = word;
      word += key_draw_words(jobs[i].kind, N, L);
    }
    OpScope sc(c);
    const KeyDrawJob* dj = (const KeyDrawJob*)sc.upload(jobs.data() + j, (nj - j) * sizeof(KeyDrawJob));
    const uint32_t none = 0xFFFFFFFFu;
    void* h = c->ring.reserve(4, c->stream);
    memcpy(h, &none, 4);
    HIPCHK(hipMemcpyAsync(c->key_reject, h, 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(launch_key_draws(dj, nj - j, N, L, c->d_bc, c->key_reject, band_from(band, j), c->stream));
    uint32_t r = 0;
    download(c, &r, c->key_reject, 4);
    if (c->force_serial) r = 0;  // TH_OPT_FORCE_SERIAL_SAMPLER: every job drawn serially (testing)
    if (r >= nj - j) break;
    // job j + r and the ones after it move: their flags from this pass do not count
    memset(c->bflag_host + off + j + r, 0, nj - j - r);
    HIPCHK(launch_key_replay(dj + r, N, L, c->d_bc, c->key_end, band_from(band, j + r), c->stream));
    download(c, &word, c->key_end, 8);
    j += r + 1;
  }
  const bool flagged = any_flag(c, off, nj);
  release_flags(c, off);
  return flagged;
}

// GPU encode of `count` padded inputs (device, count x N/2) into dst + i*dst_stride:
// M = m (+ e0), and E1, U when those are given (encoding.rs:173-207).
void queue_encode(OpScope& sc, const double* z, size_t count, const uint8_t* u, const int64_t* e0,
                  const int64_t* e1, uint64_t* dst, size_t dst_stride, uint32_t rep_d = 0, uint32_t rep_cols = 0) {
  th_ctx* c = sc.c;
  const uint32_t N = c->N, S = N / 2;
  double* parts = (double*)sc.dev(count * encode_parts_doubles(c->logn) * 8);
  std::vector<EncodeJob> ej(count);
  for (size_t i = 0; i < count; ++i) {
    ej[i].z = rep_d ? z + i * rep_d : z + i * S;
    ej[i].rep_d = rep_d;
    ej[i].rep_cols = rep_cols;
    ej[i].u = u ? u + i * N : nullptr;
    ej[i].e0 = e0 ? e0 + i * N : nullptr;
    ej[i].e1 = e1 ? e1 + i * N : nullptr;
    ej[i].dst = dst + i * dst_stride;
    ej[i].parts = parts + i * encode_parts_doubles(c->logn);
  }
  HIPCHK(launch_encode(sc.up(ej), (uint32_t)count, c->d_bc, c->d_twist_re, c->d_twist_im, c->d_stage_re,
                       c->d_stage_im, c->logn, c->L, c->stream));
}

// encrypt_pk's draws on the host (ciphertext.rs:255-273): u, then e0, then e1.
void draw_pk_randomness(uint64_t seed, int has_seed, uint32_t N, uint8_t* u, int64_t* e0, int64_t* e1) {
  ChaChaStream s = has_seed ? ChaChaStream(seed) : ChaChaStream::from_os_entropy();
  draw_ternary(s, N, u);
  draw_gaussian(s, N, e0);
  draw_gaussian(s, N, e1);
}

// encrypt_pk's randomness of `count` seeded inputs drawn on the host with
// glibc, exactly as the reference draws it, in device buffers u, e0, e1
// (count x N each) of the caller's scope.
void upload_host_draws(OpScope& sc, const uint64_t* seeds, size_t count, uint8_t* u, int64_t* e0, int64_t* e1) {
  th_ctx* c = sc.c;
  const uint32_t N = c->N;
  std::vector<uint8_t> hu(count * N);
  std::vector<int64_t> he0(count * N), he1(count * N);
  parallel_for(count, [&](size_t i) { draw_pk_randomness(seeds[i], 1, N, &hu[i * N], &he0[i * N], &he1[i * N]); });
  HIPCHK(hipMemcpyAsync(u, sc.up(hu), hu.size(), hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(hipMemcpyAsync(e0, sc.up(he0), he0.size() * 8, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(hipMemcpyAsync(e1, sc.up(he1), he1.size() * 8, hipMemcpyDeviceToDevice, c->stream));
}

// Queue encrypt_pk of `count` inputs already on the device (z: count x N/2
// padded slots, or count x rep_d values replicated rep_cols times) into the
// ciphertext buffers out[i] (2 x L limb-polys each). The randomness comes from
// the device sampler (seeds, band flags `band`), or, with host_draw, from the
// host (upload_host_draws).
void queue_encrypt_pk(OpScope& sc, const th_pk* pk, const double* z, size_t count, const uint64_t* seeds,
                      uint32_t rep_d, uint32_t rep_cols, uint64_t* const* out, bool host_draw, BandArgs band) {
  th_ctx* c = sc.c;
  const uint32_t N = c->N, L = c->L;
  uint8_t* u = (uint8_t*)sc.dev(count * N);
  int64_t* e0 = (int64_t*)sc.dev(count * N * 8);
  int64_t* e1 = (int64_t*)sc.dev(count * N * 8);
  if (host_draw) {
    upload_host_draws(sc, seeds, count, u, e0, e1);
  } else {
    std::vector<SampleJob> sj(count);
    for (size_t i = 0; i < count; ++i) sj[i] = SampleJob{seeds[i], u + i * N, e0 + i * N, e1 + i * N, nullptr};
    HIPCHK(launch_sample_pk(sc.up(sj), (uint32_t)count, N, c->force_serial, c->stream, nullptr, false, false, band));
  }
  uint64_t* prep = (uint64_t*)sc.dev(count * 3 * L * poly_bytes(c));
  queue_encode(sc, z, count, u, e0, e1, prep, (size_t)3 * L * N, rep_d, rep_cols);
  ntt_strided(c, false, prep, prep, (uint32_t)(count * 3 * L), L);
  std::vector<EncCombineJob> cj(count);
  for (size_t i = 0; i < count; ++i) cj[i] = EncCombineJob{prep + i * 3 * L * N, pk->d, pk->d + (size_t)L * N, out[i]};
  HIPCHK(launch_encrypt_combine(sc.up(cj), (uint32_t)count, c->d_bc, N, L, c->stream));
}

// Queue encrypt_pk of `count` padded inputs (device z, count x N/2) with
// host-supplied randomness (host arrays, count x N each) into out[i].
void queue_encrypt_pk_explicit(OpScope& sc, const th_pk* pk, const double* z, size_t count, const uint8_t* hu,
                               const int64_t* he0, const int64_t* he1, uint64_t* const* out) {
  th_ctx* c = sc.c;
  const uint32_t N = c->N, L = c->L;
  const uint8_t* u = (const uint8_t*)sc.upload(hu, count * N);
  const int64_t* e0 = (const int64_t*)sc.upload(he0, count * N * 8);
  const int64_t* e1 = (const int64_t*)sc.upload(he1, count * N * 8);
  uint64_t* prep = (uint64_t*)sc.dev(count * 3 * L * poly_bytes(c));
  queue_encode(sc, z, count, u, e0, e1, prep, (size_t)3 * L * N);
  ntt_strided(c, false, prep, prep, (uint32_t)(count * 3 * L), L);
  std::vector<EncCombineJob> cj(count);
  for (size_t i = 0; i < count; ++i) cj[i] = EncCombineJob{prep + i * 3 * L * N, pk->d, pk->d + (size_t)L * N, out[i]};
  HIPCHK(launch_encrypt_combine(sc.up(cj), (uint32_t)count, c->d_bc, N, L, c->stream));
}

// New ciphertexts for `count` encrypt_pk outputs (ciphertext.rs:314-318).
std::vector<th_ct*> new_encrypt_outputs(th_ctx* c, size_t count) {
  std::vector<th_ct*> made;
  try {
    for (size_t i = 0; i < count; ++i) made.push_back(new_ct(c, c->L, kScale));
  } catch (...) {
    drop_all_rethrow(made);
  }
  return made;
}

// encrypt_pk of `count` padded inputs zh (host, count x N/2) with
// host-supplied randomness (count x N each).
void encrypt_pk_explicit_many(th_ctx* c, const th_pk* pk, const double* zh, size_t count, const uint8_t* hu,
                              const int64_t* he0, const int64_t* he1, th_ct** outs) {
  std::vector<th_ct*> made = new_encrypt_outputs(c, count);
  try {
    OpScope sc(c);
    const double* z = (const double*)sc.upload(zh, count * (c->N / 2) * 8);
    std::vector<uint64_t*> dst(count);
    for (size_t i = 0; i < count; ++i) dst[i] = made[i]->d;
    queue_encrypt_pk_explicit(sc, pk, z, count, hu, he0, he1, dst.data());
  } catch (...) {
    drop_all_rethrow(made);
  }
  for (size_t i = 0; i < count; ++i) outs[i] = made[i];
}

// Seeded encrypt_pk of `count` padded inputs through the configured sampler.
// With the device sampler the call waits for its work: if a Gaussian draw
// landed in the band, the inputs are encrypted again from glibc draws
// (host sampler) into the same ciphertexts before they are returned.
void encrypt_pk_seeded(th_ctx* c, const th_pk* pk, const double* zh, size_t count, const uint64_t* seeds,
                       th_ct** outs) {
  const uint32_t N = c->N, S = N / 2;
  std::vector<th_ct*> made = new_encrypt_outputs(c, count);
  try {
    OpScope sc(c);
    const double* z = (const double*)sc.upload(zh, count * S * 8);
    std::vector<uint64_t*> dst(count);
    for (size_t i = 0; i < count; ++i) dst[i] = made[i]->d;
    if (c->host_sampler) {
      queue_encrypt_pk(sc, pk, z, count, seeds, 0, 0, dst.data(), true, BandArgs{nullptr, 0.0});
    } else {
      const uint32_t off = take_flags(c, (uint32_t)count);
      queue_encrypt_pk(sc, pk, z, count, seeds, 0, 0, dst.data(), false, band_args(c, off));
      wait_stream(c);
      if (any_flag(c, off, (uint32_t)count)) {
        queue_encrypt_pk(sc, pk, z, count, seeds, 0, 0, dst.data(), true, BandArgs{nullptr, 0.0});
        c->redrawn_inputs += count;
      }
      release_flags(c, off);
    }
  } catch (...) {
    drop_all_rethrow(made);
  }
  for (size_t i = 0; i < count; ++i) outs[i] = made[i];
}

// ---------------------------------------------------------------- pipelines on raw device ciphertexts
// A ciphertext in device memory: c0 then c1, `limbs` limb-polys each.
struct CtView {
  const uint64_t* d;
  uint32_t limbs;
  double scale;
};

std::vector<CtView> views_of(const th_ct* const* cts, size_t count) {
  std::vector<CtView> v(count);
  for (size_t i = 0; i < count; ++i) v[i] = CtView{cts[i]->d, cts[i]->limbs, cts[i]->scale};
  return v;
}

// Segment-sum weights for (d, cols), built on first use and kept for the
// context's lifetime (cols x N doubles).
const double* seg_weights(th_ctx* c, uint32_t d, uint32_t cols) {
  auto key = std::make_pair(d, cols);
  auto it = c->seg_w.find(key);
  if (it != c->seg_w.end()) return it->second;
  std::vector<double> w((size_t)cols * c->N);
  segment_weights(c->N, d, cols, w.data());
  double* dev = nullptr;
  HIPCHK(hipMalloc(&dev, w.size() * 8));
  c->seg_w[key] = dev;
  HIPCHK(hipMemcpy(dev, w.data(), w.size() * 8, hipMemcpyHostToDevice));
  return dev;
}

// Segment-weight pairs (segment_weight_pairs) for segments of d slots, cached
// per context; used by the decrypt transform's segment-sum epilogue.
const double* seg_pairs(th_ctx* c, uint32_t d) {
  auto it = c->seg_p.find(d);
  if (it != c->seg_p.end()) return it->second;
  std::vector<double> w((size_t)2 * c->N);
  segment_weight_pairs(c->N, d, w.data());
  double* dev = nullptr;
  HIPCHK(hipMalloc(&dev, w.size() * 8));
  c->seg_p[d] = dev;
  HIPCHK(hipMemcpy(dev, w.data(), w.size() * 8, hipMemcpyHostToDevice));
  return dev;
}

// Queue decrypt + decode of the views; slots to out_dev (count x S) and/or
// segment sums to seg_dev (count x cols). m_l = c0_l + c1_l * s_l
// (ciphertext.rs:332-341) is formed inside the inverse transform's load.
// When only segment sums are wanted (and cols <= SEGSUM_MAX_COLS) they come
// from the coefficients and the segment weights, without forming the slots.
// Scratch lives in the caller's scope.
// The decrypt transform can produce segment sums itself (NTT_STORE_SEGSUM)
// when its batch runs in the whole-polynomial kernel.
// Fewest batches for which a LoRA set rescales and decrypts with one
// workgroup per product by default (build_lora).
constexpr uint32_t RD_WHOLE_MIN_BATCHES = 160;

bool segsum_in_transform(const th_ctx* c, uint32_t jobs, uint32_t cols) {
  return c->logn <= 14 && jobs <= 256 && cols >= 1 && cols <= NTT_SEGSUM_FUSED_MAX_COLS;
}

// Decrypt transforms (c0 + c1 s on limb 0, inverse NTT) whose epilogue writes
// each job's segment sums to its dst: launches of at most one round of
// whole-polynomial workgroups (256 jobs), so that a job's sums do not depend
// on how many jobs the batch has.
void launch_dot_segsum(th_ctx* c, const NttJob* d_jobs, uint32_t n, const th_sk* sk, const double* W, uint32_t cols) {
  NttArgs a{};
  a.lc = c->d_lc;
  a.load = NTT_LOAD_DOTM;
  a.store = NTT_STORE_SEGSUM;
  a.bc = c->d_bc;
  a.key = sk_montgomery(c, sk);
  a.segw = W;
  a.cols = cols;
  for (uint32_t off = 0; off < n; off += 256) {
    a.jobs = d_jobs + off;
    HIPCHK(launch_ntt((int)c->logn, true, a, std::min<uint32_t>(256, n - off), c->stream));
  }
}

void queue_decrypt(OpScope& sc, const std::vector<CtView>& cts, const th_sk* sk, double* out_dev, double* seg_dev,
                   uint32_t d, uint32_t cols) {
  th_ctx* c = sc.c;
  const size_t count = cts.size();
  const uint32_t N = c->N, S = N / 2;
  uint64_t* dot = (uint64_t*)sc.dev(count * 2 * poly_bytes(c));
  double* parts = (double*)sc.dev(count * decode_parts_doubles(c->logn) * 8);
  std::vector<NttJob> nj;
  std::vector<DecodeJob> dec(count);
  for (size_t i = 0; i < count; ++i) {
    const CtView& ct = cts[i];
    // ciphertext.rs:351: CRT branch iff scale > 1.5 * 2^40 and at least two limbs
    const uint32_t nl = (ct.scale > kScale * 1.5 && ct.limbs >= 2) ? 2 : 1;
    uint64_t* o = dot + i * 2 * N;
    for (uint32_t l = 0; l < nl; ++l)
      nj.push_back(NttJob{ct.d + (size_t)l * N, o + (size_t)l * N, ct.d + (size_t)(ct.limbs + l) * N, nullptr, l, 0});
    dec[i].m = o;
    dec[i].parts = parts + i * decode_parts_doubles(c->logn);
    dec[i].out = out_dev ? out_dev + i * S : nullptr;
    dec[i].seg = seg_dev ? seg_dev + i * cols : nullptr;
    dec[i].scale = ct.scale;
    dec[i].crt = nl == 2;
  }
  const bool seg_only = seg_dev && !out_dev && cols >= 1 && cols <= SEGSUM_MAX_COLS;
  if (seg_only && nj.size() == count && segsum_in_transform(c, (uint32_t)count, cols)) {
    // every ciphertext takes the limb-0 branch: the segment sums come out of
    // the decrypt transform itself
    for (size_t i = 0; i < count; ++i) {
      nj[i].dst = reinterpret_cast<uint64_t*>(seg_dev + i * cols);
      nj[i].scale = cts[i].scale;
    }
    launch_dot_segsum(c, sc.up(nj), (uint32_t)count, sk, seg_pairs(c, d), cols);
    return;
  }
  ntt_list(sc, true, nj, NTT_LOAD_DOT, nullptr, sk->d);
  if (seg_only)
    HIPCHK(launch_segsum(sc.up(dec), (uint32_t)count, c->d_dc, seg_weights(c, d, cols), c->logn, cols, c->stream));
  else
    HIPCHK(launch_decode(sc.up(dec), (uint32_t)count, c->d_dc, c->d_twist_re, c->d_twist_im, c->d_stage_re,
                         c->d_stage_im, c->logn, d, cols, c->stream));
}

// out[i] = in[i] x pt[i] on in[i]'s limbs (ciphertext.rs:422-429); out[i] has 2 x limbs limb-polys.
void queue_ct_pt(OpScope& sc, const std::vector<CtView>& in, const uint64_t* const* pts, uint64_t* const* out) {
  th_ctx* c = sc.c;
  std::vector<CtPtJob> jobs(in.size());
  uint32_t maxl = 1;
  for (size_t i = 0; i < in.size(); ++i) {
    const size_t ln = (size_t)in[i].limbs * c->N;
    jobs[i] = CtPtJob{in[i].d, in[i].d + ln, pts[i], out[i], in[i].limbs, 0};
    maxl = std::max(maxl, in[i].limbs);
  }
  HIPCHK(launch_ct_pt_mul(sc.up(jobs), (uint32_t)in.size(), maxl, c->d_bc, c->N, c->stream));
}

// Rescale (ciphertext.rs:476-535) of views that all have L >= 2 limbs into
// out[i] (2 x (L-1) limb-polys each), in the evaluation domain: for each
// component, inverse NTT of the last limb only, then for l < L-1 a forward
// NTT of (c_last mod q_l) whose store forms (C_l - NTT(c_last mod q_l)) *
// (q_last mod q_l)^{-1}; equal residue for residue to the reference's
// coefficient-domain rescale because the NTT is linear mod q_l. With pts,
// input i is first multiplied by pts[i] (ct_pt_mul_ntt, ciphertext.rs:
// 422-429): C_l = ct_l * pt_l in the store and ct_last * pt_last in the
// inverse transform's load, so the product ciphertext is never stored.
void queue_rescale(OpScope& sc, const std::vector<CtView>& in, uint64_t* const* out,
                   const uint64_t* const* pts = nullptr) {
  th_ctx* c = sc.c;
  const uint32_t N = c->N;
  const size_t count = in.size();
  const uint32_t L = in[0].limbs;
  uint64_t* last = (uint64_t*)sc.dev(count * 2 * poly_bytes(c));  // coefficient-domain last limbs
  std::vector<NttJob> inv, fwd;
  inv.reserve(count * 2);
  fwd.reserve(count * 2 * (L - 1));
  for (size_t i = 0; i < count; ++i)
    for (uint32_t comp = 0; comp < 2; ++comp) {
      const uint64_t* cc = in[i].d + (size_t)comp * L * N;
      uint64_t* lc = last + (i * 2 + comp) * N;
      inv.push_back(NttJob{cc + (size_t)(L - 1) * N, lc, pts ? pts[i] + (size_t)(L - 1) * N : nullptr, nullptr,
                           L - 1, 0});
      for (uint32_t l = 0; l + 1 < L; ++l)
        fwd.push_back(NttJob{lc, out[i] + (size_t)(comp * (L - 1) + l) * N, cc + (size_t)l * N,
                             pts ? pts[i] + (size_t)l * N : nullptr, l, 0});
    }
  NttArgs ia{}, fa{};
  ia.lc = fa.lc = c->d_lc;
  ia.bc = fa.bc = c->d_bc;
  ia.jobs = sc.up(inv);
  ia.load = pts ? NTT_LOAD_MUL : NTT_LOAD_NONE;
  fa.jobs = sc.up(fwd);
  fa.load = NTT_LOAD_REDUCE;
  fa.store = pts ? NTT_STORE_MUL_RESCALE : NTT_STORE_RESCALE;
  fa.rc = c->d_rc + (size_t)L * c->L;
  HIPCHK(launch_rescale((int)c->logn, ia, (uint32_t)inv.size(), fa, (uint32_t)fwd.size(), c->stream));
}

void check_decrypt_args(th_ctx* c, const th_ct* const* cts, size_t count, const th_sk* sk) {
  need(sk && sk->ctx == c, "secret key belongs to another context");
  need(cts != nullptr || count == 0, "null ciphertext list");
  for (size_t i = 0; i < count; ++i) check_ct(c, cts[i]);
}

// D2H through the staging ring, then wait.
void download(th_ctx* c, void* dst, const void* src_dev, size_t bytes) {
  void* h = c->ring.reserve(bytes, c->stream);
  HIPCHK(hipMemcpyAsync(h, src_dev, bytes, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(hipStreamSynchronize(c->stream));
  memcpy(dst, h, bytes);
}

void rescale_many(th_ctx* c, const th_ct* const* cts, size_t count, th_ct** outs) {
  const uint32_t L = cts[0]->limbs;
  for (size_t i = 0; i < count; ++i) {
    check_ct(c, cts[i]);
    need(cts[i]->limbs == L, "rescale_batch: all ciphertexts must have the same limb count");
  }
  need(L >= 2, "Cannot rescale: only 1 limb left", TH_ESTATE);  // ciphertext.rs:479
  std::vector<th_ct*> made;
  try {
    std::vector<uint64_t*> dst(count);
    for (size_t i = 0; i < count; ++i) {
      made.push_back(new_ct(c, L - 1, cts[i]->scale / (double)c->q[L - 1]));  // ciphertext.rs:533
      dst[i] = made.back()->d;
    }
    OpScope sc(c);
    queue_rescale(sc, views_of(cts, count), dst.data());
  } catch (...) {
    drop_all_rethrow(made);
  }
  for (size_t i = 0; i < count; ++i) outs[i] = made[i];
}

th_pt* encode_pt(th_ctx* c, const double* z, size_t n) {
  std::vector<double> pad(c->N / 2);
  pad_input(c, z, n, pad.data());
  th_pt* pt = adopt(new th_pt{c, c->L, nullptr});
  try {
    pt->d = (uint64_t*)c->pool.get(c->L * poly_bytes(c));
    OpScope sc(c);
    const double* zd = sc.up(pad);
    queue_encode(sc, zd, 1, nullptr, nullptr, nullptr, pt->d, 0);
    ntt_strided(c, false, pt->d, pt->d, c->L, c->L);
  } catch (...) {
    drop(pt);
    throw;
  }
  return pt;
}

void ct_pt_many(th_ctx* c, const th_ct* const* cts, const th_pt* const* pts, size_t count, th_ct** outs) {
  std::vector<th_ct*> made;
  try {
    std::vector<const uint64_t*> p(count);
    std::vector<uint64_t*> dst(count);
    for (size_t i = 0; i < count; ++i) {
      check_ct(c, cts[i]);
      need(pts[i] && pts[i]->ctx == c, "plaintext belongs to another context");
      need(pts[i]->limbs >= cts[i]->limbs, "plaintext has fewer limbs than the ciphertext");
      made.push_back(new_ct(c, cts[i]->limbs, cts[i]->scale * cts[i]->scale));  // ciphertext.rs:427
      dst[i] = made.back()->d;
      p[i] = pts[i]->d;
    }
    OpScope sc(c);
    queue_ct_pt(sc, views_of(cts, count), p.data(), dst.data());
  } catch (...) {
    drop_all_rethrow(made);
  }
  for (size_t i = 0; i < count; ++i) outs[i] = made[i];
}

// ct_add / ct_sub (ciphertext.rs:435-466): the result has a's limbs and
// scale; RnsPoly::add/sub (rns.rs:217-240) run over self's limbs and index
// the other operand's, so b may have more limbs (a rescaled ciphertext plus
// one at the top level) and fewer is the reference's out-of-bounds panic.
void add_sub(th_ctx* c, const th_ct* a, const th_ct* b, bool sub, th_ct** out) {
  check_ct(c, a);
  check_ct(c, b);
  // ciphertext.rs:436-441
  need(fabs(a->scale - b->scale) < 1.0, std::string("Scale mismatch in ") + (sub ? "ct_sub" : "ct_add"));
  need(b->limbs >= a->limbs, std::string(sub ? "ct_sub" : "ct_add") + ": the second ciphertext has " +
                                 std::to_string(b->limbs) + " limbs, fewer than the first's " +
                                 std::to_string(a->limbs));
  th_ct* o = new_ct(c, a->limbs, a->scale);
  const size_t N = c->N;
  AddJob j{a->d, a->d + (size_t)a->limbs * N, b->d, b->d + (size_t)b->limbs * N, o->d, a->limbs, sub ? 1u : 0u};
  try {
    OpScope sc(c);
    HIPCHK(launch_ct_addsub(sc.up(std::vector<AddJob>{j}), 1, a->limbs, c->d_q, c->N, c->stream));
  } catch (...) {
    drop(o);
    throw;
  }
  *out = o;
}

void ntt_batch(th_ctx* c, uint64_t* polys, size_t count, uint32_t limbs, int on_device, bool inverse) {
  need(limbs >= 1 && limbs <= c->L, "limbs must be in [1, L]");
  const size_t bytes = count * limbs * poly_bytes(c);
  if (!count) return;
  if (on_device) {
    ntt_strided(c, inverse, polys, polys, (uint32_t)(count * limbs), limbs);
    return;
  }
  OpScope sc(c);
  uint64_t* d = (uint64_t*)sc.upload(polys, bytes);
  ntt_strided(c, inverse, d, d, (uint32_t)(count * limbs), limbs);
  download(c, polys, d, bytes);
}

}  // namespace

// ================================================================ C ABI
extern "C" {

const char* th_last_error(void) { return g_err.c_str(); }
const char* th_version(void) { return "tensafe-he-mi355x 0.1.0 (gfx950)"; }

int th_device_count(int* count) {
  return guarded([&] {
    need(count != nullptr, "null output");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    *count = n;
  });
}

int th_ctx_create(uint32_t N, const uint64_t* moduli, uint32_t L, uint32_t scale_bits, int device, th_ctx** out) {
  return guarded([&] {
    need(out != nullptr, "null output");
    *out = nullptr;
    need(N >= (1u << NTT_MIN_LOGN) && N <= (1u << NTT_MAX_LOGN) && (N & (N - 1)) == 0,
         "Unsupported poly_mod_degree: " + std::to_string(N) + ". Use a power of two in [1024, 32768].");
    need(scale_bits == 40, "scale_bits must be 40");
    std::vector<uint64_t> q;
    if (moduli) {
      need(L >= 1 && L <= 16, "L must be in [1, 16]");
      q.assign(moduli, moduli + L);
      for (uint32_t i = 0; i < L; ++i) {
        need(q[i] < (1ULL << 61), "moduli must be below 2^61");
        need(q[i] % (2ULL * N) == 1, "modulus " + std::to_string(q[i]) + " is not 1 mod 2N");
        need(is_prime(q[i]), "modulus " + std::to_string(q[i]) + " is not prime");
        for (uint32_t j = 0; j < i; ++j) need(q[i] != q[j], "moduli must be distinct");
      }
    } else {
      need(default_chain(N, q), "Unsupported poly_mod_degree: " + std::to_string(N) +
                                    ". Use 8192, 16384, or 32768.");  // lib.rs:38-47
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
      (void)hipGetLastError();
      raise(TH_EDEVICE, "no HIP device available (the tensafe_he engine requires an MI355X / gfx950 GPU)");
    }
    need(device >= 0 && device < ndev, "device index out of range", TH_EDEVICE);
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      raise(TH_EDEVICE, std::string("device is ") + prop.gcnArchName + ", the engine is built for gfx950");
    th_ctx* c = new th_ctx();
    try {
      c->device = device;
      c->N = N;
      c->logn = (uint32_t)__builtin_ctz(N);
      c->L = (uint32_t)q.size();
      c->q = q;
      HIPCHK(hipSetDevice(device));
      c->scratch = scratch_base(device);
      HIPCHK(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
      build_tables(c);
      c->ring.init(64u << 20);
      c->bflag_cap = 1u << 16;
      HIPCHK(hipHostMalloc((void**)&c->bflag_host, c->bflag_cap, hipHostMallocMapped | hipHostMallocCoherent));
      HIPCHK(hipHostGetDevicePointer((void**)&c->bflag_dev, c->bflag_host, 0));
      HIPCHK(hipMalloc((void**)&c->bflag_gen, (size_t)c->bflag_cap * 4));
      HIPCHK(hipMemset(c->bflag_gen, 0, (size_t)c->bflag_cap * 4));
      HIPCHK(hipMalloc((void**)&c->key_end, 16));  // the end word, then the reject word
      c->key_reject = reinterpret_cast<uint32_t*>(c->key_end + 1);
    } catch (...) {
      destroy_ctx(c);
      throw;
    }
    *out = c;
  });
}

int th_ctx_free(th_ctx* ctx) {
  return guarded([&] {
    if (!ctx) return;
    need(!ctx->closed.exchange(true), "context already freed", TH_ESTATE);
    {
      // settle queued tokens while their handles are certainly alive
      std::lock_guard<std::mutex> lk(ctx->mu);
      use_device(ctx);
      drain(ctx);
    }
    ctx_release(ctx);  // the last handle released frees the context
  });
}

int th_ctx_info(const th_ctx* ctx, uint32_t* N, uint32_t* L, uint64_t* moduli_out) {
  return guarded([&] {
    need(ctx != nullptr, "null context");
    if (N) *N = ctx->N;
    if (L) *L = ctx->L;
    if (moduli_out) memcpy(moduli_out, ctx->q.data(), ctx->L * 8);
  });
}

int th_ctx_sync(th_ctx* ctx) {
  return guarded([&] {
    need(ctx != nullptr, "null context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    use_device(ctx);
    drain(ctx);
  });
}

int th_ctx_stats(th_ctx* ctx, uint64_t* redrawn_inputs) {
  return guarded([&] {
    need(ctx && redrawn_inputs, "null argument");
    std::lock_guard<std::mutex> lk(ctx->mu);
    *redrawn_inputs = ctx->redrawn_inputs;
  });
}

int th_ctx_stream(th_ctx* ctx, void** stream) {
  return guarded([&] {
    need(ctx && stream, "null argument");
    *stream = (void*)ctx->stream;
  });
}

#define TH_LOCK(c)                                                      \
  need((c) != nullptr, "null context");                                 \
  need(!(c)->closed.load(), "the context has been freed", TH_ESTATE);  \
  std::lock_guard<std::mutex> _lk((c)->mu);                             \
  use_device(c)

int th_keygen(th_ctx* ctx, uint64_t seed, int has_seed, th_sk** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr, "null output");
    const uint32_t N = ctx->N, L = ctx->L;
    const uint64_t sd = has_seed ? seed : os_entropy_seed();  // rng.rs:73-76
    th_sk* sk = adopt(new th_sk{ctx, nullptr});
    try {
      sk->d = (uint64_t*)ctx->pool.get(L * poly_bytes(ctx));
      OpScope sc(ctx);
      int64_t* v = (int64_t*)sc.dev((size_t)N * 8);
      // s: N x range_u32(3) as -1, 0, 1 (ciphertext.rs:86-97), on every limb, then NTT
      device_key_draws(ctx, {KeyDrawJob{sd, 0, KEY_TERNARY, 0, v, nullptr, nullptr}});
      HIPCHK(launch_signed_to_rns(v, sk->d, ctx->d_bc, N, L, ctx->stream));
      ntt_strided(ctx, false, sk->d, sk->d, L, L);
    } catch (...) {
      drop(sk);
      throw;
    }
    *out = sk;
  });
}

int th_keygen_public(th_ctx* ctx, const th_sk* sk, uint64_t seed, int has_seed, th_pk** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr && sk != nullptr && sk->ctx == ctx, "bad secret key");
    const uint32_t N = ctx->N, L = ctx->L;
    const uint64_t sd = has_seed ? seed : os_entropy_seed();
    th_pk* pk = adopt(new th_pk{ctx, nullptr});
    try {
      pk->d = (uint64_t*)ctx->pool.get(2 * L * poly_bytes(ctx));
      uint64_t* b = pk->d;
      uint64_t* ad = pk->d + (size_t)L * N;
      OpScope sc(ctx);
      int64_t* e = (int64_t*)sc.dev((size_t)N * 8);
      uint64_t* etmp = (uint64_t*)sc.dev(L * poly_bytes(ctx));
      // ciphertext.rs:119-127: a for every limb, then e, drawn on the device;
      // a Gaussian draw in the sampler's band: all of it again with glibc
      if (device_key_draws(ctx, {KeyDrawJob{sd, 0, KEY_UNIFORM_GAUSS, 0, nullptr, ad, e}})) {
        host_key_draws(sc, sd, 1, &ad, e);
        ctx->redrawn_inputs += 1;
      }
      HIPCHK(launch_signed_to_rns(e, etmp, ctx->d_bc, N, L, ctx->stream));
      ntt_strided(ctx, false, ad, ad, L, L);
      ntt_strided(ctx, false, etmp, etmp, L, L);
      HIPCHK(launch_sub_product(etmp, ad, sk->d, b, ctx->d_bc, N, L, ctx->stream));  // b = e - a*s
    } catch (...) {
      drop(pk);
      throw;
    }
    *out = pk;
  });
}

int th_sk_free(th_sk* sk) {
  return guarded([&] {
    if (!sk) return;
    settle_before_free(sk->ctx, sk);
    drop(sk);
  });
}

int th_pk_free(th_pk* pk) {
  return guarded([&] {
    if (!pk) return;
    settle_before_free(pk->ctx, pk);
    drop(pk);
  });
}

int th_sk_download(th_ctx* ctx, const th_sk* sk, uint64_t* out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(sk && sk->ctx == ctx && out, "bad argument");
    download(ctx, out, sk->d, ctx->L * poly_bytes(ctx));
  });
}

int th_pk_download(th_ctx* ctx, const th_pk* pk, uint64_t* b, uint64_t* a) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(pk && pk->ctx == ctx && b && a, "bad argument");
    const size_t bytes = ctx->L * poly_bytes(ctx);
    download(ctx, b, pk->d, bytes);
    download(ctx, a, pk->d + (size_t)ctx->L * ctx->N, bytes);
  });
}

}  // extern "C"

namespace {
// Secret-key encryption (ciphertext.rs:167-229) of `count` padded inputs
// (host, count x N/2) drawing from ONE stream seeded with `seed`, input after
// input (batch_encrypt's shared RNG, lib.rs:230-258): per input, a on every
// limb then e (on the device; all of it again with glibc on the host when a
// Gaussian lands in the sampler's band); encode m + e; c1 = NTT(a),
// c0 = NTT(m + e) - c1 s.
std::vector<th_ct*> encrypt_sk_many(th_ctx* ctx, const th_sk* sk, const std::vector<double>& pads, size_t count,
                                    uint64_t seed) {
  const uint32_t N = ctx->N, L = ctx->L;
  std::vector<th_ct*> made;
  try {
    for (size_t i = 0; i < count; ++i) made.push_back(new_ct(ctx, L, kScale));
    if (!count) return made;
    OpScope sc(ctx);
    int64_t* e = (int64_t*)sc.dev(count * N * 8);
    uint64_t* me = (uint64_t*)sc.dev(count * L * poly_bytes(ctx));
    std::vector<KeyDrawJob> jobs(count);
    std::vector<uint64_t*> a(count);
    for (size_t i = 0; i < count; ++i) {
      a[i] = made[i]->d + (size_t)L * N;  // c1 = a, transformed below
      jobs[i] = KeyDrawJob{seed, 0, KEY_UNIFORM_GAUSS, 0, nullptr, a[i], e + i * N};
    }
    if (device_key_draws(ctx, jobs)) {
      host_key_draws(sc, seed, count, a.data(), e);
      ctx->redrawn_inputs += count;
    }
    queue_encode(sc, sc.up(pads), count, nullptr, e, nullptr, me, (size_t)L * N);  // M = m + e
    for (size_t i = 0; i < count; ++i) {
      uint64_t* m = me + i * L * N;
      ntt_strided(ctx, false, m, m, L, L);
      ntt_strided(ctx, false, a[i], a[i], L, L);
      HIPCHK(launch_sub_product(m, a[i], sk->d, made[i]->d, ctx->d_bc, N, L, ctx->stream));  // c0 = (m + e) - a*s
    }
  } catch (...) {
    drop_all_rethrow(made);
  }
  return made;
}
}  // namespace

extern "C" {

int th_encrypt(th_ctx* ctx, const th_sk* sk, const double* z, size_t n, uint64_t seed, int has_seed, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out && sk && sk->ctx == ctx, "bad argument");
    need(z != nullptr || n == 0, "null input");
    std::vector<double> pad(ctx->N / 2);
    pad_input(ctx, z, n, pad.data());
    *out = encrypt_sk_many(ctx, sk, pad, 1, has_seed ? seed : os_entropy_seed())[0];
  });
}

int th_encrypt_batch(th_ctx* ctx, const th_sk* sk, const double* z, const uint64_t* lens, size_t stride,
                     size_t count, uint64_t seed, int has_seed, th_ct** outs) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(outs && sk && sk->ctx == ctx && (count == 0 || (z && lens)), "bad argument");
    const size_t S = ctx->N / 2;
    std::vector<double> pads(count * S);
    for (size_t i = 0; i < count; ++i) pad_input(ctx, z + i * stride, (size_t)lens[i], pads.data() + i * S);
    const std::vector<th_ct*> made =
        encrypt_sk_many(ctx, sk, pads, count, has_seed ? seed : os_entropy_seed());  // lib.rs:238-241
    for (size_t i = 0; i < count; ++i) outs[i] = made[i];
  });
}

int th_encrypt_pk(th_ctx* ctx, const th_pk* pk, const double* z, size_t n, uint64_t seed, int has_seed, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out && pk && pk->ctx == ctx, "bad argument");
    need(z != nullptr || n == 0, "null input");
    std::vector<double> pad(ctx->N / 2);
    pad_input(ctx, z, n, pad.data());
    if (!has_seed) {  // OS entropy: draw the seed on the host like TenSafeRng::from_entropy
      uint64_t s = 0;
      FILE* f = fopen("/dev/urandom", "rb");
      bool ok = f && fread(&s, 1, 8, f) == 8;
      if (f) fclose(f);
      if (!ok) s = (uint64_t)(uintptr_t)&s ^ 0xdeadbeefcafebabeULL;
      seed = s;
    }
    encrypt_pk_seeded(ctx, pk, pad.data(), 1, &seed, out);
  });
}

int th_encrypt_pk_explicit(th_ctx* ctx, const th_pk* pk, const double* z, size_t n, const uint8_t* u,
                           const int64_t* e0, const int64_t* e1, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out && pk && pk->ctx == ctx && u && e0 && e1, "bad argument");
    need(z != nullptr || n == 0, "null input");
    const uint32_t N = ctx->N;
    for (uint32_t i = 0; i < N; ++i) need(u[i] <= 2, "u values must be in {0, 1, 2}");
    std::vector<double> pad(N / 2);
    pad_input(ctx, z, n, pad.data());
    encrypt_pk_explicit_many(ctx, pk, pad.data(), 1, u, e0, e1, out);
  });
}

int th_encrypt_pk_batch(th_ctx* ctx, const th_pk* pk, const double* z, size_t n, size_t stride, size_t count,
                        const uint64_t* seeds, th_ct** outs) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(outs && pk && pk->ctx == ctx && seeds, "bad argument");
    need(z != nullptr || count == 0, "null input");
    if (!count) return;
    const size_t S = ctx->N / 2;
    std::vector<double> pad(count * S);
    for (size_t i = 0; i < count; ++i) pad_input(ctx, z + i * stride, n, pad.data() + i * S);
    encrypt_pk_seeded(ctx, pk, pad.data(), count, seeds, outs);
  });
}

int th_ctx_set_option(th_ctx* ctx, int option, int64_t value) {
  return guarded([&] {
    TH_LOCK(ctx);
    switch (option) {
      case TH_OPT_SAMPLER:
        need(value == TH_SAMPLER_DEVICE || value == TH_SAMPLER_HOST, "unknown sampler");
        ctx->host_sampler = value == TH_SAMPLER_HOST;
        break;
      case TH_OPT_FORCE_SERIAL_SAMPLER:
        ctx->force_serial = value != 0;
        break;
      case TH_OPT_SAMPLER_BAND:
        need(value >= -40 && value <= -1, "sampler band must be 2^v for v in [-40, -1]");
        ctx->band = std::ldexp(1.0, (int)value);
        break;
      case TH_OPT_RESCALE_DECRYPT:
        need(value == TH_RD_AUTO || value == TH_RD_SPLIT || value == TH_RD_WHOLE, "unknown rescale-decrypt kernels");
        ctx->rd_kernels = (int)value;
        break;
      default:
        raise(TH_EINVAL, "unknown option " + std::to_string(option));
    }
  });
}

int th_encode_to_ntt(th_ctx* ctx, const double* z, size_t n, th_pt** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out && (z || n == 0), "bad argument");
    need(n <= ctx->N / 2, "Input length exceeds slot count");  // encoding.rs:174-179
    *out = encode_pt(ctx, z, n);
  });
}

int th_pt_free(th_pt* pt) {
  return guarded([&] {
    if (pt) drop(pt);
  });
}

int th_pt_download(th_ctx* ctx, const th_pt* pt, uint64_t* out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(pt && pt->ctx == ctx && out, "bad argument");
    download(ctx, out, pt->d, pt->limbs * poly_bytes(ctx));
  });
}

int th_ct_pt_mul(th_ctx* ctx, const th_ct* ct, const double* pt, size_t n, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out && (pt || n == 0), "bad argument");
    check_ct(ctx, ct);
    th_pt* p = encode_pt(ctx, pt, n);  // lib.rs:184-187 pads/truncates to N/2
    try {
      const th_ct* cs[1] = {ct};
      const th_pt* ps[1] = {p};
      ct_pt_many(ctx, cs, ps, 1, out);
    } catch (...) {
      drop(p);
      throw;
    }
    drop(p);
  });
}

int th_ct_pt_mul_ntt(th_ctx* ctx, const th_ct* ct, const th_pt* pt, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr, "null output");
    const th_ct* cs[1] = {ct};
    const th_pt* ps[1] = {pt};
    ct_pt_many(ctx, cs, ps, 1, out);
  });
}

int th_ct_pt_mul_ntt_batch(th_ctx* ctx, const th_ct* const* cts, const th_pt* const* pts, size_t count,
                           th_ct** outs) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(outs && ((cts && pts) || count == 0), "bad argument");
    if (count) ct_pt_many(ctx, cts, pts, count, outs);
  });
}

int th_ct_add(th_ctx* ctx, const th_ct* a, const th_ct* b, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr, "null output");
    add_sub(ctx, a, b, false, out);
  });
}

int th_ct_sub(th_ctx* ctx, const th_ct* a, const th_ct* b, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr, "null output");
    add_sub(ctx, a, b, true, out);
  });
}

int th_rescale(th_ctx* ctx, const th_ct* ct, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr, "null output");
    check_ct(ctx, ct);
    const th_ct* cs[1] = {ct};
    rescale_many(ctx, cs, 1, out);
  });
}

int th_rescale_batch(th_ctx* ctx, const th_ct* const* cts, size_t count, th_ct** outs) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(outs && (cts || count == 0), "bad argument");
    if (count) rescale_many(ctx, cts, count, outs);
  });
}

int th_decrypt(th_ctx* ctx, const th_ct* ct, const th_sk* sk, double* out) {
  return th_batch_decrypt(ctx, &ct, 1, sk, out);
}

int th_batch_decrypt(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk, double* out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out || count == 0, "null output");
    check_decrypt_args(ctx, cts, count, sk);
    if (!count) return;
    const size_t S = ctx->N / 2;
    OpScope sc(ctx);
    double* dev = (double*)sc.dev(count * S * 8);
    queue_decrypt(sc, views_of(cts, count), sk, dev, nullptr, 0, 0);
    download(ctx, out, dev, count * S * 8);
  });
}

int th_batch_decrypt_segsum(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk, uint32_t d,
                            uint32_t cols, double* out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out || count == 0, "null output");
    need(d >= 1 && cols >= 1 && (uint64_t)d * cols <= ctx->N / 2, "segments must fit in N/2 slots");
    check_decrypt_args(ctx, cts, count, sk);
    if (!count) return;
    OpScope sc(ctx);
    double* dev = (double*)sc.dev(count * cols * 8);
    queue_decrypt(sc, views_of(cts, count), sk, nullptr, dev, d, cols);
    download(ctx, out, dev, count * cols * 8);
  });
}

// th_batch_decrypt_segsum without any allocation: every device buffer beyond
// the ciphertexts, the key and the context's tables lives in this device's
// scratch (job lists, segment weights, decrypted coefficients, partial and
// final sums), and host staging uses the context's pinned ring. The decrypt
// multiplies c1 by the key as stored (NTT_LOAD_DOT, no Montgomery copy of the
// key); the residues, and so the sums, equal th_batch_decrypt_segsum's.
int th_batch_decrypt_segsum_noalloc(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk, uint32_t d,
                                    uint32_t cols, double* out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out || count == 0, "null output");
    const uint32_t N = ctx->N;
    need(d >= 1 && cols >= 1 && (uint64_t)d * cols <= N / 2, "segments must fit in N/2 slots");
    check_decrypt_args(ctx, cts, count, sk);
    if (!count) return;
    const size_t P = poly_bytes(ctx);
    // decrypt branch per ciphertext (ciphertext.rs:351)
    size_t ntt_jobs = 0;
    bool all_limb0 = true;
    for (size_t i = 0; i < count; ++i) {
      const bool crt = cts[i]->scale > kScale * 1.5 && cts[i]->limbs >= 2;
      ntt_jobs += crt ? 2 : 1;
      all_limb0 &= !crt;
    }
    // the three paths of queue_decrypt: segment sums in the decrypt transform's
    // epilogue, segment-sum kernels on the decrypted coefficients, or the full
    // decode summed per segment
    const bool fused = all_limb0 && segsum_in_transform(ctx, (uint32_t)count, cols);
    const bool standalone = !fused && cols <= SEGSUM_MAX_COLS;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    size_t off = 0;
    const size_t o_ntt = off;
    off += al(ntt_jobs * sizeof(NttJob));
    const size_t o_dec = off;
    if (!fused) off += al(count * sizeof(DecodeJob));
    const size_t w_doubles = fused ? (size_t)2 * N : (standalone ? (size_t)cols * N : 0);
    const size_t o_w = off;
    off += al(w_doubles * 8);
    const size_t o_dot = off;
    if (!fused) off += al(count * 2 * P);
    const size_t parts_per = fused ? 0 : (standalone ? segsum_parts_doubles(cols) : decode_parts_doubles(ctx->logn));
    const size_t o_parts = off;
    off += al(count * parts_per * 8);
    const size_t o_sum = off;
    off += al(count * cols * 8);
    need(off <= TH_NOALLOC_SCRATCH_BYTES,
         "th_batch_decrypt_segsum_noalloc: " + std::to_string(count) + " ciphertexts need " + std::to_string(off) +
             " bytes of scratch, more than its " + std::to_string(TH_NOALLOC_SCRATCH_BYTES) + " bytes");
    std::lock_guard<std::mutex> dl(g_scratch[ctx->device].mu);
    unsigned char* base = ctx->scratch;  // the device address of this GPU's scratch
    hipStream_t st = ctx->stream;
    NttJob* d_ntt = reinterpret_cast<NttJob*>(base + o_ntt);
    DecodeJob* d_dec = reinterpret_cast<DecodeJob*>(base + o_dec);
    double* d_sum = reinterpret_cast<double*>(base + o_sum);
    // job lists built in the pinned ring and copied into the scratch, one
    // region at a time (a reservation may wrap the ring once earlier copies
    // are queued)
    auto dot_of = [&](size_t i) { return reinterpret_cast<uint64_t*>(base + o_dot) + i * 2 * N; };
    auto limbs_of = [&](const th_ct* ct) -> uint32_t { return (ct->scale > kScale * 1.5 && ct->limbs >= 2) ? 2 : 1; };
    NttJob* h_ntt = (NttJob*)ctx->ring.reserve(ntt_jobs * sizeof(NttJob), st);
    size_t k = 0;
    for (size_t i = 0; i < count; ++i) {
      const th_ct* ct = cts[i];
      if (fused) {
        h_ntt[k++] = NttJob{ct->d, reinterpret_cast<uint64_t*>(d_sum + i * cols), ct->d + (size_t)ct->limbs * N,
                            nullptr, 0, 0, ct->scale};
      } else {
        for (uint32_t l = 0; l < limbs_of(ct); ++l)
          h_ntt[k++] = NttJob{ct->d + (size_t)l * N, dot_of(i) + (size_t)l * N, ct->d + (size_t)(ct->limbs + l) * N,
                              nullptr, l, 0, 0.0};
      }
    }
    HIPCHK(hipMemcpyAsync(d_ntt, h_ntt, ntt_jobs * sizeof(NttJob), hipMemcpyHostToDevice, st));
    if (!fused) {
      DecodeJob* h_dec = (DecodeJob*)ctx->ring.reserve(count * sizeof(DecodeJob), st);
      for (size_t i = 0; i < count; ++i)
        h_dec[i] = DecodeJob{dot_of(i), reinterpret_cast<double*>(base + o_parts) + i * parts_per, nullptr,
                             d_sum + i * cols, cts[i]->scale, limbs_of(cts[i]) == 2, 0};
      HIPCHK(hipMemcpyAsync(d_dec, h_dec, count * sizeof(DecodeJob), hipMemcpyHostToDevice, st));
    }
    // segment weights: the context's cached copy when it has one, else made
    // on the host into the ring and copied into the scratch
    const double* W = nullptr;
    if (w_doubles) {
      if (fused) {
        auto it = ctx->seg_p.find(d);
        if (it != ctx->seg_p.end()) W = it->second;
      } else {
        auto it = ctx->seg_w.find(std::make_pair(d, cols));
        if (it != ctx->seg_w.end()) W = it->second;
      }
      if (!W) {
        double* hw = (double*)ctx->ring.reserve(w_doubles * 8, st);
        if (fused)
          segment_weight_pairs(N, d, hw);
        else
          segment_weights(N, d, cols, hw);
        double* dw = reinterpret_cast<double*>(base + o_w);
        HIPCHK(hipMemcpyAsync(dw, hw, w_doubles * 8, hipMemcpyHostToDevice, st));
        W = dw;
      }
    }
    NttArgs a{};
    a.lc = ctx->d_lc;
    a.jobs = d_ntt;
    a.load = NTT_LOAD_DOT;
    a.bc = ctx->d_bc;
    a.key = sk->d;
    if (fused) {
      a.store = NTT_STORE_SEGSUM;
      a.segw = W;
      a.cols = cols;
      HIPCHK(launch_ntt((int)ctx->logn, true, a, (uint32_t)count, st));
    } else {
      HIPCHK(launch_ntt((int)ctx->logn, true, a, (uint32_t)ntt_jobs, st));
      if (standalone)
        HIPCHK(launch_segsum(d_dec, (uint32_t)count, ctx->d_dc, W, ctx->logn, cols, st));
      else
        HIPCHK(launch_decode(d_dec, (uint32_t)count, ctx->d_dc, ctx->d_twist_re, ctx->d_twist_im, ctx->d_stage_re,
                             ctx->d_stage_im, ctx->logn, d, cols, st));
    }
    download(ctx, out, d_sum, count * cols * 8);
  });
}

int th_batch_decrypt_device(th_ctx* ctx, const th_ct* const* cts, size_t count, const th_sk* sk, double* dev_out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(dev_out || count == 0, "null output");
    check_decrypt_args(ctx, cts, count, sk);
    if (!count) return;
    OpScope sc(ctx);
    queue_decrypt(sc, views_of(cts, count), sk, dev_out, nullptr, 0, 0);
    HIPCHK(hipStreamSynchronize(ctx->stream));
  });
}

int th_lora_a_pass(th_ctx* ctx, const th_pk* pk, const th_sk* sk, const double* hidden, uint32_t n_inputs,
                   uint32_t d, const uint64_t* seeds, const th_pt* const* pts, const uint32_t* pt_input,
                   uint32_t n_pts, int do_rescale, double* out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(pk && pk->ctx == ctx && sk && sk->ctx == ctx, "keys belong to another context");
    need(n_inputs > 0 && hidden && seeds && out, "bad argument");
    need(n_pts == 0 || (pts && pt_input), "bad argument");
    const uint32_t N = ctx->N, S = N / 2, L = ctx->L;
    need(d >= 1 && d <= S, "d must be in [1, N/2]");
    need(!do_rescale || L >= 2, "Cannot rescale: only 1 limb left", TH_ESTATE);
    const uint32_t cols = S / d;  // inference_engine.py:1258
    for (uint32_t j = 0; j < n_pts; ++j) {
      need(pt_input[j] < n_inputs, "pt_input index out of range");
      need(pts[j] && pts[j]->ctx == ctx && pts[j]->limbs == L, "plaintext belongs to another context");
    }
    if (!n_pts) return;
    const size_t ctb = 2 * L * poly_bytes(ctx);
    OpScope sc(ctx);
    const double* z = (const double*)sc.upload(hidden, (size_t)n_inputs * d * 8);
    uint64_t* cts = (uint64_t*)sc.dev(n_inputs * ctb);
    std::vector<uint64_t*> ct_ptr(n_inputs);
    for (uint32_t i = 0; i < n_inputs; ++i) ct_ptr[i] = cts + (size_t)i * 2 * L * N;
    double* seg = (double*)sc.dev((size_t)n_pts * cols * 8);
    // the whole pass, randomness from the device sampler or from the host
    auto queue_pass = [&](bool host_draw, BandArgs band) {
      queue_encrypt_pk(sc, pk, z, n_inputs, seeds, d, cols, ct_ptr.data(), host_draw, band);
      // products ct[pt_input[j]] x pts[j] (inference_engine.py:1311)
      std::vector<CtView> in(n_pts), views(n_pts);
      std::vector<const uint64_t*> p(n_pts);
      for (uint32_t j = 0; j < n_pts; ++j) {
        in[j] = CtView{ct_ptr[pt_input[j]], L, kScale};
        p[j] = pts[j]->d;
      }
      if (do_rescale) {
        // the product is formed inside the rescale's inverse transforms
        uint64_t* res = (uint64_t*)sc.dev(n_pts * 2 * (L - 1) * poly_bytes(ctx));
        std::vector<uint64_t*> rdst(n_pts);
        for (uint32_t j = 0; j < n_pts; ++j) rdst[j] = res + (size_t)j * 2 * (L - 1) * N;
        queue_rescale(sc, in, rdst.data(), p.data());
        for (uint32_t j = 0; j < n_pts; ++j)
          views[j] = CtView{rdst[j], L - 1, kScale * kScale / (double)ctx->q[L - 1]};
      } else {
        uint64_t* prods = (uint64_t*)sc.dev(n_pts * ctb);
        std::vector<uint64_t*> dst(n_pts);
        for (uint32_t j = 0; j < n_pts; ++j) {
          dst[j] = prods + (size_t)j * 2 * L * N;
          views[j] = CtView{dst[j], L, kScale * kScale};
        }
        queue_ct_pt(sc, in, p.data(), dst.data());
      }
      queue_decrypt(sc, views, sk, nullptr, seg, d, cols);
    };
    if (ctx->host_sampler) {
      queue_pass(true, BandArgs{nullptr, 0.0});
    } else {
      const uint32_t off = take_flags(ctx, n_inputs);
      queue_pass(false, band_args(ctx, off));
      wait_stream(ctx);
      if (any_flag(ctx, off, n_inputs)) {  // glibc draws
        queue_pass(true, BandArgs{nullptr, 0.0});
        ctx->redrawn_inputs += n_inputs;
      }
      release_flags(ctx, off);
    }
    download(ctx, out, seg, (size_t)n_pts * cols * 8);
  });
}

}  // extern "C"

namespace {

// Device copy of a host vector that lives as long as the set.
template <class T>
const T* persist(th_lora* set, const std::vector<T>& v) {
  th_ctx* c = set->ctx;
  const size_t bytes = v.size() * sizeof(T);
  T* d = (T*)set->alloc(bytes);
  void* h = c->ring.reserve(bytes, c->stream);
  memcpy(h, v.data(), bytes);
  HIPCHK(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, c->stream));
  return d;
}

void launch_jobs_ntt(th_ctx* c, bool inverse, const NttJob* jobs, uint32_t n, NttLoad load,
                     const RescaleConst* rc = nullptr, const uint64_t* key = nullptr,
                     NttStore store = NTT_STORE_NONE) {
  NttArgs a{};
  a.lc = c->d_lc;
  a.jobs = jobs;
  a.load = load;
  a.store = store;
  a.bc = c->d_bc;
  a.rc = rc;
  a.key = key;
  HIPCHK(launch_ntt((int)c->logn, inverse, a, n, c->stream));
}

// Queue the plaintexts and mixed B of a mixture set for its gates (set->d_gates,
// n_proj x k): every batch's plaintext is sum_x encode_to_ntt(g_x * A_x rows)
// (the encoder and transforms of th_encode_to_ntt), in Montgomery form (and
// plain where a token reads it), and B = sum_x g_x B_x. The encoder gates the
// experts' packed rows as it reads them, and its last launch sums the k
// experts' residues of each batch (the k encoded residue polynomials summed
// mod q_l); each batch's forward transform then runs once per limb, in place,
// and writes the Montgomery form in its store (NTT_STORE_MONT). The
// transform is linear mod q_l, so this is the sum of the k transforms,
// residue by residue. Only the limbs a token reads are formed.
void queue_regate(OpScope& sc, th_lora* set) {
  th_ctx* c = sc.c;
  const uint32_t N = c->N, S = N / 2, L = c->L, nb = set->n_batches, k = set->k;
  const size_t nv = (size_t)nb * k, pd = encode_parts_doubles(c->logn);
  double* parts = (double*)sc.dev(nv * pd * 8);
  std::vector<EncodeJob> ej(nv);
  for (size_t v = 0; v < nv; ++v) {
    const MoeBatch& mb = set->moe_b[v / k];
    ej[v].z = set->apack + v * S;
    ej[v].gate = set->d_gates + (size_t)mb.proj * k + v % k;
    ej[v].n_valid = mb.n_valid;
    ej[v].dst = set->ptm + (v / k) * L * N;  // the group's sums, transformed in place below
    ej[v].parts = parts + v * pd;
  }
  // the fold sums at most ENC_FOLD_MAX_LIMBS limbs per launch: longer chains
  // encode once per group of limbs
  const EncodeJob* d_ej = sc.up(ej);
  uint32_t rest = set->moe_limbs;
  while (rest) {
    uint32_t group = 0;
    for (uint32_t l = 0, n = 0; l < 32 && n < ENC_FOLD_MAX_LIMBS; ++l)
      if (rest >> l & 1) {
        group |= 1u << l;
        ++n;
      }
    rest &= ~group;
    HIPCHK(launch_encode(d_ej, (uint32_t)nv, c->d_bc, c->d_twist_re, c->d_twist_im, c->d_stage_re, c->d_stage_im,
                         c->logn, L, c->stream, nullptr, nullptr, nullptr, 0, BandArgs{nullptr, 0.0}, k, group));
  }
  launch_jobs_ntt(c, false, set->d_moe_ntt, set->moe_ntt_jobs, NTT_LOAD_NONE, nullptr, nullptr, NTT_STORE_MONT);
  HIPCHK(launch_moe_mix_b(set->bexp, set->d_moe_p, set->d_gates, set->n_proj, k, set->max_b_count, set->bmix,
                          c->stream));
}

// New gates (host, n_proj x k) into the set's device copy, on the stream.
void upload_gates(th_lora* set, const double* gates) {
  th_ctx* c = set->ctx;
  const size_t bytes = (size_t)set->n_proj * set->k * 8;
  void* h = c->ring.reserve(bytes, c->stream);
  memcpy(h, gates, bytes);
  HIPCHK(hipMemcpyAsync(set->d_gates, h, bytes, hipMemcpyHostToDevice, c->stream));
}

// k experts per projection. Expert x of projection j has A = a[j * k + x],
// B = b[j * k + x] and gate weight gates[j * k + x]; gates == nullptr (k == 1)
// is a plain LoRA set.
// Each packed batch holds, per expert, the gate-scaled A rows; the k encoded
// plaintexts of a batch are folded into one (queue_regate), which makes the
// batch's product the ct_add of the k experts' products, bit for bit. The
// B side applies sum_x g_x B_x to the decrypted intermediate.
void build_lora(th_lora* set, const uint32_t* input_of, const uint32_t* ranks, const uint32_t* d_out,
                uint32_t k, const double* gates, const double* const* a, const double* const* b) {
  th_ctx* c = set->ctx;
  const uint32_t N = c->N, S = N / 2, L = c->L, d = set->d, cols = set->cols;
  const size_t P = poly_bytes(c);
  // plaintext batches (inference_engine.py:1300-1308) and the B jobs
  // Batches hold the A rows as they are (no gates) or ungated per expert
  // (gated sets: the gate is applied on the device, queue_regate). B is stored
  // rank-major on the device (element (i, r) at r * d_out + i), so the B
  // kernel's lanes, one output row each, read consecutive addresses; with
  // experts, each one's B in turn (MoeProj), mixed on the device.
  set->k = k;
  std::vector<double> packed;
  std::vector<uint32_t> batch_input;
  std::vector<MoeBatch> moe_b;
  std::vector<MoeProj> moe_p(set->n_proj);
  std::vector<LoraBJob> bj(set->n_proj);
  std::vector<double> bmat;
  uint64_t out_off = 0, boff = 0;
  for (uint32_t j = 0; j < set->n_proj; ++j) {
    const uint32_t nb = (ranks[j] + cols - 1) / cols;
    bj[j] = LoraBJob{nullptr, d_out[j], ranks[j], (uint32_t)batch_input.size(), input_of[j], out_off};
    for (uint32_t bt = 0; bt < nb; ++bt) {
      const uint32_t rows = std::min(cols, ranks[j] - bt * cols);
      for (uint32_t x = 0; x < k; ++x) {
        const double* ax = a[(size_t)j * k + x];
        packed.resize(packed.size() + S, 0.0);
        double* p = packed.data() + packed.size() - S;
        for (uint32_t i = 0; i < rows; ++i) memcpy(p + (size_t)i * d, ax + (size_t)(bt * cols + i) * d, (size_t)d * 8);
      }
      batch_input.push_back(input_of[j]);
      moe_b.push_back(MoeBatch{j, rows * d});
    }
    const size_t bn = (size_t)d_out[j] * ranks[j];
    moe_p[j] = MoeProj{boff, (uint32_t)bn, 0};
    for (uint32_t x = 0; x < k; ++x) {
      const double* bx = b[(size_t)j * k + x];
      const size_t b0 = bmat.size();
      bmat.resize(b0 + bn);
      for (uint32_t i = 0; i < d_out[j]; ++i)
        for (uint32_t r = 0; r < ranks[j]; ++r) bmat[b0 + (size_t)r * d_out[j] + i] = bx[(size_t)i * ranks[j] + r];
    }
    boff += bn;
    out_off += d_out[j];
    set->max_d_out = std::max(set->max_d_out, d_out[j]);
    set->max_b_count = std::max(set->max_b_count, (uint32_t)bn);
  }
  set->n_batches = (uint32_t)batch_input.size();
  set->n_deltas = out_off;
  const uint32_t nb = set->n_batches, ni = set->n_in;
  const bool gated = gates != nullptr;
  const uint32_t Lr = L > 1 ? L - 1 : 1;
  // decrypt branch (ciphertext.rs:351): CRT over limbs 0, 1 iff scale > 1.5 * 2^40 and >= 2 limbs
  const double scale_n = kScale * kScale, scale_r = scale_n / (double)c->q[L - 1];
  const uint32_t nl_n = (scale_n > 1.5 * kScale && L >= 2) ? 2 : 1;
  const uint32_t nl_r = (scale_r > 1.5 * kScale && Lr >= 2) ? 2 : 1;
  // rescaled products straight into segment sums where the decryption reads
  // limb 0: one workgroup per product (rescale_decrypt_kernel) or the split
  // kernels (launch_rescale_decrypt_split). The first serves one round of
  // workgroups (at most 256 batches, N <= 16384); it takes two transforms'
  // time whatever the batch count, while the split kernels' time grows with
  // it: at N = 16384 a token measured 0.153 against 0.097 ms with 8 batches,
  // 0.180 against 0.176 with 128, 0.216 against 0.220 with 192 and 0.230
  // against 0.241 with 224 (one workgroup per product first).
  const bool rd_ok = L >= 2 && nl_r == 1 && cols >= 1 && cols <= NTT_SEGSUM_FUSED_MAX_COLS;
  const bool split_ok = c->logn >= 13;
  const bool whole_ok = segsum_in_transform(c, nb, cols);
  bool rd_whole = rd_ok && whole_ok;
  if (split_ok && c->rd_kernels == TH_RD_SPLIT) rd_whole = false;
  if (split_ok && c->rd_kernels == TH_RD_AUTO && nb < RD_WHOLE_MIN_BATCHES) rd_whole = false;
  const bool rd_split = rd_ok && !rd_whole && split_ok;
  const bool fused_rd = rd_whole || rd_split;
  set->rd_split = rd_split;
  if (rd_split) set->rd_partials = (double*)set->alloc((size_t)nb * cols * (N / 16) * 8);
  if (!gated) {
    set->bmix = const_cast<double*>(persist(set, bmat));
  } else {
    set->bexp = persist(set, bmat);
    set->bmix = (double*)set->alloc((size_t)boff * 8);
    set->d_moe_p = persist(set, moe_p);
  }
  for (uint32_t j = 0; j < set->n_proj; ++j) bj[j].b = set->bmix + moe_p[j].off;
  // device memory
  set->pts = (uint64_t*)set->alloc(nb * L * P);
  set->ptm = (uint64_t*)set->alloc(nb * L * P);
  set->hidden = (double*)set->alloc((size_t)ni * d * 8);
  set->u = (uint8_t*)set->alloc((size_t)ni * N);
  set->e0 = (int64_t*)set->alloc((size_t)ni * N * 8);
  set->e1 = (int64_t*)set->alloc((size_t)ni * N * 8);
  set->mvals = (int64_t*)set->alloc((size_t)ni * N * 8);
  set->prep = (uint64_t*)set->alloc(ni * 3 * L * P);
  double* enc_parts = (double*)set->alloc(ni * encode_parts_doubles(c->logn) * 8);
  set->cts = (uint64_t*)set->alloc(ni * 2 * L * P);
  set->work = (uint64_t*)set->alloc(nb * 2 * P);
  set->m = (uint64_t*)set->alloc(nb * 2 * P);
  double* dec_parts = (double*)set->alloc(nb * decode_parts_doubles(c->logn) * 8);
  set->sums = (double*)set->alloc((size_t)nb * cols * 8);
  {
    // sampler and combine jobs; seeds and the public key come with each launch
    std::vector<SampleJob> sj(ni);
    std::vector<EncCombineJob> cj(ni);
    uint32_t* reject = const_cast<uint32_t*>(persist(set, std::vector<uint32_t>(ni, 0)));
    for (uint32_t i = 0; i < ni; ++i) {
      sj[i] = SampleJob{0, set->u + (size_t)i * N, set->e0 + (size_t)i * N, set->e1 + (size_t)i * N, reject + i};
      cj[i] = EncCombineJob{set->prep + (size_t)i * 3 * L * N, nullptr, nullptr, set->cts + (size_t)i * 2 * L * N};
    }
    set->d_sample = persist(set, sj);
    set->d_comb = persist(set, cj);
  }
  // encode the plaintext batches (th_encode_to_ntt of each packed vector); with
  // gates, the gated batches, folded (queue_regate)
  if (!gated) {
    OpScope sc(c);
    queue_encode(sc, sc.up(packed), nb, nullptr, nullptr, nullptr, set->pts, (size_t)L * N);
    ntt_strided(c, false, set->pts, set->pts, nb * L, L);
    HIPCHK(launch_to_montgomery(set->pts, set->ptm, c->d_bc, N, L, nb, c->stream));
    HIPCHK(hipStreamSynchronize(c->stream));  // the scope's buffers return to the pool
  } else {
    set->apack = persist(set, packed);
    set->moe_b = moe_b;
    set->d_gates = (double*)set->alloc((size_t)set->n_proj * k * 8);
    // A complete token (ct x pt on every limb) reads every limb of the
    // plaintexts in plain form (the rescale's store, the products) and limb
    // L-1 in Montgomery form (the rescale's inverse loads); a fused token
    // reads limbs 0..nl-1 and L-1 in Montgomery form: the regated plaintexts
    // are formed on every limb, in both forms.
    set->moe_limbs = L >= 32 ? ~0u : (1u << L) - 1;
    std::vector<NttJob> mj;
    for (uint32_t bt = 0; bt < nb; ++bt)
      for (uint32_t l = 0; l < L; ++l) {
        const size_t off = ((size_t)bt * L + l) * N;
        mj.push_back(NttJob{set->ptm + off, set->ptm + off, set->pts + off, nullptr, l, 0});
      }
    set->d_moe_ntt = persist(set, mj);
    set->moe_ntt_jobs = (uint32_t)mj.size();
    upload_gates(set, gates);
    OpScope sc(c);
    queue_regate(sc, set);
    HIPCHK(hipStreamSynchronize(c->stream));
  }
  // per-token job lists
  std::vector<EncodeJob> ej(ni);
  for (uint32_t i = 0; i < ni; ++i) {
    ej[i].z = set->hidden + (size_t)i * d;
    ej[i].rep_d = d;
    ej[i].rep_cols = cols;
    ej[i].u = set->u + (size_t)i * N;
    ej[i].e0 = set->e0 + (size_t)i * N;
    ej[i].e1 = set->e1 + (size_t)i * N;
    ej[i].dst = set->prep + (size_t)i * 3 * L * N;
    ej[i].mvals = set->mvals + (size_t)i * N;
    ej[i].parts = enc_parts + i * encode_parts_doubles(c->logn);
  }
  set->d_enc = persist(set, ej);
  std::vector<NttJob> inv, fwd, dot_r, inv_nr;
  std::vector<RescaleDecryptJob> rd;
  std::vector<DecodeJob> dec_r(nb), dec_n(nb);
  set->nl_n = nl_n;
  set->nl_r = nl_r;
  {
    // the encrypt inputs' forward transforms read m, e0, e1 and u and form
    // each limb's residues as they load them: [M_l = m + e0 | E1_l | U_l] per
    // input, for the limbs in mask
    auto enc_jobs = [&](uint32_t mask) {
      std::vector<NttJob> ej2;
      for (uint32_t i = 0; i < ni; ++i) {
        uint64_t* pr = set->prep + (size_t)i * 3 * L * N;
        const uint64_t* m = reinterpret_cast<const uint64_t*>(set->mvals + (size_t)i * N);
        const uint64_t* e0 = reinterpret_cast<const uint64_t*>(set->e0 + (size_t)i * N);
        const uint64_t* e1 = reinterpret_cast<const uint64_t*>(set->e1 + (size_t)i * N);
        const uint64_t* u = reinterpret_cast<const uint64_t*>(set->u + (size_t)i * N);
        for (uint32_t l = 0; l < L; ++l)
          if (mask >> l & 1) ej2.push_back(NttJob{m, pr + (size_t)l * N, e0, nullptr, l, 0});
        for (uint32_t l = 0; l < L; ++l)
          if (mask >> l & 1) ej2.push_back(NttJob{e1, pr + (size_t)(L + l) * N, nullptr, nullptr, l, 1});
        for (uint32_t l = 0; l < L; ++l)
          if (mask >> l & 1) ej2.push_back(NttJob{u, pr + (size_t)(2 * L + l) * N, nullptr, nullptr, l, 2});
      }
      return ej2;
    };
    // A token reads only some limbs of its input ciphertexts: the decryption
    // reads limb 0 (limbs 0 and 1 in the CRT branch) of what it decrypts, a
    // product's limb l depends on the input's limb l only, and a rescaled
    // limb l on limbs l and L-1. So a token with a rescale needs limbs
    // 0..nl_r-1 and L-1 of each input, one without a rescale limbs 0..nl_n-1;
    // the encryptions form only those limbs where the transform size allows
    // it (the other limbs would be the same residues as th_encrypt_pk's).
    const uint32_t full = L >= 32 ? ~0u : (1u << L) - 1;
    const NttJob* all = persist(set, enc_jobs(full));
    set->d_enc_all = all;
    auto plan = [&](uint32_t mask) {
      if (mask != full && encrypt_limbs_supported((int)c->logn))
        return std::make_pair(persist(set, enc_jobs(mask)), mask);
      return std::make_pair(all, full);
    };
    std::tie(set->d_enc_r, set->enc_mask_r) = plan(((1u << nl_r) - 1) | (L >= 2 ? 1u << (L - 1) : 0u));
    std::tie(set->d_enc_n, set->enc_mask_n) = plan((1u << nl_n) - 1);
  }
  if (!fused_rd) set->res = (uint64_t*)set->alloc(nb * 2 * nl_r * P);
  set->dkey = (uint64_t*)set->alloc((size_t)set->n_in * nl_n * P);
  for (uint32_t bt = 0; bt < nb; ++bt) {
    const uint64_t* ct = set->cts + (size_t)batch_input[bt] * 2 * L * N;
    const uint64_t* pt = set->pts + (size_t)bt * L * N;
    const uint64_t* ptm = set->ptm + (size_t)bt * L * N;
    uint64_t* w = set->work + (size_t)bt * 2 * N;
    uint64_t* r = fused_rd ? nullptr : set->res + (size_t)bt * 2 * nl_r * N;
    uint64_t* mm = set->m + (size_t)bt * 2 * N;
    if (L >= 2) {
      // evaluation-domain rescale of ct x pt (see queue_rescale): inverse NTT of the product's
      // last limb (into the batch's work area), forward NTTs of it reduced to the limbs the
      // decryption reads. Limb l of the rescaled ciphertext depends on limbs l and L-1 of the
      // product only, and the decryption reads limb 0 (limbs 0 and 1 in the CRT branch,
      // ciphertext.rs:351-353, encoding.rs:221-226), so the other limbs are not formed; their
      // residues would be those of th_rescale.
      for (uint32_t comp = 0; comp < 2; ++comp) {
        const uint64_t* cc = ct + (size_t)comp * L * N;
        uint64_t* lc = w + (size_t)comp * N;
        inv.push_back(NttJob{cc + (size_t)(L - 1) * N, lc, ptm + (size_t)(L - 1) * N, nullptr, L - 1, 0});
        if (!fused_rd)
          for (uint32_t l = 0; l < nl_r; ++l)
            fwd.push_back(
                NttJob{lc, r + (size_t)(comp * nl_r + l) * N, cc + (size_t)l * N, pt + (size_t)l * N, l, 0});
      }
      if (fused_rd)
        rd.push_back(RescaleDecryptJob{w + N, w, set->dkey + (size_t)batch_input[bt] * N, ptm,
                                       set->sums + (size_t)bt * cols, scale_r});
      else
        for (uint32_t l = 0; l < nl_r; ++l)
          dot_r.push_back(NttJob{r + (size_t)l * N, mm + (size_t)l * N, r + (size_t)(nl_r + l) * N, nullptr, l, 0});
    }
    for (uint32_t l = 0; l < nl_n; ++l) {
      inv_nr.push_back(NttJob{set->dkey + ((size_t)batch_input[bt] * nl_n + l) * N, mm + (size_t)l * N,
                              ptm + (size_t)l * N, nullptr, l, 0});
    }
    dec_r[bt] = DecodeJob{mm, dec_parts + bt * decode_parts_doubles(c->logn), nullptr, set->sums + (size_t)bt * cols,
                          scale_r, nl_r == 2, 0};
    dec_n[bt] = DecodeJob{mm, dec_parts + bt * decode_parts_doubles(c->logn), nullptr, set->sums + (size_t)bt * cols,
                          scale_n, nl_n == 2, 0};
  }
  if (L >= 2) {
    set->d_inv_mul = persist(set, inv);
    set->d_dec_r = persist(set, dec_r);
  }
  if (fused_rd) {
    set->d_rd = persist(set, rd);
  } else if (L >= 2) {
    set->d_fwd_rs = persist(set, fwd);
    set->d_dot_r = persist(set, dot_r);
    if (nl_r == 1 && segsum_in_transform(c, nb, cols)) {
      std::vector<NttJob> ds(nb);
      for (uint32_t bt = 0; bt < nb; ++bt) {
        const uint64_t* r = set->res + (size_t)bt * 2 * N;
        ds[bt] = NttJob{r, reinterpret_cast<uint64_t*>(set->sums + (size_t)bt * cols), r + N, nullptr, 0, 0, scale_r};
      }
      set->d_dot_seg = persist(set, ds);
    }
  }
  set->d_inv_nr = persist(set, inv_nr);
  set->inv_nr_jobs = (uint32_t)inv_nr.size();
  set->dot_r_jobs = (uint32_t)dot_r.size();
  set->d_dec_n = persist(set, dec_n);
  {
    // The complete pass: the encryptions form every limb of c0 and c1
    // (d_enc_all); each batch's rescale forms every limb of the rescaled
    // product in outs, after the inverse transforms of its last limb
    // (d_inv_mul, the product in their loads): forward jobs of the last limb
    // reduced modulo limbs 0..L-2, the product ct_l pt_l, the subtraction and
    // the scaling in their stores (queue_rescale's algebra; inverse job i
    // owns forward jobs i (L-1) .. i (L-1) + L-2); without a rescale each
    // batch's product ct x pt is formed on every limb. The decryption reads
    // limb 0 of each (limbs 0 and 1 in the CRT branch): one transform with c0
    // + c1 s in its load and the segment sums in its epilogue where the
    // whole-polynomial kernel serves (N <= 16384, at most 8 segments; in
    // launches of one round of workgroups), else transforms into m and the
    // segment-sum (or decode) kernels.
    set->outs = (uint64_t*)set->alloc(nb * 2 * L * P);
    std::vector<NttJob> fa, seg, dr, dn;
    std::vector<CtPtJob> cp(nb);
    for (uint32_t bt = 0; bt < nb; ++bt) {
      const uint64_t* ct = set->cts + (size_t)batch_input[bt] * 2 * L * N;
      const uint64_t* pt = set->pts + (size_t)bt * L * N;
      uint64_t* o = set->outs + (size_t)bt * 2 * L * N;
      uint64_t* mm = set->m + (size_t)bt * 2 * N;
      if (L >= 2) {
        const uint64_t* w = set->work + (size_t)bt * 2 * N;
        for (uint32_t comp = 0; comp < 2; ++comp)
          for (uint32_t l = 0; l + 1 < L; ++l)
            fa.push_back(NttJob{w + (size_t)comp * N, o + (size_t)(comp * (L - 1) + l) * N,
                                ct + (size_t)(comp * L + l) * N, pt + (size_t)l * N, l, 0});
        for (uint32_t l = 0; l < nl_r; ++l)
          dr.push_back(NttJob{o + (size_t)l * N, mm + (size_t)l * N, o + (size_t)(L - 1 + l) * N, nullptr, l, 0});
        seg.push_back(NttJob{o, reinterpret_cast<uint64_t*>(set->sums + (size_t)bt * cols), o + (size_t)(L - 1) * N,
                             nullptr, 0, 0, scale_r});
      }
      cp[bt] = CtPtJob{ct, ct + (size_t)L * N, pt, o, L, 0};
      for (uint32_t l = 0; l < nl_n; ++l)
        dn.push_back(NttJob{o + (size_t)l * N, mm + (size_t)l * N, o + (size_t)(L + l) * N, nullptr, l, 0});
    }
    if (L >= 2) {
      set->d_fwd_all = persist(set, fa);
      set->d_dot_all_r = persist(set, dr);
      set->dot_all_r_jobs = (uint32_t)dr.size();
      if (nl_r == 1 && segsum_in_transform(c, std::min<uint32_t>(nb, 256), cols)) set->d_seg_all = persist(set, seg);
    }
    set->d_ctpt = persist(set, cp);
    set->d_dot_all_n = persist(set, dn);
    set->dot_all_n_jobs = (uint32_t)dn.size();
  }
  set->d_bjobs = persist(set, bj);
  if (cols <= SEGSUM_MAX_COLS) set->seg_w = seg_weights(c, d, cols);
  if (set->d_dot_seg || set->d_rd || set->d_seg_all) set->seg_p = seg_pairs(c, d);
  // Host-I/O tokens stage through one pinned buffer of the set, written once
  // here: a token staged through fresh pinned pages (the context's ring on
  // its first pass) measured about twice the time of one staged through
  // pages used before.
  set->io_in_off = ((size_t)(set->n_deltas + (uint64_t)nb * cols) * 8 + 255) & ~(size_t)255;
  set->io_bytes = set->io_in_off + (size_t)ni * d * 8;
  HIPCHK(hipHostMalloc(&set->io_host, set->io_bytes, hipHostMallocMapped));
  memset(set->io_host, 0, set->io_bytes);
  HIPCHK(hipHostGetDevicePointer(reinterpret_cast<void**>(&set->io_dev), set->io_host, 0));
  HIPCHK(hipStreamSynchronize(c->stream));
}

void free_lora(th_lora* set) {
  th_ctx* c = set->ctx;
  if (set->io_host) (void)hipHostFree(set->io_host);
  for (void* p : set->owned) c->pool.put(p);
  delete set;
  ctx_release(c);
}

// Host hidden states up to this size are read by the encoder from the set's
// mapped staging pages instead of being copied to the device first: a single
// delta's 12 KiB. The encoder reads all N FFT inputs, each hidden value about
// N / d times (replicas and the mirrored half: 11 at d = 1536), which for the
// 1.5B shape's 344 KiB would be several MB across PCIe.
constexpr size_t HOST_INPUT_MAPPED_MAX = 32 * 1024;

// The rest of a TH_LORA_SK_FUSED token after the encoder: only the limbs the
// decryptions read, with the secret key inside the encryption (D = c0 + c1 s
// on the decrypted limbs instead of c0 and c1) and the rescale fused into the
// decryption; no complete ciphertext is formed.
void queue_fused_rest(th_ctx* ctx, th_lora* set, const th_pk* pk, const th_sk* sk, bool do_rescale) {
  const uint32_t N = ctx->N, L = ctx->L, ni = set->n_in, nb = set->n_batches;
  hipStream_t st = ctx->stream;
  // D = c0 + c1 s, all the decryption reads of an input's limbs 0..nl-1
  // (k_key_dot, or formed by the encrypt row passes in place of those limbs
  // where they run): limb 0 before the fused rescale-decrypt, limbs
  // 0..nl_n-1 without a rescale
  const bool fused_rd = do_rescale && set->d_rd;
  const uint32_t nl_d = fused_rd ? 1 : (do_rescale ? 0 : set->nl_n);
  const uint64_t* skm = nl_d ? sk_montgomery(ctx, sk) : nullptr;
  bool d_formed = false;
  {
    NttArgs ea{};
    ea.lc = ctx->d_lc;
    ea.jobs = do_rescale ? set->d_enc_r : set->d_enc_n;
    ea.load = NTT_LOAD_ENC;
    ea.bc = ctx->d_bc;
    EncDot dot{};
    if (nl_d && encrypt_limbs_supported((int)ctx->logn)) dot = EncDot{(1u << nl_d) - 1, skm, set->dkey};
    bool combined = false;
    HIPCHK(launch_encrypt((int)ctx->logn, ea, ni, L, do_rescale ? set->enc_mask_r : set->enc_mask_n, dot,
                          pk_pairs(ctx, pk), set->cts, &combined, st));
    if (!combined) HIPCHK(launch_encrypt_combine(set->d_comb, ni, ctx->d_bc, N, L, st, pk->d));
    d_formed = combined && dot.mask;
  }
  if (nl_d && !d_formed)
    HIPCHK(launch_key_dot(set->cts, (uint64_t)2 * L * N, skm, set->dkey, ctx->d_bc, N, L, nl_d, ni, st));
  if (do_rescale && set->d_rd) {
    // the last limb of (c0 pt, c1 pt) as coefficients (ct x pt in the inverse
    // transforms' loads), D = c0 + c1 s on limb 0 per input, then each batch's
    // rescale and decryption on limb 0 in one kernel, which writes the sums
    RescaleDecryptArgs ra{};
    ra.lc = ctx->d_lc;
    ra.bc = ctx->d_bc;
    ra.rc = ctx->d_rc + (size_t)L * L;
    ra.skm = skm;
    ra.segw = set->seg_p;
    ra.jobs = set->d_rd;
    ra.cols = set->cols;
    if (set->rd_split) {
      NttArgs ia{};
      ia.lc = ctx->d_lc;
      ia.bc = ctx->d_bc;
      ia.jobs = set->d_inv_mul;
      ia.load = NTT_LOAD_MULM;
      HIPCHK(launch_rescale_decrypt_split((int)ctx->logn, ia, ra, nb, set->rd_partials, st));
    } else {
      launch_jobs_ntt(ctx, true, set->d_inv_mul, nb * 2, NTT_LOAD_MULM);
      HIPCHK(launch_rescale_decrypt((int)ctx->logn, ra, nb, st));
    }
  } else if (do_rescale) {
    // ct x pt inside the rescale's inverse transforms, rescale combine inside the forward ones
    NttArgs ia{}, fa{};
    ia.lc = fa.lc = ctx->d_lc;
    ia.bc = fa.bc = ctx->d_bc;
    ia.jobs = set->d_inv_mul;
    ia.load = NTT_LOAD_MULM;
    fa.jobs = set->d_fwd_rs;
    fa.load = NTT_LOAD_REDUCE;
    fa.store = NTT_STORE_MUL_RESCALE;
    fa.rc = ctx->d_rc + (size_t)L * L;
    HIPCHK(launch_rescale((int)ctx->logn, ia, nb * 2, fa, nb * 2 * set->nl_r, st));
    if (!set->d_dot_seg) launch_jobs_ntt(ctx, true, set->d_dot_r, set->dot_r_jobs, NTT_LOAD_DOT, nullptr, sk->d);
  } else {
    // the product ciphertexts (c0 pt, c1 pt) decrypt to pt (c0 + c1 s): with
    // D (above), each batch's inverse transforms with pt * D in their loads
    launch_jobs_ntt(ctx, true, set->d_inv_nr, set->inv_nr_jobs, NTT_LOAD_MULM);
  }
  const DecodeJob* dec = do_rescale ? set->d_dec_r : set->d_dec_n;
  if (do_rescale && set->d_rd) {
    // the sums are written
  } else if (do_rescale && set->d_dot_seg)
    launch_dot_segsum(ctx, set->d_dot_seg, nb, sk, set->seg_p, set->cols);
  else if (set->seg_w)
    HIPCHK(launch_segsum(dec, nb, ctx->d_dc, set->seg_w, ctx->logn, set->cols, st));
  else
    HIPCHK(launch_decode(dec, nb, ctx->d_dc, ctx->d_twist_re, ctx->d_twist_im, ctx->d_stage_re,
                         ctx->d_stage_im, ctx->logn, set->d, set->cols, st));
}

// The rest of a complete token after the encoder: the reference's
// client/server sequence (inference_engine.py:1477-1482). encrypt_pk forms
// every limb of c0 and c1 of each input from the public key (ciphertext.rs:
// 240-319), ct x pt and the rescale every limb of each batch's product
// (ciphertext.rs:422-429, :476-535) without the secret key, into the set's
// working memory; then the batched decrypt (ciphertext.rs:327-400) reads the
// limbs it decodes with the secret key.
void queue_complete_rest(th_ctx* ctx, th_lora* set, const th_pk* pk, const th_sk* sk, bool do_rescale) {
  const uint32_t N = ctx->N, L = ctx->L, ni = set->n_in, nb = set->n_batches;
  hipStream_t st = ctx->stream;
  {
    NttArgs ea{};
    ea.lc = ctx->d_lc;
    ea.jobs = set->d_enc_all;
    ea.load = NTT_LOAD_ENC;
    ea.bc = ctx->d_bc;
    const uint32_t full = L >= 32 ? ~0u : (1u << L) - 1;
    bool combined = false;
    HIPCHK(launch_encrypt((int)ctx->logn, ea, ni, L, full, EncDot{}, pk_pairs(ctx, pk), set->cts, &combined, st));
    if (!combined) HIPCHK(launch_encrypt_combine(set->d_comb, ni, ctx->d_bc, N, L, st, pk->d));
  }
  const DecodeJob* dec = nullptr;
  if (do_rescale) {
    // inverse transforms of the products' last limb (ct x pt in their loads),
    // forward transforms of its reductions with the product, the subtraction
    // and the scaling in their stores: every limb of each rescaled product
    NttArgs ia{}, fa{};
    ia.lc = fa.lc = ctx->d_lc;
    ia.bc = fa.bc = ctx->d_bc;
    ia.jobs = set->d_inv_mul;
    ia.load = NTT_LOAD_MULM;
    fa.jobs = set->d_fwd_all;
    fa.load = NTT_LOAD_REDUCE;
    fa.store = NTT_STORE_MUL_RESCALE;
    fa.rc = ctx->d_rc + (size_t)L * L;
    HIPCHK(launch_rescale((int)ctx->logn, ia, nb * 2, fa, nb * 2 * (L - 1), st));
    if (set->d_seg_all) {
      launch_dot_segsum(ctx, set->d_seg_all, nb, sk, set->seg_p, set->cols);
    } else {
      launch_jobs_ntt(ctx, true, set->d_dot_all_r, set->dot_all_r_jobs, NTT_LOAD_DOTM, nullptr,
                      sk_montgomery(ctx, sk));
      dec = set->d_dec_r;
    }
  } else {
    HIPCHK(launch_ct_pt_mul(set->d_ctpt, nb, L, ctx->d_bc, N, st));
    launch_jobs_ntt(ctx, true, set->d_dot_all_n, set->dot_all_n_jobs, NTT_LOAD_DOTM, nullptr, sk_montgomery(ctx, sk));
    dec = set->d_dec_n;
  }
  if (dec) {
    if (set->seg_w)
      HIPCHK(launch_segsum(dec, nb, ctx->d_dc, set->seg_w, ctx->logn, set->cols, st));
    else
      HIPCHK(launch_decode(dec, nb, ctx->d_dc, ctx->d_twist_re, ctx->d_twist_im, ctx->d_stage_re,
                           ctx->d_stage_im, ctx->logn, set->d, set->cols, st));
  }
}

// Queue one token of the set (the body of th_lora_deltas): encrypt_pk of every
// input z (device, n_in x d) with randomness from the device sampler (band
// flags `band`) or, with host_draw, drawn on the host with glibc; ct x pt
// (inside the rescale's transforms with TH_LORA_RESCALE); decrypt with
// segment sums; B applied into dout (device, n_deltas). mode: TH_LORA_* bits.
void queue_token(th_ctx* ctx, th_lora* set, const th_pk* pk, const th_sk* sk, const double* z,
                 const uint64_t* seeds, int mode, double* dout, bool host_draw, BandArgs band) {
  const uint32_t N = ctx->N, L = ctx->L, ni = set->n_in;
  const bool do_rescale = (mode & TH_LORA_RESCALE) != 0;
  hipStream_t st = ctx->stream;
  // encrypt_pk of every input (ciphertext.rs:240-319); seeds travel with the
  // launch. When every input's seed fits one launch, the encoder's launch
  // draws the randomness too (the sampler's workgroups beside the encoder's)
  const bool sample_in_encode = !host_draw && ni <= SEEDS_PER_LAUNCH;
  if (host_draw) {
    OpScope sc(ctx);
    upload_host_draws(sc, seeds, ni, set->u, set->e0, set->e1);
  } else if (!sample_in_encode) {
    HIPCHK(launch_sample_pk(set->d_sample, ni, N, ctx->force_serial, st, seeds, true, false, band));
  }
  HIPCHK(launch_encode(set->d_enc, ni, ctx->d_bc, ctx->d_twist_re, ctx->d_twist_im, ctx->d_stage_re,
                       ctx->d_stage_im, ctx->logn, L, st, z, sample_in_encode ? set->d_sample : nullptr, seeds,
                       ctx->force_serial, band));
  if (mode & TH_LORA_SK_FUSED)
    queue_fused_rest(ctx, set, pk, sk, do_rescale);
  else
    queue_complete_rest(ctx, set, pk, sk, do_rescale);
  HIPCHK(launch_lora_b(set->d_bjobs, set->n_proj, set->max_d_out, set->sums, dout, set->cols, st, band.dflags,
                       band.gen));
  set->last_mode = mode;
}

void resolve_pending(th_ctx* c) {
  size_t first = c->pending.size();
  for (size_t i = 0; i < c->pending.size(); ++i)
    if (any_flag(c, c->pending[i].flag_off, c->pending[i].set->n_in)) {
      first = i;
      break;
    }
  std::vector<AsyncToken> redo(c->pending.begin() + (std::ptrdiff_t)first, c->pending.end());
  std::vector<char> flagged(redo.size());
  for (size_t i = 0; i < redo.size(); ++i) flagged[i] = any_flag(c, redo[i].flag_off, redo[i].set->n_in);
  c->pending.clear();
  c->bflag_used = 0;
  if (redo.empty()) return;
  // flagged tokens from glibc draws; the others again from the device
  // sampler, which reproduces their (unflagged) draws exactly
  for (size_t i = 0; i < redo.size(); ++i) {
    const AsyncToken& t = redo[i];
    queue_token(c, t.set, t.pk, t.sk, t.hidden, t.seeds.data(), t.mode, t.deltas, flagged[i] != 0,
                BandArgs{nullptr, 0.0});
    if (flagged[i]) c->redrawn_inputs += t.set->n_in;
  }
  wait_stream(c);
}

}  // namespace

extern "C" {

int th_lora_create_moe(th_ctx* ctx, uint32_t n_inputs, uint32_t d, uint32_t n_proj, const uint32_t* input_of,
                       const uint32_t* ranks, const uint32_t* d_out, uint32_t n_experts, const double* gates,
                       const double* const* a, const double* const* b, th_lora** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr, "null output");
    need(n_inputs >= 1 && n_proj >= 1, "need at least one input and one projection");
    need(n_experts >= 1 && n_experts <= 64, "n_experts must be in [1, 64]");
    need(n_experts == 1 || gates != nullptr, "null gates");  // th_lora_create passes none
    need(d >= 1 && d <= ctx->N / 2, "d must be in [1, N/2]");
    need(input_of && ranks && d_out && a && b, "null argument");
    for (uint32_t j = 0; j < n_proj; ++j) {
      need(input_of[j] < n_inputs, "input_of index out of range");
      need(ranks[j] >= 1 && d_out[j] >= 1, "ranks and d_out must be positive");
      for (uint32_t x = 0; x < n_experts; ++x) {
        need(a[(size_t)j * n_experts + x] && b[(size_t)j * n_experts + x], "null LoRA matrix");
        if (gates) need(std::isfinite(gates[(size_t)j * n_experts + x]), "gate weights must be finite");
      }
    }
    th_lora* set = new th_lora{};
    set->ctx = ctx;
    ctx_retain(ctx);
    set->n_in = n_inputs;
    set->d = d;
    set->n_proj = n_proj;
    set->cols = (ctx->N / 2) / d;  // inference_engine.py:1258
    try {
      build_lora(set, input_of, ranks, d_out, n_experts, gates, a, b);
    } catch (...) {
      (void)hipStreamSynchronize(ctx->stream);
      free_lora(set);
      throw;
    }
    *out = set;
  });
}

int th_lora_create(th_ctx* ctx, uint32_t n_inputs, uint32_t d, uint32_t n_proj, const uint32_t* input_of,
                   const uint32_t* ranks, const uint32_t* d_out, const double* const* a, const double* const* b,
                   th_lora** out) {
  return th_lora_create_moe(ctx, n_inputs, d, n_proj, input_of, ranks, d_out, 1, nullptr, a, b, out);
}

int th_lora_set_gates(th_ctx* ctx, th_lora* set, const double* gates) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(set && set->ctx == ctx, "LoRA set belongs to another context");
    need(set->apack != nullptr, "the LoRA set was created without gates", TH_ESTATE);
    need(gates != nullptr, "null gates");
    const size_t ng = (size_t)set->n_proj * set->k;
    for (size_t i = 0; i < ng; ++i) need(std::isfinite(gates[i]), "gate weights must be finite");
    // a queued token redone later (sampler band) must see the plaintexts it was queued with
    if (!ctx->pending.empty()) drain(ctx);
    upload_gates(set, gates);
    OpScope sc(ctx);
    queue_regate(sc, set);
  });
}

int th_lora_free(th_lora* set) {
  return guarded([&] {
    if (!set) return;
    {
      std::lock_guard<std::mutex> lk(set->ctx->mu);
      use_device(set->ctx);
      drain(set->ctx);  // queued tokens of this set are settled (and finished) first
    }
    free_lora(set);  // may release the context's last reference: outside its lock
  });
}

int th_lora_info(const th_lora* set, uint64_t* n_deltas, uint32_t* n_batches, uint32_t* cols) {
  return guarded([&] {
    need(set != nullptr, "null LoRA set");
    if (n_deltas) *n_deltas = set->n_deltas;
    if (n_batches) *n_batches = set->n_batches;
    if (cols) *cols = set->cols;
  });
}

int th_lora_ct(th_ctx* ctx, th_lora* set, int which, uint32_t index, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(set && set->ctx == ctx, "LoRA set belongs to another context");
    need(out != nullptr, "null output");
    need(which == TH_LORA_CT_INPUT || which == TH_LORA_CT_PRODUCT, "which must be TH_LORA_CT_INPUT or _PRODUCT");
    // a queued token redone later (sampler band) rewrites these ciphertexts: settle first
    if (!ctx->pending.empty()) drain(ctx);
    need(set->last_mode >= 0, "the LoRA set has run no token yet", TH_ESTATE);
    need(!(set->last_mode & TH_LORA_SK_FUSED),
         "the set's last token ran with TH_LORA_SK_FUSED, which forms no complete ciphertext", TH_ESTATE);
    const uint32_t L = ctx->L, N = ctx->N;
    const uint64_t* src;
    uint32_t limbs;
    double scale;
    if (which == TH_LORA_CT_INPUT) {
      need(index < set->n_in, "input index out of range");
      src = set->cts + (size_t)index * 2 * L * N;
      limbs = L;
      scale = kScale;
    } else {
      need(index < set->n_batches, "batch index out of range");
      src = set->outs + (size_t)index * 2 * L * N;
      const bool rs = (set->last_mode & TH_LORA_RESCALE) != 0;
      limbs = rs ? L - 1 : L;
      scale = rs ? kScale * kScale / (double)ctx->q[L - 1] : kScale * kScale;  // ciphertext.rs:427, :533
    }
    th_ct* ct = new_ct(ctx, limbs, scale);
    const hipError_t e =
        hipMemcpyAsync(ct->d, src, 2 * (size_t)limbs * poly_bytes(ctx), hipMemcpyDeviceToDevice, ctx->stream);
    if (e != hipSuccess) {
      drop(ct);
      hipchk(e, "hipMemcpyAsync");
    }
    *out = ct;
  });
}

int th_lora_deltas(th_ctx* ctx, th_lora* set, const th_pk* pk, const th_sk* sk, const double* hidden,
                   int hidden_on_device, const uint64_t* seeds, int mode, double* deltas, int deltas_on_device,
                   double* inter) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(set && set->ctx == ctx, "LoRA set belongs to another context");
    need(pk && pk->ctx == ctx && sk && sk->ctx == ctx, "keys belong to another context");
    need(hidden && seeds && deltas, "null argument");
    const uint32_t L = ctx->L, ni = set->n_in, nb = set->n_batches;
    need((mode & ~(TH_LORA_RESCALE | TH_LORA_SK_FUSED)) == 0, "unknown th_lora_deltas mode bits");
    need(!(mode & TH_LORA_RESCALE) || L >= 2, "Cannot rescale: only 1 limb left", TH_ESTATE);
    const bool async = hidden_on_device && deltas_on_device && !inter;
    // tokens queued asynchronously before are settled first, so that a redo
    // of one of them cannot overwrite this call's results
    if (!async && !ctx->pending.empty()) drain(ctx);
    const size_t hbytes = (size_t)ni * set->d * 8;
    hipStream_t st = ctx->stream;
    // device-resident inputs are read where they are; host inputs go through
    // the set's staging pages (free: every host-I/O call waits for its work),
    // read there by the encoder itself when small, else copied to the device
    // first
    const double* z = hidden;
    if (!hidden_on_device) {
      char* in = (char*)set->io_host + set->io_in_off;
      memcpy(in, hidden, hbytes);
      if (hbytes <= HOST_INPUT_MAPPED_MAX) {
        z = set->io_dev + set->io_in_off / 8;
      } else {
        HIPCHK(hipMemcpyAsync(set->hidden, in, hbytes, hipMemcpyHostToDevice, st));
        z = set->hidden;
      }
    }
    // host deltas: B is applied straight into the set's mapped staging pages
    // (visible to the host once the stream is idle), read out below
    double* dout = deltas_on_device ? deltas : set->io_dev;
    if (ctx->host_sampler) {
      queue_token(ctx, set, pk, sk, z, seeds, mode, dout, true, BandArgs{nullptr, 0.0});
    } else {
      const uint32_t off = take_flags(ctx, ni);
      queue_token(ctx, set, pk, sk, z, seeds, mode, dout, false, band_args(ctx, off));
      if (async) {
        ctx->pending.push_back(
            AsyncToken{set, pk, sk, z, std::vector<uint64_t>(seeds, seeds + ni), mode, deltas, off});
        return;
      }
      wait_stream(ctx);
      if (any_flag(ctx, off, ni)) {  // a draw in the band: the token again, from glibc draws
        queue_token(ctx, set, pk, sk, z, seeds, mode, dout, true, BandArgs{nullptr, 0.0});
        ctx->redrawn_inputs += ni;
      }
      release_flags(ctx, off);
    }
    const size_t db = set->n_deltas * 8, ib = (size_t)nb * set->cols * 8;
    if (!deltas_on_device || inter) {
      char* hh = (char*)set->io_host;  // stream order: after the hidden states' copy
      if (inter) HIPCHK(hipMemcpyAsync(hh + db, set->sums, ib, hipMemcpyDeviceToHost, st));
      wait_stream(ctx);
      if (!deltas_on_device) memcpy(deltas, hh, db);
      if (inter) memcpy(inter, hh + db, ib);
    } else if (!hidden_on_device) {
      // the host input sits in the staging ring: finish reading it before returning
      wait_stream(ctx);
    }
  });
}

int th_ct_free(th_ct* ct) {
  return guarded([&] {
    if (ct) drop(ct);
  });
}

int th_ct_info(const th_ct* ct, uint32_t* limbs, double* scale) {
  return guarded([&] {
    need(ct != nullptr, "null ciphertext");
    if (limbs) *limbs = ct->limbs;
    if (scale) *scale = ct->scale;
  });
}

int th_ct_download(th_ctx* ctx, const th_ct* ct, uint64_t* c0, uint64_t* c1) {
  return guarded([&] {
    TH_LOCK(ctx);
    check_ct(ctx, ct);
    need(c0 && c1, "null output");
    const size_t bytes = ct->limbs * poly_bytes(ctx);
    download(ctx, c0, ct->d, bytes);
    download(ctx, c1, ct->d + (size_t)ct->limbs * ctx->N, bytes);
  });
}

int th_ct_upload(th_ctx* ctx, const uint64_t* c0, const uint64_t* c1, uint32_t limbs, double scale, th_ct** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out && c0 && c1, "bad argument");
    need(limbs >= 1 && limbs <= ctx->L, "limbs must be in [1, L]");
    const size_t ln = (size_t)limbs * ctx->N;
    for (uint32_t l = 0; l < limbs; ++l)
      for (uint32_t i = 0; i < ctx->N; ++i)
        need(c0[(size_t)l * ctx->N + i] < ctx->q[l] && c1[(size_t)l * ctx->N + i] < ctx->q[l],
             "residues must be reduced modulo their limb prime");
    th_ct* ct = new_ct(ctx, limbs, scale);
    try {
      OpScope sc(ctx);
      const uint64_t* u0 = (const uint64_t*)sc.upload(c0, ln * 8);
      const uint64_t* u1 = (const uint64_t*)sc.upload(c1, ln * 8);
      HIPCHK(hipMemcpyAsync(ct->d, u0, ln * 8, hipMemcpyDeviceToDevice, ctx->stream));
      HIPCHK(hipMemcpyAsync(ct->d + ln, u1, ln * 8, hipMemcpyDeviceToDevice, ctx->stream));
    } catch (...) {
      drop(ct);
      throw;
    }
    *out = ct;
  });
}

int th_ct_export(th_ctx* ctx, const th_ct* ct, uint8_t* buf, size_t cap, size_t* len) {
  return guarded([&] {
    TH_LOCK(ctx);
    check_ct(ctx, ct);
    need(len != nullptr, "null length");
    const size_t pb = ct->limbs * poly_bytes(ctx);
    *len = 8 + 2 * pb;  // serialize.rs:71-77
    if (!buf) return;
    need(cap >= *len, "buffer too small");
    memcpy(buf, &ct->scale, 8);
    download(ctx, buf + 8, ct->d, 2 * pb);
  });
}

int th_ct_import(th_ctx* ctx, const uint8_t* buf, size_t len, uint32_t limbs, th_ct** out) {
  return guarded([&] {
    need(ctx && buf && out, "bad argument");
    const size_t pb = (size_t)limbs * ctx->N * 8;
    need(limbs >= 1 && limbs <= ctx->L, "limbs must be in [1, L]");
    need(len == 8 + 2 * pb, "Expected " + std::to_string(8 + 2 * pb) + " bytes for Ciphertext, got " +
                                std::to_string(len));  // serialize.rs:82-88
    double scale;
    memcpy(&scale, buf, 8);
    std::vector<uint64_t> c0(pb / 8), c1(pb / 8);
    memcpy(c0.data(), buf + 8, pb);
    memcpy(c1.data(), buf + 8 + pb, pb);
    int rc = th_ct_upload(ctx, c0.data(), c1.data(), limbs, scale, out);
    if (rc != TH_OK) raise(rc, g_err);
  });
}

int th_pk_export(th_ctx* ctx, const th_pk* pk, uint8_t* buf, size_t cap, size_t* len) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(pk && pk->ctx == ctx && len, "bad argument");
    const size_t pb = ctx->L * poly_bytes(ctx);
    *len = 2 * pb;  // serialize.rs:48-52
    if (!buf) return;
    need(cap >= *len, "buffer too small");
    download(ctx, buf, pk->d, 2 * pb);
  });
}

int th_pk_import(th_ctx* ctx, const uint8_t* buf, size_t len, th_pk** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(buf && out, "bad argument");
    const size_t pb = ctx->L * poly_bytes(ctx);
    need(len == 2 * pb, "Expected " + std::to_string(2 * pb) + " bytes for PublicKey, got " +
                            std::to_string(len));  // serialize.rs:57-63
    const uint64_t* w = (const uint64_t*)buf;
    for (uint32_t l = 0; l < ctx->L; ++l)
      for (uint32_t i = 0; i < ctx->N; ++i) {
        uint64_t b, a;
        memcpy(&b, buf + ((size_t)l * ctx->N + i) * 8, 8);
        memcpy(&a, buf + pb + ((size_t)l * ctx->N + i) * 8, 8);
        need(b < ctx->q[l] && a < ctx->q[l], "residues must be reduced modulo their limb prime");
      }
    (void)w;
    th_pk* pk = adopt(new th_pk{ctx, nullptr});
    try {
      pk->d = (uint64_t*)ctx->pool.get(2 * pb);
      OpScope sc(ctx);
      const void* up = sc.upload(buf, 2 * pb);
      HIPCHK(hipMemcpyAsync(pk->d, up, 2 * pb, hipMemcpyDeviceToDevice, ctx->stream));
    } catch (...) {
      drop(pk);
      throw;
    }
    *out = pk;
  });
}

int th_ntt_forward_batch(th_ctx* ctx, uint64_t* polys, size_t count, uint32_t limbs, int on_device) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(polys || count == 0, "null polynomials");
    ntt_batch(ctx, polys, count, limbs, on_device, false);
  });
}

int th_ntt_inverse_batch(th_ctx* ctx, uint64_t* polys, size_t count, uint32_t limbs, int on_device) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(polys || count == 0, "null polynomials");
    ntt_batch(ctx, polys, count, limbs, on_device, true);
  });
}

int th_dev_alloc(th_ctx* ctx, size_t bytes, void** out) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(out != nullptr, "null output");
    void* p = ctx->pool.get(bytes);
    ctx->user_allocs.insert(p);
    *out = p;
  });
}

// Only buffers from th_dev_alloc that are still held may be freed: a second
// free, or a ciphertext's or key's own buffer, is refused (the pool would
// otherwise hand one buffer to two later owners).
int th_dev_free(th_ctx* ctx, void* p) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(ctx->user_allocs.count(p) == 1, "pointer was not allocated by th_dev_alloc, or was already freed");
    if (!ctx->pending.empty()) drain(ctx);  // a queued token redone later may read this buffer
    ctx->user_allocs.erase(p);
    ctx->pool.put(p);
  });
}

int th_memcpy_h2d(th_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    TH_LOCK(ctx);
    if (!ctx->pending.empty()) drain(ctx);  // a queued token redone later may read what this overwrites
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
  });
}

int th_memcpy_d2h(th_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    TH_LOCK(ctx);
    if (!ctx->pending.empty()) drain(ctx);  // queued tokens settled before their outputs are read
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
  });
}

int th_ntt_time(th_ctx* ctx, uint64_t* dev_polys, size_t count, uint32_t limbs, int inverse, int reps, float* avg_ms) {
  return guarded([&] {
    TH_LOCK(ctx);
    need(dev_polys && avg_ms && reps > 0 && count > 0, "bad argument");
    need(limbs >= 1 && limbs <= ctx->L, "limbs must be in [1, L]");
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    try {
      HIPCHK(hipEventRecord(e0, ctx->stream));
      for (int r = 0; r < reps; ++r)
        ntt_strided(ctx, inverse != 0, dev_polys, dev_polys, (uint32_t)(count * limbs), limbs);
      HIPCHK(hipEventRecord(e1, ctx->stream));
      HIPCHK(hipEventSynchronize(e1));
      float ms = 0;
      HIPCHK(hipEventElapsedTime(&ms, e0, e1));
      *avg_ms = ms / reps;
    } catch (...) {
      (void)hipEventDestroy(e0);
      (void)hipEventDestroy(e1);
      throw;
    }
    HIPCHK(hipEventDestroy(e0));
    HIPCHK(hipEventDestroy(e1));
  });
}

}  // extern "C"
