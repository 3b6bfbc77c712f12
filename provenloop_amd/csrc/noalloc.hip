// th_batch_decrypt_segsum_noalloc: th_batch_decrypt_segsum for callers that
// cannot allocate device memory, with its working memory in a file-scope
// device array per GPU.
#include "runtime.h"

// Device scratch of th_batch_decrypt_segsum_noalloc, one copy per GPU for the
// life of the process. In host code this name is only a stand-in for the
// symbol, not a device address: host code uses the pointer that
// hipGetSymbolAddress returns for each device (scratch_base).
constexpr size_t TH_NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[TH_NOALLOC_SCRATCH_BYTES];

namespace thrt {

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

}  // namespace thrt

extern "C" {

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
    // The array is idle whenever its lock is free: a failure after work was
    // queued waits for the stream before the lock is released.
    try {
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
    } catch (...) {
      (void)hipStreamSynchronize(ctx->stream);
      throw;
    }
  });
}

}  // extern "C"
