// Contexts (th_ctx_*), context options, key handles' release and download,
// device memory helpers and the raw batched transforms of the C ABI
// (include/tensafe_he.h).
#include "runtime.h"

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
