// Keys, encryption, plaintexts, ct x pt, add / sub, rescale, decryption,
// the one-call LoRA-A pass and the wire format of the C ABI
// (include/tensafe_he.h): each entry point queues its pipeline (runtime.h)
// on the context's stream.
#include "runtime.h"

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

}  // extern "C"
