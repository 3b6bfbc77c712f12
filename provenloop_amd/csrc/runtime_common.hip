// Shared helpers of the host runtime (declared in runtime.h): handle
// lifetime, sampler band flags, NTT dispatch, context tables, and the
// encode, encrypt, product, rescale and decrypt pipelines the entry points
// queue on a context's stream.
#include "runtime.h"

namespace thrt {

thread_local std::string g_err = "";







// ---------------------------------------------------------------- handle lifetime


// Drops one reference; the last one destroys the context.
void ctx_release(th_ctx* c) {
  if (c->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) destroy_ctx(c);
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
                 uint32_t limb_base) {
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
void ntt_list(OpScope& sc, bool inverse, const std::vector<NttJob>& jobs, NttLoad load,
              const RescaleConst* rc, const uint64_t* key, NttStore store) {
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
  // twiddles: per limb forward then inverse, N pairs of 16 bytes each; at the
  // split kernels' sizes followed by the row tables (row_table_index), per
  // limb forward then inverse, 15 N / 16 pairs each
  const bool split = c->logn >= (uint32_t)NTT_SPLIT_MIN_LOGN && c->logn <= (uint32_t)NTT_MAX_LOGN;
  const size_t row_n = split ? (size_t)15 * N / 16 : 0;
  const size_t main_bytes = (size_t)L * 2 * N * 16;
  const size_t tab_bytes = main_bytes + (size_t)L * 2 * row_n * 16;
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
    unsigned char* frow = host_tab.data() + main_bytes + (size_t)(2 * l) * row_n * 16;
    unsigned char* irow = host_tab.data() + main_bytes + (size_t)(2 * l + 1) * row_n * 16;
    if (split) {
      const uint32_t parts = N >> 10;
      for (int b = 0; b < 4; ++b)
        for (uint32_t p = 0; p < parts; ++p)
          for (uint32_t s = 0; s < (16u >> (b + 1)); ++s)
            for (uint32_t ln = 0; ln < 64; ++ln) {
              const uint32_t to = row_table_index(N, b, p, s, ln), from = row_table_source(N, (int)c->logn, b, p, s, ln);
              memcpy(frow + 16 * (size_t)to, fdst + 16 * (size_t)from, 16);
              memcpy(irow + 16 * (size_t)to, idst + 16 * (size_t)from, 16);
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
    lc.fwd_row = split ? (const char*)c->d_tables + main_bytes + (size_t)(2 * l) * row_n * 16 : nullptr;
    lc.inv_row = split ? (const char*)c->d_tables + main_bytes + (size_t)(2 * l + 1) * row_n * 16 : nullptr;
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
                  const int64_t* e1, uint64_t* dst, size_t dst_stride, uint32_t rep_d, uint32_t rep_cols) {
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

// Whether a batch of `jobs` limb-0 decryptions with `cols` segments can take
// the decrypt transform's segment-sum epilogue (NTT_STORE_SEGSUM) in one
// round of whole-polynomial workgroups.
bool segsum_in_transform(const th_ctx* c, uint32_t jobs, uint32_t cols) {
  return c->logn <= 14 && jobs <= 256 && cols >= 1 && cols <= NTT_SEGSUM_FUSED_MAX_COLS;
}

SumsPath decrypt_sums_path(const th_ctx* c, uint32_t jobs, uint32_t cols) {
  if (cols < 1 || cols > NTT_SEGSUM_FUSED_MAX_COLS) return SumsPath::KERNELS;
  if (c->logn < 13 || (c->logn <= 14 && jobs >= DECRYPT_WHOLE_MIN_JOBS)) return SumsPath::WHOLE;
  return SumsPath::SPLIT;
}

void launch_dec_sums_split(th_ctx* c, const NttJob* d_row, const RescaleDecryptJob* d_jobs, uint32_t n,
                           const th_sk* sk, const double* W, uint32_t cols, double* partials) {
  NttArgs row{};
  row.lc = c->d_lc;
  row.jobs = d_row;
  row.load = NTT_LOAD_DOTM;
  row.bc = c->d_bc;
  row.key = sk_montgomery(c, sk);
  RescaleDecryptArgs a{};
  a.lc = c->d_lc;
  a.bc = c->d_bc;
  a.segw = W;
  a.jobs = d_jobs;
  a.cols = cols;
  HIPCHK(launch_decrypt_sums_split((int)c->logn, row, a, n, partials, c->stream));
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

// Queue decrypt + decode of the views; slots to out_dev (count x S) and/or
// segment sums to seg_dev (count x cols). m_l = c0_l + c1_l * s_l
// (ciphertext.rs:332-341) is formed inside the inverse transform's load.
// When only segment sums are wanted (and cols <= SEGSUM_MAX_COLS) they come
// from the coefficients and the segment weights, without forming the slots;
// the decrypt transform produces them itself (NTT_STORE_SEGSUM) when its
// batch runs in the whole-polynomial kernel. Scratch lives in the caller's
// scope.
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
  const SumsPath path = seg_only && nj.size() == count ? decrypt_sums_path(c, (uint32_t)count, cols)
                                                       : SumsPath::KERNELS;
  if (path == SumsPath::WHOLE) {
    // every ciphertext takes the limb-0 branch: the segment sums come out of
    // the decrypt transform itself
    for (size_t i = 0; i < count; ++i) {
      nj[i].dst = reinterpret_cast<uint64_t*>(seg_dev + i * cols);
      nj[i].scale = cts[i].scale;
    }
    launch_dot_segsum(c, sc.up(nj), (uint32_t)count, sk, seg_pairs(c, d), cols);
    return;
  }
  if (path == SumsPath::SPLIT) {
    std::vector<RescaleDecryptJob> rj(count);
    for (size_t i = 0; i < count; ++i)
      rj[i] = RescaleDecryptJob{dot + i * 2 * N, nullptr, nullptr, nullptr, seg_dev + i * cols, cts[i].scale};
    launch_dec_sums_split(c, sc.up(nj), sc.up(rj), (uint32_t)count, sk, seg_pairs(c, d), cols,
                          (double*)sc.dev(count * cols * (N / 16) * 8));
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
                   const uint64_t* const* pts) {
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

}  // namespace thrt
