// LoRA sets (th_lora_*): the cached plaintexts and LoRA-B of a set of
// projections on the device, the per-token pass (complete or sk-fused), the
// CryptoMOE regate and tokens queued without a host synchronisation.
#include "runtime.h"

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
    std::vector<RescaleDecryptJob> rj;
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
        rj.push_back(RescaleDecryptJob{mm, nullptr, nullptr, nullptr, set->sums + (size_t)bt * cols, scale_r});
      }
      cp[bt] = CtPtJob{ct, ct + (size_t)L * N, pt, o, L, 0};
      for (uint32_t l = 0; l < nl_n; ++l)
        dn.push_back(NttJob{o + (size_t)l * N, mm + (size_t)l * N, o + (size_t)(L + l) * N, nullptr, l, 0});
    }
    if (L >= 2) {
      set->d_fwd_all = persist(set, fa);
      set->d_dot_all_r = persist(set, dr);
      set->dot_all_r_jobs = (uint32_t)dr.size();
      const SumsPath sp = nl_r == 1 ? decrypt_sums_path(c, nb, cols) : SumsPath::KERNELS;
      if (sp == SumsPath::WHOLE) {
        set->d_seg_all = persist(set, seg);
      } else if (sp == SumsPath::SPLIT) {
        // the same transforms on the split kernels: seg's jobs with the work area as dst
        for (uint32_t bt = 0; bt < nb; ++bt) seg[bt].dst = set->m + (size_t)bt * 2 * N;
        set->d_dec_row = persist(set, seg);
        set->d_dec_rj = persist(set, rj);
        set->dec_partials = (double*)set->alloc((size_t)nb * cols * (N / 16) * 8);
      }
    }
    set->d_ctpt = persist(set, cp);
    set->d_dot_all_n = persist(set, dn);
    set->dot_all_n_jobs = (uint32_t)dn.size();
  }
  set->d_bjobs = persist(set, bj);
  if (cols <= SEGSUM_MAX_COLS) set->seg_w = seg_weights(c, d, cols);
  if (set->d_dot_seg || set->d_rd || set->d_seg_all || set->d_dec_row) set->seg_p = seg_pairs(c, d);
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
    } else if (set->d_dec_row) {
      launch_dec_sums_split(ctx, set->d_dec_row, set->d_dec_rj, nb, sk, set->seg_p, set->cols, set->dec_partials);
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

}  // namespace

namespace thrt {

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

}  // namespace thrt

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

}  // extern "C"
