// Poseidon Merkle commitments of weight MLEs and their openings, and the
// weight phase after the walk (crypto/mle_opening.rs, gkr/prover.rs:2059-2200).
#include "internal.h"
#include "merkle.h"
#include "poseidon9_host.h"
/* ------------------------------------------------------------------ MLE commitments
 * Poseidon Merkle roots (merkle.h).  A batch runs level by level: launch L
 * moves every unfinished tree from level s to s + d, writing the real nodes
 * of level s + d into buffer L % 2 and reading level s from the other one.
 * d is the largest of 4..2 that still gives 2^18 output nodes over the
 * batch, else 1 (the upper levels are latency-bound: one hash per thread per
 * launch keeps them short). */
struct MerkleTreeSpec {
  uint32_t kind;  // 0 matrix, 1 QM31 vector
  const uint32_t* src;
  uint64_t rows, cols;
  uint32_t log_pk, height;
  uint64_t mle_len;
};

static uint32_t log2_ceil(uint64_t v) {
  uint32_t l = 0;
  while ((1ull << l) < v) l++;
  return l;
}

static int merkle_consts(gkr_ctx* c, const MerkleConsts** out) {
  if (!c->merkle_consts) {
    const f9::setup& S = f9::host_setup();
    std::unique_ptr<MerkleConsts> h(new MerkleConsts());
    h->hk = S.k;
    h->r2 = S.r2;
    h->one = S.one;
    const felt two124 = felt_to_mont(felt{{0, (uint64_t)1 << 60, 0, 0}});  // securefield_to_felt(0) = 2^124
    felt z = two124, zz = felt_zero();
    for (int s = 0; s < 64; s++) {
      h->z[s] = f9::from_host_mont(z);
      h->zz[s] = f9::from_host_mont(zz);
      z = poseidon_hash(z, z);
      zz = poseidon_hash(zz, zz);
    }
    MerkleConsts* d = nullptr;
    HIP_TRY(hipMalloc(&d, sizeof(MerkleConsts)));
    if (hipMemcpy(d, h.get(), sizeof(MerkleConsts), hipMemcpyHostToDevice) != hipSuccess) {
      (void)hipFree(d);
      return fail(GKR_ERR_DEVICE, "copy of the Merkle constants failed");
    }
    c->merkle_consts = d;
  }
  *out = c->merkle_consts;
  return GKR_OK;
}

// kept == nullptr: roots only (ping-pong level buffers).  Otherwise every level
// of every tree is kept in one arena (one level per launch) and described in
// (*kept)[i] for path extraction; the arena stays valid until the next call.
static int merkle_roots(gkr_ctx* c, const std::vector<MerkleTreeSpec>& trees, gkr_felt* roots,
                        std::vector<MerkleKept>* kept = nullptr) {
  const size_t nt = trees.size();
  if (nt == 0) return GKR_OK;
  const MerkleConsts* K;
  TRY(merkle_consts(c, &K));
  struct Launch {
    uint32_t s;
    size_t first_step, n_steps;
    uint64_t total;
  };
  std::vector<Launch> launches;
  std::vector<MerkleStep> steps;
  std::vector<uint64_t> step_off;  // node offset of each step's output in its buffer (arena when kept)
  std::vector<std::pair<size_t, size_t>> root_at(nt);  // (launch, step) producing each root
  uint64_t need[2] = {1, 1}, arena = 0;
  uint32_t smax = 0;
  for (const auto& t : trees) smax = std::max(smax, t.height);
  for (uint32_t s = 0; s < smax;) {
    auto outputs = [&](uint32_t D) {
      uint64_t n = 0;
      for (const auto& t : trees)
        if (t.height > s) n += merkle_real_count(t.kind, t.rows, t.cols, t.log_pk, s + std::min(D, t.height - s));
      return n;
    };
    uint32_t D = 1;
    if (!kept)
      for (uint32_t cand = kMerkleMaxD; cand >= 2; cand--)
        if (outputs(cand) >= (1ull << 18)) {
          D = cand;
          break;
        }
    Launch L{s, steps.size(), 0, 0};
    uint64_t off = 0;
    for (size_t i = 0; i < nt; i++) {
      const auto& t = trees[i];
      if (t.height <= s) continue;
      MerkleStep st{};
      st.src = t.src;
      st.rows = t.rows;
      st.cols = t.cols;
      st.mle_len = t.mle_len;
      st.kind = t.kind;
      st.log_pk = t.log_pk;
      st.d = std::min(D, t.height - s);
      st.n_out = merkle_real_count(t.kind, t.rows, t.cols, t.log_pk, s + st.d);
      st.thread_begin = L.total;
      L.total += st.n_out;
      step_off.push_back(kept ? arena : off);
      off += st.n_out;
      arena += st.n_out;
      if (s + st.d == t.height) root_at[i] = {launches.size(), steps.size()};
      steps.push_back(st);
    }
    L.n_steps = steps.size() - L.first_step;
    need[launches.size() & 1] = std::max(need[launches.size() & 1], off);
    launches.push_back(L);
    s += D;
  }
  f9::fe* buf[2] = {nullptr, nullptr};
  if (kept) {
    TRY(ensureT(c, S_MK0, arena, &buf[0]));
    kept->assign(nt, MerkleKept{});
    for (size_t i = 0; i < nt; i++) {
      MerkleKept& k = (*kept)[i];
      k.src = trees[i].src;
      k.rows = trees[i].rows;
      k.cols = trees[i].cols;
      k.mle_len = trees[i].mle_len;
      k.kind = trees[i].kind;
      k.log_pk = trees[i].log_pk;
      k.height = trees[i].height;
    }
  } else {
    TRY(ensureT(c, S_MK0, need[0], &buf[0]));
    TRY(ensureT(c, S_MK1, need[1], &buf[1]));
  }
  void* droot;
  TRY(ensure(c, S_MKROOT, nt * (sizeof(f9::fe) + sizeof(void*) + 32), &droot));
  f9::fe* root_nodes = (f9::fe*)droot;
  const f9::fe** dptr = (const f9::fe**)(root_nodes + nt);
  uint32_t* dwords = (uint32_t*)(dptr + nt);
  // wire the buffers: a tree's input is its previous output.  Roots only:
  // launch l writes buf[l & 1], and a tree's last launch writes its root to
  // root_nodes (later launches reuse the ping-pong buffers).  Kept: every
  // output has its own place in the arena.
  std::vector<const f9::fe*> prev(nt, nullptr);
  for (size_t l = 0; l < launches.size(); l++) {
    size_t k = launches[l].first_step;
    for (size_t i = 0; i < nt; i++) {
      if (trees[i].height <= launches[l].s) continue;
      steps[k].in = prev[i];
      if (kept) {
        steps[k].out = buf[0] + step_off[k];
        (*kept)[i].level[launches[l].s + steps[k].d] = steps[k].out;
      } else {
        steps[k].out = root_at[i].second == k ? root_nodes + i : buf[l & 1] + step_off[k];
      }
      prev[i] = steps[k].out;
      k++;
    }
  }
  MerkleStep* dsteps;
  TRY(ensureT(c, S_MKSTEP, steps.size(), &dsteps));
  HIP_TRY(hipMemcpyAsync(dsteps, steps.data(), steps.size() * sizeof(MerkleStep), hipMemcpyHostToDevice, c->stream));
  for (const auto& L : launches) {
    const uint64_t blocks = (L.total + kMerkleBlock - 1) / kMerkleBlock;
    uint64_t hashes = 0;  // the timer's byte counter holds the hash count of this kernel
    for (size_t k = L.first_step; k < L.first_step + L.n_steps; k++) hashes += steps[k].n_out * ((1ull << steps[k].d) - 1);
    TimedLaunch tl(c, K_MERKLE, hashes);
    GKR_LAUNCH(c, k_merkle_level, dim3((uint32_t)blocks), dim3(kMerkleBlock), 0, dsteps + L.first_step, (int)L.n_steps,
                                                                              L.s, L.total, K);
    HIP_TRY(hipGetLastError());
  }
  std::vector<const f9::fe*> rp(nt);
  for (size_t i = 0; i < nt; i++) rp[i] = kept ? steps[root_at[i].second].out : root_nodes + i;
  HIP_TRY(hipMemcpyAsync(dptr, rp.data(), nt * sizeof(void*), hipMemcpyHostToDevice, c->stream));
  GKR_LAUNCH(c, k_merkle_roots, dim3((uint32_t)((nt + 63) / 64)), dim3(64), 0, dptr, (int)nt, K, dwords);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipMemcpyAsync(roots, dwords, nt * 32, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return GKR_OK;
}

static int weight_tree(const gkr_matrix* m, MerkleTreeSpec* t) {
  if (!m || !m->dev || m->rows == 0 || m->cols == 0) return fail(GKR_ERR_INVALID, "weight commitment: empty matrix");
  t->kind = 0;
  t->src = m->dev;
  t->rows = m->rows;
  t->cols = m->cols;
  t->log_pk = log2_ceil(m->rows);
  const uint32_t log_pn = log2_ceil(m->cols);
  if (t->log_pk + log_pn > 48) return fail(GKR_ERR_INVALID, "weight commitment: padded MLE above 2^48 entries");
  t->mle_len = 1ull << (t->log_pk + log_pn);
  t->height = std::max(1u, t->log_pk + log_pn);
  return GKR_OK;
}

extern "C" int gkr_weight_commitment(gkr_ctx* c, const gkr_matrix* b, gkr_felt* root) {
  if (!c || !root) return fail(GKR_ERR_INVALID, "null argument");
  return gkr_weight_commitments(c, &b, 1, root);
}

// Roots already on a matrix (computed before, or supplied with
// gkr_matrix_set_commitment) are taken from it; the others are computed in
// one batch and kept on their matrices, until the contents change
// (gkr_matrix_invalidate, gkr_matmul_forward_into).  The reference keeps the
// same root per weight in WeightCommitmentCache (weight_cache.rs:283-327).
extern "C" int gkr_weight_commitments(gkr_ctx* c, const gkr_matrix* const* mats, size_t count, gkr_felt* roots) {
  if (!c || (count && (!mats || !roots))) return fail(GKR_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(c->device));
  std::vector<MerkleTreeSpec> trees;
  std::vector<size_t> todo;
  for (size_t i = 0; i < count; i++) {
    MerkleTreeSpec t;
    TRY(weight_tree(mats[i], &t));  // validates every matrix, cached or not
    if (mats[i]->have_root) {
      roots[i] = mats[i]->root;
      continue;
    }
    trees.push_back(t);
    todo.push_back(i);
  }
  if (trees.empty()) return GKR_OK;
  std::vector<gkr_felt> fresh(trees.size());
  TRY(merkle_roots(c, trees, fresh.data()));
  for (size_t j = 0; j < todo.size(); j++) {
    gkr_matrix* m = const_cast<gkr_matrix*>(mats[todo[j]]);
    roots[todo[j]] = fresh[j];
    if (m->ctx == c) {
      m->root = fresh[j];
      m->have_root = true;
    }
  }
  return GKR_OK;
}
extern "C" int gkr_matrix_commitment_cached(const gkr_matrix* m, gkr_felt* root, int* cached) {
  if (!m || !root || !cached) return fail(GKR_ERR_INVALID, "null argument");
  *cached = m->have_root ? 1 : 0;
  if (m->have_root) *root = m->root;
  return GKR_OK;
}
extern "C" int gkr_matrix_set_commitment(gkr_ctx* c, gkr_matrix* m, const gkr_felt* root) {
  if (!c || !m || !root) return fail(GKR_ERR_INVALID, "null argument");
  if (m->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another (or a destroyed) context");
  if (!felt_abi_canonical(*root)) return fail(GKR_ERR_INVALID, "commitment root not canonical");
  m->root = *root;
  m->have_root = true;
  return GKR_OK;
}

extern "C" int gkr_mle_commitment(gkr_ctx* c, const gkr_qvec* evals, gkr_felt* root) {
  if (!c || !evals || !root) return fail(GKR_ERR_INVALID, "null argument");
  if (evals->n == 0) return fail(GKR_ERR_INVALID, "MLE commitment: empty vector");
  HIP_TRY(hipSetDevice(c->device));
  MerkleTreeSpec t{};
  t.kind = 1;
  t.src = (const uint32_t*)evals->dev;
  t.rows = evals->n;
  t.cols = 1;
  t.mle_len = evals->n;
  t.height = std::max(1u, log2_ceil(evals->n));
  if (t.height > 48) return fail(GKR_ERR_INVALID, "MLE commitment: above 2^48 entries");
  return merkle_roots(c, {t}, root);
}

/* ------------------------------------------------------------------ weight openings
 * prove_mle_opening_with_commitment (engine/src/crypto/mle_opening.rs:1654-1915)
 * over matrix_to_mle_col_major_padded(B):
 *   layer 0 = the padded MLE (read from B), layer t+1 = fold of layer t on its
 *   top variable with eval_point[t]; the Merkle tree of every layer longer
 *   than 1 is built once with all its levels kept (the reference rebuilds
 *   them for the query phase); roots are mixed in layer order; query pairs are
 *   drawn (low 64 bits of draw_felt252 mod len/2, then mod max(mid/2, 1) per
 *   round); values and auth paths are gathered on the device.
 * Layers 1..log2(pn) keep B's zero rows (a grid with `rows` real rows, kind 2
 * trees); later layers are plain QM31 vectors (kind 1).  The record holds the
 * serialized claim and MleOpeningProof (cairo_serde.rs:341-369, 1759-1767). */
constexpr size_t kMleQueries = 10;  // MLE_N_QUERIES, mle_opening.rs:47

// src: a weight matrix (its column-major padded MLE) or a resident QM31
// vector of a power-of-two length.  with_claim: the record starts with the
// claim (point, expected value) as serialize_gkr_model_proof writes openings;
// otherwise it holds the MleOpeningProof alone.
int mle_opening(gkr_ctx* c, const OpenSrc& src, const gkr_qm31* point, uint32_t n_point, const gkr_qm31* expected,
                PoseidonChannel& C, felt* commitment, std::vector<felt>& rec, bool with_claim) {
  const gkr_matrix* b = src.b;
  MerkleTreeSpec t0{};
  uint32_t log_pk = 0, log_pn = 0, nv = 0;
  if (b) {
    TRY(weight_tree(b, &t0));
    log_pk = t0.log_pk;
    log_pn = log2_ceil(b->cols);
    nv = log_pk + log_pn;
  } else {
    if (!src.q || src.qn == 0 || (src.qn & (src.qn - 1))) return fail(GKR_ERR_INVALID, "MLE opening: bad vector");
    nv = log2_ceil(src.qn);
    t0.kind = 1;
    t0.src = (const uint32_t*)src.q;
    t0.rows = src.qn;
    t0.cols = 1;
    t0.mle_len = src.qn;
    t0.height = std::max(1u, nv);
  }
  if (n_point != nv) return fail(GKR_ERR_INVALID, "weight opening: point has %u vars, the padded MLE has %u", n_point, nv);
  for (uint32_t t = 0; t < nv; t++)
    if (!canonical_q(point[t])) return fail(GKR_ERR_INVALID, "weight opening: point not canonical");
  const uint64_t N = 1ull << nv;
  // folded layers 1..nv, back to back (N - 1 values)
  qm31* lay = nullptr;
  TRY(ensureT(c, S_OPL, N, &lay));
  std::vector<qm31*> L(nv + 1, nullptr);
  for (uint64_t t = 1, off = 0; t <= nv; t++) {
    L[t] = lay + off;
    off += N >> t;
  }
  for (uint32_t t = 0; t < nv; t++) {
    const uint64_t mid = N >> (t + 1);
    const uint32_t blocks = (uint32_t)((mid + 255) / 256);
    if (t == 0 && b)
      GKR_LAUNCH(c, k_open_fold_matrix, dim3(blocks), dim3(256), 0, b->dev, b->rows, b->cols, log_pk, mid,
                                                                    Q(point[0]), L[1]);
    else if (t == 0)
      GKR_LAUNCH(c, k_open_fold, dim3(blocks), dim3(256), 0, src.q, mid, Q(point[0]), L[1]);
    else
      GKR_LAUNCH(c, k_open_fold, dim3(blocks), dim3(256), 0, L[t], mid, Q(point[t]), L[t + 1]);
    HIP_TRY(hipGetLastError());
  }
  // trees of layers 0..nv-1 (layer 0 also when nv == 0: one leaf padded to two)
  std::vector<MerkleTreeSpec> trees(1, t0);
  for (uint32_t t = 1; t < nv; t++) {
    MerkleTreeSpec s{};
    s.src = (const uint32_t*)L[t];
    s.mle_len = N >> t;
    s.height = nv - t;
    if (b && t <= log_pn) {
      s.kind = 2;
      s.rows = b->rows;
      s.cols = 1ull << (log_pn - t);
      s.log_pk = log_pk;
    } else {
      s.kind = 1;
      s.rows = N >> t;
      s.cols = 1;
    }
    trees.push_back(s);
  }
  std::vector<gkr_felt> roots(trees.size());
  std::vector<MerkleKept> kept;
  TRY(merkle_roots(c, trees, roots.data(), &kept));
  qm31 final_value;
  if (nv == 0 && b) {
    uint32_t v;
    HIP_TRY(hipMemcpy(&v, b->dev, 4, hipMemcpyDeviceToHost));
    final_value = qm31_from_m31(v);
  } else if (nv == 0) {
    HIP_TRY(hipMemcpy(&final_value, src.q, sizeof(qm31), hipMemcpyDeviceToHost));
  } else {
    HIP_TRY(hipMemcpy(&final_value, L[nv], sizeof(qm31), hipMemcpyDeviceToHost));
  }
  if (expected && !qm31_eq(final_value, Q(*expected)))
    return fail(GKR_ERR_INVALID, "weight opening: the MLE at the point differs from the expected value");
  std::vector<felt> rf(trees.size());
  for (size_t t = 0; t < trees.size(); t++) rf[t] = felt_canon_from_words(roots[t].w);
  *commitment = rf[0];
  for (size_t t = 0; t < trees.size(); t++) C.mix_felt(felt_to_mont(rf[t]));
  // queries
  const uint64_t half = N / 2;
  const size_t nq = (size_t)std::min<uint64_t>(kMleQueries, half);
  std::vector<uint64_t> pairs(nq);
  for (size_t q = 0; q < nq; q++) {
    const felt f = felt_from_mont(C.draw_felt252());
    pairs[q] = f.l[0] % half;
  }
  std::vector<MerkleGather> items;
  for (size_t q = 0; q < nq; q++) {
    uint64_t idx = pairs[q];
    for (uint32_t t = 0; t < nv; t++) {
      const uint64_t mid = (N >> t) / 2, li = idx, ri = mid + idx;
      items.push_back(MerkleGather{t, 0, 1, 0, li});
      items.push_back(MerkleGather{t, 0, 1, 0, ri});
      for (uint64_t k0 : {li, ri}) {
        uint64_t k = k0;
        for (uint32_t lv = 0; lv < trees[t].height; lv++) {
          items.push_back(MerkleGather{t, lv, 0, 0, k ^ 1});
          k >>= 1;
        }
      }
      idx %= std::max<uint64_t>(mid / 2, 1);
    }
  }
  std::vector<uint32_t> got(8 * items.size());
  if (!items.empty()) {
    void* dio;
    const size_t kbytes = kept.size() * sizeof(MerkleKept), ibytes = items.size() * sizeof(MerkleGather);
    TRY(ensure(c, S_OPI, kbytes + ibytes + got.size() * 4, &dio));
    MerkleKept* dk = (MerkleKept*)dio;
    MerkleGather* di = (MerkleGather*)((char*)dio + kbytes);
    uint32_t* dout = (uint32_t*)((char*)dio + kbytes + ibytes);
    HIP_TRY(hipMemcpyAsync(dk, kept.data(), kbytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(di, items.data(), ibytes, hipMemcpyHostToDevice, c->stream));
    const MerkleConsts* K;
    TRY(merkle_consts(c, &K));
    GKR_LAUNCH(c, k_merkle_gather, dim3((uint32_t)((items.size() + 63) / 64)), dim3(64), 0, dk, di, (int)items.size(),
                                                                                          K, dout);
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipMemcpyAsync(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
  }
  // record: claim point, expected value, MleOpeningProof
  auto fu = [&](uint64_t v) { rec.push_back(felt{{v, 0, 0, 0}}); };
  auto fq = [&](const qm31& x) { fu(x.a); fu(x.b); fu(x.c); fu(x.d); };
  if (with_claim) {
    fu(nv);
    for (uint32_t t = 0; t < nv; t++) fq(Q(point[t]));
    fq(expected ? Q(*expected) : final_value);
  }
  fu(nv > 0 ? nv - 1 : 0);
  for (uint32_t t = 1; t < nv; t++) rec.push_back(rf[t]);
  fu(nq);
  size_t it = 0;
  for (size_t q = 0; q < nq; q++) {
    fu(pairs[q]);
    fu(nv);
    for (uint32_t t = 0; t < nv; t++) {
      for (int side = 0; side < 2; side++, it++) fq(qm31{got[8 * it], got[8 * it + 1], got[8 * it + 2], got[8 * it + 3]});
      for (int side = 0; side < 2; side++) {
        fu(trees[t].height);
        for (uint32_t lv = 0; lv < trees[t].height; lv++, it++) rec.push_back(felt_canon_from_words(&got[8 * it]));
      }
    }
  }
  fq(final_value);
  return GKR_OK;
}

extern "C" int gkr_prove_weight_opening(gkr_ctx* c, const gkr_matrix* b, const gkr_qm31* eval_point, uint32_t n_point,
                                        const gkr_qm31* expected_value, gkr_channel* ch, gkr_proof* proof,
                                        gkr_felt* commitment) {
  CH_CHECK(ch);
  if (!c || !b || !proof || (!eval_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (expected_value && !canonical_q(*expected_value)) return fail(GKR_ERR_INVALID, "expected value not canonical");
  HIP_TRY(hipSetDevice(c->device));
  felt cm;
  std::vector<felt> rec;
  TRY(mle_opening(c, OpenSrc{b, nullptr, 0}, eval_point, n_point, expected_value, ch->ch, &cm, rec, true));
  proof->weight_commitments.push_back(cm);
  proof->weight_openings.push_back(std::move(rec));
  if (commitment) felt_canon_to_words(cm, commitment->w);
  return GKR_OK;
}

extern "C" int gkr_prove_weight_openings(gkr_ctx* c, gkr_channel* ch, gkr_proof* proof) {
  return gkr_prove_weight_binding(c, ch, proof, GKR_WEIGHT_SEQUENTIAL);
}

// The weight phase of the GKR prover (prover.rs:2059-2200) over the claims the
// proof recorded, in recording order.
//   SEQUENTIAL: one opening per claim on the main channel (prover.rs:2160-2190).
//   AGGREGATED_RLC: the reference default, the aggregated oracle sumcheck without
//     the full binding proof (prover.rs:368-658): the commitment of every claimed
//     weight (one batch) goes into the proof, then rho = draw_qm31 and
//     mix_secure_field(sum rho^i v_i) (prover.rs:1335-1345); no openings.
//   RLC_DIRECT: apply_aggregated_rlc_binding (prover.rs:669-699): rho and the
//     combined value only, no commitments.
extern "C" int gkr_prove_weight_binding(gkr_ctx* c, gkr_channel* ch, gkr_proof* proof, int mode) {
  CH_CHECK(ch);
  if (!c || !proof) return fail(GKR_ERR_INVALID, "null argument");
  if (mode != GKR_WEIGHT_SEQUENTIAL && mode != GKR_WEIGHT_AGGREGATED_RLC && mode != GKR_WEIGHT_RLC_DIRECT &&
      mode != GKR_WEIGHT_AGGREGATED_FULL)
    return fail(GKR_ERR_INVALID, "unknown weight binding mode %d", mode);
  auto& claims = proof->weight_claims;
  if (mode == GKR_WEIGHT_SEQUENTIAL) {
    for (const WeightClaimRec& w : claims) {
      const gkr_qm31* pt = reinterpret_cast<const gkr_qm31*>(w.point.data());
      const gkr_qm31 v = {{w.value.a, w.value.b, w.value.c, w.value.d}};
      TRY(gkr_prove_weight_opening(c, w.b, pt, (uint32_t)w.point.size(), &v, ch, proof, nullptr));
    }
    claims.clear();
    return GKR_OK;
  }
  if (claims.empty()) return GKR_OK;
  std::vector<gkr_felt> claim_roots;
  if (mode == GKR_WEIGHT_AGGREGATED_RLC || mode == GKR_WEIGHT_AGGREGATED_FULL) {
    // one root per distinct matrix, repeated per claim
    std::vector<const gkr_matrix*> uniq;
    std::map<const gkr_matrix*, size_t> at;
    for (const auto& w : claims)
      if (at.emplace(w.b, uniq.size()).second) uniq.push_back(w.b);
    std::vector<gkr_felt> roots(uniq.size());
    TRY(gkr_weight_commitments(c, uniq.data(), uniq.size(), roots.data()));
    for (const auto& w : claims) {
      proof->weight_commitments.push_back(felt_canon_from_words(roots[at[w.b]].w));
      claim_roots.push_back(roots[at[w.b]]);
    }
  }
  if (mode == GKR_WEIGHT_AGGREGATED_FULL) {  // groups of BINDING_GROUP_SIZE claims (prover.rs:1276-1300)
    constexpr size_t kGroup = 4;
    for (size_t g0 = 0; g0 < claims.size(); g0 += kGroup) {
      const size_t ng = std::min(kGroup, claims.size() - g0);
      std::vector<gkr_binding_claim> bc(ng);
      for (size_t i = 0; i < ng; i++) {
        const WeightClaimRec& w = claims[g0 + i];
        bc[i].weight = w.b;
        bc[i].eval_point = reinterpret_cast<const gkr_qm31*>(w.point.data());
        bc[i].n_point = (uint32_t)w.point.size();
        bc[i].expected_value = G(w.value);
        bc[i].commitment = claim_roots[g0 + i];
      }
      size_t n = 0;
      const int rc = gkr_prove_aggregated_binding(c, ch, bc.data(), ng, nullptr, 0, &n);
      if (rc != GKR_ERR_BUFFER) return rc == GKR_OK ? fail(GKR_ERR_INVALID, "binding proof size") : rc;
      std::vector<gkr_felt> out(n);
      TRY(gkr_prove_aggregated_binding(c, ch, bc.data(), ng, out.data(), n, &n));
      proof->binding_groups.push_back(std::move(out));
    }
    claims.clear();
    return GKR_OK;
  }
  PoseidonChannel& C = ch->ch;
  const qm31 rho = C.draw_qm31();
  qm31 pw = qm31_one(), combined = qm31_zero();
  for (const auto& w : claims) {
    combined = qm31_add(combined, qm31_mul(pw, w.value));
    pw = qm31_mul(pw, rho);
  }
  C.mix_secure_field(combined);
  claims.clear();
  return GKR_OK;
}


extern "C" size_t gkr_proof_num_binding_groups(const gkr_proof* p) { return p ? p->binding_groups.size() : 0; }
extern "C" int gkr_proof_binding_group(const gkr_proof* p, size_t g, gkr_felt* out, size_t cap, size_t* n_felts) {
  if (!p || !n_felts || (!out && cap)) return fail(GKR_ERR_INVALID, "null argument");
  if (g >= p->binding_groups.size()) return fail(GKR_ERR_INVALID, "binding group %zu of %zu", g, p->binding_groups.size());
  const auto& v = p->binding_groups[g];
  *n_felts = v.size();
  if (cap < v.size()) return fail(GKR_ERR_BUFFER, "need %zu felts, have %zu", v.size(), cap);
  std::copy(v.begin(), v.end(), out);
  return GKR_OK;
}
