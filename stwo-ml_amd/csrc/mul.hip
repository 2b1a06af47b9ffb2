// Element-wise Mul layer (reduce_mul_layer, gkr/prover.rs:6172-6271).
#include "internal.h"
// ------------------------------------------------------------------ Mul layer
// reduce_mul_layer (gkr/prover.rs:6172-6271) over the padded QM31 MLEs held in
// S_W0 (lhs) and S_D0 (rhs), n = 2^nv entries each.
static int mul_layer_core(gkr_ctx* c, const std::vector<qm31>& cpt, const qm31& claim, int nv, gkr_channel* ch,
                          gkr_proof* proof, gkr_mul_out* out) {
  const uint64_t n = 1ull << nv;
  qm31 *d_w0, *d_w1, *d_d0, *d_d1;
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_W1, n / 2 + 1, &d_w1));
  TRY(ensureT(c, S_D0, n, &d_d0));
  TRY(ensureT(c, S_D1, n / 2 + 1, &d_d1));
  TraceScope trace;
  PoseidonChannel& C = ch->ch;
  Eq3Plan epl;  // eq over the first nv claim coordinates, kept factored
  TRY(eq3_prepare(c, cpt.data(), nv, &epl));
  C.mix_u64(0x4D554Cull);  // "MUL"
  C.mix_secure_field(claim);
  std::vector<qm31> chal(nv);
  qm31 fin[3];
  TRY(eq3_sumcheck(c, C, cpt.data(), epl, d_w0, d_d0, d_w1, d_d1, out->eq_round_polys, chal.data(), fin));
  trace_point(C, "mul.eq");
  const qm31 lhs = fin[1], rhs = fin[2];
  C.mix_secure_field(lhs);
  C.mix_secure_field(rhs);
  const qm31 alpha = C.draw_qm31();
  trace_point(C, "mul");
  const qm31 comb = qm31_add(qm31_mul(alpha, lhs), qm31_mul(qm31_sub(qm31_one(), alpha), rhs));
  out->lhs_eval = G(lhs);
  out->rhs_eval = G(rhs);
  out->alpha = G(alpha);
  out->next_value = G(comb);
  out->n_vars = (uint32_t)nv;
  if (proof) {
    LayerRec L;
    L.tag = 2;
    L.claim_value = claim;
    L.rp.resize(4 * (size_t)nv);
    for (size_t i = 0; i < L.rp.size(); i++) L.rp[i] = Q(out->eq_round_polys[i]);
    L.final_a = lhs;
    L.final_b = rhs;
    proof_add_layer(proof, std::move(L));
  }
  return GKR_OK;
}
static int mul_check_claim(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value, int nv,
                           gkr_mul_out* out, std::vector<qm31>* cpt) {
  if (!claim_value || !out || (!claim_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (nv > kMaxVars) return fail(GKR_ERR_INVALID, "mul layer too large");
  if ((int)n_point < nv) return fail(GKR_ERR_INVALID, "claim point too short for MLE size (%u < %d)", n_point, nv);
  if (!out->eq_round_polys && nv > 0) return fail(GKR_ERR_INVALID, "null eq_round_polys");
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  cpt->resize(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(claim_point[l])) return fail(GKR_ERR_INVALID, "claim point not canonical");
    (*cpt)[l] = Q(claim_point[l]);
  }
  return GKR_OK;
}
// Padded QM31 MLEs of two resident matrices into S_W0 / S_D0; returns nv.
static int mul_stage_matrices(gkr_ctx* c, const gkr_matrix* lhs, const gkr_matrix* rhs, int* nv_out) {
  if (!lhs || !rhs) return fail(GKR_ERR_INVALID, "null matrix");
  if (lhs->ctx != c || rhs->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another context");
  const uint64_t nl = next_pow2(lhs->rows) * next_pow2(lhs->cols);
  const uint64_t nr = next_pow2(rhs->rows) * next_pow2(rhs->cols);
  if (nl != nr) return fail(GKR_ERR_INVALID, "lhs and rhs must have same length (%llu vs %llu)",
                            (unsigned long long)nl, (unsigned long long)nr);
  const int nv = log2_exact(nl);
  if (nv > kMaxVars) return fail(GKR_ERR_INVALID, "mul layer too large");
  qm31 *d_w0, *d_d0;
  TRY(ensureT(c, S_W0, nl, &d_w0));
  TRY(ensureT(c, S_D0, nl, &d_d0));
  GKR_LAUNCH(c, k_pad_q, dim3(grid_for(nl)), dim3(kBlock), 0, lhs->dev, lhs->rows, lhs->cols,
                     log2_exact(next_pow2(lhs->cols)), nl, d_w0);
  TRY(check_launch(c));
  GKR_LAUNCH(c, k_pad_q, dim3(grid_for(nl)), dim3(kBlock), 0, rhs->dev, rhs->rows, rhs->cols,
                     log2_exact(next_pow2(rhs->cols)), nl, d_d0);
  TRY(check_launch(c));
  *nv_out = nv;
  return GKR_OK;
}

extern "C" int gkr_prove_mul_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                   const gkr_qm31* claim_value, const gkr_matrix* lhs, const gkr_matrix* rhs,
                                   gkr_channel* ch, gkr_proof* proof, gkr_mul_out* out) {
  CH_CHECK(ch);
  if (!c) return fail(GKR_ERR_INVALID, "null context");
  HIP_TRY(hipSetDevice(c->device));
  int nv = 0;
  TRY(mul_stage_matrices(c, lhs, rhs, &nv));
  std::vector<qm31> cpt;
  TRY(mul_check_claim(claim_point, n_point, claim_value, nv, out, &cpt));
  c->mm.valid = false;
  return mul_layer_core(c, cpt, Q(*claim_value), nv, ch, proof, out);
}

extern "C" int gkr_reduce_mul_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                    const gkr_qm31* claim_value, const gkr_qm31* lhs_vals, const gkr_qm31* rhs_vals,
                                    uint64_t n, gkr_channel* ch, gkr_proof* proof, gkr_mul_out* out) {
  CH_CHECK(ch);
  if (!c || !lhs_vals || !rhs_vals) return fail(GKR_ERR_INVALID, "null argument");
  if (n == 0 || (n & (n - 1))) return fail(GKR_ERR_INVALID, "MLE size must be power of 2 (got %llu)",
                                          (unsigned long long)n);
  const int nv = log2_exact(n);
  std::vector<qm31> cpt;
  TRY(mul_check_claim(claim_point, n_point, claim_value, nv, out, &cpt));
  for (uint64_t i = 0; i < n; i++)
    if (!canonical_q(lhs_vals[i]) || !canonical_q(rhs_vals[i]))
      return fail(GKR_ERR_INVALID, "MLE value %llu not canonical", (unsigned long long)i);
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  qm31 *d_w0, *d_d0;
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_D0, n, &d_d0));
  HIP_TRY(hipMemcpyAsync(d_w0, lhs_vals, n * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(d_d0, rhs_vals, n * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
  return mul_layer_core(c, cpt, Q(*claim_value), nv, ch, proof, out);
}

// MLE of lhs (.) rhs (padded) at `point`: sum_x eq(point, x) lhs(x) rhs(x),
// one eq-weighted pass (a trip of no rounds; eq as a product of two tables).
extern "C" int gkr_mul_output_claim(gkr_ctx* c, const gkr_matrix* lhs, const gkr_matrix* rhs,
                                    const gkr_qm31* point, uint32_t n_point, gkr_qm31* out) {
  if (!c || !out || (!point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(c->device));
  int nv = 0;
  TRY(mul_stage_matrices(c, lhs, rhs, &nv));
  if ((int)n_point != nv) return fail(GKR_ERR_INVALID, "point has %u vars, product MLE has %d", n_point, nv);
  std::vector<qm31> pt(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(point[l])) return fail(GKR_ERR_INVALID, "point not canonical");
    pt[l] = Q(point[l]);
  }
  c->mm.valid = false;
  const uint64_t n = 1ull << nv;
  qm31 *d_w0, *d_d0;
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_D0, n, &d_d0));
  const int h = nv < kEqLoMax ? nv : kEqLoMax;
  EqPartsArg arg;
  memset(&arg, 0, sizeof arg);
  arg.z = make_point(pt.data(), nv);
  arg.count = 2;
  arg.s[0] = 0;
  arg.m[0] = nv - h;
  arg.off[0] = 0;
  arg.s[1] = nv - h;
  arg.m[1] = h;
  arg.off[1] = 1u << (nv - h);
  const uint32_t total = arg.off[1] + (1u << h);
  qm31* parts;
  TRY(ensureT(c, S_EQPARTS, total, &parts));
  Posted ps;
  memset(&ps, 0, sizeof ps);
  GKR_LAUNCH(c, k_eq_parts, dim3(grid_for(kEqLanes * (uint64_t)total)), dim3(kBlock), 0, arg, total, parts, ps);
  TRY(check_launch(c));
  RoundSink sk;
  TRY(launch_trip(c, 1, 0, d_w0, d_d0, n, 0, nullptr, nullptr, nullptr, parts, parts + arg.off[1], h, 0, &sk));
  qm31 v[1];
  TRY(wait_trip(c, sk, 1, v));
  *out = G(v[0]);
  return GKR_OK;
}

