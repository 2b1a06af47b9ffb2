// Host verifier replay of layer reductions and serialized walks
// (engine/src/gkr/verifier.rs).
#include "internal.h"
#include "activations.h"
#include "norm.h"
#include "verifier.h"
// ------------------------------------------------------------------ verifier replay
static bool read_point(const gkr_qm31* p, uint32_t n, std::vector<qm31>* out) {
  out->resize(n);
  for (uint32_t l = 0; l < n; l++) {
    if (!canonical_q(p[l])) return false;
    (*out)[l] = Q(p[l]);
  }
  return true;
}
static int verify_fail(const VerifyError& e) { return fail(GKR_ERR_VERIFY, "%s", e.why.c_str()); }

extern "C" int gkr_verify_matmul_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                                       uint64_t m, uint64_t k, uint64_t n, const gkr_qm31* round_polys,
                                       uint32_t n_rounds, const gkr_qm31* final_a, const gkr_qm31* final_b,
                                       gkr_channel* ch, gkr_qm31* next_point, uint32_t* n_next,
                                       gkr_qm31* next_value) {
  CH_CHECK(ch);
  TraceScope trace;
  if (!claim_value || !final_a || !final_b || !next_point || !n_next || !next_value ||
      (!claim_point && n_point) || (!round_polys && n_rounds))
    return fail(GKR_ERR_INVALID, "null argument");
  if (m == 0 || k == 0 || n == 0) return fail(GKR_ERR_INVALID, "empty dimension");
  std::vector<qm31> pt, polys(3 * (size_t)n_rounds);
  if (!read_point(claim_point, n_point, &pt)) return fail(GKR_ERR_INVALID, "claim point not canonical");
  for (size_t i = 0; i < polys.size(); i++) {
    if (!canonical_q(round_polys[i])) return fail(GKR_ERR_INVALID, "round polynomial not canonical");
    polys[i] = Q(round_polys[i]);
  }
  std::vector<qm31> np;
  qm31 nv;
  VerifyError e;
  if (!verify_matmul(pt, Q(*claim_value), m, k, n, polys, Q(*final_a), Q(*final_b), ch->ch, &np, &nv, &e))
    return verify_fail(e);
  for (size_t l = 0; l < np.size(); l++) next_point[l] = G(np[l]);
  *n_next = (uint32_t)np.size();
  *next_value = G(nv);
  return GKR_OK;
}

extern "C" int gkr_verify_mul_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                                    const gkr_qm31* eq_round_polys, uint32_t n_rounds, const gkr_qm31* lhs_eval,
                                    const gkr_qm31* rhs_eval, gkr_channel* ch, gkr_qm31* next_value) {
  CH_CHECK(ch);
  TraceScope trace;
  if (!claim_value || !lhs_eval || !rhs_eval || !next_value || (!claim_point && n_point) ||
      (!eq_round_polys && n_rounds))
    return fail(GKR_ERR_INVALID, "null argument");
  std::vector<qm31> pt, polys(4 * (size_t)n_rounds);
  if (!read_point(claim_point, n_point, &pt)) return fail(GKR_ERR_INVALID, "claim point not canonical");
  for (size_t i = 0; i < polys.size(); i++) polys[i] = Q(eq_round_polys[i]);
  qm31 nv;
  VerifyError e;
  if (!verify_mul(pt, Q(*claim_value), polys, Q(*lhs_eval), Q(*rhs_eval), ch->ch, &nv, &e)) return verify_fail(e);
  *next_value = G(nv);
  return GKR_OK;
}

static const std::vector<uint32_t>& verifier_table(uint32_t tag, uint32_t log) {
  static std::mutex mu;
  static std::map<uint64_t, std::vector<uint32_t>> tables;
  std::lock_guard<std::mutex> lock(mu);
  const uint64_t key = ((uint64_t)tag << 32) | log;
  auto it = tables.find(key);
  if (it == tables.end()) it = tables.emplace(key, act_table(tag, log)).first;
  return it->second;
}

extern "C" int gkr_verify_activation_layer(const gkr_qm31* claim_point, uint32_t n_point, uint32_t activation_type,
                                           uint32_t table_log_size, uint32_t n_eq_rounds, const gkr_logup_out* proof,
                                           gkr_channel* ch, gkr_qm31* next_value) {
  CH_CHECK(ch);
  TraceScope trace;
  if (!proof || !next_value || (!claim_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (!act_valid(activation_type)) return fail(GKR_ERR_INVALID, "unknown activation type %u", activation_type);
  if (!act_logup_valid(activation_type))
    return fail(GKR_ERR_INVALID, "activation type %u (ReLU) is proved algebraically, not by LogUp", activation_type);
  if (table_log_size == 0) table_log_size = act_default_log_size(activation_type);
  if (table_log_size > 24) return fail(GKR_ERR_INVALID, "table_log_size %u too large", table_log_size);
  if ((n_eq_rounds && !proof->eq_round_polys) || !proof->multiplicities || !proof->mult_round_polys)
    return fail(GKR_ERR_INVALID, "null proof arrays");
  std::vector<qm31> pt;
  if (!read_point(claim_point, n_point, &pt)) return fail(GKR_ERR_INVALID, "claim point not canonical");
  LogUpProofIn p;
  p.claimed_sum = Q(proof->claimed_sum);
  for (uint32_t i = 0; i < 4 * n_eq_rounds; i++) p.eq_polys.push_back(Q(proof->eq_round_polys[i]));
  p.w_eval = Q(proof->w_eval);
  p.in_eval = Q(proof->in_eval);
  p.out_eval = Q(proof->out_eval);
  p.mults.assign(proof->multiplicities, proof->multiplicities + (1ull << table_log_size));
  for (uint32_t i = 0; i < 2 * table_log_size; i++) p.mult_polys.push_back(Q(proof->mult_round_polys[i]));
  p.mult_final = Q(proof->mult_final_eval);
  p.mult_sum = Q(proof->mult_claimed_sum);
  p.input_eval = Q(proof->input_eval);
  p.output_eval = Q(proof->output_eval);
  if (!felt_abi_canonical(proof->table_commitment)) return fail(GKR_ERR_INVALID, "table commitment not canonical");
  p.table_commitment = felt_canon_from_words(proof->table_commitment.w);
  qm31 nv;
  VerifyError e;
  if (!verify_activation(pt, activation_type, table_log_size, verifier_table(activation_type, table_log_size), p,
                         ch->ch, &nv, &e))
    return verify_fail(e);
  *next_value = G(nv);
  return GKR_OK;
}

static const std::vector<uint32_t>& rsqrt_table() {
  static const std::vector<uint32_t> t = [] {
    std::vector<uint32_t> v(1u << kNormTableLog);
    for (uint32_t j = 0; j < v.size(); j++) v[j] = norm_rsqrt(j);
    return v;
  }();
  return t;
}
static int verify_norm_abi(bool ln, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                           uint64_t dim, const gkr_norm_out* o, gkr_channel* ch, gkr_qm31* next_value) {
  CH_CHECK(ch);
  TraceScope trace;
  if (!o || !claim_value || !next_value || (!claim_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (!o->p0_round_polys || !o->lin_round_polys || !o->logup_round_polys || !o->multiplicities ||
      !o->mult_round_polys || (o->n_rows && (!o->row_stats0 || !o->row_stats1)))
    return fail(GKR_ERR_INVALID, "null proof arrays");
  std::vector<qm31> pt;
  if (!read_point(claim_point, n_point, &pt)) return fail(GKR_ERR_INVALID, "claim point not canonical");
  NormProofIn p;
  p.input_eval = Q(o->input_eval);
  p.output_eval = Q(o->output_eval);
  p.key_eval = Q(o->mean_eval);
  p.rsqrt_eval = Q(o->rsqrt_eval);
  p.var_eval = Q(o->var_eval);
  p.n_active = o->n_active;
  p.sum0 = Q(o->sum0);
  p.sum1 = Q(o->sum1);
  for (uint32_t i = 0; i < 4 * n_point; i++) {
    p.p0.push_back(Q(o->p0_round_polys[i]));
    p.lin.push_back(Q(o->lin_round_polys[i]));
    p.lu.eq_polys.push_back(Q(o->logup_round_polys[i]));
  }
  p.p0_final0 = Q(o->p0_final0);
  p.p0_final1 = Q(o->p0_final1);
  p.lin_final0 = Q(o->lin_final0);
  p.lin_final1 = Q(o->lin_final1);
  p.cb_input = Q(o->cb_input);
  p.cb_mean = Q(o->cb_mean);
  p.lu.claimed_sum = Q(o->claimed_sum);
  p.lu.w_eval = Q(o->w_eval);
  p.lu.in_eval = Q(o->in_eval);
  p.lu.out_eval = Q(o->out_eval);
  p.lu.mults.assign(o->multiplicities, o->multiplicities + (1u << kNormTableLog));
  for (uint32_t i = 0; i < 2 * kNormTableLog; i++) p.lu.mult_polys.push_back(Q(o->mult_round_polys[i]));
  p.lu.mult_final = Q(o->mult_final_eval);
  p.lu.mult_sum = Q(o->mult_claimed_sum);
  if (!felt_abi_canonical(o->table_commitment)) return fail(GKR_ERR_INVALID, "table commitment not canonical");
  p.lu.table_commitment = felt_canon_from_words(o->table_commitment.w);
  if (o->n_rows > 1) {  // per-row statistics are part of the proof only for several rows
    p.rows0.assign(o->row_stats0, o->row_stats0 + o->n_rows);
    p.rows1.assign(o->row_stats1, o->row_stats1 + o->n_rows);
  }
  qm31 nv;
  VerifyError e;
  if (!verify_norm(ln, pt, Q(*claim_value), dim, p, rsqrt_table(), ch->ch, &nv, &e)) return verify_fail(e);
  *next_value = G(nv);
  return GKR_OK;
}
extern "C" int gkr_verify_layernorm_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                                          uint64_t dim, const gkr_norm_out* proof, gkr_channel* ch,
                                          gkr_qm31* next_value) {
  return verify_norm_abi(true, claim_point, n_point, claim_value, dim, proof, ch, next_value);
}
extern "C" int gkr_verify_rmsnorm_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                                        uint64_t dim, const gkr_norm_out* proof, gkr_channel* ch,
                                        gkr_qm31* next_value) {
  return verify_norm_abi(false, claim_point, n_point, claim_value, dim, proof, ch, next_value);
}

// A chained walk from serialize_gkr_model_proof calldata: every layer's
// claim is the previous layer's input claim, starting from init_*.  Checks
// the layer proofs and the input-claim section; the weight commitments,
// openings and IO commitment that follow are not examined.
extern "C" int gkr_verify_walk(const gkr_felt* calldata, size_t n_felts, const gkr_layer_shape* layers,
                               size_t n_layers, const gkr_qm31* init_point, uint32_t n_init,
                               const gkr_qm31* init_value, const gkr_qm31* fresh_values, size_t n_fresh,
                               gkr_channel* ch, gkr_qm31* final_point, uint32_t* n_final, gkr_qm31* final_value,
                               size_t* n_consumed) {
  CH_CHECK(ch);
  TraceScope trace;
  if (!calldata || !layers || !final_point || !n_final || !final_value || (!init_point && n_init) ||
      (!fresh_values && n_fresh))
    return fail(GKR_ERR_INVALID, "null argument");
  if (n_layers && layers[0].claim != GKR_CLAIM_FRESH && !init_value)
    return fail(GKR_ERR_INVALID, "the first layer's claim is chained but no initial claim is given");
  std::vector<qm31> point;
  if (!read_point(init_point, n_init, &point)) return fail(GKR_ERR_INVALID, "initial point not canonical");
  qm31 value = init_value ? Q(*init_value) : qm31_zero();
  size_t fresh_used = 0;
  FeltReader R{reinterpret_cast<const uint32_t*>(calldata), n_felts};
  auto bad = [&](const std::string& why) { return fail(GKR_ERR_VERIFY, "%s", why.c_str()); };
  const uint64_t nl = R.u();
  if (!R.ok) return bad(R.why);
  if (nl != n_layers) return bad("proof has " + std::to_string(nl) + " layers, circuit " + std::to_string(n_layers));
  for (size_t li = 0; li < n_layers; li++) {
    const gkr_layer_shape& L = layers[li];
    const std::string at = "layer " + std::to_string(li) + ": ";
    const uint64_t tag = R.u();
    if (!R.ok) return bad(R.why);
    if (L.claim == GKR_CLAIM_FRESH) {  // the prover's fresh-claim rule (gkr_prove_walk)
      if (L.kind != GKR_STEP_MATMUL && L.kind != GKR_STEP_MUL && L.kind != GKR_STEP_ACTIVATION &&
          L.kind != GKR_STEP_LAYERNORM && L.kind != GKR_STEP_RMSNORM)
        return fail(GKR_ERR_INVALID, "layer %zu: unknown kind %u", li, L.kind);
      const uint64_t out_cols = L.kind == GKR_STEP_MATMUL ? L.cols_b : L.cols;
      const int nv = v_log2(v_next_pow2(L.rows)) + v_log2(v_next_pow2(out_cols));
      if (nv > 64) return fail(GKR_ERR_INVALID, "layer %zu: output claim of %d variables", li, nv);
      point.resize(nv);
      ch->ch.draw_qm31s(point.data(), (size_t)nv);
      if (L.kind == GKR_STEP_ACTIVATION) {
        value = ch->ch.draw_qm31();
      } else {
        if (fresh_used >= n_fresh) return fail(GKR_ERR_INVALID, "layer %zu: no fresh claim value left", li);
        if (!canonical_q(fresh_values[fresh_used])) return fail(GKR_ERR_INVALID, "fresh claim value not canonical");
        value = Q(fresh_values[fresh_used++]);
        ch->ch.mix_secure_field(value);
      }
    } else if (L.claim != GKR_CLAIM_CHAINED) {
      return fail(GKR_ERR_INVALID, "layer %zu: unknown claim rule %u", li, L.claim);
    }
    VerifyError e;
    if (L.kind == GKR_STEP_MATMUL) {
      if (tag != 0) return bad(at + "expected a MatMul proof (tag 0), found tag " + std::to_string(tag));
      const uint64_t nr = R.u(64);
      std::vector<qm31> polys;
      for (uint64_t t = 0; t < nr && R.ok; t++) {
        const qm31 c0 = R.q(), c2 = R.q();
        polys.push_back(c0);
        polys.push_back(qm31_zero());
        polys.push_back(c2);
      }
      const qm31 fa = R.q(), fb = R.q();
      if (!R.ok) return bad(at + R.why);
      std::vector<qm31> np;
      if (!verify_matmul(point, value, L.rows, L.cols, L.cols_b, polys, fa, fb, ch->ch, &np, &value, &e, true))
        return bad(at + e.why);
      point = np;
    } else if (L.kind == GKR_STEP_MUL) {
      if (tag != 2) return bad(at + "expected a Mul proof (tag 2), found tag " + std::to_string(tag));
      const uint64_t nr = R.u(64);
      std::vector<qm31> polys;
      for (uint64_t t = 0; t < nr && R.ok; t++) {
        const qm31 c0 = R.q(), c2 = R.q(), c3 = R.q();
        polys.push_back(c0);
        polys.push_back(qm31_zero());
        polys.push_back(c2);
        polys.push_back(c3);
      }
      const qm31 lhs = R.q(), rhs = R.q();
      if (!R.ok) return bad(at + R.why);
      if (nr != (uint64_t)v_log2(v_next_pow2(L.rows) * v_next_pow2(L.cols)))
        return bad(at + "Mul proof has " + std::to_string(nr) + " rounds for a " + std::to_string(L.rows) + " x " +
                   std::to_string(L.cols) + " operand");
      if (!verify_mul(point, value, polys, lhs, rhs, ch->ch, &value, &e, true)) return bad(at + e.why);
    } else if (L.kind == GKR_STEP_ACTIVATION) {
      if (tag != 3) return bad(at + "expected an Activation proof (tag 3), found tag " + std::to_string(tag));
      const uint32_t act = (uint32_t)R.u(0xFFFFFFFFull);
      if (R.ok && act != L.activation_type)
        return bad(at + "activation type " + std::to_string(act) + ", circuit " + std::to_string(L.activation_type));
      if (!act_valid(act)) return bad(at + "unknown activation type");
      if (!act_logup_valid(act)) return bad(at + "ReLU is proved algebraically, not by LogUp");
      const uint32_t tlog = L.table_log_size ? L.table_log_size : act_default_log_size(act);
      if (tlog > 24) return bad(at + "table size too large");
      LogUpProofIn p;
      p.input_eval = R.q();
      p.output_eval = R.q();
      p.table_commitment = R.f();
      if (R.u(1) != 1 || !R.ok) return bad(at + "activation proof without a LogUp proof");
      p.claimed_sum = R.q();
      const uint64_t nr = R.u(64);
      for (uint64_t t = 0; t < nr && R.ok; t++) {
        const qm31 c0 = R.q(), c2 = R.q(), c3 = R.q();
        p.eq_polys.push_back(c0);
        p.eq_polys.push_back(qm31_zero());
        p.eq_polys.push_back(c2);
        p.eq_polys.push_back(c3);
      }
      p.w_eval = R.q();
      p.in_eval = R.q();
      p.out_eval = R.q();
      const uint64_t nm = R.u(1ull << 24);
      for (uint64_t j = 0; j < nm && R.ok; j++) p.mults.push_back((uint32_t)R.u(0xFFFFFFFFull));
      if (R.u(1) != 1 || !R.ok) return bad(at + "activation proof without a multiplicity sumcheck");
      const uint64_t nmr = R.u(64);
      for (uint64_t t = 0; t < nmr && R.ok; t++) {
        p.mult_polys.push_back(R.q());
        p.mult_polys.push_back(R.q());
      }
      p.mult_final = R.q();
      p.mult_sum = R.q();
      const uint64_t has_prod = R.u(1), has_pw = R.u(1);
      if (!R.ok) return bad(at + R.why);
      if (has_prod || has_pw) return bad(at + "product / piecewise activation proofs are not supported");
      if (nr != (uint64_t)v_log2(v_next_pow2(L.rows) * v_next_pow2(L.cols)))
        return bad(at + "activation proof has " + std::to_string(nr) + " eq rounds for a " + std::to_string(L.rows) +
                   " x " + std::to_string(L.cols) + " input");
      if (nmr != tlog) return bad(at + "multiplicity sumcheck has " + std::to_string(nmr) + " rounds");
      if (!verify_activation(point, act, tlog, verifier_table(act, tlog), p, ch->ch, &value, &e, true))
        return bad(at + e.why);
    } else if (L.kind == GKR_STEP_LAYERNORM) {
      if (tag != 4) return bad(at + "expected a LayerNorm proof (tag 4), found tag " + std::to_string(tag));
      NormProofIn p;
      p.input_eval = R.q();
      p.output_eval = R.q();
      p.key_eval = R.q();
      p.rsqrt_eval = R.q();
      p.lu.table_commitment = R.f();
      if (R.u(1) != 0) return bad(at + "SIMD-combined LayerNorm proofs are not supported");
      if (R.u(1) != 1) return bad(at + "LayerNorm proof without the mean-variance part");
      p.n_active = R.u(0xFFFFFFFFull);
      p.sum0 = R.q();
      p.sum1 = R.q();
      auto rounds = [&](std::vector<qm31>* v) {
        const uint64_t nr = R.u(64);
        for (uint64_t t = 0; t < nr && R.ok; t++) {
          const qm31 c0 = R.q(), c2 = R.q(), c3 = R.q();
          v->insert(v->end(), {c0, qm31_zero(), c2, c3});
        }
      };
      rounds(&p.p0);
      p.p0_final0 = R.q();
      p.p0_final1 = R.q();
      rounds(&p.lin);
      p.lin_final0 = R.q();
      p.lin_final1 = R.q();
      p.cb_input = R.q();
      p.cb_mean = R.q();
      if (R.u(1) != 1) return bad(at + "LayerNorm proof without the rsqrt LogUp");
      p.lu.claimed_sum = R.q();
      rounds(&p.lu.eq_polys);
      p.lu.w_eval = R.q();
      p.lu.in_eval = R.q();
      p.lu.out_eval = R.q();
      const uint64_t nm = R.u(1ull << 24);
      for (uint64_t j = 0; j < nm && R.ok; j++) p.lu.mults.push_back((uint32_t)R.u(0xFFFFFFFFull));
      if (R.u(1) != 1) return bad(at + "LayerNorm proof without the multiplicity sumcheck");
      const uint64_t nmr = R.u(64);
      for (uint64_t t = 0; t < nmr && R.ok; t++) {
        p.lu.mult_polys.push_back(R.q());
        p.lu.mult_polys.push_back(R.q());
      }
      p.lu.mult_final = R.q();
      p.lu.mult_sum = R.q();
      p.var_eval = R.q();
      for (std::vector<uint32_t>* rv : {&p.rows0, &p.rows1})
        if (R.u(1)) {
          const uint64_t nr = R.u(1ull << 24);
          for (uint64_t i = 0; i < nr && R.ok; i++) rv->push_back((uint32_t)R.u(P - 1));
        }
      if (!R.ok) return bad(at + R.why);
      if (p.lin.size() / 4 != (uint64_t)v_log2(v_next_pow2(L.rows) * v_next_pow2(L.cols)))
        return bad(at + "LayerNorm proof has " + std::to_string(p.lin.size() / 4) + " rounds for a " +
                   std::to_string(L.rows) + " x " + std::to_string(L.cols) + " input");
      if (nmr != kNormTableLog) return bad(at + "multiplicity sumcheck has " + std::to_string(nmr) + " rounds");
      const uint64_t dim = L.dim ? L.dim : L.cols;
      if (!verify_norm(true, point, value, dim, p, rsqrt_table(), ch->ch, &value, &e, true)) return bad(at + e.why);
    } else if (L.kind == GKR_STEP_RMSNORM) {
      return bad(at + "RMSNorm proofs cannot be replayed from serialize_gkr_model_proof calldata: the format omits "
                      "their multiplicity sumcheck (cairo_serde.rs:1648-1720); use gkr_verify_rmsnorm_layer");
    } else {
      return fail(GKR_ERR_INVALID, "layer %zu: unknown kind %u", li, L.kind);
    }
    trace_point(ch->ch, "walk.step", (long)li);
  }
  // the input claim the proof states must be the one the walk arrived at
  const uint64_t npt = R.u(64);
  std::vector<qm31> ipt;
  for (uint64_t l = 0; l < npt && R.ok; l++) ipt.push_back(R.q());
  const qm31 ival = R.q();
  if (!R.ok) return bad(R.why);
  bool same = ipt.size() == point.size() && qm31_eq(ival, value);
  for (size_t l = 0; same && l < ipt.size(); l++) same = qm31_eq(ipt[l], point[l]);
  if (!same) return bad("input claim in the proof differs from the claim the walk reached");
  if (fresh_used != n_fresh)
    return fail(GKR_ERR_INVALID, "%zu fresh claim values given, the circuit uses %zu", n_fresh, fresh_used);
  if (point.size() > 64) return fail(GKR_ERR_BUFFER, "final claim has %zu variables", point.size());
  for (size_t l = 0; l < point.size(); l++) final_point[l] = G(point[l]);
  *n_final = (uint32_t)point.size();
  *final_value = G(value);
  if (n_consumed) *n_consumed = R.pos;
  return GKR_OK;
}

