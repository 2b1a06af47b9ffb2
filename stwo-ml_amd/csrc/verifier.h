// Verifier replay of the GKR layer reductions, on the host.
//
// Restated from engine/src/gkr/verifier.rs: verify_matmul_reduction
// (2675-2788), verify_mul_reduction (2963-3045), the LogUp branch of
// verify_activation_reduction (3058-3290), verify_multiplicity_sumcheck
// (5818-5842) and compute_eq_eval (5791-5798).  Each check replays the
// prover's transcript on the caller's channel and returns the claim on the
// layer's input.  A failed check returns false with the reason in `why`.
#pragma once
#include <stdint.h>
#include <stdio.h>

#include <string>
#include <vector>

#include "activations.h"
#include "field.h"
#include "poseidon.h"
#include "trace.h"

namespace gkr {

struct VerifyError {
  std::string why;
};

// p(r) for coefficients c[0..deg] (Horner).
inline qm31 poly_eval(const qm31* c, int deg, const qm31& r) {
  qm31 acc = c[deg];
  for (int i = deg - 1; i >= 0; i--) acc = qm31_add(qm31_mul(acc, r), c[i]);
  return acc;
}

// prod_l ((1 - a_l)(1 - b_l) + a_l b_l)
inline qm31 eq_eval(const qm31* a, const qm31* b, size_t n) {
  qm31 acc = qm31_one();
  for (size_t l = 0; l < n; l++) {
    const qm31 t = qm31_add(qm31_mul(qm31_sub(qm31_one(), a[l]), qm31_sub(qm31_one(), b[l])), qm31_mul(a[l], b[l]));
    acc = qm31_mul(acc, t);
  }
  return acc;
}

inline std::string q_str(const qm31& x) {
  char b[64];
  snprintf(b, sizeof b, "(%u,%u,%u,%u)", x.a, x.b, x.c, x.d);
  return b;
}

static inline uint64_t v_next_pow2(uint64_t v) {
  uint64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}
static inline int v_log2(uint64_t v) {
  int l = 0;
  while ((1ull << l) < v) l++;
  return l;
}

// Round polynomials arrive either in full or compressed as serialized
// (cairo_serde.rs: c1 omitted); a compressed c1 is rebuilt from the running
// sum, c1 = sum - 2 c0 - c2 (- c3), as the reference's calldata verifier does
// (components/matmul.rs:1031-1039, gkr/types.rs:94-103).

// verify_matmul_reduction.  polys: (c0, c1, c2) per round.
inline bool verify_matmul(const std::vector<qm31>& point, const qm31& value, uint64_t m, uint64_t k, uint64_t n,
                          const std::vector<qm31>& polys, const qm31& final_a, const qm31& final_b, PoseidonChannel& ch,
                          std::vector<qm31>* next_point, qm31* next_value, VerifyError* err, bool compressed = false) {
  const int log_m = v_log2(v_next_pow2(m)), log_k = v_log2(v_next_pow2(k)), log_n = v_log2(v_next_pow2(n));
  const size_t rounds = polys.size() / 3;
  if ((int)rounds != log_k) {
    err->why = "expected " + std::to_string(log_k) + " sumcheck rounds, got " + std::to_string(rounds);
    return false;
  }
  if ((int)point.size() < log_m + log_n) {
    err->why = "output claim point too short";
    return false;
  }
  ch.mix_u64(m);
  ch.mix_u64(k);
  ch.mix_u64(n);
  ch.mix_secure_field(value);
  qm31 sum = value;
  std::vector<qm31> chal;
  for (size_t t = 0; t < rounds; t++) {
    qm31 c[3] = {polys[3 * t], polys[3 * t + 1], polys[3 * t + 2]};
    if (compressed) c[1] = qm31_sub(qm31_sub(qm31_sub(sum, c[0]), c[0]), c[2]);
    const qm31 p01 = qm31_add(c[0], qm31_add(qm31_add(c[0], c[1]), c[2]));
    if (!qm31_eq(p01, sum)) {
      err->why = "round " + std::to_string(t) + ": p(0)+p(1) = " + q_str(p01) + " != claimed sum " + q_str(sum);
      return false;
    }
    ch.mix_poly_coeffs(c[0], c[1], c[2]);
    const qm31 r = ch.draw_qm31();
    chal.push_back(r);
    sum = poly_eval(c, 2, r);
  }
  const qm31 prod = qm31_mul(final_a, final_b);
  if (!qm31_eq(sum, prod)) {
    err->why = "final eval check failed: sum=" + q_str(sum) + " != a*b=" + q_str(prod);
    return false;
  }
  trace_point(ch, "matmul.rounds");
  ch.mix_secure_field(final_a);
  ch.mix_secure_field(final_b);
  trace_point(ch, "matmul");
  next_point->assign(point.begin(), point.begin() + log_m);
  next_point->insert(next_point->end(), chal.begin(), chal.end());
  *next_value = final_a;
  return true;
}

// verify_mul_reduction.  polys: (c0, c1, c2, c3) per round.
inline bool verify_mul(const std::vector<qm31>& point, const qm31& value, const std::vector<qm31>& polys,
                       const qm31& lhs, const qm31& rhs, PoseidonChannel& ch, qm31* next_value, VerifyError* err,
                       bool compressed = false) {
  const size_t nv = polys.size() / 4;
  if (point.size() < nv) {
    err->why = "mul: claim point has " + std::to_string(point.size()) + " vars, need at least " + std::to_string(nv);
    return false;
  }
  ch.mix_u64(0x4D554Cull);
  ch.mix_secure_field(value);
  qm31 sum = value;
  std::vector<qm31> chal;
  for (size_t t = 0; t < nv; t++) {
    qm31 c[4] = {polys[4 * t], polys[4 * t + 1], polys[4 * t + 2], polys[4 * t + 3]};
    if (compressed) c[1] = qm31_sub(qm31_sub(qm31_sub(qm31_sub(sum, c[0]), c[0]), c[2]), c[3]);
    const qm31 p01 = qm31_add(c[0], qm31_add(qm31_add(qm31_add(c[0], c[1]), c[2]), c[3]));
    if (!qm31_eq(p01, sum)) {
      err->why = "mul round " + std::to_string(t) + ": p(0)+p(1) = " + q_str(p01) + " != claimed sum " + q_str(sum);
      return false;
    }
    ch.mix_poly_coeffs_deg3(c[0], c[1], c[2], c[3]);
    const qm31 r = ch.draw_qm31();
    chal.push_back(r);
    sum = poly_eval(c, 3, r);
  }
  const qm31 expected = qm31_mul(qm31_mul(eq_eval(point.data(), chal.data(), nv), lhs), rhs);
  if (!qm31_eq(sum, expected)) {
    err->why = "mul final check failed: sum=" + q_str(sum) + " != eq*a*b=" + q_str(expected);
    return false;
  }
  trace_point(ch, "mul.eq");
  ch.mix_secure_field(lhs);
  ch.mix_secure_field(rhs);
  const qm31 alpha = ch.draw_qm31();
  trace_point(ch, "mul");
  *next_value = qm31_add(qm31_mul(alpha, lhs), qm31_mul(qm31_sub(qm31_one(), alpha), rhs));
  return true;
}

// The proof fields of the LogUp activation reduction.
struct LogUpProofIn {
  qm31 claimed_sum;
  std::vector<qm31> eq_polys;  // (c0, c1, c2, c3) per round
  qm31 w_eval, in_eval, out_eval;
  std::vector<uint32_t> mults;
  std::vector<qm31> mult_polys;  // (c0, c1) per round
  qm31 mult_final, mult_sum;
  qm31 input_eval, output_eval;
  felt table_commitment;  // canonical (not Montgomery)
};

// verify_activation_reduction, LogUp branch (with its multiplicity
// sumcheck).  The reference additionally refuses LogUp-only proofs of
// non-ReLU activations unless STWO_ALLOW_LOGUP_ACTIVATION is set; this
// replay corresponds to that setting.  table: the activation's outputs.
inline bool verify_activation(const std::vector<qm31>& point, uint32_t tag, uint32_t table_log,
                              const std::vector<uint32_t>& table, const LogUpProofIn& p, PoseidonChannel& ch,
                              qm31* next_value, VerifyError* err, bool compressed = false) {
  const size_t nv = p.eq_polys.size() / 4;
  if (nv == 0) {
    err->why = "activation eq-sumcheck has 0 rounds";
    return false;
  }
  if (point.size() < nv) {
    err->why = "activation: claim point has " + std::to_string(point.size()) + " vars, need at least " +
               std::to_string(nv);
    return false;
  }
  ch.mix_u64(0x4C4F47ull);
  ch.mix_u64(tag);
  const qm31 gamma = ch.draw_qm31();
  const qm31 beta = ch.draw_qm31();
  trace_point(ch, "logup.gamma_beta");
  felt tc_in[2] = {felt_from_u64(tag), felt_from_u64(table_log)};
  const felt expected_tc = felt_from_mont(poseidon_hash_many(tc_in, 2));
  if (!felt_eq(expected_tc, p.table_commitment)) {
    err->why = "activation table commitment mismatch";
    return false;
  }
  const uint64_t tsize = 1ull << table_log;
  if (p.mults.size() != tsize) {
    err->why = "multiplicities length " + std::to_string(p.mults.size()) + " != table size " + std::to_string(tsize);
    return false;
  }
  qm31 table_sum = qm31_zero();
  for (uint64_t j = 0; j < tsize; j++) {
    if (p.mults[j] == 0) continue;
    const qm31 d = qm31_sub(qm31_sub(gamma, qm31_from_m31(m31_from_u32((uint32_t)j))),
                            qm31_mul(beta, qm31_from_m31(table[j])));
    table_sum = qm31_add(table_sum, qm31_mul(qm31_from_m31(m31_from_u32(p.mults[j])), qm31_inv(d)));
  }
  if (!qm31_eq(p.claimed_sum, table_sum)) {
    err->why = "LogUp sum mismatch: claimed=" + q_str(p.claimed_sum) + ", table=" + q_str(table_sum);
    return false;
  }
  ch.mix_secure_field(p.claimed_sum);
  qm31 sum = qm31_one();
  std::vector<qm31> chal;
  for (size_t t = 0; t < nv; t++) {
    qm31 c[4] = {p.eq_polys[4 * t], p.eq_polys[4 * t + 1], p.eq_polys[4 * t + 2], p.eq_polys[4 * t + 3]};
    if (compressed) c[1] = qm31_sub(qm31_sub(qm31_sub(qm31_sub(sum, c[0]), c[0]), c[2]), c[3]);
    const qm31 p01 = qm31_add(c[0], qm31_add(qm31_add(qm31_add(c[0], c[1]), c[2]), c[3]));
    if (!qm31_eq(p01, sum)) {
      err->why = "activation eq-sumcheck round " + std::to_string(t) + ": p(0)+p(1) = " + q_str(p01) +
                 " != sum " + q_str(sum);
      return false;
    }
    ch.mix_poly_coeffs_deg3(c[0], c[1], c[2], c[3]);
    const qm31 r = ch.draw_qm31();
    chal.push_back(r);
    sum = poly_eval(c, 3, r);
  }
  const qm31 d_eval = qm31_sub(qm31_sub(gamma, p.in_eval), qm31_mul(beta, p.out_eval));
  const qm31 expected = qm31_mul(qm31_mul(eq_eval(point.data(), chal.data(), nv), p.w_eval), d_eval);
  if (!qm31_eq(sum, expected)) {
    err->why = "activation final check failed: sum=" + q_str(sum) + " != eq*w*d=" + q_str(expected);
    return false;
  }
  trace_point(ch, "logup.eq");
  // verify_multiplicity_sumcheck
  qm31 msum = p.mult_sum;
  for (size_t t = 0; t < p.mult_polys.size() / 2; t++) {
    const qm31 c0 = p.mult_polys[2 * t], c1 = p.mult_polys[2 * t + 1];
    if (!qm31_eq(qm31_add(c0, qm31_add(c0, c1)), msum)) {
      err->why = "multiplicity sumcheck round check failed";
      return false;
    }
    ch.mix_secure_field(c0);
    ch.mix_secure_field(c1);
    const qm31 r = ch.draw_qm31();
    msum = qm31_add(c0, qm31_mul(c1, r));
  }
  if (!qm31_eq(msum, p.mult_final)) {
    err->why = "multiplicity sumcheck final eval mismatch";
    return false;
  }
  trace_point(ch, "logup.mult");
  ch.mix_secure_field(p.input_eval);
  ch.mix_secure_field(p.output_eval);
  trace_point(ch, "logup");
  *next_value = p.input_eval;
  return true;
}

// A LayerNorm / RMSNorm layer proof (types.rs LayerProof::LayerNorm /
// RMSNorm) with full round polynomials (c0..c3 per round).  RMSNorm keeps
// rms^2 in key_eval, the square sum in sum0, the Part 0 final input in
// p0_final0, the per-row rms^2 in rows0; has_mult is false when the format
// carries no multiplicity sumcheck (serialize_gkr_model_proof's RMSNorm).
struct NormProofIn {
  qm31 input_eval, output_eval, key_eval /* LN mean, RMS rms^2 */, rsqrt_eval, var_eval;
  uint64_t n_active = 0;
  qm31 sum0, sum1;
  std::vector<qm31> p0, lin;
  qm31 p0_final0, p0_final1, lin_final0, lin_final1, cb_input, cb_mean;
  LogUpProofIn lu;  // claimed_sum, eq_polys, w/in/out evals, mults, mult_polys, mult_final/sum, table_commitment
  bool has_mult = true;
  std::vector<uint32_t> rows0, rows1;
};

inline uint32_t norm_inv_or_zero(uint64_t n) { return n ? m31_inv(m31_from_u32((uint32_t)(n % P))) : 0u; }
inline qm31 norm_row_mle(const std::vector<uint32_t>& v, int log_rows, const qm31* s) {
  qm31 acc = qm31_zero();
  for (size_t r = 0; r < v.size(); r++) {
    qm31 e = qm31_one();
    for (int k = 0; k < log_rows; k++) e = qm31_mul(e, ((r >> (log_rows - 1 - k)) & 1) ? s[k] : qm31_sub(qm31_one(), s[k]));
    acc = qm31_add(acc, qm31_mul(e, qm31_from_m31(v[r])));
  }
  return acc;
}
// p(0) + p(1) = sum per round, mix, draw; the challenges and the final sum.
inline bool norm_rounds(const std::vector<qm31>& polys, qm31* sum, PoseidonChannel& ch, std::vector<qm31>* chal,
                        const char* what, VerifyError* err, bool compressed) {
  for (size_t t = 0; t < polys.size() / 4; t++) {
    qm31 c[4] = {polys[4 * t], polys[4 * t + 1], polys[4 * t + 2], polys[4 * t + 3]};
    if (compressed) c[1] = qm31_sub(qm31_sub(qm31_sub(qm31_sub(*sum, c[0]), c[0]), c[2]), c[3]);
    const qm31 p01 = qm31_add(c[0], qm31_add(qm31_add(qm31_add(c[0], c[1]), c[2]), c[3]));
    if (!qm31_eq(p01, *sum)) {
      err->why = std::string(what) + " round " + std::to_string(t) + ": p(0)+p(1) = " + q_str(p01) + " != sum " +
                 q_str(*sum);
      return false;
    }
    ch.mix_poly_coeffs_deg3(c[0], c[1], c[2], c[3]);
    const qm31 r = ch.draw_qm31();
    if (chal) chal->push_back(r);
    *sum = poly_eval(c, 3, r);
  }
  return true;
}

// verify_layernorm_reduction (verifier.rs:4153-4690) and verify_rmsnorm_reduction
// (4693-5076), non-SIMD, with the Part 0 proof present.  The multi-row
// LayerNorm variance binding is the reference's: the row variances weighted at
// the mean-variance challenges must equal var_eval at the claim point, which
// holds when every row has the same variance.
inline bool verify_norm(bool ln, const std::vector<qm31>& point, const qm31& value, uint64_t dim, const NormProofIn& p,
                        const std::vector<uint32_t>& rsqrt_table, PoseidonChannel& ch, qm31* next_value,
                        VerifyError* err, bool compressed = false) {
  const char* name = ln ? "layernorm" : "rmsnorm";
  const size_t nv = p.lin.size() / 4;
  if (nv == 0) {
    err->why = std::string(name) + " linear eq-sumcheck has 0 rounds";
    return false;
  }
  if (point.size() < nv) {
    err->why = std::string(name) + ": claim point too short";
    return false;
  }
  if (p.lu.eq_polys.size() / 4 != nv || p.p0.size() / 4 != nv) {
    err->why = std::string(name) + ": part 0 / LogUp round counts differ from the linear sumcheck";
    return false;
  }
  const uint64_t total = 1ull << nv;
  const uint64_t n_active = dim < total ? dim : total;
  const uint64_t cols_padded = v_next_pow2(dim);
  const uint64_t rows = total / cols_padded;
  const int log_rows = (int)nv - v_log2(cols_padded);
  // Part 0
  std::vector<qm31> mv;
  qm31 sum;
  if (ln) {
    ch.mix_u64(0x4D56ull);
    ch.mix_u64(n_active);
    ch.mix_secure_field(p.sum0);
    ch.mix_secure_field(p.sum1);
    const qm31 eta0 = ch.draw_qm31(), eta1 = qm31_mul(eta0, eta0);
    sum = qm31_add(qm31_mul(eta0, p.sum0), qm31_mul(eta1, p.sum1));
    if (!norm_rounds(p.p0, &sum, ch, &mv, "layernorm mean-variance", err, compressed)) return false;
    ch.mix_secure_field(p.p0_final0);
    ch.mix_secure_field(p.p0_final1);
    const qm31 cf = qm31_sub(p.p0_final0, p.p0_final1);
    if (!qm31_eq(sum, qm31_add(qm31_mul(eta0, p.p0_final0), qm31_mul(eta1, qm31_sqr(cf))))) {
      err->why = "layernorm mean-variance final check failed";
      return false;
    }
    if (rows == 1) {
      const uint32_t inv_n = norm_inv_or_zero(n_active);
      if (m31_mul(p.sum0.a, inv_n) != p.key_eval.a) {
        err->why = "layernorm mean derivation mismatch";
        return false;
      }
      if (n_active == cols_padded && (m31_mul(p.sum1.a, inv_n) & 0xFFFFu) != p.var_eval.a) {
        err->why = "layernorm variance derivation mismatch";
        return false;
      }
    } else {
      if (p.rows0.size() != rows || p.rows1.size() != rows) {
        err->why = "layernorm row statistics length differs from " + std::to_string(rows) + " rows";
        return false;
      }
      if (!qm31_eq(p.p0_final1, norm_row_mle(p.rows0, log_rows, mv.data()))) {
        err->why = "layernorm multi-row mean binding failed";
        return false;
      }
      if (!qm31_eq(p.var_eval, norm_row_mle(p.rows1, log_rows, mv.data()))) {
        err->why = "layernorm multi-row variance binding failed";
        return false;
      }
    }
  } else {
    ch.mix_u64(0x5251ull);
    ch.mix_u64(n_active);
    ch.mix_secure_field(p.sum0);
    sum = p.sum0;
    if (!norm_rounds(p.p0, &sum, ch, nullptr, "rmsnorm RMS^2", err, compressed)) return false;
    ch.mix_secure_field(p.p0_final0);
    if (!qm31_eq(qm31_sqr(p.p0_final0), sum)) {
      err->why = "rmsnorm RMS^2 final check failed";
      return false;
    }
    if (rows == 1) {
      if ((m31_mul(p.sum0.a, norm_inv_or_zero(n_active)) & 0xFFFFu) != p.key_eval.a) {
        err->why = "rmsnorm RMS^2 derivation mismatch";
        return false;
      }
    } else {
      if (p.rows0.size() != rows) {
        err->why = "rmsnorm row_rms_sq length differs from " + std::to_string(rows) + " rows";
        return false;
      }
      if (!qm31_eq(p.key_eval, norm_row_mle(p.rows0, log_rows, point.data()))) {
        err->why = "rmsnorm multi-row rms_sq binding failed";
        return false;
      }
    }
  }
  // Part 1
  ch.mix_u64(ln ? 0x4C4Eull : 0x524Eull);
  ch.mix_secure_field(p.key_eval);
  ch.mix_secure_field(p.rsqrt_eval);
  ch.mix_secure_field(value);
  sum = value;
  std::vector<qm31> chal;
  if (!norm_rounds(p.lin, &sum, ch, &chal, ln ? "layernorm linear" : "rmsnorm linear", err, compressed)) return false;
  if (!qm31_eq(sum, qm31_mul(qm31_mul(eq_eval(point.data(), chal.data(), nv), p.lin_final0), p.lin_final1))) {
    err->why = std::string(name) + " linear final check failed";
    return false;
  }
  ch.mix_secure_field(p.lin_final0);
  ch.mix_secure_field(p.lin_final1);
  if (ln) {
    ch.mix_secure_field(p.cb_input);
    ch.mix_secure_field(p.cb_mean);
    if (!qm31_eq(p.lin_final0, qm31_sub(p.cb_input, p.cb_mean))) {
      err->why = "layernorm centered binding failed";
      return false;
    }
  }
  // Part 2: rsqrt LogUp
  ch.mix_u64(0x4C4F47ull);
  ch.mix_u64(ln ? 0x5253ull : 0x524Eull);
  const qm31 gamma = ch.draw_qm31(), beta = ch.draw_qm31();
  felt tc_in[2] = {felt_from_u64(0x5253), felt_from_u64(16)};
  if (!felt_eq(felt_from_mont(poseidon_hash_many(tc_in, 2)), p.lu.table_commitment)) {
    err->why = std::string(name) + " rsqrt table commitment mismatch";
    return false;
  }
  if (p.lu.mults.size() != rsqrt_table.size()) {
    err->why = std::string(name) + " rsqrt multiplicities length " + std::to_string(p.lu.mults.size());
    return false;
  }
  qm31 table_sum = qm31_zero();
  for (size_t j = 0; j < rsqrt_table.size(); j++) {
    if (!p.lu.mults[j]) continue;
    const qm31 d = qm31_sub(qm31_sub(gamma, qm31_from_m31((uint32_t)j)), qm31_mul(beta, qm31_from_m31(rsqrt_table[j])));
    table_sum = qm31_add(table_sum, qm31_mul(qm31_from_m31(m31_from_u32(p.lu.mults[j])), qm31_inv(d)));
  }
  if (!qm31_eq(p.lu.claimed_sum, table_sum)) {
    err->why = std::string(name) + " rsqrt LogUp sum mismatch";
    return false;
  }
  ch.mix_secure_field(p.lu.claimed_sum);
  sum = qm31_one();
  std::vector<qm31> lchal;
  if (!norm_rounds(p.lu.eq_polys, &sum, ch, &lchal, ln ? "layernorm LogUp" : "rmsnorm LogUp", err, compressed))
    return false;
  const qm31 d_eval = qm31_sub(qm31_sub(gamma, p.lu.in_eval), qm31_mul(beta, p.lu.out_eval));
  if (!qm31_eq(sum, qm31_mul(qm31_mul(eq_eval(point.data(), lchal.data(), nv), p.lu.w_eval), d_eval))) {
    err->why = std::string(name) + " LogUp final check failed";
    return false;
  }
  if (p.has_mult) {  // verify_multiplicity_sumcheck
    qm31 msum = p.lu.mult_sum;
    for (size_t t = 0; t < p.lu.mult_polys.size() / 2; t++) {
      const qm31 c0 = p.lu.mult_polys[2 * t], c1 = p.lu.mult_polys[2 * t + 1];
      if (!qm31_eq(qm31_add(c0, qm31_add(c0, c1)), msum)) {
        err->why = "multiplicity sumcheck round check failed";
        return false;
      }
      ch.mix_secure_field(c0);
      ch.mix_secure_field(c1);
      msum = qm31_add(c0, qm31_mul(c1, ch.draw_qm31()));
    }
    if (!qm31_eq(msum, p.lu.mult_final)) {
      err->why = "multiplicity sumcheck final eval mismatch";
      return false;
    }
  }
  ch.mix_secure_field(p.input_eval);
  ch.mix_secure_field(p.output_eval);
  trace_point(ch, name);
  *next_value = p.input_eval;
  return true;
}

// Reader of serialize_gkr_model_proof calldata (felt252 words).
struct FeltReader {
  const uint32_t* w;  // 8 words per felt
  size_t n, pos = 0;
  bool ok = true;
  std::string why;
  bool take(const uint32_t** f) {
    if (pos >= n) {
      ok = false;
      why = "calldata ends early at felt " + std::to_string(pos);
      return false;
    }
    *f = w + 8 * pos++;
    return true;
  }
  uint64_t u(uint64_t max = ~0ull) {
    const uint32_t* f;
    if (!take(&f)) return 0;
    for (int i = 2; i < 8; i++)
      if (f[i]) {
        ok = false;
        why = "felt " + std::to_string(pos - 1) + " is not a small integer";
        return 0;
      }
    const uint64_t v = (uint64_t)f[0] | ((uint64_t)f[1] << 32);
    if (v > max) {
      ok = false;
      why = "felt " + std::to_string(pos - 1) + " out of range";
      return 0;
    }
    return v;
  }
  uint32_t m31() {
    const uint64_t v = u((1ull << 31) - 2);
    return (uint32_t)v;
  }
  qm31 q() {
    const uint32_t a = m31(), b = m31(), c = m31(), d = m31();
    return qm31{a, b, c, d};
  }
  felt f() {
    const uint32_t* x;
    if (!take(&x)) return felt{{0, 0, 0, 0}};
    return felt_canon_from_words(x);
  }
};

}  // namespace gkr
