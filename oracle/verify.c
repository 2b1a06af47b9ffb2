/* Verifier replay of the matmul and LogUp activation layers, restated from
 * engine/src/gkr/verifier.rs:2675-2788 (verify_matmul_reduction),
 * 3058-3290 (verify_activation_reduction, LogUp branch), 5791-5798
 * (compute_eq_eval) and 5818-5842 (verify_multiplicity_sumcheck).
 * Round polynomials arrive compressed as in the serialized proof (c1
 * omitted) and c1 is rebuilt from the running sum
 * (components/matmul.rs:1031-1039, gkr/types.rs:94-103).
 * Returns 0 on acceptance, a positive step number on rejection.
 * TEST INFRASTRUCTURE ONLY. */
#include "oracle_internal.h"

static size_t next_pow2(size_t v) {
  size_t p = 1;
  while (p < v) p <<= 1;
  return p;
}
static int ilog2(size_t v) {
  int l = 0;
  while (((size_t)1 << l) < v) l++;
  return l;
}
static void mix_q(orc_channel* ch, qm v) {
  uint32_t w[4];
  q_store(w, v);
  orc_mix_secure_field(ch, w);
}
static qm draw_q(orc_channel* ch) {
  uint32_t w[4];
  orc_draw_qm31(ch, w);
  return q_load(w);
}

int orc_verify_matmul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value, size_t m,
                            size_t k, size_t n, const uint32_t* c0c2, int n_rounds, const uint32_t* final_a,
                            const uint32_t* final_b, orc_channel* ch, uint32_t* next_point, uint32_t* next_value) {
  const int log_m = ilog2(next_pow2(m)), log_k = ilog2(next_pow2(k)), log_n = ilog2(next_pow2(n));
  if (n_rounds != log_k) return 1;
  if (n_point < log_m + log_n) return 2;
  orc_mix_u64(ch, m);
  orc_mix_u64(ch, k);
  orc_mix_u64(ch, n);
  orc_mix_secure_field(ch, claim_value);
  qm sum = q_load(claim_value);
  qm* chal = (qm*)malloc((size_t)(log_k + 1) * sizeof(qm));
  for (int t = 0; t < n_rounds; t++) {
    qm c0 = q_load(c0c2 + 8 * t), c2 = q_load(c0c2 + 8 * t + 4);
    /* p(0) + p(1) = 2 c0 + c1 + c2 = sum  =>  c1 = sum - 2 c0 - c2 */
    qm c1 = q_sub(q_sub(q_sub(sum, c0), c0), c2);
    uint32_t cw[12];
    q_store(cw, c0);
    q_store(cw + 4, c1);
    q_store(cw + 8, c2);
    orc_mix_poly_coeffs(ch, cw);
    qm r = draw_q(ch);
    chal[t] = r;
    sum = q_add(q_add(c0, q_mul(c1, r)), q_mul(q_mul(c2, r), r));
  }
  qm fa = q_load(final_a), fb = q_load(final_b);
  if (!q_eq(sum, q_mul(fa, fb))) {
    free(chal);
    return 3;
  }
  mix_q(ch, fa);
  mix_q(ch, fb);
  if (next_point) {
    memcpy(next_point, claim_point, (size_t)log_m * 16);
    for (int t = 0; t < log_k; t++) q_store(next_point + 4 * (log_m + t), chal[t]);
  }
  if (next_value) q_store(next_value, fa);
  free(chal);
  return 0;
}

int orc_verify_activation_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                                uint32_t tag, uint32_t table_log, const uint32_t* claimed_sum,
                                const uint32_t* c0c2c3, int n_rounds, const uint32_t* final_evals,
                                const uint32_t* multiplicities, const uint32_t* mult_round_polys,
                                const uint32_t* mult_final, const uint32_t* mult_sum, const uint32_t* input_eval,
                                orc_channel* ch) {
  if (n_rounds == 0) return 1;
  if (n_point < n_rounds) return 2;
  orc_mix_u64(ch, 0x4C4F47ull);
  orc_mix_u64(ch, tag);
  qm gamma = draw_q(ch), beta = draw_q(ch);
  /* LogUp table-side sum over multiplicities */
  const size_t tsize = (size_t)1 << table_log;
  qm table_sum = q_zero();
  for (size_t j = 0; j < tsize; j++) {
    if (!multiplicities[j]) continue;
    qm d = q_sub(q_sub(gamma, q_from_m31(m31_from((uint32_t)j))),
                 q_mul(beta, q_from_m31(orc_activation(tag, (uint32_t)j))));
    table_sum = q_add(table_sum, q_mul(q_from_m31(m31_from(multiplicities[j])), q_inv(d)));
  }
  qm cs = q_load(claimed_sum);
  if (!q_eq(cs, table_sum)) return 3;
  mix_q(ch, cs);
  qm sum = q_one();
  qm* chal = (qm*)malloc((size_t)n_rounds * sizeof(qm));
  for (int t = 0; t < n_rounds; t++) {
    qm c0 = q_load(c0c2c3 + 12 * t), c2 = q_load(c0c2c3 + 12 * t + 4), c3 = q_load(c0c2c3 + 12 * t + 8);
    qm c1 = q_sub(q_sub(q_sub(q_sub(sum, c0), c0), c2), c3);
    uint32_t cw[16];
    q_store(cw, c0);
    q_store(cw + 4, c1);
    q_store(cw + 8, c2);
    q_store(cw + 12, c3);
    orc_mix_poly_coeffs_deg3(ch, cw);
    qm r = draw_q(ch);
    chal[t] = r;
    qm r2 = q_mul(r, r);
    sum = q_add(q_add(c0, q_mul(c1, r)), q_add(q_mul(c2, r2), q_mul(c3, q_mul(r2, r))));
  }
  qm w_eval = q_load(final_evals), in_s = q_load(final_evals + 4), out_s = q_load(final_evals + 8);
  qm d_eval = q_sub(q_sub(gamma, in_s), q_mul(beta, out_s));
  qm eq = q_one();
  const qm* r = (const qm*)claim_point;
  for (int t = 0; t < n_rounds; t++) {
    qm a = r[t], b = chal[t];
    eq = q_mul(eq, q_add(q_mul(q_sub(q_one(), a), q_sub(q_one(), b)), q_mul(a, b)));
  }
  free(chal);
  if (!q_eq(sum, q_mul(q_mul(eq, w_eval), d_eval))) return 4;
  /* multiplicity sumcheck chain */
  qm msum = q_load(mult_sum);
  for (uint32_t t = 0; t < table_log; t++) {
    qm c0 = q_load(mult_round_polys + 8 * t), c1 = q_load(mult_round_polys + 8 * t + 4);
    if (!q_eq(q_add(c0, q_add(c0, c1)), msum)) return 5;
    mix_q(ch, c0);
    mix_q(ch, c1);
    qm rr = draw_q(ch);
    msum = q_add(c0, q_mul(c1, rr));
  }
  if (!q_eq(msum, q_load(mult_final))) return 6;
  orc_mix_secure_field(ch, input_eval);
  orc_mix_secure_field(ch, claim_value);
  return 0;
}

/* verify_mul_reduction (verifier.rs:2963-3045): transcript replay, the final
 * check sum == eq(r, s) * lhs * rhs, then the combiner draw. */
int orc_verify_mul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                         const uint32_t* c0c2c3, int n_rounds, const uint32_t* lhs_eval, const uint32_t* rhs_eval,
                         orc_channel* ch, uint32_t* next_value) {
  if (n_point < n_rounds) return 1;
  orc_mix_u64(ch, 0x4D554Cull);
  orc_mix_secure_field(ch, claim_value);
  qm sum = q_load(claim_value);
  qm eq = q_one();
  const qm* r = (const qm*)claim_point;
  for (int t = 0; t < n_rounds; t++) {
    qm c0 = q_load(c0c2c3 + 12 * t), c2 = q_load(c0c2c3 + 12 * t + 4), c3 = q_load(c0c2c3 + 12 * t + 8);
    qm c1 = q_sub(q_sub(q_sub(q_sub(sum, c0), c0), c2), c3);
    uint32_t cw[16];
    q_store(cw, c0);
    q_store(cw + 4, c1);
    q_store(cw + 8, c2);
    q_store(cw + 12, c3);
    orc_mix_poly_coeffs_deg3(ch, cw);
    qm s = draw_q(ch);
    qm s2 = q_mul(s, s);
    sum = q_add(q_add(c0, q_mul(c1, s)), q_add(q_mul(c2, s2), q_mul(c3, q_mul(s2, s))));
    eq = q_mul(eq, q_add(q_mul(q_sub(q_one(), r[t]), q_sub(q_one(), s)), q_mul(r[t], s)));
  }
  qm le = q_load(lhs_eval), re = q_load(rhs_eval);
  if (!q_eq(sum, q_mul(q_mul(eq, le), re))) return 2;
  mix_q(ch, le);
  mix_q(ch, re);
  qm alpha = draw_q(ch);
  q_store(next_value, q_add(q_mul(alpha, le), q_mul(q_sub(q_one(), alpha), re)));
  return 0;
}
