/* Mul layer (element-wise product) eq-sumcheck, restated from
 * engine/src/gkr/prover.rs:6162-6271 (reduce_mul_layer) with the helpers
 * compute_mul_eq_sum_at_t (9236-9270), fold_mle (9424-9430) and
 * build_eq_evals (9201-9233).  TEST INFRASTRUCTURE ONLY. */
#include "oracle_internal.h"

static qm mul_sum_at_t(const qm* eq, const qm* a, const qm* b, size_t mid, qm t) {
  qm omt = q_sub(q_one(), t);
  qm sum = q_zero();
  for (size_t i = 0; i < mid; i++) {
    qm et = q_add(q_mul(omt, eq[i]), q_mul(t, eq[mid + i]));
    qm at = q_add(q_mul(omt, a[i]), q_mul(t, a[mid + i]));
    qm bt = q_add(q_mul(omt, b[i]), q_mul(t, b[mid + i]));
    sum = q_add(sum, q_mul(q_mul(et, at), bt));
  }
  return sum;
}
static void fold(qm* v, qm r, size_t mid) {
  qm omr = q_sub(q_one(), r);
  for (size_t i = 0; i < mid; i++) v[i] = q_add(q_mul(omr, v[i]), q_mul(r, v[mid + i]));
}
static void mix_qv(orc_channel* ch, qm v) {
  uint32_t w[4];
  q_store(w, v);
  orc_mix_secure_field(ch, w);
}
static qm draw_qv(orc_channel* ch) {
  uint32_t w[4];
  orc_draw_qm31(ch, w);
  return q_load(w);
}

/* lhs, rhs: n QM31 each (n a power of two); claim_point has n_point >= log2 n
 * entries.  Outputs: eq_round_polys 4 x log2 n QM31 (c0..c3), lhs_eval,
 * rhs_eval, the combiner alpha and the next claim value
 * alpha * lhs + (1 - alpha) * rhs (the next claim point is claim_point). */
int orc_reduce_mul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                         const uint32_t* lhs, const uint32_t* rhs, size_t n, orc_channel* ch,
                         uint32_t* eq_round_polys, uint32_t* lhs_eval, uint32_t* rhs_eval, uint32_t* alpha_out,
                         uint32_t* next_value) {
  if (n == 0 || (n & (n - 1))) return 1;
  int nv = 0;
  while (((size_t)1 << nv) < n) nv++;
  if (n_point < nv) return 2;
  qm* eq = (qm*)malloc(n * sizeof(qm));
  qm* fa = (qm*)malloc(n * sizeof(qm));
  qm* fb = (qm*)malloc(n * sizeof(qm));
  mle_eq_evals((const qm*)claim_point, nv, eq);
  for (size_t i = 0; i < n; i++) {
    fa[i] = q_load(lhs + 4 * i);
    fb[i] = q_load(rhs + 4 * i);
  }
  orc_mix_u64(ch, 0x4D554Cull);
  mix_qv(ch, q_load(claim_value));
  const qm two = q_from_m31(2), three = q_from_m31(3);
  const qm inv2 = q_inv(two), inv6 = q_inv(q_from_m31(6));
  size_t cur = n;
  for (int t = 0; t < nv; t++) {
    size_t mid = cur / 2;
    qm s0 = mul_sum_at_t(eq, fa, fb, mid, q_zero());
    qm s1 = mul_sum_at_t(eq, fa, fb, mid, q_one());
    qm s2 = mul_sum_at_t(eq, fa, fb, mid, two);
    qm s3 = mul_sum_at_t(eq, fa, fb, mid, three);
    qm d1 = q_sub(s1, s0);
    qm d2 = q_mul(q_add(q_sub(q_sub(s2, s1), s1), s0), inv2);
    qm d3 = q_mul(q_sub(q_sub(s3, s0), q_mul(three, q_sub(s2, s1))), inv6);
    qm c[4] = {s0, q_add(q_sub(d1, d2), q_mul(two, d3)), q_sub(d2, q_mul(three, d3)), d3};
    for (int k = 0; k < 4; k++) q_store(eq_round_polys + 16 * t + 4 * k, c[k]);
    orc_mix_poly_coeffs_deg3(ch, eq_round_polys + 16 * t);
    qm r = draw_qv(ch);
    fold(eq, r, mid);
    fold(fa, r, mid);
    fold(fb, r, mid);
    cur = mid;
  }
  qm le = fa[0], re = fb[0];
  free(eq); free(fa); free(fb);
  orc_trace(ch, "mul.eq", -1);
  mix_qv(ch, le);
  mix_qv(ch, re);
  qm alpha = draw_qv(ch);
  orc_trace(ch, "mul", -1);
  qm comb = q_add(q_mul(alpha, le), q_mul(q_sub(q_one(), alpha), re));
  q_store(lhs_eval, le);
  q_store(rhs_eval, re);
  q_store(alpha_out, alpha);
  q_store(next_value, comb);
  return 0;
}
