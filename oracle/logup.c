/* LogUp activation layer, restated from engine/src/gkr/prover.rs:6400-6600
 * (+ helpers 9236-9270, 9424-9511, 8365-8373), the activation functions of
 * engine/src/gadgets/lookup_table.rs:192-342 and the type tags of
 * engine/src/components/activation.rs:63-71.  TEST INFRASTRUCTURE ONLY. */
#include <math.h>

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

/* ---------------------------------------------------------------- activations */
static const uint64_t AP = (1ull << 31) - 1;
static const uint32_t HALF_P = (1u << 30) - 1;
static double signed_real(uint32_t val) {
  return val <= HALF_P ? (double)val / 65536.0 : -((double)(AP - val)) / 65536.0;
}
static uint32_t fixed_point(double y) {
  if (y >= 0.0) {
    uint64_t r = (uint64_t)round(y * 65536.0);
    return (uint32_t)(r < AP - 1 ? r : AP - 1);
  }
  uint64_t neg = (uint64_t)round(-y * 65536.0);
  if (neg > AP - 1) neg = AP - 1;
  return (uint32_t)(AP - neg);
}
uint32_t orc_activation(uint32_t tag, uint32_t v) {
  uint32_t r;
  switch (tag) {
    case 1: /* relu */
      r = v <= HALF_P ? v : 0;
      break;
    case 2: { /* gelu_approx */
      if (v == 0) return 0;
      double x = signed_real(v);
      double inner = sqrt(2.0 / M_PI) * (x + 0.044715 * x * x * x);
      r = fixed_point(0.5 * x * (1.0 + tanh(inner)));
      break;
    }
    case 3: /* sigmoid_approx */
      r = v > HALF_P ? 0 : (v == 0 ? 32768u : 65536u);
      break;
    case 4: { /* softmax_exp */
      if (v > HALF_P) {
        uint32_t neg = ((1u << 31) - 2) - v;
        uint32_t decay = neg / 65536u;
        if (decay > 20) decay = 20;
        uint32_t res = 65536u >> decay;
        r = res > 1 ? res : 1;
      } else if (v == 0) {
        r = 65536u;
      } else {
        uint32_t growth = v / 65536u;
        if (growth > 10) growth = 10;
        uint64_t res = (uint64_t)65536u << growth;
        r = (uint32_t)(res < (1ull << 31) - 2 ? res : (1ull << 31) - 2);
      }
      break;
    }
    default: { /* silu_approx */
      if (v == 0) return 0;
      double x = signed_real(v);
      r = fixed_point(x / (1.0 + exp(-x)));
      break;
    }
  }
  return m31_from(r);
}

/* compute_mul_eq_sum_at_t (prover.rs:9236-9270) */
static qm mul_eq_sum_at_t(const qm* eq, const qm* a, const qm* b, size_t mid, qm t) {
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
/* fold_mle (prover.rs:9424-9430) */
static void fold_mle(qm* v, qm r, size_t mid) {
  qm omr = q_sub(q_one(), r);
  for (size_t i = 0; i < mid; i++) v[i] = q_add(q_mul(omr, v[i]), q_mul(r, v[mid + i]));
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

int orc_prove_activation_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                               const uint32_t* X, size_t rows, size_t cols, uint32_t tag, uint32_t table_log,
                               orc_channel* ch, uint32_t* claimed_sum, uint32_t* eq_round_polys,
                               uint32_t* final_evals, uint32_t* multiplicities, uint32_t* mult_round_polys,
                               uint32_t* mult_final, uint32_t* mult_sum, uint32_t* input_eval,
                               uint32_t* table_commitment) {
  const size_t prow = next_pow2(rows), pcol = next_pow2(cols), n = prow * pcol;
  const int nv = ilog2(n);
  if (n_point != nv) return 1;
  const qm* point = (const qm*)claim_point;
  /* pad + matrix_to_mle + evaluate_mle(input, claim.point) (6411-6417) */
  qm* input_mle = (qm*)calloc(n, sizeof(qm));
  uint32_t* padded = (uint32_t*)calloc(n, sizeof(uint32_t));
  for (size_t i = 0; i < rows; i++)
    for (size_t j = 0; j < cols; j++) padded[i * pcol + j] = X[i * cols + j];
  for (size_t p = 0; p < n; p++) input_mle[p] = q_from_m31(padded[p]);
  qm in_eval_claim = mle_evaluate(input_mle, nv, point);
  free(input_mle);

  /* table (PrecomputedTable::build_parallel) + masking + lookups (6423-6443) */
  const size_t tsize = (size_t)1 << table_log;
  const uint32_t mask = (uint32_t)(tsize - 1);
  uint32_t* table = (uint32_t*)malloc(tsize * sizeof(uint32_t));
  for (size_t j = 0; j < tsize; j++) table[j] = orc_activation(tag, (uint32_t)j);
  qm* masked_in = (qm*)malloc(n * sizeof(qm));
  qm* masked_out = (qm*)malloc(n * sizeof(qm));
  memset(multiplicities, 0, tsize * sizeof(uint32_t));
  for (size_t p = 0; p < n; p++) {
    uint32_t mi = padded[p] & mask;
    masked_in[p] = q_from_m31(mi);
    masked_out[p] = q_from_m31(table[mi]);
    multiplicities[mi]++; /* compute_multiplicities (activation.rs:211-221) */
  }
  free(padded);

  /* Fiat-Shamir (6451-6454) */
  orc_mix_u64(ch, 0x4C4F47ull);
  orc_mix_u64(ch, tag);
  qm gamma = draw_q(ch);
  qm beta = draw_q(ch);
  orc_trace(ch, "logup.gamma_beta", -1);
  /* d_i = gamma - in_i - beta out_i; w = batch_inverse(d) (6457-6464) */
  qm* d = (qm*)malloc(n * sizeof(qm));
  qm* w = (qm*)malloc(n * sizeof(qm));
  for (size_t p = 0; p < n; p++) d[p] = q_sub(q_sub(gamma, masked_in[p]), q_mul(beta, masked_out[p]));
  q_batch_inverse(d, w, n);
  qm trace_sum = q_zero();
  for (size_t p = 0; p < n; p++) trace_sum = q_add(trace_sum, w[p]);
  /* table side (6470-6486) */
  size_t nz = 0;
  for (size_t j = 0; j < tsize; j++) nz += multiplicities[j] > 0;
  qm* td = (qm*)malloc((nz ? nz : 1) * sizeof(qm));
  qm* tinv = (qm*)malloc((nz ? nz : 1) * sizeof(qm));
  size_t* tj = (size_t*)malloc((nz ? nz : 1) * sizeof(size_t));
  size_t q = 0;
  for (size_t j = 0; j < tsize; j++)
    if (multiplicities[j] > 0) {
      td[q] = q_sub(q_sub(gamma, q_from_m31(m31_from((uint32_t)j))), q_mul(beta, q_from_m31(table[j])));
      tj[q++] = j;
    }
  q_batch_inverse(td, tinv, nz);
  qm table_sum = q_zero();
  for (size_t i = 0; i < nz; i++) table_sum = q_add(table_sum, q_mul(q_from_m31(m31_from(multiplicities[tj[i]])), tinv[i]));
  free(td);
  free(tinv);
  free(tj);
  free(table);
  if (!q_eq(trace_sum, table_sum)) {
    free(masked_in); free(masked_out); free(d); free(w);
    return 2;
  }
  mix_q(ch, trace_sum);
  q_store(claimed_sum, trace_sum);

  /* eq-sumcheck rounds (6501-6556) */
  qm* eq = (qm*)malloc(n * sizeof(qm));
  mle_eq_evals(point, nv, eq);
  qm* chal = (qm*)malloc((size_t)(nv ? nv : 1) * sizeof(qm));
  const qm two = q_from_m31(2), three = q_from_m31(3);
  const qm inv2 = q_inv(two), inv6 = q_inv(q_from_m31(6));
  size_t cur_n = n;
  for (int t = 0; t < nv; t++) {
    size_t mid = cur_n / 2;
    qm s0 = mul_eq_sum_at_t(eq, w, d, mid, q_zero());
    qm s1 = mul_eq_sum_at_t(eq, w, d, mid, q_one());
    qm s2 = mul_eq_sum_at_t(eq, w, d, mid, two);
    qm s3 = mul_eq_sum_at_t(eq, w, d, mid, three);
    qm dd1 = q_sub(s1, s0);
    qm dd2 = q_mul(q_add(q_sub(q_sub(s2, s1), s1), s0), inv2);
    qm dd3 = q_mul(q_sub(q_sub(s3, s0), q_mul(three, q_sub(s2, s1))), inv6);
    qm c[4] = {s0, q_add(q_sub(dd1, dd2), q_mul(two, dd3)), q_sub(dd2, q_mul(three, dd3)), dd3};
    for (int k = 0; k < 4; k++) q_store(eq_round_polys + 16 * t + 4 * k, c[k]);
    orc_mix_poly_coeffs_deg3(ch, eq_round_polys + 16 * t);
    qm r = draw_q(ch);
    chal[t] = r;
    fold_mle(eq, r, mid);
    fold_mle(w, r, mid);
    fold_mle(d, r, mid);
    cur_n = mid;
  }
  orc_trace(ch, "logup.eq", -1);
  qm w_eval = w[0];
  qm in_eval_s = mle_evaluate(masked_in, nv, chal);
  qm out_eval_s = mle_evaluate(masked_out, nv, chal);
  q_store(final_evals, w_eval);
  q_store(final_evals + 4, in_eval_s);
  q_store(final_evals + 8, out_eval_s);
  free(eq); free(w); free(d); free(masked_in); free(masked_out); free(chal);

  /* build_multiplicity_sumcheck (9449-9511) */
  qm* vals = (qm*)malloc(tsize * sizeof(qm));
  for (size_t j = 0; j < tsize; j++) vals[j] = q_from_m31(m31_from(multiplicities[j]));
  qm msum = q_zero();
  for (size_t j = 0; j < tsize; j++) msum = q_add(msum, vals[j]);
  size_t cur = tsize;
  for (uint32_t t = 0; t < table_log; t++) {
    size_t half = cur / 2;
    qm lo = q_zero(), hi = q_zero();
    for (size_t i = 0; i < half; i++) lo = q_add(lo, vals[i]);
    for (size_t i = half; i < cur; i++) hi = q_add(hi, vals[i]);
    qm c0 = lo, c1 = q_sub(hi, lo);
    q_store(mult_round_polys + 8 * t, c0);
    q_store(mult_round_polys + 8 * t + 4, c1);
    mix_q(ch, c0);
    mix_q(ch, c1);
    qm r = draw_q(ch);
    qm omr = q_sub(q_one(), r);
    for (size_t i = 0; i < half; i++) vals[i] = q_add(q_mul(omr, vals[i]), q_mul(r, vals[i + half]));
    cur = half;
  }
  orc_trace(ch, "logup.mult", -1);
  q_store(mult_final, vals[0]);
  q_store(mult_sum, msum);
  free(vals);

  /* compute_activation_table_commitment (8365-8373) */
  uint32_t tc_in[16] = {0};
  tc_in[0] = tag;
  tc_in[8] = table_log;
  orc_hash_many(tc_in, 2, table_commitment);
  /* final mixes (6578-6579) */
  mix_q(ch, in_eval_claim);
  orc_mix_secure_field(ch, claim_value);
  orc_trace(ch, "logup", -1);
  q_store(input_eval, in_eval_claim);
  return 0;
}
