/* LayerNorm and RMSNorm layer reducers and verifiers of the CPU oracle.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates engine/src/gkr/prover.rs:7944-8395 (reduce_layernorm_layer),
 * 8407-8801 (reduce_rmsnorm_layer_with_gamma), the sum helpers 9236-9330,
 * fold_mle 9424-9430 and build_multiplicity_sumcheck 9449-9511, the rsqrt
 * table engine/src/components/layernorm.rs:116-151 (shared by rmsnorm.rs:125),
 * and the verifiers engine/src/gkr/verifier.rs:4153-4690 (LayerNorm) and
 * 4693-5076 (RMSNorm) with verify_multiplicity_sumcheck 5818-5842. */
#include "oracle_internal.h"

#define NM_TABLE_LOG 16u /* LayerNormConfig / RMSNormConfig::new: rsqrt_table_log_size (layernorm.rs:41-47) */

static size_t nm_next_pow2(size_t v) {
  size_t p = 1;
  while (p < v) p <<= 1;
  return p;
}
static int nm_log2(size_t v) {
  int l = 0;
  while (((size_t)1 << l) < v) l++;
  return l;
}
static uint32_t madd(uint32_t a, uint32_t b) { return m31_reduce((uint64_t)a + b); }
static uint32_t msub(uint32_t a, uint32_t b) { return m31_reduce((uint64_t)a + ORC_P - b); }
static uint32_t mmul(uint32_t a, uint32_t b) { return m31_reduce((uint64_t)a * b); }
/* m31_mod_inverse (prover.rs:8378-8395): Fermat, 0 -> 0 */
static uint32_t m31_inv_fermat(uint32_t n) {
  if (n == 0) return 0;
  uint64_t result = 1, base = n % ORC_P, e = ORC_P - 2;
  while (e) {
    if (e & 1) result = result * base % ORC_P;
    base = base * base % ORC_P;
    e >>= 1;
  }
  return (uint32_t)result;
}

/* isqrt (layernorm.rs:139-151): floor(sqrt(n)) by Newton from 2^ceil(bits/2) */
static uint64_t nm_isqrt(uint64_t n) {
  if (n < 2) return n;
  const int bits = 64 - __builtin_clzll(n);
  uint64_t x = 1ull << ((bits + 1) / 2);
  for (;;) {
    const uint64_t x1 = (x + n / x) / 2;
    if (x1 >= x) return x;
    x = x1;
  }
}
/* build_rsqrt_table entry (layernorm.rs:116-135): 2^16 / isqrt(x), x = 0 -> 2^16 - 1 */
uint32_t orc_rsqrt(uint32_t v) {
  if (v == 0) return (1u << 16) - 1;
  const uint64_t s = nm_isqrt(v);
  if (s == 0) return (1u << 16) - 1;
  uint64_t r = (1ull << 16) / s;
  if (r > (1ull << 31) - 2) r = (1ull << 31) - 2;
  return m31_from((uint32_t)r);
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
/* compute_mul_eq_sum_at_t (prover.rs:9236-9270) */
static qm mul_eq_sum_at_t(const qm* eq, const qm* a, const qm* b, size_t mid, qm t) {
  const qm omt = q_sub(q_one(), t);
  qm sum = q_zero();
  for (size_t i = 0; i < mid; i++) {
    const qm et = q_add(q_mul(omt, eq[i]), q_mul(t, eq[mid + i]));
    const qm at = q_add(q_mul(omt, a[i]), q_mul(t, a[mid + i]));
    const qm bt = q_add(q_mul(omt, b[i]), q_mul(t, b[mid + i]));
    sum = q_add(sum, q_mul(q_mul(et, at), bt));
  }
  return sum;
}
/* compute_plain_sq_sum_at_t (prover.rs:9275-9289) */
static qm plain_sq_sum_at_t(const qm* a, size_t mid, qm t) {
  const qm omt = q_sub(q_one(), t);
  qm sum = q_zero();
  for (size_t j = 0; j < mid; j++) {
    const qm at = q_add(q_mul(omt, a[j]), q_mul(t, a[mid + j]));
    sum = q_add(sum, q_mul(at, at));
  }
  return sum;
}
/* compute_plain_mean_var_sum_at_t (prover.rs:9292-9310) */
static qm plain_mean_var_sum_at_t(const qm* in, const qm* c, qm eta0, qm eta1, size_t mid, qm t) {
  const qm omt = q_sub(q_one(), t);
  qm sum = q_zero();
  for (size_t j = 0; j < mid; j++) {
    const qm it = q_add(q_mul(omt, in[j]), q_mul(t, in[mid + j]));
    const qm ct = q_add(q_mul(omt, c[j]), q_mul(t, c[mid + j]));
    sum = q_add(sum, q_add(q_mul(eta0, it), q_mul(q_mul(eta1, ct), ct)));
  }
  return sum;
}
/* fold_mle (prover.rs:9424-9430) */
static void fold_mle(qm* v, qm r, size_t mid) {
  const qm omr = q_sub(q_one(), r);
  for (size_t i = 0; i < mid; i++) v[i] = q_add(q_mul(omr, v[i]), q_mul(r, v[mid + i]));
}
/* degree-2 Newton form from s0, s1, s2, with c3 = 0 (prover.rs:8074-8082) */
static void newton_deg2(qm s0, qm s1, qm s2, qm c[4]) {
  const qm inv2 = q_inv(q_from_m31(2));
  const qm dd1 = q_sub(s1, s0);
  const qm dd2 = q_mul(q_sub(q_sub(s2, s1), dd1), inv2);
  c[0] = s0;
  c[1] = q_sub(dd1, dd2);
  c[2] = dd2;
  c[3] = q_zero();
}
/* degree-3 Newton form from s0..s3 (prover.rs:8134-8145) */
static void newton_deg3(qm s0, qm s1, qm s2, qm s3, qm c[4]) {
  const qm two = q_from_m31(2), three = q_from_m31(3);
  const qm inv2 = q_inv(two), inv6 = q_inv(q_from_m31(6));
  const qm dd1 = q_sub(s1, s0);
  const qm dd2 = q_mul(q_add(q_sub(q_sub(s2, s1), s1), s0), inv2);
  const qm dd3 = q_mul(q_sub(q_sub(s3, s0), q_mul(three, q_sub(s2, s1))), inv6);
  c[0] = s0;
  c[1] = q_add(q_sub(dd1, dd2), q_mul(two, dd3));
  c[2] = q_sub(dd2, q_mul(three, dd3));
  c[3] = dd3;
}
static void store_poly(uint32_t* out, const qm c[4]) {
  for (int k = 0; k < 4; k++) q_store(out + 4 * k, c[k]);
}
/* The eq-weighted degree-3 sumcheck sum_x eq(r, x) a(x) b(x) over n = 2^nv
 * entries (prover.rs:8113-8160, 8270-8319): per round s(0..3), Newton
 * coefficients, mix_poly_coeffs_deg3, draw, fold eq / a / b.  a, b are
 * folded in place (a[0], b[0] hold the final values); chal receives nv. */
static void eq_sumcheck(orc_channel* ch, const qm* r, int nv, qm* a, qm* b, uint32_t* polys, qm* chal) {
  const size_t n = (size_t)1 << nv;
  qm* eq = (qm*)malloc(n * sizeof(qm));
  mle_eq_evals(r, nv, eq);
  size_t cur = n;
  for (int t = 0; t < nv; t++) {
    const size_t mid = cur / 2;
    const qm s0 = mul_eq_sum_at_t(eq, a, b, mid, q_zero());
    const qm s1 = mul_eq_sum_at_t(eq, a, b, mid, q_one());
    const qm s2 = mul_eq_sum_at_t(eq, a, b, mid, q_from_m31(2));
    const qm s3 = mul_eq_sum_at_t(eq, a, b, mid, q_from_m31(3));
    qm c[4];
    newton_deg3(s0, s1, s2, s3, c);
    store_poly(polys + 16 * t, c);
    orc_mix_poly_coeffs_deg3(ch, polys + 16 * t);
    const qm x = draw_q(ch);
    chal[t] = x;
    fold_mle(eq, x, mid);
    fold_mle(a, x, mid);
    fold_mle(b, x, mid);
    cur = mid;
  }
  free(eq);
}
/* build_multiplicity_sumcheck (prover.rs:9449-9511) */
static void multiplicity_sumcheck(orc_channel* ch, const uint32_t* mults, uint32_t log, uint32_t* rp, uint32_t* fin,
                                  uint32_t* sum) {
  const size_t tsize = (size_t)1 << log;
  qm* vals = (qm*)malloc(tsize * sizeof(qm));
  qm s = q_zero();
  for (size_t j = 0; j < tsize; j++) {
    vals[j] = q_from_m31(m31_from(mults[j]));
    s = q_add(s, vals[j]);
  }
  size_t cur = tsize;
  for (uint32_t t = 0; t < log; t++) {
    const size_t half = cur / 2;
    qm lo = q_zero(), hi = q_zero();
    for (size_t i = 0; i < half; i++) lo = q_add(lo, vals[i]);
    for (size_t i = half; i < cur; i++) hi = q_add(hi, vals[i]);
    const qm c0 = lo, c1 = q_sub(hi, lo);
    q_store(rp + 8 * t, c0);
    q_store(rp + 8 * t + 4, c1);
    mix_q(ch, c0);
    mix_q(ch, c1);
    const qm r = draw_q(ch);
    fold_mle(vals, r, half);
    cur = half;
  }
  q_store(fin, vals[0]);
  q_store(sum, s);
  free(vals);
}
/* compute_rsqrt_table_commitment (prover.rs:8357-8363): hash_many([0x5253, log]) */
static void rsqrt_table_commitment(uint32_t out[8]) {
  uint32_t in[16] = {0};
  in[0] = 0x5253;
  in[8] = NM_TABLE_LOG;
  orc_hash_many(in, 2, out);
}
/* The rsqrt LogUp of both layers (prover.rs:8184-8342, 8632-8727): tags, gamma,
 * beta, d = gamma - key - beta * rsqrt, w = 1/d, trace and table sums, the
 * eq-sumcheck, final evaluations at its challenges, the multiplicity
 * sumcheck.  key / rsqrt: the per-entry MLE values (n = 2^nv).  Returns 2
 * when the trace and table sums differ. */
static int rsqrt_logup(orc_channel* ch, uint64_t type_tag, const qm* r, int nv, const qm* key, const qm* rsq,
                       orc_norm_out* out) {
  const size_t n = (size_t)1 << nv, tsize = (size_t)1 << NM_TABLE_LOG;
  memset(out->multiplicities, 0, tsize * sizeof(uint32_t));
  for (size_t p = 0; p < n; p++) { /* compute_multiplicities (activation.rs:211-221) */
    const uint32_t k = key[p].lo.a;
    if (k < tsize) out->multiplicities[k]++;
  }
  orc_mix_u64(ch, 0x4C4F47ull);
  orc_mix_u64(ch, type_tag);
  const qm gamma = draw_q(ch), beta = draw_q(ch);
  qm* d = (qm*)malloc(n * sizeof(qm));
  qm* w = (qm*)malloc(n * sizeof(qm));
  for (size_t p = 0; p < n; p++) d[p] = q_sub(q_sub(gamma, key[p]), q_mul(beta, rsq[p]));
  q_batch_inverse(d, w, n);
  qm trace = q_zero();
  for (size_t p = 0; p < n; p++) trace = q_add(trace, w[p]);
  qm table = q_zero();
  for (size_t j = 0; j < tsize; j++)
    if (out->multiplicities[j]) {
      const qm dj = q_sub(q_sub(gamma, q_from_m31((uint32_t)j)), q_mul(beta, q_from_m31(orc_rsqrt((uint32_t)j))));
      table = q_add(table, q_mul(q_from_m31(m31_from(out->multiplicities[j])), q_inv(dj)));
    }
  if (!q_eq(trace, table)) {
    free(d);
    free(w);
    return 2;
  }
  mix_q(ch, trace);
  q_store(out->claimed_sum, trace);
  qm* chal = (qm*)malloc((size_t)(nv ? nv : 1) * sizeof(qm));
  eq_sumcheck(ch, r, nv, w, d, out->logup_round_polys, chal);
  q_store(out->w_eval, w[0]);
  q_store(out->in_eval, mle_evaluate(key, nv, chal));
  q_store(out->out_eval, mle_evaluate(rsq, nv, chal));
  free(chal);
  free(d);
  free(w);
  multiplicity_sumcheck(ch, out->multiplicities, NM_TABLE_LOG, out->mult_round_polys, out->mult_final, out->mult_sum);
  rsqrt_table_commitment(out->table_commitment);
  return 0;
}

/* pad_matrix_pow2 + matrix_to_mle of X (rows x cols) */
static uint32_t* pad(const uint32_t* X, size_t rows, size_t cols, size_t prow, size_t pcol) {
  uint32_t* p = (uint32_t*)calloc(prow * pcol, sizeof(uint32_t));
  for (size_t i = 0; i < rows; i++)
    for (size_t j = 0; j < cols; j++) p[i * pcol + j] = X[i * cols + j];
  return p;
}

/* Forward statistics of reduce_layernorm_layer (prover.rs:7968-8020): per padded
 * row the mean over the n_active = min(dim, pcol) first columns, the masked
 * variance and its rsqrt; centered = x - mean and output = centered * rsqrt on
 * every column (padding included). */
static void layernorm_rows(const uint32_t* xp, size_t prow, size_t pcol, size_t n_active, uint32_t* mean,
                           uint32_t* var, uint32_t* rsq) {
  const uint32_t inv_n = m31_inv_fermat((uint32_t)n_active);
  for (size_t r = 0; r < prow; r++) {
    uint32_t s = 0;
    for (size_t c = 0; c < n_active; c++) s = madd(s, xp[r * pcol + c]);
    const uint32_t m = mmul(s, inv_n);
    uint32_t vs = 0;
    for (size_t c = 0; c < n_active; c++) {
      const uint32_t diff = msub(xp[r * pcol + c], m);
      vs = madd(vs, mmul(diff, diff));
    }
    const uint32_t v = mmul(vs, inv_n) & ((1u << NM_TABLE_LOG) - 1);
    mean[r] = m;
    var[r] = v;
    rsq[r] = orc_rsqrt(v);
  }
}
void orc_layernorm_forward(const uint32_t* X, size_t rows, size_t cols, size_t dim, uint32_t* out_padded) {
  const size_t prow = nm_next_pow2(rows), pcol = nm_next_pow2(cols);
  const size_t n_active = dim < pcol ? dim : pcol;
  uint32_t* xp = pad(X, rows, cols, prow, pcol);
  uint32_t *mean = (uint32_t*)malloc(prow * 4), *var = (uint32_t*)malloc(prow * 4), *rsq = (uint32_t*)malloc(prow * 4);
  layernorm_rows(xp, prow, pcol, n_active, mean, var, rsq);
  for (size_t r = 0; r < prow; r++)
    for (size_t c = 0; c < pcol; c++) out_padded[r * pcol + c] = mmul(msub(xp[r * pcol + c], mean[r]), rsq[r]);
  free(xp);
  free(mean);
  free(var);
  free(rsq);
}

int orc_prove_layernorm_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                              const uint32_t* X, size_t rows, size_t cols, size_t dim, orc_channel* ch,
                              orc_norm_out* out) {
  const size_t prow = nm_next_pow2(rows), pcol = nm_next_pow2(cols), n = prow * pcol;
  const int nv = nm_log2(n);
  if (n_point != nv || nv == 0) return 1;
  const size_t n_active = dim < pcol ? dim : pcol;
  const qm* r = (const qm*)claim_point;
  uint32_t* xp = pad(X, rows, cols, prow, pcol);
  uint32_t *mean = (uint32_t*)malloc(prow * 4), *var = (uint32_t*)malloc(prow * 4), *rsq = (uint32_t*)malloc(prow * 4);
  layernorm_rows(xp, prow, pcol, n_active, mean, var, rsq);
  qm *input = (qm*)malloc(n * sizeof(qm)), *centered = (qm*)malloc(n * sizeof(qm));
  qm *mean_m = (qm*)malloc(n * sizeof(qm)), *var_m = (qm*)malloc(n * sizeof(qm));
  qm *rsq_m = (qm*)malloc(n * sizeof(qm)), *output = (qm*)malloc(n * sizeof(qm));
  for (size_t i = 0; i < prow; i++)
    for (size_t c = 0; c < pcol; c++) {
      const size_t p = i * pcol + c;
      const uint32_t cen = msub(xp[p], mean[i]);
      input[p] = q_from_m31(xp[p]);
      centered[p] = q_from_m31(cen);
      mean_m[p] = q_from_m31(mean[i]);
      var_m[p] = q_from_m31(var[i]);
      rsq_m[p] = q_from_m31(rsq[i]);
      output[p] = q_from_m31(mmul(cen, rsq[i]));
    }
  free(xp);
  /* evaluations at the claim point (8023-8028) */
  const qm input_eval = mle_evaluate(input, nv, r), output_eval = mle_evaluate(output, nv, r);
  const qm mean_eval = mle_evaluate(mean_m, nv, r), rsqrt_eval = mle_evaluate(rsq_m, nv, r);
  const qm var_eval = mle_evaluate(var_m, nv, r);
  q_store(out->input_eval, input_eval);
  q_store(out->output_eval, output_eval);
  q_store(out->mean_eval, mean_eval);
  q_store(out->rsqrt_eval, rsqrt_eval);
  q_store(out->var_eval, var_eval);
  free(output);

  /* Part 0: batched mean + variance plain sumcheck (8030-8097) */
  qm tin = q_zero(), tcs = q_zero();
  for (size_t p = 0; p < n; p++) {
    tin = q_add(tin, input[p]);
    tcs = q_add(tcs, q_mul(centered[p], centered[p]));
  }
  orc_mix_u64(ch, 0x4D56ull);
  orc_mix_u64(ch, n_active);
  mix_q(ch, tin);
  mix_q(ch, tcs);
  const qm eta0 = draw_q(ch), eta1 = q_mul(eta0, eta0);
  out->n_active = (uint32_t)n_active;
  q_store(out->sum0, tin);
  q_store(out->sum1, tcs);
  qm *in0 = (qm*)malloc(n * sizeof(qm)), *c0v = (qm*)malloc(n * sizeof(qm)), *m0 = (qm*)malloc(n * sizeof(qm));
  memcpy(in0, input, n * sizeof(qm));
  memcpy(c0v, centered, n * sizeof(qm));
  memcpy(m0, mean_m, n * sizeof(qm));
  size_t cur = n;
  for (int t = 0; t < nv; t++) {
    const size_t mid = cur / 2;
    const qm s0 = plain_mean_var_sum_at_t(in0, c0v, eta0, eta1, mid, q_zero());
    const qm s1 = plain_mean_var_sum_at_t(in0, c0v, eta0, eta1, mid, q_one());
    const qm s2 = plain_mean_var_sum_at_t(in0, c0v, eta0, eta1, mid, q_from_m31(2));
    qm c[4];
    newton_deg2(s0, s1, s2, c);
    store_poly(out->p0_round_polys + 16 * t, c);
    orc_mix_poly_coeffs_deg3(ch, out->p0_round_polys + 16 * t);
    const qm x = draw_q(ch);
    fold_mle(in0, x, mid);
    fold_mle(c0v, x, mid);
    fold_mle(m0, x, mid);
    cur = mid;
  }
  q_store(out->p0_final0, in0[0]);
  q_store(out->p0_final1, m0[0]);
  mix_q(ch, in0[0]);
  mix_q(ch, m0[0]);
  free(in0);
  free(c0v);
  free(m0);

  /* Part 1: linear eq-sumcheck sum eq(r, x) centered(x) rsqrt(x) (8099-8182) */
  orc_mix_u64(ch, 0x4C4Eull);
  mix_q(ch, mean_eval);
  mix_q(ch, rsqrt_eval);
  orc_mix_secure_field(ch, claim_value);
  qm *ca = (qm*)malloc(n * sizeof(qm)), *rb = (qm*)malloc(n * sizeof(qm));
  memcpy(ca, centered, n * sizeof(qm));
  memcpy(rb, rsq_m, n * sizeof(qm));
  qm* chal = (qm*)malloc((size_t)nv * sizeof(qm));
  eq_sumcheck(ch, r, nv, ca, rb, out->lin_round_polys, chal);
  const qm cb_in = mle_evaluate(input, nv, chal), cb_mean = mle_evaluate(mean_m, nv, chal);
  q_store(out->lin_final0, ca[0]);
  q_store(out->lin_final1, rb[0]);
  q_store(out->cb_input, cb_in);
  q_store(out->cb_mean, cb_mean);
  mix_q(ch, ca[0]);
  mix_q(ch, rb[0]);
  mix_q(ch, cb_in);
  mix_q(ch, cb_mean);
  free(ca);
  free(rb);
  free(chal);

  /* Part 2: rsqrt LogUp (8184-8342), type tag "RS" */
  int rc = rsqrt_logup(ch, 0x5253ull, r, nv, var_m, rsq_m, out);
  if (rc == 0) {
    mix_q(ch, input_eval); /* 8348-8349 */
    mix_q(ch, output_eval);
    orc_trace(ch, "layernorm", -1);
    out->n_rows = (uint32_t)prow;
    for (size_t i = 0; i < prow; i++) {
      out->row_stats0[i] = mean[i];
      out->row_stats1[i] = var[i];
    }
  }
  free(input);
  free(centered);
  free(mean_m);
  free(var_m);
  free(rsq_m);
  free(mean);
  free(var);
  free(rsq);
  return rc;
}

/* Forward statistics of reduce_rmsnorm_layer_with_gamma (prover.rs:8447-8487):
 * per padded row rms_sq = (sum of squares over the n_active first columns /
 * n_active) & mask, its rsqrt; scale = rsqrt * gamma[min(col, len - 1)] on the
 * active columns (rsqrt on the others), output = x * scale (x on the others). */
static void rmsnorm_rows(const uint32_t* xp, size_t prow, size_t pcol, size_t n_active, uint32_t* ms, uint32_t* rsq) {
  const uint32_t inv_n = m31_inv_fermat((uint32_t)n_active);
  for (size_t r = 0; r < prow; r++) {
    uint32_t s = 0;
    for (size_t c = 0; c < n_active; c++) s = madd(s, mmul(xp[r * pcol + c], xp[r * pcol + c]));
    ms[r] = mmul(s, inv_n) & ((1u << NM_TABLE_LOG) - 1);
    rsq[r] = orc_rsqrt(ms[r]);
  }
}
static uint32_t rms_scale(size_t c, size_t n_active, uint32_t rsq, const uint32_t* gamma, size_t ng) {
  if (c >= n_active || !gamma || !ng) return rsq;
  return mmul(rsq, gamma[c < ng - 1 ? c : ng - 1]);
}
void orc_rmsnorm_forward(const uint32_t* X, size_t rows, size_t cols, size_t dim, const uint32_t* gamma, size_t ng,
                         uint32_t* out_padded) {
  const size_t prow = nm_next_pow2(rows), pcol = nm_next_pow2(cols);
  const size_t n_active = dim < pcol ? dim : pcol;
  uint32_t* xp = pad(X, rows, cols, prow, pcol);
  uint32_t *ms = (uint32_t*)malloc(prow * 4), *rsq = (uint32_t*)malloc(prow * 4);
  rmsnorm_rows(xp, prow, pcol, n_active, ms, rsq);
  for (size_t r = 0; r < prow; r++)
    for (size_t c = 0; c < pcol; c++) {
      const uint32_t x = xp[r * pcol + c];
      out_padded[r * pcol + c] = c < n_active ? mmul(x, rms_scale(c, n_active, rsq[r], gamma, ng)) : x;
    }
  free(xp);
  free(ms);
  free(rsq);
}

int orc_prove_rmsnorm_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value, const uint32_t* X,
                            size_t rows, size_t cols, size_t dim, const uint32_t* gamma, size_t ng, orc_channel* ch,
                            orc_norm_out* out) {
  const size_t prow = nm_next_pow2(rows), pcol = nm_next_pow2(cols), n = prow * pcol;
  const int nv = nm_log2(n);
  if (n_point != nv || nv == 0) return 1;
  const size_t n_active = dim < pcol ? dim : pcol;
  const qm* r = (const qm*)claim_point;
  uint32_t* xp = pad(X, rows, cols, prow, pcol);
  uint32_t *ms = (uint32_t*)malloc(prow * 4), *rsq = (uint32_t*)malloc(prow * 4);
  rmsnorm_rows(xp, prow, pcol, n_active, ms, rsq);
  qm *input = (qm*)malloc(n * sizeof(qm)), *rsq_m = (qm*)malloc(n * sizeof(qm)), *scale = (qm*)malloc(n * sizeof(qm));
  qm *ms_m = (qm*)malloc(n * sizeof(qm)), *output = (qm*)malloc(n * sizeof(qm));
  for (size_t i = 0; i < prow; i++)
    for (size_t c = 0; c < pcol; c++) {
      const size_t p = i * pcol + c;
      const uint32_t x = xp[p], sc = rms_scale(c, n_active, rsq[i], gamma, ng);
      input[p] = q_from_m31(x);
      ms_m[p] = q_from_m31(ms[i]);
      rsq_m[p] = q_from_m31(rsq[i]);
      scale[p] = q_from_m31(sc);
      output[p] = q_from_m31(c < n_active ? mmul(x, sc) : x);
    }
  free(xp);
  const qm input_eval = mle_evaluate(input, nv, r), output_eval = mle_evaluate(output, nv, r);
  const qm rsqrt_eval = mle_evaluate(rsq_m, nv, r), ms_eval = mle_evaluate(ms_m, nv, r);
  q_store(out->input_eval, input_eval);
  q_store(out->output_eval, output_eval);
  q_store(out->mean_eval, ms_eval);
  q_store(out->rsqrt_eval, rsqrt_eval);
  memset(out->var_eval, 0, sizeof out->var_eval);
  free(output);
  if (gamma && ng) { /* gamma commitment and evaluation (8758-8781), not mixed or serialized */
    orc_channel g;
    orc_channel_init(&g);
    orc_mix_u64(&g, 0x47414D4D41ull);
    for (size_t i = 0; i < ng; i++) {
      uint32_t q[4] = {gamma[i], 0, 0, 0};
      orc_mix_secure_field(&g, q);
    }
    orc_digest(&g, out->gamma_commitment);
    qm* gm = (qm*)malloc(n * sizeof(qm));
    for (size_t p = 0; p < n; p++) gm[p] = (p % pcol) < ng ? q_from_m31(gamma[p % pcol]) : q_one();
    q_store(out->gamma_eval, mle_evaluate(gm, nv, r));
    free(gm);
  }

  /* Part 0: plain sumcheck sum_x input(x)^2 (8497-8540) */
  qm tsq = q_zero();
  for (size_t p = 0; p < n; p++) tsq = q_add(tsq, q_mul(input[p], input[p]));
  orc_mix_u64(ch, 0x5251ull);
  orc_mix_u64(ch, n_active);
  mix_q(ch, tsq);
  out->n_active = (uint32_t)n_active;
  q_store(out->sum0, tsq);
  memset(out->sum1, 0, sizeof out->sum1);
  qm* in0 = (qm*)malloc(n * sizeof(qm));
  memcpy(in0, input, n * sizeof(qm));
  size_t cur = n;
  for (int t = 0; t < nv; t++) {
    const size_t mid = cur / 2;
    const qm s0 = plain_sq_sum_at_t(in0, mid, q_zero());
    const qm s1 = plain_sq_sum_at_t(in0, mid, q_one());
    const qm s2 = plain_sq_sum_at_t(in0, mid, q_from_m31(2));
    qm c[4];
    newton_deg2(s0, s1, s2, c);
    store_poly(out->p0_round_polys + 16 * t, c);
    orc_mix_poly_coeffs_deg3(ch, out->p0_round_polys + 16 * t);
    fold_mle(in0, draw_q(ch), mid);
    cur = mid;
  }
  q_store(out->p0_final0, in0[0]);
  memset(out->p0_final1, 0, sizeof out->p0_final1);
  mix_q(ch, in0[0]);
  free(in0);

  /* Part 1: eq-sumcheck sum eq(r, x) input(x) scale(x) (8553-8630) */
  orc_mix_u64(ch, 0x524Eull);
  mix_q(ch, ms_eval);
  mix_q(ch, rsqrt_eval);
  orc_mix_secure_field(ch, claim_value);
  qm* chal = (qm*)malloc((size_t)nv * sizeof(qm));
  qm* ia = (qm*)malloc(n * sizeof(qm));
  memcpy(ia, input, n * sizeof(qm));
  eq_sumcheck(ch, r, nv, ia, scale, out->lin_round_polys, chal);
  q_store(out->lin_final0, ia[0]);
  q_store(out->lin_final1, scale[0]);
  memset(out->cb_input, 0, sizeof out->cb_input);
  memset(out->cb_mean, 0, sizeof out->cb_mean);
  mix_q(ch, ia[0]);
  mix_q(ch, scale[0]);
  free(ia);
  free(chal);

  /* Part 2: rsqrt LogUp (8632-8733), type tag "RN" */
  int rc = rsqrt_logup(ch, 0x524Eull, r, nv, ms_m, rsq_m, out);
  if (rc == 0) {
    mix_q(ch, input_eval); /* 8740-8741 */
    mix_q(ch, output_eval);
    orc_trace(ch, "rmsnorm", -1);
    out->n_rows = (uint32_t)prow;
    for (size_t i = 0; i < prow; i++) {
      out->row_stats0[i] = ms[i];
      out->row_stats1[i] = 0;
    }
  }
  free(input);
  free(rsq_m);
  free(scale);
  free(ms_m);
  free(ms);
  free(rsq);
  return rc;
}

/* ------------------------------------------------------------------ verifiers */
static qm poly_eval(const uint32_t* c4, qm x) { /* RoundPolyDeg3::eval */
  const qm c0 = q_load(c4), c1 = q_load(c4 + 4), c2 = q_load(c4 + 8), c3 = q_load(c4 + 12);
  return q_add(c0, q_mul(x, q_add(c1, q_mul(x, q_add(c2, q_mul(x, c3))))));
}
static qm poly_sum01(const uint32_t* c4) { /* p(0) + p(1) */
  const qm c0 = q_load(c4), c1 = q_load(c4 + 4), c2 = q_load(c4 + 8), c3 = q_load(c4 + 12);
  return q_add(c0, q_add(q_add(q_add(c0, c1), c2), c3));
}
static qm eq_eval(const qm* r, const qm* s, int n) { /* compute_eq_eval */
  qm e = q_one();
  for (int i = 0; i < n; i++)
    e = q_mul(e, q_add(q_mul(r[i], s[i]), q_mul(q_sub(q_one(), r[i]), q_sub(q_one(), s[i]))));
  return e;
}
/* rounds of a sumcheck starting at `sum`: p(0) + p(1) = sum, mix, draw; returns
 * 0 and the final sum / challenges, or 1 */
static int replay_rounds(orc_channel* ch, const uint32_t* polys, int nv, qm* sum, qm* chal) {
  for (int t = 0; t < nv; t++) {
    if (!q_eq(poly_sum01(polys + 16 * t), *sum)) return 1;
    orc_mix_poly_coeffs_deg3(ch, polys + 16 * t);
    const qm x = draw_q(ch);
    if (chal) chal[t] = x;
    *sum = poly_eval(polys + 16 * t, x);
  }
  return 0;
}
/* verify_multiplicity_sumcheck (verifier.rs:5818-5842) */
static int verify_mult(orc_channel* ch, const orc_norm_out* p) {
  qm cur = q_load(p->mult_sum);
  for (uint32_t t = 0; t < NM_TABLE_LOG; t++) {
    const qm c0 = q_load(p->mult_round_polys + 8 * t), c1 = q_load(p->mult_round_polys + 8 * t + 4);
    if (!q_eq(q_add(c0, q_add(c0, c1)), cur)) return 1;
    mix_q(ch, c0);
    mix_q(ch, c1);
    cur = q_add(c0, q_mul(c1, draw_q(ch)));
  }
  return q_eq(cur, q_load(p->mult_final)) ? 0 : 1;
}
/* the rsqrt LogUp part of both verifiers (verifier.rs:4561-4672, 4957-5063) */
static int verify_rsqrt_logup(orc_channel* ch, uint64_t type_tag, const qm* r, int nv, const orc_norm_out* p) {
  orc_mix_u64(ch, 0x4C4F47ull);
  orc_mix_u64(ch, type_tag);
  const qm gamma = draw_q(ch), beta = draw_q(ch);
  uint32_t tc[8];
  rsqrt_table_commitment(tc);
  if (memcmp(tc, p->table_commitment, sizeof tc)) return 10;
  qm table = q_zero();
  for (size_t j = 0; j < ((size_t)1 << NM_TABLE_LOG); j++)
    if (p->multiplicities[j]) {
      const qm dj = q_sub(q_sub(gamma, q_from_m31((uint32_t)j)), q_mul(beta, q_from_m31(orc_rsqrt((uint32_t)j))));
      table = q_add(table, q_mul(q_from_m31(m31_from(p->multiplicities[j])), q_inv(dj)));
    }
  if (!q_eq(table, q_load(p->claimed_sum))) return 11;
  mix_q(ch, q_load(p->claimed_sum));
  qm sum = q_one();
  qm* chal = (qm*)malloc((size_t)nv * sizeof(qm));
  if (replay_rounds(ch, p->logup_round_polys, nv, &sum, chal)) {
    free(chal);
    return 12;
  }
  const qm d = q_sub(q_sub(gamma, q_load(p->in_eval)), q_mul(beta, q_load(p->out_eval)));
  const qm expected = q_mul(q_mul(eq_eval(r, chal, nv), q_load(p->w_eval)), d);
  free(chal);
  return q_eq(sum, expected) ? 0 : 13;
}
/* sum_r v_r eq(s[0..log_rows), r) over the row bits (the first variables) */
static qm row_mle(const uint32_t* v, size_t rows, int log_rows, const qm* s) {
  qm acc = q_zero();
  for (size_t rr = 0; rr < rows; rr++) {
    qm e = q_one();
    for (int k = 0; k < log_rows; k++)
      e = q_mul(e, ((rr >> (log_rows - 1 - k)) & 1) ? s[k] : q_sub(q_one(), s[k]));
    acc = q_add(acc, q_mul(e, q_from_m31(v[rr])));
  }
  return acc;
}

int orc_verify_layernorm_layer(const uint32_t* claim_point, int nv, const uint32_t* claim_value, size_t dim,
                               const orc_norm_out* p, orc_channel* ch, uint32_t next_value[4]) {
  if (nv <= 0) return 1;
  const qm* r = (const qm*)claim_point;
  /* Part 0 (verifier.rs:4214-4489) */
  const size_t n_active = dim < ((size_t)1 << nv) ? dim : ((size_t)1 << nv);
  orc_mix_u64(ch, 0x4D56ull);
  orc_mix_u64(ch, n_active);
  const qm tin = q_load(p->sum0), tcs = q_load(p->sum1);
  mix_q(ch, tin);
  mix_q(ch, tcs);
  const qm eta0 = draw_q(ch), eta1 = q_mul(eta0, eta0);
  qm sum = q_add(q_mul(eta0, tin), q_mul(eta1, tcs));
  qm* mv = (qm*)malloc((size_t)nv * sizeof(qm));
  if (replay_rounds(ch, p->p0_round_polys, nv, &sum, mv)) {
    free(mv);
    return 2;
  }
  const qm in_f = q_load(p->p0_final0), mean_f = q_load(p->p0_final1);
  mix_q(ch, in_f);
  mix_q(ch, mean_f);
  const qm cf = q_sub(in_f, mean_f);
  if (!q_eq(sum, q_add(q_mul(eta0, in_f), q_mul(q_mul(eta1, cf), cf)))) {
    free(mv);
    return 3;
  }
  size_t cols_padded = 1;
  while (cols_padded < dim) cols_padded <<= 1;
  const size_t rows = ((size_t)1 << nv) / cols_padded;
  const qm mean_eval = q_load(p->mean_eval), var_eval = q_load(p->var_eval);
  if (rows == 1) { /* single-row derivations (4289-4372) */
    const uint32_t inv_n = m31_inv_fermat((uint32_t)n_active);
    if (mmul(tin.lo.a, inv_n) != mean_eval.lo.a) {
      free(mv);
      return 4;
    }
    const uint32_t var_expected = mmul(tcs.lo.a, inv_n) & ((1u << NM_TABLE_LOG) - 1);
    if (n_active == cols_padded && var_expected != var_eval.lo.a) {
      free(mv);
      return 5;
    }
  } else { /* multi-row bindings (4373-4463), as the reference states them */
    if (p->n_rows != rows) {
      free(mv);
      return 6;
    }
    const int log_rows = nv - nm_log2(cols_padded);
    if (!q_eq(mean_f, row_mle(p->row_stats0, rows, log_rows, mv)) ||
        !q_eq(var_eval, row_mle(p->row_stats1, rows, log_rows, mv))) {
      free(mv);
      return 7;
    }
  }
  free(mv);
  /* Part 1 (4491-4555) */
  orc_mix_u64(ch, 0x4C4Eull);
  mix_q(ch, mean_eval);
  mix_q(ch, q_load(p->rsqrt_eval));
  orc_mix_secure_field(ch, claim_value);
  sum = q_load(claim_value);
  qm* chal = (qm*)malloc((size_t)nv * sizeof(qm));
  if (replay_rounds(ch, p->lin_round_polys, nv, &sum, chal)) {
    free(chal);
    return 8;
  }
  const qm cen = q_load(p->lin_final0), rsf = q_load(p->lin_final1);
  const int ok1 = q_eq(sum, q_mul(q_mul(eq_eval(r, chal, nv), cen), rsf));
  free(chal);
  if (!ok1) return 9;
  mix_q(ch, cen);
  mix_q(ch, rsf);
  const qm cbi = q_load(p->cb_input), cbm = q_load(p->cb_mean);
  mix_q(ch, cbi);
  mix_q(ch, cbm);
  if (!q_eq(cen, q_sub(cbi, cbm))) return 14;
  /* Part 2 + multiplicity sumcheck + final mixes (4557-4690) */
  int rc = verify_rsqrt_logup(ch, 0x5253ull, r, nv, p);
  if (rc) return rc;
  if (verify_mult(ch, p)) return 15;
  mix_q(ch, q_load(p->input_eval));
  mix_q(ch, q_load(p->output_eval));
  memcpy(next_value, p->input_eval, 16);
  return 0;
}

int orc_verify_rmsnorm_layer(const uint32_t* claim_point, int nv, const uint32_t* claim_value, size_t dim,
                             const orc_norm_out* p, orc_channel* ch, uint32_t next_value[4]) {
  if (nv <= 0) return 1;
  const qm* r = (const qm*)claim_point;
  /* Part 0 (verifier.rs:4752-4885) */
  const size_t n_active = dim < ((size_t)1 << nv) ? dim : ((size_t)1 << nv);
  const qm tsq = q_load(p->sum0);
  orc_mix_u64(ch, 0x5251ull);
  orc_mix_u64(ch, n_active);
  mix_q(ch, tsq);
  qm sum = tsq;
  if (replay_rounds(ch, p->p0_round_polys, nv, &sum, NULL)) return 2;
  const qm in_f = q_load(p->p0_final0);
  mix_q(ch, in_f);
  if (!q_eq(q_mul(in_f, in_f), sum)) return 3;
  size_t cols_padded = 1;
  while (cols_padded < dim) cols_padded <<= 1;
  const size_t rows = ((size_t)1 << nv) / cols_padded;
  const qm ms_eval = q_load(p->mean_eval);
  if (rows == 1) {
    const uint32_t expected = mmul(tsq.lo.a, m31_inv_fermat((uint32_t)n_active)) & ((1u << NM_TABLE_LOG) - 1);
    if (expected != ms_eval.lo.a) return 4;
  } else {
    if (p->n_rows != rows) return 6;
    if (!q_eq(ms_eval, row_mle(p->row_stats0, rows, nv - nm_log2(cols_padded), r))) return 7;
  }
  /* Part 1 (4887-4937) */
  orc_mix_u64(ch, 0x524Eull);
  mix_q(ch, ms_eval);
  mix_q(ch, q_load(p->rsqrt_eval));
  orc_mix_secure_field(ch, claim_value);
  sum = q_load(claim_value);
  qm* chal = (qm*)malloc((size_t)nv * sizeof(qm));
  if (replay_rounds(ch, p->lin_round_polys, nv, &sum, chal)) {
    free(chal);
    return 8;
  }
  const qm inf = q_load(p->lin_final0), rsf = q_load(p->lin_final1);
  const int ok1 = q_eq(sum, q_mul(q_mul(eq_eval(r, chal, nv), inf), rsf));
  free(chal);
  if (!ok1) return 9;
  mix_q(ch, inf);
  mix_q(ch, rsf);
  int rc = verify_rsqrt_logup(ch, 0x524Eull, r, nv, p);
  if (rc) return rc;
  if (verify_mult(ch, p)) return 15;
  mix_q(ch, q_load(p->input_eval));
  mix_q(ch, q_load(p->output_eval));
  memcpy(next_value, p->input_eval, 16);
  return 0;
}
