/* MLE helpers and the matmul sumcheck reducer, restated from
 * engine/src/components/matmul.rs, engine/src/backend.rs and
 * engine/src/gkr/prover.rs.  OpenMP stands in for rayon where the reference
 * parallelises.  TEST INFRASTRUCTURE ONLY (see oracle.h). */
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

/* evaluate_mle (matmul.rs:118-136): in-place folding, first variable = MSB */
qm mle_evaluate(const qm* evals, int n_vars, const qm* point) {
  size_t size = (size_t)1 << n_vars;
  qm* cur = (qm*)malloc(size * sizeof(qm));
  memcpy(cur, evals, size * sizeof(qm));
  for (int v = 0; v < n_vars; v++) {
    size_t mid = size / 2;
    for (size_t i = 0; i < mid; i++) cur[i] = q_add(cur[i], q_mul(point[v], q_sub(cur[mid + i], cur[i])));
    size = mid;
  }
  qm r = cur[0];
  free(cur);
  return r;
}
void orc_evaluate_mle(const uint32_t* evals, int n_vars, const uint32_t* point, uint32_t out[4]) {
  q_store(out, mle_evaluate((const qm*)evals, n_vars, (const qm*)point));
}

/* sum_i fa[i] * fb[i]: the claim the product round loop starts from
 * (backend.rs:146-157 at round 0: s0 + s1 = the sum over the whole hypercube) */
void orc_inner_product_q(const uint32_t* fa, const uint32_t* fb, size_t n, uint32_t out[4]) {
  const qm* a = (const qm*)fa;
  const qm* b = (const qm*)fb;
  qm total = q_zero();
#pragma omp parallel
  {
    qm part = q_zero();
#pragma omp for schedule(static)
    for (size_t i = 0; i < n; i++) part = q_add(part, q_mul(a[i], b[i]));
#pragma omp critical
    total = q_add(total, part);
  }
  q_store(out, total);
}

/* restrict_mle (matmul.rs:144-169): fold the first s variables; parallel when mid >= 8192 */
static qm* restrict_mle(const qm* evals, size_t len, const qm* assign, int s) {
  qm* cur = (qm*)malloc(len * sizeof(qm));
  memcpy(cur, evals, len * sizeof(qm));
  size_t size = len;
  for (int v = 0; v < s; v++) {
    size_t mid = size / 2;
    const qm r = assign[v];
    if (mid >= 8192) {
#pragma omp parallel for schedule(static)
      for (size_t i = 0; i < mid; i++) cur[i] = q_add(cur[i], q_mul(r, q_sub(cur[mid + i], cur[i])));
    } else {
      for (size_t i = 0; i < mid; i++) cur[i] = q_add(cur[i], q_mul(r, q_sub(cur[mid + i], cur[i])));
    }
    size = mid;
  }
  return cur; /* first `size` entries valid */
}
void orc_restrict_mle(const uint32_t* evals, size_t len, const uint32_t* assign, int s, uint32_t* out) {
  qm* r = restrict_mle((const qm*)evals, len, (const qm*)assign, s);
  memcpy(out, r, (len >> s) * sizeof(qm));
  free(r);
}

/* compute_lagrange_basis (matmul.rs:342-355): each challenge doubles the table,
 * weights[2w] = w(1-c), weights[2w+1] = w c  => c[0] on the MSB */
void orc_lagrange_basis(const uint32_t* c, int n, uint32_t* out) {
  qm* w = (qm*)out;
  w[0] = q_one();
  size_t len = 1;
  qm* tmp = (qm*)malloc(((size_t)1 << n) * sizeof(qm));
  for (int l = 0; l < n; l++) {
    qm cl = q_load(c + 4 * l);
    qm omc = q_sub(q_one(), cl);
    for (size_t i = 0; i < len; i++) {
      tmp[2 * i] = q_mul(w[i], omc);
      tmp[2 * i + 1] = q_mul(w[i], cl);
    }
    len *= 2;
    memcpy(w, tmp, len * sizeof(qm));
  }
  free(tmp);
}
/* build_eq_evals (gkr/prover.rs:9201-9233): seeded with the last coordinate,
 * then doubled for r[n-2] .. r[0]  => r[0] on the MSB */
void mle_eq_evals(const qm* r, int n, qm* out) {
  if (n == 0) {
    out[0] = q_one();
    return;
  }
  out[0] = q_sub(q_one(), r[n - 1]);
  out[1] = r[n - 1];
  size_t len = 2;
  for (int i = n - 2; i >= 0; i--) {
    qm one_minus = q_sub(q_one(), r[i]);
    for (size_t j = 0; j < len; j++) out[len + j] = q_mul(out[j], r[i]);
    for (size_t j = 0; j < len; j++) out[j] = q_mul(out[j], one_minus);
    len *= 2;
  }
}
void orc_eq_evals(const uint32_t* r, int n, uint32_t* out) { mle_eq_evals((const qm*)r, n, (qm*)out); }

/* matmul_m31 (matmul.rs:571-625): C = A B over M31 */
void orc_matmul_forward(const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n, uint32_t* Cm) {
  uint32_t* bt = (uint32_t*)malloc(k * n * sizeof(uint32_t));
  for (size_t i = 0; i < k; i++)
    for (size_t j = 0; j < n; j++) bt[j * k + i] = B[i * n + j];
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < m; i++) {
    for (size_t j = 0; j < n; j++) {
      uint32_t s = 0;
      for (size_t l = 0; l < k; l++) s = orc_m31_add(s, orc_m31_mul(A[i * k + l], bt[j * k + l]));
      Cm[i * n + j] = s;
    }
  }
  free(bt);
}

/* pad_matrix_pow2 + matrix_to_mle (matmul.rs:174-192, 649-665): row-major QM31 MLE */
static qm* row_major_mle(const uint32_t* M, size_t rows, size_t cols, size_t* out_len) {
  size_t pr = next_pow2(rows), pc = next_pow2(cols);
  qm* e = (qm*)calloc(pr * pc, sizeof(qm));
#pragma omp parallel for schedule(static) if (pr * pc >= 65536)
  for (size_t i = 0; i < rows; i++)
    for (size_t j = 0; j < cols; j++) e[i * pc + j] = q_from_m31(M[i * cols + j]);
  *out_len = pr * pc;
  return e;
}
/* pad_matrix_pow2 + matrix_to_mle_col_major (matmul.rs:194-220): B[i][j] at j*rows + i */
static qm* col_major_mle(const uint32_t* M, size_t rows, size_t cols, size_t* out_len) {
  size_t pr = next_pow2(rows), pc = next_pow2(cols);
  qm* e = (qm*)calloc(pr * pc, sizeof(qm));
#pragma omp parallel for schedule(static) if (pr * pc >= 65536)
  for (size_t j = 0; j < cols; j++)
    for (size_t i = 0; i < rows; i++) e[j * pr + i] = q_from_m31(M[i * cols + j]);
  *out_len = pr * pc;
  return e;
}

/* MLE of the padded output C at r_out, the driver's output claim (prover.rs:1543-1553) */
void orc_matmul_output_claim(const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n,
                             const uint32_t* r_out, int n_vars, uint32_t out[4]) {
  uint32_t* Cm = (uint32_t*)malloc(m * n * sizeof(uint32_t));
  orc_matmul_forward(A, m, k, B, n, Cm);
  size_t len;
  qm* e = row_major_mle(Cm, m, n, &len);
  q_store(out, mle_evaluate(e, n_vars, (const qm*)r_out));
  free(e);
  free(Cm);
}

/* SimdBackend::reduce_matmul_layer (backend.rs:111-197) */
/* Round loop of SimdBackend::reduce_matmul_layer (backend.rs:146-177):
 * s0 = sum a0 b0, s1 = sum a1 b1, s2 = sum (2a1 - a0)(2b1 - b0); c0 = s0,
 * c2 = (s2 - 2 s1 + s0) / 2, c1 = s1 - s0 - c2; mix_poly_coeffs, draw, fold
 * x + r (y - x).  fa/fb (length cur) are folded in place. */
static void product_rounds(qm* fa, qm* fb, size_t cur, int log_k, orc_channel* ch, uint32_t* round_polys,
                           uint32_t* challenges, uint32_t* final_a, uint32_t* final_b) {
  const qm inv2 = q_inv(q_from_m31(2));
  for (int t = 0; t < log_k; t++) {
    size_t mid = cur / 2;
    qm s0 = q_zero(), s1 = q_zero(), s2 = q_zero();
    for (size_t i = 0; i < mid; i++) {
      s0 = q_add(s0, q_mul(fa[i], fb[i]));
      s1 = q_add(s1, q_mul(fa[mid + i], fb[mid + i]));
      qm a2 = q_sub(q_add(fa[mid + i], fa[mid + i]), fa[i]);
      qm b2 = q_sub(q_add(fb[mid + i], fb[mid + i]), fb[i]);
      s2 = q_add(s2, q_mul(a2, b2));
    }
    qm c0 = s0;
    qm c2 = q_mul(q_add(q_sub(q_sub(s2, s1), s1), s0), inv2);
    qm c1 = q_sub(q_sub(s1, s0), c2);
    q_store(round_polys + 12 * t, c0);
    q_store(round_polys + 12 * t + 4, c1);
    q_store(round_polys + 12 * t + 8, c2);
    orc_mix_poly_coeffs(ch, round_polys + 12 * t);
    uint32_t al[4];
    orc_draw_qm31(ch, al);
    memcpy(challenges + 4 * t, al, 16);
    qm alpha = q_load(al);
    for (size_t i = 0; i < mid; i++) {
      fa[i] = q_add(fa[i], q_mul(alpha, q_sub(fa[mid + i], fa[i])));
      fb[i] = q_add(fb[i], q_mul(alpha, q_sub(fb[mid + i], fb[i])));
    }
    cur = mid;
  }
  q_store(final_a, cur ? fa[0] : q_zero());
  q_store(final_b, cur ? fb[0] : q_zero());
}

int orc_reduce_matmul_layer(const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n,
                            const uint32_t* r_i, int n_ri, const uint32_t* r_j, int n_rj, size_t pk,
                            orc_channel* ch, uint32_t* round_polys, uint32_t* challenges, uint32_t* final_a,
                            uint32_t* final_b) {
  size_t la, lb;
  qm* a_mle = row_major_mle(A, m, k, &la);
  qm* b_mle = col_major_mle(B, k, n, &lb);
  qm* fa = restrict_mle(a_mle, la, (const qm*)r_i, n_ri);
  qm* fb = restrict_mle(b_mle, lb, (const qm*)r_j, n_rj);
  free(a_mle);
  free(b_mle);
  size_t cur = la >> n_ri; /* f_a length */
  if ((lb >> n_rj) != cur) {
    free(fa);
    free(fb);
    return 1;
  }
  product_rounds(fa, fb, cur, ilog2(pk), ch, round_polys, challenges, final_a, final_b);
  free(fa);
  free(fb);
  return 0;
}

/* The round loop alone over given QM31 vectors of length n (a power of two):
 * config-2 style product sumcheck sum_x f_a(x) f_b(x). */
int orc_sumcheck_product(const uint32_t* fa_in, const uint32_t* fb_in, size_t n, orc_channel* ch,
                         uint32_t* round_polys, uint32_t* challenges, uint32_t* final_a, uint32_t* final_b) {
  if (n == 0 || (n & (n - 1))) return 1;
  qm* fa = (qm*)malloc(n * sizeof(qm));
  qm* fb = (qm*)malloc(n * sizeof(qm));
  for (size_t i = 0; i < n; i++) {
    fa[i] = q_load(fa_in + 4 * i);
    fb[i] = q_load(fb_in + 4 * i);
  }
  product_rounds(fa, fb, n, ilog2(n), ch, round_polys, challenges, final_a, final_b);
  free(fa);
  free(fb);
  return 0;
}

static void mix_sf(orc_channel* ch, qm v) {
  uint32_t w[4];
  q_store(w, v);
  orc_mix_secure_field(ch, w);
}

/* reduce_matmul_layer_with_backend (gkr/prover.rs:5959-6070) */
int orc_prove_matmul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                           const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n, orc_channel* ch,
                           uint32_t* round_polys, uint32_t* final_a, uint32_t* final_b, uint32_t* next_point,
                           uint32_t* next_value) {
  const size_t pm = next_pow2(m), pk = next_pow2(k), pn = next_pow2(n);
  const int log_m = ilog2(pm), log_n = ilog2(pn), T = ilog2(pk);
  if (n_point != log_m + log_n) return 1;
  orc_mix_u64(ch, m);
  orc_mix_u64(ch, k);
  orc_mix_u64(ch, n);
  orc_mix_secure_field(ch, claim_value);
  uint32_t* chal = (uint32_t*)malloc((size_t)(T + 1) * 16);
  int rc = orc_reduce_matmul_layer(A, m, k, B, n, claim_point, log_m, claim_point + 4 * log_m, log_n, pk, ch,
                                   round_polys, chal, final_a, final_b);
  if (rc) {
    free(chal);
    return rc;
  }
  orc_trace(ch, "matmul.rounds", -1);
  orc_mix_secure_field(ch, final_a);
  orc_mix_secure_field(ch, final_b);
  orc_trace(ch, "matmul", -1);
  memcpy(next_point, claim_point, (size_t)log_m * 16);
  memcpy(next_point + 4 * log_m, chal, (size_t)T * 16);
  memcpy(next_value, final_a, 16);
  free(chal);
  (void)mix_sf;
  return 0;
}

/* restrict_cols_unpadded (matmul.rs:470-514): f_b[i] = sum_{j<n} B[i][j] L_j, padded to pk */
void orc_restrict_cols_fused(const uint32_t* B, size_t k, size_t n, const uint32_t* r_j, int n_rj, size_t pk,
                             uint32_t* out) {
  qm* L = (qm*)malloc(((size_t)1 << n_rj) * sizeof(qm));
  orc_lagrange_basis(r_j, n_rj, (uint32_t*)L);
  qm* f = (qm*)out;
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < k; i++) {
    qm s = q_zero();
    for (size_t j = 0; j < n; j++) s = q_add(s, q_mul(q_from_m31(B[i * n + j]), L[j]));
    f[i] = s;
  }
  for (size_t i = k; i < pk; i++) f[i] = q_zero();
  free(L);
}
/* restrict_rows_unpadded (matmul.rs:523-565): f_a[j] = sum_{i<m} A[i][j] L_i, padded to pk */
void orc_restrict_rows_fused(const uint32_t* A, size_t m, size_t k, const uint32_t* r_i, int n_ri, size_t pk,
                             uint32_t* out) {
  qm* L = (qm*)malloc(((size_t)1 << n_ri) * sizeof(qm));
  orc_lagrange_basis(r_i, n_ri, (uint32_t*)L);
  qm* f = (qm*)out;
#pragma omp parallel for schedule(static)
  for (size_t j = 0; j < k; j++) {
    qm s = q_zero();
    for (size_t i = 0; i < m; i++) s = q_add(s, q_mul(q_from_m31(A[i * k + j]), L[i]));
    f[j] = s;
  }
  for (size_t j = k; j < pk; j++) f[j] = q_zero();
  free(L);
}

/* Synthetic inputs: counter-mode SplitMix64 (value i = (i+1)-th output of the
 * sequential generator seeded with `seed`).  kind 0: uniform M31 (31-bit draw,
 * P rejected by re-mixing); kind 1: int8-range (z >> 32) % 255 - 127, negative v
 * stored as P + v. */
static uint64_t sm_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
uint32_t orc_synthetic_value(int kind, uint64_t seed, uint64_t i) {
  uint64_t z = sm_mix(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
  if (kind == 0) {
    uint32_t v = (uint32_t)(z >> 33);
    while (v == ORC_P) {
      z = sm_mix(z + 0x9E3779B97F4A7C15ull);
      v = (uint32_t)(z >> 33);
    }
    return v;
  }
  int s = (int)((z >> 32) % 255ull) - 127;
  return s < 0 ? (uint32_t)((int64_t)ORC_P + s) : (uint32_t)s;
}
void orc_synthetic_fill(uint32_t* out, size_t n, int kind, uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) out[i] = orc_synthetic_value(kind, seed, i);
}
