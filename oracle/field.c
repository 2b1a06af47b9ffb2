/* M31 / CM31 / QM31 restated from stwo-gpu/crates/stwo/src/core/fields.
 * TEST INFRASTRUCTURE ONLY (see oracle.h). */
#include "oracle_internal.h"

/* m31.rs:41-61, 77-104 */
uint32_t orc_m31_add(uint32_t a, uint32_t b) { return m31_partial_reduce(a + b); }
uint32_t orc_m31_sub(uint32_t a, uint32_t b) { return m31_partial_reduce(a + ORC_P - b); }
uint32_t orc_m31_mul(uint32_t a, uint32_t b) { return m31_reduce((uint64_t)a * (uint64_t)b); }
uint32_t orc_m31_inv(uint32_t a) {
  /* a^(P-2) by square-and-multiply (m31.rs:63-66 uses an addition chain for
   * the same exponent 2147483645) */
  uint32_t r = 1, b = a, e = ORC_P - 2;
  while (e) {
    if (e & 1) r = orc_m31_mul(r, b);
    b = orc_m31_mul(b, b);
    e >>= 1;
  }
  return r;
}

/* cm31.rs:47-57: (a + bi)(c + di) = (ac - bd) + (ad + bc)i */
cm cm_mul(cm x, cm y) {
  cm r;
  r.a = orc_m31_sub(orc_m31_mul(x.a, y.a), orc_m31_mul(x.b, y.b));
  r.b = orc_m31_add(orc_m31_mul(x.a, y.b), orc_m31_mul(x.b, y.a));
  return r;
}
cm cm_add(cm x, cm y) { cm r = {orc_m31_add(x.a, y.a), orc_m31_add(x.b, y.b)}; return r; }
cm cm_sub(cm x, cm y) { cm r = {orc_m31_sub(x.a, y.a), orc_m31_sub(x.b, y.b)}; return r; }
cm cm_neg(cm x) { cm r = {m31_partial_reduce(ORC_P - x.a), m31_partial_reduce(ORC_P - x.b)}; return r; }
/* cm31.rs:70-76: 1/(a+bi) = (a - bi)/(a^2 + b^2) */
cm cm_inv(cm x) {
  uint32_t n = orc_m31_add(orc_m31_mul(x.a, x.a), orc_m31_mul(x.b, x.b));
  uint32_t ni = orc_m31_inv(n);
  cm c = {x.a, m31_partial_reduce(ORC_P - x.b)};
  cm r = {orc_m31_mul(c.a, ni), orc_m31_mul(c.b, ni)};
  return r;
}

/* qm31.rs:81-88: (a + bu)(c + du) = (ac + R bd) + (ad + bc)u, R = 2 + i */
qm q_mul(qm x, qm y) {
  static const cm R = {2, 1};
  qm r;
  r.lo = cm_add(cm_mul(x.lo, y.lo), cm_mul(R, cm_mul(x.hi, y.hi)));
  r.hi = cm_add(cm_mul(x.lo, y.hi), cm_mul(x.hi, y.lo));
  return r;
}
qm q_add(qm x, qm y) { qm r = {cm_add(x.lo, y.lo), cm_add(x.hi, y.hi)}; return r; }
qm q_sub(qm x, qm y) { qm r = {cm_sub(x.lo, y.lo), cm_sub(x.hi, y.hi)}; return r; }
qm q_neg(qm x) { qm r = {cm_neg(x.lo), cm_neg(x.hi)}; return r; }
/* qm31.rs:120-129: (a + bu)^-1 = (a - bu) / (a^2 - (2+i) b^2) */
qm q_inv(qm x) {
  cm b2 = cm_mul(x.hi, x.hi);
  cm ib2 = {m31_partial_reduce(ORC_P - b2.b), b2.a};
  cm denom = cm_sub(cm_mul(x.lo, x.lo), cm_add(cm_add(b2, b2), ib2));
  cm di = cm_inv(denom);
  qm r = {cm_mul(x.lo, di), cm_mul(cm_neg(x.hi), di)};
  return r;
}
qm q_from_m31(uint32_t v) { qm r = {{v, 0}, {0, 0}}; return r; }
qm q_zero(void) { return q_from_m31(0); }
qm q_one(void) { return q_from_m31(1); }
int q_eq(qm x, qm y) { return x.lo.a == y.lo.a && x.lo.b == y.lo.b && x.hi.a == y.hi.a && x.hi.b == y.hi.b; }
qm q_load(const uint32_t* w) { qm r = {{w[0], w[1]}, {w[2], w[3]}}; return r; }
void q_store(uint32_t* w, qm x) { w[0] = x.lo.a; w[1] = x.lo.b; w[2] = x.hi.a; w[3] = x.hi.b; }

void orc_qm31_add(const uint32_t* x, const uint32_t* y, uint32_t* out) { q_store(out, q_add(q_load(x), q_load(y))); }
void orc_qm31_sub(const uint32_t* x, const uint32_t* y, uint32_t* out) { q_store(out, q_sub(q_load(x), q_load(y))); }
void orc_qm31_mul(const uint32_t* x, const uint32_t* y, uint32_t* out) { q_store(out, q_mul(q_load(x), q_load(y))); }
void orc_qm31_inv(const uint32_t* x, uint32_t* out) { q_store(out, q_inv(q_load(x))); }

/* Montgomery batch inversion exactly as stwo core/fields/mod.rs:44-101
 * (WIDTH = 4 interleaved cumulative products when n > 4 and n % 4 == 0). */
static void batch_inverse_classic(const qm* col, qm* dst, size_t n) {
  if (n == 0) return;
  dst[0] = col[0];
  for (size_t i = 1; i < n; i++) dst[i] = q_mul(dst[i - 1], col[i]);
  qm cur = q_inv(dst[n - 1]);
  for (size_t i = n - 1; i >= 1; i--) {
    dst[i] = q_mul(dst[i - 1], cur);
    cur = q_mul(cur, col[i]);
  }
  dst[0] = cur;
}
void q_batch_inverse(const qm* col, qm* dst, size_t n) {
  const size_t W = 4;
  if (n <= W || n % W != 0) {
    batch_inverse_classic(col, dst, n);
    return;
  }
  qm cum[4] = {q_one(), q_one(), q_one(), q_one()};
  for (size_t i = 0; i < n; i++) {
    cum[i % W] = q_mul(cum[i % W], col[i]);
    dst[i] = cum[i % W];
  }
  qm tail[4];
  batch_inverse_classic(dst + n - W, tail, W);
  for (size_t i = n - 1; i >= W; i--) {
    dst[i] = q_mul(dst[i - W], tail[i % W]);
    tail[i % W] = q_mul(tail[i % W], col[i]);
  }
  for (size_t i = 0; i < W; i++) dst[i] = tail[i];
}
