// M31 / CM31 / QM31 arithmetic shared by host code and gfx950 kernels.
//
// Field tower (reference: stwo-gpu/crates/stwo/src/core/fields/m31.rs:14,
// cm31.rs:47, qm31.rs:14 and the product rule at qm31.rs:81-88):
//   M31  = Z / (2^31 - 1)
//   CM31 = M31[i] / (i^2 + 1)
//   QM31 = CM31[u] / (u^2 - (2 + i))
// A QM31 value is stored as four u32 words {a, b, c, d} meaning
// (a + b*i) + (c + d*i)*u, the same array-of-structs order the reference's
// device code uses (engine/src/gpu_sumcheck.rs:3614-3625).  Every function
// here returns canonical representatives in [0, P); because the arithmetic is
// exact, any evaluation order yields bit-identical results.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define GKR_HD __host__ __device__ __forceinline__

namespace gkr {

constexpr uint32_t P = 0x7fffffffu;

GKR_HD uint32_t umin32(uint32_t x, uint32_t y) { return x < y ? x : y; }

// ---------------------------------------------------------------- M31
GKR_HD uint32_t m31_add(uint32_t a, uint32_t b) {
  uint32_t s = a + b;          // < 2P < 2^32
  return umin32(s, s - P);     // s - P wraps to a huge value when s < P
}
GKR_HD uint32_t m31_sub(uint32_t a, uint32_t b) {
  uint32_t d = a - b;          // wraps when a < b
  return umin32(d, d + P);
}
GKR_HD uint32_t m31_neg(uint32_t a) { return m31_sub(0u, a); }
// Reduce x < 2^62 (a product of two canonical values, or a short sum of them).
GKR_HD uint32_t m31_reduce62(uint64_t x) {
  uint32_t r = (uint32_t)(x & P) + (uint32_t)(x >> 31);  // < 2^32
  return umin32(r, r - P);
}
// Reduce any x < 2^64.
GKR_HD uint32_t m31_reduce64(uint64_t x) {
  uint64_t y = (x & P) + (x >> 31);                       // < 2^34
  uint32_t r = (uint32_t)(y & P) + (uint32_t)(y >> 31);   // < 2^31 + 8
  return umin32(r, r - P);
}
GKR_HD uint32_t m31_mul(uint32_t a, uint32_t b) {
  return m31_reduce62((uint64_t)a * (uint64_t)b);
}
GKR_HD uint32_t m31_from_u32(uint32_t v) {  // M31::from(u32): v mod P
  uint32_t r = (v & P) + (v >> 31);
  return umin32(r, r - P);
}
GKR_HD uint32_t m31_pow(uint32_t a, uint32_t e) {
  uint32_t r = 1;
  while (e) {
    if (e & 1) r = m31_mul(r, a);
    a = m31_mul(a, a);
    e >>= 1;
  }
  return r;
}
// Fermat inverse a^(P-2); returns 0 for a == 0 (callers reject zero first).
GKR_HD uint32_t m31_inv(uint32_t a) { return m31_pow(a, P - 2); }

// ---------------------------------------------------------------- CM31
struct cm31 {
  uint32_t a, b;  // a + b*i
};
GKR_HD cm31 cm31_add(cm31 x, cm31 y) { return {m31_add(x.a, y.a), m31_add(x.b, y.b)}; }
GKR_HD cm31 cm31_sub(cm31 x, cm31 y) { return {m31_sub(x.a, y.a), m31_sub(x.b, y.b)}; }
GKR_HD cm31 cm31_neg(cm31 x) { return {m31_neg(x.a), m31_neg(x.b)}; }
GKR_HD cm31 cm31_mul(cm31 x, cm31 y) {
  // (a + bi)(c + di) = (ac - bd) + (ad + bc)i, with one reduction per part:
  // ac + (P - b)d < 2^63 and ad + bc < 2^63.
  uint64_t re = (uint64_t)x.a * y.a + (uint64_t)(P - x.b) * y.b;
  uint64_t im = (uint64_t)x.a * y.b + (uint64_t)x.b * y.a;
  return {m31_reduce64(re), m31_reduce64(im)};
}
GKR_HD cm31 cm31_mul_m31(cm31 x, uint32_t s) { return {m31_mul(x.a, s), m31_mul(x.b, s)}; }
GKR_HD cm31 cm31_inv(cm31 x) {
  // 1 / (a + bi) = (a - bi) / (a^2 + b^2)
  uint32_t n = m31_reduce64((uint64_t)x.a * x.a + (uint64_t)x.b * x.b);
  uint32_t ni = m31_inv(n);
  return {m31_mul(x.a, ni), m31_mul(m31_neg(x.b), ni)};
}
// Multiply by R = 2 + i (u^2 = R): (2 + i)(e + fi) = (2e - f) + (e + 2f)i.
GKR_HD cm31 cm31_mul_r(cm31 x) {
  uint32_t e2 = m31_add(x.a, x.a), f2 = m31_add(x.b, x.b);
  return {m31_sub(e2, x.b), m31_add(x.a, f2)};
}

// ---------------------------------------------------------------- QM31
struct qm31 {
  uint32_t a, b, c, d;  // (a + b*i) + (c + d*i)*u
};
GKR_HD qm31 qm31_make(cm31 lo, cm31 hi) { return {lo.a, lo.b, hi.a, hi.b}; }
GKR_HD cm31 qm31_lo(qm31 x) { return {x.a, x.b}; }
GKR_HD cm31 qm31_hi(qm31 x) { return {x.c, x.d}; }
GKR_HD qm31 qm31_zero() { return {0u, 0u, 0u, 0u}; }
GKR_HD qm31 qm31_one() { return {1u, 0u, 0u, 0u}; }
GKR_HD qm31 qm31_from_m31(uint32_t v) { return {v, 0u, 0u, 0u}; }
GKR_HD bool qm31_eq(qm31 x, qm31 y) { return x.a == y.a && x.b == y.b && x.c == y.c && x.d == y.d; }
GKR_HD bool qm31_is_zero(qm31 x) { return (x.a | x.b | x.c | x.d) == 0u; }
GKR_HD qm31 qm31_add(qm31 x, qm31 y) {
  return {m31_add(x.a, y.a), m31_add(x.b, y.b), m31_add(x.c, y.c), m31_add(x.d, y.d)};
}
GKR_HD qm31 qm31_sub(qm31 x, qm31 y) {
  return {m31_sub(x.a, y.a), m31_sub(x.b, y.b), m31_sub(x.c, y.c), m31_sub(x.d, y.d)};
}
GKR_HD qm31 qm31_neg(qm31 x) { return {m31_neg(x.a), m31_neg(x.b), m31_neg(x.c), m31_neg(x.d)}; }
GKR_HD qm31 qm31_mul_m31(qm31 x, uint32_t s) {
  return {m31_mul(x.a, s), m31_mul(x.b, s), m31_mul(x.c, s), m31_mul(x.d, s)};
}

// Full QM31 product with one modular reduction per output word.
//   x = (x0 + x1 i) + (x2 + x3 i) u,  y likewise,  u^2 = 2 + i.
//   lo = x_lo*y_lo + (2+i) * x_hi*y_hi,  hi = x_lo*y_hi + x_hi*y_lo.
// Each word is a signed combination of 32-bit products; subtractions are
// turned into additions of (P - v) so every intermediate is a non-negative
// u64 below 2^64.  Canonical inputs and P - v are at most P, so a product is
// at most P^2 and four of them sum to at most 4P^2 = 2^64 - 2^34 + 4: each
// output word takes a single reduction.
GKR_HD qm31 qm31_mul(qm31 x, qm31 y) {
  // t = x_hi * y_hi (CM31), kept unreduced: t.re = x2y2 - x3y3, t.im = x2y3 + x3y2
  uint64_t tre = (uint64_t)x.c * y.c + (uint64_t)(P - x.d) * y.d;   // < 2^63
  uint64_t tim = (uint64_t)x.c * y.d + (uint64_t)x.d * y.c;         // < 2^63
  uint32_t tr = m31_reduce64(tre), ti = m31_reduce64(tim);
  // (2 + i)(tr + ti i) = (2tr - ti) + (tr + 2ti) i
  uint64_t lo_re = (uint64_t)x.a * y.a + (uint64_t)(P - x.b) * y.b   // < 2^63
                   + 2ull * tr + (uint64_t)(P - ti);                  // + < 2^33
  uint64_t lo_im = (uint64_t)x.a * y.b + (uint64_t)x.b * y.a
                   + (uint64_t)tr + 2ull * ti;
  uint64_t hi_re = (uint64_t)x.a * y.c + (uint64_t)(P - x.b) * y.d    // <= 4P^2 < 2^64
                   + (uint64_t)x.c * y.a + (uint64_t)(P - x.d) * y.b;
  uint64_t hi_im = (uint64_t)x.a * y.d + (uint64_t)x.b * y.c
                   + (uint64_t)x.c * y.b + (uint64_t)x.d * y.a;
  return {m31_reduce64(lo_re), m31_reduce64(lo_im), m31_reduce64(hi_re), m31_reduce64(hi_im)};
}
GKR_HD qm31 qm31_sqr(qm31 x) { return qm31_mul(x, x); }
GKR_HD qm31 qm31_inv(qm31 x) {
  // (a + bu)^-1 = (a - bu) / (a^2 - (2 + i) b^2)   (qm31.rs:120-129)
  cm31 lo = qm31_lo(x), hi = qm31_hi(x);
  cm31 b2 = cm31_mul(hi, hi);
  cm31 denom = cm31_sub(cm31_mul(lo, lo), cm31_mul_r(b2));
  cm31 di = cm31_inv(denom);
  return qm31_make(cm31_mul(lo, di), cm31_mul(cm31_neg(hi), di));
}
// fold: x + r*(y - x)  ==  (1 - r)*x + r*y
GKR_HD qm31 qm31_fold(qm31 x, qm31 y, qm31 r) { return qm31_add(x, qm31_mul(r, qm31_sub(y, x))); }

}  // namespace gkr
