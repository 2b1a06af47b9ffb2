// Host arithmetic in the Stark prime field p = 2^251 + 17*2^192 + 1.
//
// Elements are four little-endian u64 limbs in Montgomery form (R = 2^256).
// p's limbs are {1, 0, 0, 0x0800000000000011}, so -p^-1 mod 2^64 is
// 0xffff_ffff_ffff_ffff and each Montgomery reduction step needs only one
// 64x64 product (m * p3) besides the addition of m itself.  Additions and
// subtractions are branch-free (masked select of the reduced value).  This is the
// field of the reference's Poseidon channel (engine/src/crypto/
// poseidon_channel.rs, via starknet-ff 0.3.7).
#pragma once
#include <stdint.h>
#include <string.h>

namespace gkr {

typedef unsigned __int128 u128;

struct felt {
  uint64_t l[4];
};

namespace felt_detail {
constexpr uint64_t P0 = 1ull, P1 = 0ull, P2 = 0ull, P3 = 0x0800000000000011ull;

inline bool geq_p(const uint64_t t[4]) {
  if (t[3] != P3) return t[3] > P3;
  if (t[2] != P2) return t[2] > P2;
  if (t[1] != P1) return t[1] > P1;
  return t[0] >= P0;
}
inline void sub_p(uint64_t t[4]) {
  u128 c = (u128)t[0] - P0;
  t[0] = (uint64_t)c;
  uint64_t borrow = (uint64_t)(c >> 64) & 1;
  c = (u128)t[1] - P1 - borrow; t[1] = (uint64_t)c; borrow = (uint64_t)(c >> 64) & 1;
  c = (u128)t[2] - P2 - borrow; t[2] = (uint64_t)c; borrow = (uint64_t)(c >> 64) & 1;
  t[3] = t[3] - P3 - borrow;
}
}  // namespace felt_detail

inline felt felt_raw(uint64_t l0, uint64_t l1, uint64_t l2, uint64_t l3) { return felt{{l0, l1, l2, l3}}; }

inline bool felt_eq(const felt& x, const felt& y) {
  return x.l[0] == y.l[0] && x.l[1] == y.l[1] && x.l[2] == y.l[2] && x.l[3] == y.l[3];
}

// Branch-free: r = x + y, s = r - p, keep s when the subtraction did not borrow.
inline felt felt_add(const felt& x, const felt& y) {
  u128 c = (u128)x.l[0] + y.l[0];
  const uint64_t r0 = (uint64_t)c;
  c = (u128)x.l[1] + y.l[1] + (uint64_t)(c >> 64);
  const uint64_t r1 = (uint64_t)c;
  c = (u128)x.l[2] + y.l[2] + (uint64_t)(c >> 64);
  const uint64_t r2 = (uint64_t)c;
  const uint64_t r3 = x.l[3] + y.l[3] + (uint64_t)(c >> 64);  // x, y < p < 2^252: no carry out
  u128 d = (u128)r0 - felt_detail::P0;
  const uint64_t s0 = (uint64_t)d;
  d = (u128)r1 - ((uint64_t)(d >> 64) & 1);
  const uint64_t s1 = (uint64_t)d;
  d = (u128)r2 - ((uint64_t)(d >> 64) & 1);
  const uint64_t s2 = (uint64_t)d;
  d = (u128)r3 - felt_detail::P3 - ((uint64_t)(d >> 64) & 1);
  const uint64_t s3 = (uint64_t)d;
  const uint64_t keep_r = (uint64_t)0 - ((uint64_t)(d >> 64) & 1);  // all ones when r < p
  return felt{{(r0 & keep_r) | (s0 & ~keep_r), (r1 & keep_r) | (s1 & ~keep_r), (r2 & keep_r) | (s2 & ~keep_r),
               (r3 & keep_r) | (s3 & ~keep_r)}};
}

// Branch-free: r = x - y, add p back (masked) when it borrowed.
inline felt felt_sub(const felt& x, const felt& y) {
  u128 d = (u128)x.l[0] - y.l[0];
  const uint64_t r0 = (uint64_t)d;
  d = (u128)x.l[1] - y.l[1] - ((uint64_t)(d >> 64) & 1);
  const uint64_t r1 = (uint64_t)d;
  d = (u128)x.l[2] - y.l[2] - ((uint64_t)(d >> 64) & 1);
  const uint64_t r2 = (uint64_t)d;
  d = (u128)x.l[3] - y.l[3] - ((uint64_t)(d >> 64) & 1);
  const uint64_t r3 = (uint64_t)d;
  const uint64_t add_p = (uint64_t)0 - ((uint64_t)(d >> 64) & 1);
  u128 c = (u128)r0 + (felt_detail::P0 & add_p);
  const uint64_t o0 = (uint64_t)c;
  c = (u128)r1 + (uint64_t)(c >> 64);
  const uint64_t o1 = (uint64_t)c;
  c = (u128)r2 + (uint64_t)(c >> 64);
  const uint64_t o2 = (uint64_t)c;
  const uint64_t o3 = r3 + (felt_detail::P3 & add_p) + (uint64_t)(c >> 64);
  return felt{{o0, o1, o2, o3}};
}

// Add/subtract with carry (clang builtins; they compile to adc/sbb chains).
inline uint64_t adc64(uint64_t a, uint64_t b, uint64_t cin, uint64_t* cout) {
  unsigned long long co;
  const uint64_t r = __builtin_addcll(a, b, cin, &co);
  *cout = co;
  return r;
}
inline uint64_t sbb64(uint64_t a, uint64_t b, uint64_t bin, uint64_t* bout) {
  unsigned long long bo;
  const uint64_t r = __builtin_subcll(a, b, bin, &bo);
  *bout = bo;
  return r;
}

// Montgomery product x*y*2^-256 mod p without the final subtraction,
// coarsely integrated (row by row): t += x_i * y, then with -p^-1 = -1 mod
// 2^64 the multiplier is m = -t0, which clears limb 0 with a carry of
// (t0 != 0), and m*p adds m*P3 at limb 3 because p = 1 + P3*2^192.  For
// x*y < 8p^2 (e.g. x < 4p, y < 2p) the result is below 2p.
inline felt felt_mul_lazy(const felt& x, const felt& y) {
  const uint64_t b0 = y.l[0], b1 = y.l[1], b2 = y.l[2], b3 = y.l[3];
  uint64_t t0 = 0, t1 = 0, t2 = 0, t3 = 0, t4 = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint64_t ai = x.l[i];
    const u128 q0 = (u128)ai * b0, q1 = (u128)ai * b1, q2 = (u128)ai * b2, q3 = (u128)ai * b3;
    uint64_t c, l1, l2, l3, h3 = (uint64_t)(q3 >> 64);
    l1 = adc64((uint64_t)q1, (uint64_t)(q0 >> 64), 0, &c);
    l2 = adc64((uint64_t)q2, (uint64_t)(q1 >> 64), c, &c);
    l3 = adc64((uint64_t)q3, (uint64_t)(q2 >> 64), c, &c);
    h3 += c;  // x_i * y < 2^64 * 2^254: the top limb cannot overflow
    t0 = adc64(t0, (uint64_t)q0, 0, &c);
    t1 = adc64(t1, l1, c, &c);
    t2 = adc64(t2, l2, c, &c);
    t3 = adc64(t3, l3, c, &c);
    t4 += h3 + c;
    const uint64_t m = (uint64_t)0 - t0;
    const u128 mp = (u128)m * felt_detail::P3;
    const uint64_t n1 = adc64(t1, 0, t0 != 0, &c);
    const uint64_t n2 = adc64(t2, 0, c, &c);
    const uint64_t n3 = adc64(t3, (uint64_t)mp, c, &c);
    const uint64_t n4 = adc64(t4, (uint64_t)(mp >> 64), c, &c);
    t0 = n1; t1 = n2; t2 = n3; t3 = n4; t4 = c;
  }
  return felt{{t0, t1, t2, t3}};
}
// Montgomery square x*x*2^-256 mod p without the final subtraction, for
// x < 4p (result < 2p).  The 512-bit square takes 10 products (the six cross
// products, doubled, plus the four diagonal ones); the reduction is done in
// one step: the multiplier M with T + M*p = 0 mod 2^256 is
// M = -L - X*2^192 where L = T mod 2^256 and X = (-t0)*P3 mod 2^64 (because
// M*p = M + M*P3*2^192 and only M's lowest limb reaches limb 3 of the
// second term), and the result is T_hi + (M*P3 >> 64) + c with the carry
// c = (L != 0) + (n3 < X) out of the vanishing low half.
inline felt felt_sqr_lazy(const felt& x) {
  const uint64_t a0 = x.l[0], a1 = x.l[1], a2 = x.l[2], a3 = x.l[3];
  const u128 p01 = (u128)a0 * a1, p02 = (u128)a0 * a2, p03 = (u128)a0 * a3;
  const u128 p12 = (u128)a1 * a2, p13 = (u128)a1 * a3, p23 = (u128)a2 * a3;
  uint64_t c;
  uint64_t c1 = (uint64_t)p01;
  uint64_t c2 = adc64((uint64_t)(p01 >> 64), (uint64_t)p02, 0, &c);
  uint64_t c3 = adc64((uint64_t)(p02 >> 64), (uint64_t)p03, c, &c);
  uint64_t c4 = adc64((uint64_t)(p03 >> 64), (uint64_t)p13, c, &c);
  uint64_t c5 = adc64((uint64_t)(p13 >> 64), (uint64_t)p23, c, &c);
  uint64_t c6 = (uint64_t)(p23 >> 64) + c;
  c3 = adc64(c3, (uint64_t)p12, 0, &c);
  c4 = adc64(c4, (uint64_t)(p12 >> 64), c, &c);
  c5 = adc64(c5, 0, c, &c);
  c6 += c;
  const uint64_t c7 = c6 >> 63;  // doubling
  c6 = (c6 << 1) | (c5 >> 63);
  c5 = (c5 << 1) | (c4 >> 63);
  c4 = (c4 << 1) | (c3 >> 63);
  c3 = (c3 << 1) | (c2 >> 63);
  c2 = (c2 << 1) | (c1 >> 63);
  c1 = c1 << 1;
  const u128 d0 = (u128)a0 * a0, d1 = (u128)a1 * a1, d2 = (u128)a2 * a2, d3 = (u128)a3 * a3;
  const uint64_t t0 = (uint64_t)d0;
  const uint64_t t1 = adc64(c1, (uint64_t)(d0 >> 64), 0, &c);
  const uint64_t t2 = adc64(c2, (uint64_t)d1, c, &c);
  const uint64_t t3 = adc64(c3, (uint64_t)(d1 >> 64), c, &c);
  const uint64_t t4 = adc64(c4, (uint64_t)d2, c, &c);
  const uint64_t t5 = adc64(c5, (uint64_t)(d2 >> 64), c, &c);
  const uint64_t t6 = adc64(c6, (uint64_t)d3, c, &c);
  const uint64_t t7 = adc64(c7, (uint64_t)(d3 >> 64), c, &c);
  uint64_t b;
  const uint64_t n0 = sbb64(0, t0, 0, &b);
  const uint64_t n1 = sbb64(0, t1, b, &b);
  const uint64_t n2 = sbb64(0, t2, b, &b);
  const uint64_t n3 = sbb64(0, t3, b, &b);
  const uint64_t X = n0 * felt_detail::P3;
  const uint64_t m3 = n3 - X;
  const uint64_t cc = b + (n3 < X);
  const u128 q0 = (u128)n0 * felt_detail::P3, q1 = (u128)n1 * felt_detail::P3;
  const u128 q2 = (u128)n2 * felt_detail::P3, q3 = (u128)m3 * felt_detail::P3;
  uint64_t e;
  const uint64_t w1 = adc64((uint64_t)(q0 >> 64), (uint64_t)q1, 0, &e);
  const uint64_t w2 = adc64((uint64_t)(q1 >> 64), (uint64_t)q2, e, &e);
  const uint64_t w3 = adc64((uint64_t)(q2 >> 64), (uint64_t)q3, e, &e);
  const uint64_t w4 = (uint64_t)(q3 >> 64) + e;
  const uint64_t r0 = adc64(t4, w1, cc, &e);
  const uint64_t r1 = adc64(t5, w2, e, &e);
  const uint64_t r2 = adc64(t6, w3, e, &e);
  const uint64_t r3 = t7 + w4 + e;
  return felt{{r0, r1, r2, r3}};
}
// [0, 2p) -> [0, p): one branch-free conditional subtraction of p.
inline felt felt_reduce_once(const felt& r) {
  uint64_t b;
  const uint64_t s0 = sbb64(r.l[0], felt_detail::P0, 0, &b);
  const uint64_t s1 = sbb64(r.l[1], 0, b, &b);
  const uint64_t s2 = sbb64(r.l[2], 0, b, &b);
  const uint64_t s3 = sbb64(r.l[3], felt_detail::P3, b, &b);
  const uint64_t keep = (uint64_t)0 - b;  // all ones when r < p
  return felt{{(r.l[0] & keep) | (s0 & ~keep), (r.l[1] & keep) | (s1 & ~keep), (r.l[2] & keep) | (s2 & ~keep),
               (r.l[3] & keep) | (s3 & ~keep)}};
}
// Montgomery product x*y*2^-256 mod p of canonical inputs, canonical output.
inline felt felt_mul(const felt& x, const felt& y) { return felt_reduce_once(felt_mul_lazy(x, y)); }

// Lazy domain [0, 2p) for the permutation's inner loop: sums and differences
// are brought back below 2p with one masked correction by 2p.
inline felt felt_add_lazy(const felt& x, const felt& y) {
  constexpr uint64_t TP0 = 2 * felt_detail::P0, TP3 = 2 * felt_detail::P3;
  uint64_t c, b;
  const uint64_t r0 = adc64(x.l[0], y.l[0], 0, &c);
  const uint64_t r1 = adc64(x.l[1], y.l[1], c, &c);
  const uint64_t r2 = adc64(x.l[2], y.l[2], c, &c);
  const uint64_t r3 = adc64(x.l[3], y.l[3], c, &c);  // < 4p < 2^254: no carry out
  const uint64_t s0 = sbb64(r0, TP0, 0, &b);
  const uint64_t s1 = sbb64(r1, 0, b, &b);
  const uint64_t s2 = sbb64(r2, 0, b, &b);
  const uint64_t s3 = sbb64(r3, TP3, b, &b);
  const uint64_t keep = (uint64_t)0 - b;
  return felt{{(r0 & keep) | (s0 & ~keep), (r1 & keep) | (s1 & ~keep), (r2 & keep) | (s2 & ~keep),
               (r3 & keep) | (s3 & ~keep)}};
}
inline felt felt_sub_lazy(const felt& x, const felt& y) {
  constexpr uint64_t TP0 = 2 * felt_detail::P0, TP3 = 2 * felt_detail::P3;
  uint64_t b, c;
  const uint64_t r0 = sbb64(x.l[0], y.l[0], 0, &b);
  const uint64_t r1 = sbb64(x.l[1], y.l[1], b, &b);
  const uint64_t r2 = sbb64(x.l[2], y.l[2], b, &b);
  const uint64_t r3 = sbb64(x.l[3], y.l[3], b, &b);
  const uint64_t m = (uint64_t)0 - b;
  const uint64_t o0 = adc64(r0, TP0 & m, 0, &c);
  const uint64_t o1 = adc64(r1, 0, c, &c);
  const uint64_t o2 = adc64(r2, 0, c, &c);
  const uint64_t o3 = adc64(r3, TP3 & m, c, &c);
  return felt{{o0, o1, o2, o3}};
}

// Montgomery constants.  R mod p and R^2 mod p are derived once by doubling.
struct felt_consts {
  felt one_m;   // R mod p (Montgomery 1)
  felt r2;      // R^2 mod p
  felt_consts() {
    felt x{{1, 0, 0, 0}};           // plain 1 (valid as a canonical integer)
    for (int i = 0; i < 256; i++) x = felt_add(x, x);
    one_m = x;
    for (int i = 0; i < 256; i++) x = felt_add(x, x);
    r2 = x;
  }
};
inline const felt_consts& felt_k() {
  static const felt_consts k;
  return k;
}

// Canonical integer (< p) -> Montgomery form.
inline felt felt_to_mont(const felt& canon) { return felt_mul(canon, felt_k().r2); }
// Montgomery form -> canonical integer (< p).
inline felt felt_from_mont(const felt& m) { return felt_mul(m, felt{{1, 0, 0, 0}}); }

inline felt felt_from_u64(uint64_t v) { return felt_to_mont(felt{{v, 0, 0, 0}}); }
inline felt felt_zero() { return felt{{0, 0, 0, 0}}; }
inline felt felt_one() { return felt_k().one_m; }

// Canonical value <-> 8 little-endian u32 words (the reference's GPU/channel
// state layout, engine/src/crypto/poseidon_constants.rs:75-86).
inline void felt_canon_to_words(const felt& canon, uint32_t w[8]) {
  for (int i = 0; i < 4; i++) {
    w[2 * i] = (uint32_t)canon.l[i];
    w[2 * i + 1] = (uint32_t)(canon.l[i] >> 32);
  }
}
inline felt felt_canon_from_words(const uint32_t w[8]) {
  felt r;
  for (int i = 0; i < 4; i++) r.l[i] = (uint64_t)w[2 * i] | ((uint64_t)w[2 * i + 1] << 32);
  return r;
}

}  // namespace gkr
