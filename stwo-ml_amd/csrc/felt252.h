// Host arithmetic in the Stark prime field p = 2^251 + 17*2^192 + 1.
//
// Elements are four little-endian u64 limbs in Montgomery form (R = 2^256).
// p's limbs are {1, 0, 0, 0x0800000000000011}, so -p^-1 mod 2^64 is
// 0xffff_ffff_ffff_ffff and each Montgomery reduction step needs only one
// 64x64 product (m * p3) besides the addition of m itself.  This is the
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

inline felt felt_add(const felt& x, const felt& y) {
  felt r;
  u128 c = 0;
  for (int i = 0; i < 4; i++) {
    c = (u128)x.l[i] + y.l[i] + (uint64_t)(c >> 64);
    r.l[i] = (uint64_t)c;
  }
  // x, y < p < 2^252, so no carry out of limb 3.
  if (felt_detail::geq_p(r.l)) felt_detail::sub_p(r.l);
  return r;
}

inline felt felt_sub(const felt& x, const felt& y) {
  felt r;
  uint64_t borrow = 0;
  for (int i = 0; i < 4; i++) {
    u128 d = (u128)x.l[i] - y.l[i] - borrow;
    r.l[i] = (uint64_t)d;
    borrow = (uint64_t)(d >> 64) & 1;
  }
  if (borrow) {  // add p back
    u128 c = (u128)r.l[0] + felt_detail::P0;
    r.l[0] = (uint64_t)c;
    c = (u128)r.l[1] + felt_detail::P1 + (uint64_t)(c >> 64); r.l[1] = (uint64_t)c;
    c = (u128)r.l[2] + felt_detail::P2 + (uint64_t)(c >> 64); r.l[2] = (uint64_t)c;
    r.l[3] = r.l[3] + felt_detail::P3 + (uint64_t)(c >> 64);
  }
  return r;
}

// Montgomery product x*y*2^-256 mod p (coarsely integrated operand scanning).
inline felt felt_mul(const felt& x, const felt& y) {
  uint64_t t0 = 0, t1 = 0, t2 = 0, t3 = 0, t4 = 0;
  for (int i = 0; i < 4; i++) {
    const uint64_t yi = y.l[i];
    u128 c = (u128)x.l[0] * yi + t0;
    t0 = (uint64_t)c;
    c = (u128)x.l[1] * yi + t1 + (uint64_t)(c >> 64); t1 = (uint64_t)c;
    c = (u128)x.l[2] * yi + t2 + (uint64_t)(c >> 64); t2 = (uint64_t)c;
    c = (u128)x.l[3] * yi + t3 + (uint64_t)(c >> 64); t3 = (uint64_t)c;
    u128 top = (u128)t4 + (uint64_t)(c >> 64);
    // m = t0 * (-p^-1) = -t0;  t + m*p = t + m + m*P3*2^192, low limb cancels.
    const uint64_t m = (uint64_t)0 - t0;
    uint64_t carry = (t0 != 0);  // t0 + m == 2^64 exactly when t0 != 0
    c = (u128)t1 + carry; uint64_t n0 = (uint64_t)c;
    c = (u128)t2 + (uint64_t)(c >> 64); uint64_t n1 = (uint64_t)c;
    c = (u128)t3 + (u128)m * felt_detail::P3 + (uint64_t)(c >> 64); uint64_t n2 = (uint64_t)c;
    top += (uint64_t)(c >> 64);
    t0 = n0; t1 = n1; t2 = n2; t3 = (uint64_t)top; t4 = (uint64_t)(top >> 64);
  }
  felt r{{t0, t1, t2, t3}};
  // result < 2p < 2^253, so t4 == 0 here
  if (felt_detail::geq_p(r.l)) felt_detail::sub_p(r.l);
  return r;
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
