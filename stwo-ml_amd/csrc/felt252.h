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

// Montgomery product x*y*2^-256 mod p.  The 512-bit product is formed
// first (16 independent 64x64 products, so the multiplier pipelines), then
// reduced word by word: with -p^-1 = -1 mod 2^64, step i takes m = -t[i],
// which clears limb i with a carry of (t[i] != 0), and adds m*P3 at limb
// i+3 -- one product per step because p = 1 + P3*2^192.
inline felt felt_mul(const felt& x, const felt& y) {
  const uint64_t* a = x.l;
  const uint64_t* b = y.l;
  uint64_t t[8];
  u128 c;
  uint64_t k;
  c = (u128)a[0] * b[0];
  t[0] = (uint64_t)c;
  k = (uint64_t)(c >> 64);
  c = (u128)a[0] * b[1] + k;
  t[1] = (uint64_t)c;
  k = (uint64_t)(c >> 64);
  c = (u128)a[0] * b[2] + k;
  t[2] = (uint64_t)c;
  k = (uint64_t)(c >> 64);
  c = (u128)a[0] * b[3] + k;
  t[3] = (uint64_t)c;
  t[4] = (uint64_t)(c >> 64);
  for (int i = 1; i < 4; i++) {
    c = (u128)a[i] * b[0] + t[i];
    t[i] = (uint64_t)c;
    k = (uint64_t)(c >> 64);
    c = (u128)a[i] * b[1] + t[i + 1] + k;
    t[i + 1] = (uint64_t)c;
    k = (uint64_t)(c >> 64);
    c = (u128)a[i] * b[2] + t[i + 2] + k;
    t[i + 2] = (uint64_t)c;
    k = (uint64_t)(c >> 64);
    c = (u128)a[i] * b[3] + t[i + 3] + k;
    t[i + 3] = (uint64_t)c;
    t[i + 4] = (uint64_t)(c >> 64);
  }
  for (int i = 0; i < 4; i++) {
    const uint64_t m = (uint64_t)0 - t[i];
    uint64_t cc = (t[i] != 0);
    u128 s = (u128)t[i + 1] + cc;
    t[i + 1] = (uint64_t)s;
    cc = (uint64_t)(s >> 64);
    s = (u128)t[i + 2] + cc;
    t[i + 2] = (uint64_t)s;
    cc = (uint64_t)(s >> 64);
    s = (u128)t[i + 3] + (u128)m * felt_detail::P3 + cc;
    t[i + 3] = (uint64_t)s;
    cc = (uint64_t)(s >> 64);
    for (int j = i + 4; j < 8; j++) {
      s = (u128)t[j] + cc;
      t[j] = (uint64_t)s;
      cc = (uint64_t)(s >> 64);
    }
  }
  felt r{{t[4], t[5], t[6], t[7]}};
  // r < 2p: one branch-free conditional subtraction
  u128 d = (u128)r.l[0] - felt_detail::P0;
  const uint64_t s0 = (uint64_t)d;
  d = (u128)r.l[1] - ((uint64_t)(d >> 64) & 1);
  const uint64_t s1 = (uint64_t)d;
  d = (u128)r.l[2] - ((uint64_t)(d >> 64) & 1);
  const uint64_t s2 = (uint64_t)d;
  d = (u128)r.l[3] - felt_detail::P3 - ((uint64_t)(d >> 64) & 1);
  const uint64_t s3 = (uint64_t)d;
  const uint64_t keep = (uint64_t)0 - ((uint64_t)(d >> 64) & 1);
  r.l[0] = (r.l[0] & keep) | (s0 & ~keep);
  r.l[1] = (r.l[1] & keep) | (s1 & ~keep);
  r.l[2] = (r.l[2] & keep) | (s2 & ~keep);
  r.l[3] = (r.l[3] & keep) | (s3 & ~keep);
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
