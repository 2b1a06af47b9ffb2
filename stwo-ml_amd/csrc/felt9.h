// felt252 arithmetic for GPU lanes: p = 2^251 + 17*2^192 + 1 held in nine
// 29-bit limbs (261 bits), Montgomery form with R = 2^261.
//
// Why 29 bits: a product of two limbs below 2^30 is below 2^60, so a column
// of at most nine such products plus the reduction terms stays below 2^64.
// Every partial product is then one v_mad_u64_u32 into a 64-bit column
// accumulator with no carry handling; carries are resolved once, during the
// reduction.  The prime has three non-zero limbs (limb 0 = 1, limb 6 =
// 17*2^18, limb 8 = 2^19) and -p^-1 = -1 mod 2^29, so each of the nine
// Montgomery steps is m = -t_i mod 2^29, a shift for the carry, one mad for
// m*limb6 and one shift-add for m*limb8.
//
// Representation rules (all values are representatives, not canonical):
//   normalized: limbs in [0, 2^29), value below 2^261;
//   mul/sqr inputs: limbs below 2^30 (the sum of two normalized values is
//     fine), output normalized with value < p + a*b/R;
//   the linear layer adds limb-wise and subtracts through kD4, a
//     representation of 4p whose limbs dominate any normalized subtrahend
//     below 1.1p (limbs 0-7 at least 2^30 - 2, limb 8 at least 2^21 - 2).
// Functions are __host__ __device__ so the same code runs in CPU tests.
#pragma once
#include <stdint.h>

#ifndef GKR_HD
#if defined(__HIPCC__)
#define GKR_HD __host__ __device__ __forceinline__
#else
#define GKR_HD inline
#endif
#endif

namespace gkr {
namespace f9 {

constexpr int kLimbs = 9;
constexpr uint32_t kMask = (1u << 29) - 1;
constexpr uint32_t kP6 = 17u << 18;  // limb 6 of p
constexpr uint32_t kP8 = 1u << 19;   // limb 8 of p

struct fe {
  uint32_t l[kLimbs];
};

// kD4: 4p = 2^253 + 68*2^192 + 4 with 2^30 moved from each limb i+1 into limb i
// (adds 2^30 to limb i and subtracts 2 from limb i+1, value unchanged).
struct consts {
  static constexpr uint32_t d4(int i) {
    return i == 0 ? 4u + (1u << 30)
           : i == 6 ? (68u << 18) + (1u << 30) - 2u
           : i == 8 ? (1u << 21) - 2u
                    : (1u << 30) - 2u;
  }
};

// t (18 unnormalized 64-bit columns of a product, with 1 pre-added to columns
// 1..9) -> t / 2^261 mod p, normalized.  Step i takes m = 2^29 - (t_i mod 2^29),
// in [1, 2^29] and congruent to -t_i, so t_i + m = (floor(t_i / 2^29) + 1) 2^29:
// the carry into t_(i+1) is one shift, its "+1" being the pre-added 1.  The sum
// of the m's stays below 2^261 (1 + 2^-29), so the result is below p (1 + 2^-29)
// + t / 2^261.
// Hides a constant from the optimizer, so that it stays a multiplier or an
// addend of v_mad_u64_u32 instead of being rewritten as separate shifts/adds.
template <typename T>
GKR_HD T opaque(T v) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm("" : "+s"(v));
#endif
  return v;
}

GKR_HD void mont_reduce(uint64_t t[18], fe& r) {
  const uint32_t p6 = opaque(kP6), p8 = opaque(kP8);
#pragma unroll
  for (int i = 0; i < 9; i++) {
    const uint32_t m = (((uint32_t)t[i] & kMask) ^ kMask) + 1u;  // 2^29 - (t_i mod 2^29)
    t[i + 1] += t[i] >> 29;
    t[i + 6] += (uint64_t)m * p6;
    t[i + 8] += (uint64_t)m * p8;
  }
  uint64_t c = t[9];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    r.l[k] = (uint32_t)c & kMask;
    c = (c >> 29) + t[10 + k];
  }
  r.l[8] = (uint32_t)c;
}

// Product columns start at 1 for k = 1..9 (the reduction's carry increments).
GKR_HD void mul(const fe& a, const fe& b, fe& r) {
  uint64_t t[18];
  const uint64_t one = opaque((uint64_t)1);
#pragma unroll
  for (int k = 0; k < 18; k++) t[k] = (k >= 1 && k <= 9) ? one : 0u;
#pragma unroll
  for (int i = 0; i < 9; i++)
#pragma unroll
    for (int j = 0; j < 9; j++) t[i + j] += (uint64_t)a.l[i] * b.l[j];
  mont_reduce(t, r);
}

// Off-diagonal products taken once against the doubled limbs (2 a_i < 2^31,
// so a column stays below 4 * 2^61 + 2^60 plus the reduction terms).
GKR_HD void sqr(const fe& a, fe& r) {
  uint64_t t[18];
  const uint64_t one = opaque((uint64_t)1);
#pragma unroll
  for (int k = 0; k < 18; k++) t[k] = (k >= 1 && k <= 9) ? one : 0u;
  uint32_t d[9];
#pragma unroll
  for (int i = 0; i < 9; i++) d[i] = a.l[i] << 1;
#pragma unroll
  for (int i = 0; i < 9; i++) {
    t[2 * i] += (uint64_t)a.l[i] * a.l[i];
#pragma unroll
    for (int j = i + 1; j < 9; j++) t[i + j] += (uint64_t)d[i] * a.l[j];
  }
  mont_reduce(t, r);
}

// x^3
GKR_HD void cube(const fe& x, fe& r) {
  fe x2;
  sqr(x, x2);
  mul(x2, x, r);
}

// Carry propagation of non-negative limbs below 2^32; value must be below 2^261.
GKR_HD void normalize(fe& a) {
  uint32_t c = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const uint32_t v = a.l[k] + c;  // a.l[k] < 2^32 - 8 and c < 8 in every caller
    a.l[k] = v & kMask;
    c = v >> 29;
  }
  a.l[8] += c;
}

// Signed carry propagation (limbs read as int32); value must be in [0, 2^261).
GKR_HD void normalize_signed(fe& a) {
  int32_t c = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int32_t v = (int32_t)a.l[k] + c;
    a.l[k] = (uint32_t)v & kMask;
    c = v >> 29;  // arithmetic shift
  }
  a.l[8] = (uint32_t)((int32_t)a.l[8] + c);
}

// Normalized a -> normalized value congruent mod p and below 2^252: with
// h = a >> 251, subtract max(h - 1, 0) * p.
// Requires h < 2^7 (value below 2^258) so the limb 6 adjustment fits.
GKR_HD void fold(fe& a) {
  const int32_t h = (int32_t)(a.l[8] >> 19);
  const int32_t k = h > 0 ? h - 1 : 0;
  a.l[8] -= (uint32_t)k << 19;
  a.l[6] = (uint32_t)((int32_t)a.l[6] - k * (int32_t)kP6);
  a.l[0] = (uint32_t)((int32_t)a.l[0] - k);
  normalize_signed(a);
}

// a / 2 mod p for normalized a: add p when odd, then shift right by one bit.
// Output limbs below 2^29 + 2^28.
GKR_HD void halve(fe& a) {
  const uint32_t odd = a.l[0] & 1u;
  a.l[0] += odd;
  a.l[6] += odd * kP6;
  a.l[8] += odd * kP8;
#pragma unroll
  for (int k = 0; k < 8; k++) a.l[k] = (a.l[k] >> 1) + ((a.l[k + 1] & 1u) << 28);
  a.l[8] >>= 1;
}

// Canonical 256-bit little-endian words <-> limbs (no Montgomery conversion).
GKR_HD void from_words(const uint32_t w[8], fe& r) {
#pragma unroll
  for (int k = 0; k < 9; k++) {
    const int bit = 29 * k, wi = bit >> 5, off = bit & 31;
    uint64_t v = (uint64_t)w[wi] >> off;
    if (wi + 1 < 8) v |= (uint64_t)w[wi + 1] << (32 - off);
    r.l[k] = (uint32_t)v & kMask;
  }
}
GKR_HD void to_words(const fe& a, uint32_t w[8]) {
  uint64_t acc = 0;
  int have = 0, k = 0;
#pragma unroll
  for (int wi = 0; wi < 8; wi++) {
    while (have < 32 && k < 9) {
      acc |= (uint64_t)a.l[k++] << have;
      have += 29;
    }
    w[wi] = (uint32_t)acc;
    acc >>= 32;
    have -= 32;
  }
}

// Normalized value in [0, 2^253) -> canonical residue in [0, p).
GKR_HD void canonicalize(fe& a) {
  // subtract p up to 4 times (value < 2^253 < 5p)
#pragma unroll
  for (int rep = 0; rep < 4; rep++) {
    fe d;
    int32_t c = 0;
#pragma unroll
    for (int k = 0; k < 9; k++) {
      const uint32_t pk = k == 0 ? 1u : k == 6 ? kP6 : k == 8 ? kP8 : 0u;
      int32_t v = (int32_t)a.l[k] - (int32_t)pk + c;
      c = v >> 29;
      d.l[k] = k < 8 ? ((uint32_t)v & kMask) : (uint32_t)v;
    }
    if ((int32_t)d.l[8] >= 0) a = d;
  }
}

}  // namespace f9
}  // namespace gkr
