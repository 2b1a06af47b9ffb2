// Poseidon hash of two felt252 (hades([a, b, 2])[0]) on the nine-limb
// device representation of felt9.h, for GPU Merkle trees.
//
// Same permutation as the host code (poseidon.h): 4 full rounds, 83 partial
// rounds with the compressed constants (one constant per partial round, the
// rest folded into the first of the last four full rounds), 4 full rounds;
// MDS [[3,1,1],[1,-1,1],[1,1,-2]].
//
// Full rounds are written as s0 = 3y0 + y1 + y2, s1 = y0 - y1 + y2,
// s2 = y0 + y1 - 2y2.  Partial rounds run on (u, w, x) = (s0 + s1, s0 - s1,
// s2): with y = x^3 and k the next partial constant,
//   u' = 2(u + w + y),  w' = 2u,  x' = u + k - 2y,
// which is the round s0' = 3s0 + s1 + y, s1' = s0 - s1 + y,
// s2' = s0 + s1 + k - 2y in sum/difference coordinates.  s0 = (u + w)/2 and
// s1 = (u - w)/2 are recovered once after the last partial round.
//
// Value bounds (p ~ 2^251, R = 2^261): hash inputs below 8p; S-box inputs
// below 9p (full) and 8p (partial) give cubes below 1.1p; u is folded below
// 2^252 every partial round; outputs are normalized and below 5.2p.
#pragma once
#include "felt9.h"

namespace gkr {
namespace f9 {

struct hades_consts {
  fe first[4][3];  // rounds 0-3 (round 0, lane 2 unused: see y2_round0)
  fe y2_round0;    // (2 + first[0][2])^3: lane 2 of round 0 when the input lane 2 is 2
  fe partial0;     // constant added to lane 2 before partial round 0
  fe kd[83];       // partial constant r + 1 plus kD4 (r < 82); kD4 alone for r = 82
  fe last[4][3];   // rounds 87-90
};

GKR_HD void add(const fe& a, const fe& b, fe& r) {
#pragma unroll
  for (int k = 0; k < kLimbs; k++) r.l[k] = a.l[k] + b.l[k];
}

GKR_HD void full_linear(const fe& y0, const fe& y1, const fe& y2, fe& a, fe& b, fe& c) {
#pragma unroll
  for (int k = 0; k < kLimbs; k++) {
    const uint32_t d = consts::d4(k);
    a.l[k] = 3u * y0.l[k] + y1.l[k] + y2.l[k];
    b.l[k] = y0.l[k] + y2.l[k] + d - y1.l[k];
    c.l[k] = y0.l[k] + y1.l[k] + d - 2u * y2.l[k];
  }
  normalize(a);
  normalize(b);
  normalize(c);
}

template <typename K>
GKR_HD void full_round(fe& a, fe& b, fe& c, const K& rc0, const K& rc1, const K& rc2) {
  fe x0, x1, x2, y0, y1, y2;
  add(a, rc0, x0);
  add(b, rc1, x1);
  add(c, rc2, x2);
  cube(x0, y0);
  cube(x1, y1);
  cube(x2, y2);
  full_linear(y0, y1, y2, a, b, c);
}

// out = hades([l, r, 2])[0]; l, r normalized, Montgomery, below 8p.
GKR_HD void hash2(const fe& l, const fe& r, const hades_consts& K, fe& out) {
  fe a, b, c;
  {
    fe x0, x1, y0, y1;
    add(l, K.first[0][0], x0);
    add(r, K.first[0][1], x1);
    cube(x0, y0);
    cube(x1, y1);
    full_linear(y0, y1, K.y2_round0, a, b, c);
  }
#pragma unroll 1
  for (int rr = 1; rr < 4; rr++) full_round(a, b, c, K.first[rr][0], K.first[rr][1], K.first[rr][2]);

  fe u, w, x;
#pragma unroll
  for (int k = 0; k < kLimbs; k++) {
    u.l[k] = a.l[k] + b.l[k];
    w.l[k] = a.l[k] + consts::d4(k) - b.l[k];
  }
  normalize(u);
  fold(u);
  normalize(w);
  add(c, K.partial0, x);
#pragma unroll 1
  for (int r = 0; r < 83; r++) {
    fe y;
    cube(x, y);
    const fe& kd = K.kd[r];
#pragma unroll
    for (int k = 0; k < kLimbs; k++) {
      const uint32_t un = u.l[k];
      u.l[k] = 2u * (un + w.l[k] + y.l[k]);
      w.l[k] = 2u * un;
      x.l[k] = un + kd.l[k] - 2u * y.l[k];
    }
    normalize(u);
    fold(u);
    normalize(x);
  }
  c = x;
#pragma unroll
  for (int k = 0; k < kLimbs; k++) {
    a.l[k] = u.l[k] + w.l[k];
    b.l[k] = u.l[k] + consts::d4(k) - w.l[k];
  }
  normalize(a);
  halve(a);
  normalize(a);
  normalize(b);
  halve(b);
  normalize(b);
#pragma unroll 1
  for (int rr = 0; rr < 3; rr++) full_round(a, b, c, K.last[rr][0], K.last[rr][1], K.last[rr][2]);
  {
    fe x0, x1, x2, y0, y1, y2;
    add(a, K.last[3][0], x0);
    add(b, K.last[3][1], x1);
    add(c, K.last[3][2], x2);
    cube(x0, y0);
    cube(x1, y1);
    cube(x2, y2);
#pragma unroll
    for (int k = 0; k < kLimbs; k++) out.l[k] = 3u * y0.l[k] + y1.l[k] + y2.l[k];
    normalize(out);
  }
}

}  // namespace f9
}  // namespace gkr
