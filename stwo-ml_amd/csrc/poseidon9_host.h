// Host-side set-up for the device Poseidon (poseidon9.h): round constants and
// Montgomery conversion constants in the nine-limb, R = 2^261 representation,
// derived from the host permutation's compressed constants (poseidon.h).
#pragma once
#include "poseidon.h"
#include "poseidon9.h"

namespace gkr {
namespace f9 {

// Canonical integer below p -> limbs (no Montgomery conversion).
inline fe from_canonical(const felt& canon) {
  uint32_t w[8];
  felt_canon_to_words(canon, w);
  fe r;
  from_words(w, r);
  return r;
}

// Host Montgomery form (x * 2^256 mod p) -> device Montgomery form (x * 2^261 mod p).
inline fe from_host_mont(const felt& m) {
  felt v = m;
  for (int i = 0; i < 5; i++) v = felt_add(v, v);
  return from_canonical(v);
}

struct setup {
  hades_consts k;
  fe r2;   // 2^522 mod p: mul(x, r2) takes a canonical x to Montgomery form
  fe one;  // plain 1: mul(x, one) takes Montgomery form back to a representative of x
  setup() {
    const hades_rc& h = hades_constants();
    for (int r = 0; r < 4; r++)
      for (int j = 0; j < 3; j++) {
        k.first[r][j] = from_host_mont(h.full_first[r][j]);
        k.last[r][j] = from_host_mont(h.full_last[r][j]);
      }
    fe x2;
    add(from_host_mont(felt_from_u64(2)), k.first[0][2], x2);
    cube(x2, k.y2_round0);
    k.partial0 = from_host_mont(h.partial[0]);
    for (int r = 0; r < 83; r++) {
      fe c = r + 1 < 83 ? from_host_mont(h.partial[r + 1]) : fe{};
      for (int i = 0; i < kLimbs; i++) k.kd[r].l[i] = c.l[i] + consts::d4(i);
    }
    felt x{{1, 0, 0, 0}};
    for (int i = 0; i < 522; i++) x = felt_add(x, x);
    r2 = from_canonical(x);
    one = fe{};
    one.l[0] = 1;
  }
};

inline const setup& host_setup() {
  static const setup s;
  return s;
}

}  // namespace f9
}  // namespace gkr
