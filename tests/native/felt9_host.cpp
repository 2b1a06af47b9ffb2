// Test-only host build of the device felt252 arithmetic (stwo-ml_amd/csrc/
// felt9.h, poseidon9.h): the same source the GPU kernels use, compiled for the
// CPU so tests can compare it with the oracle's Poseidon without a GPU.
#include "../../stwo-ml_amd/csrc/poseidon9_host.h"

using namespace gkr;

namespace {
f9::fe to_mont(const uint32_t w[8]) {
  f9::fe x, m;
  f9::from_words(w, x);
  f9::mul(x, f9::host_setup().r2, m);
  return m;
}
void to_canonical(const f9::fe& m, uint32_t w[8]) {
  f9::fe x;
  f9::mul(m, f9::host_setup().one, x);
  f9::canonicalize(x);
  f9::to_words(x, w);
}
}  // namespace

extern "C" {
// out = hades([a, b, 2])[0] for canonical a, b (8 little-endian words each).
// ka, kb add ka * p and kb * p to the Montgomery inputs (representatives up to 8p).
int f9_hash2(const uint32_t* a, const uint32_t* b, uint32_t ka, uint32_t kb, uint32_t* out) {
  f9::fe A = to_mont(a), B = to_mont(b), O;
  f9::canonicalize(A);
  f9::canonicalize(B);
  A.l[0] += ka; A.l[6] += ka * f9::kP6; A.l[8] += ka * f9::kP8;
  B.l[0] += kb; B.l[6] += kb * f9::kP6; B.l[8] += kb * f9::kP8;
  f9::normalize(A);
  f9::normalize(B);
  f9::hash2(A, B, f9::host_setup().k, O);
  for (int k = 0; k < 9; k++)
    if (O.l[k] >> 29) return 1;  // output must be normalized
  to_canonical(O, out);
  return 0;
}
// n chained hashes: (x, y) <- (H(x, y), x), Montgomery values never canonicalized.
void f9_chain(const uint32_t* x0, const uint32_t* y0, int n, uint32_t* out) {
  f9::fe x = to_mont(x0), y = to_mont(y0);
  for (int i = 0; i < n; i++) {
    f9::fe o;
    f9::hash2(x, y, f9::host_setup().k, o);
    y = x;
    x = o;
  }
  to_canonical(x, out);
}
// Montgomery round trip and product: out = a * b mod p (canonical).
void f9_mulmod(const uint32_t* a, const uint32_t* b, uint32_t* out) {
  f9::fe A = to_mont(a), B = to_mont(b), O;
  f9::mul(A, B, O);
  to_canonical(O, out);
}
}
