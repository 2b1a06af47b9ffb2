// Host-side QM31 arithmetic four values at a time (AVX2), for the sumcheck
// rounds the host finishes on the last few hundred entries of a vector: the
// host thread is the prover's critical path there, and a scalar QM31 product
// with its six reductions costs it ~70 instructions.
//
// Values are canonical QM31 in the array-of-structs layout of field.h (four
// u32 words a, b, c, d per value, meaning (a + b i) + (c + d i) u, u^2 = 2 + i).
// In registers, word w of four values sits in the low halves of the four
// 64-bit lanes of one vector, so _mm256_mul_epu32 forms the 32 x 32 -> 64-bit
// products.  Every result is the canonical representative, the same as the
// scalar field code gives (the arithmetic is exact).
//
// Self-contained (no HIP headers), so that a host-only test can compile it.
#pragma once
#include <immintrin.h>
#include <stddef.h>
#include <stdint.h>

namespace hostfield {

constexpr uint32_t kP = 0x7fffffffu;

// ------------------------------------------------------------------ scalar
inline uint32_t m_add(uint32_t a, uint32_t b) {
  const uint32_t s = a + b;
  const uint32_t t = s - kP;
  return s < t ? s : t;
}
inline uint32_t m_sub(uint32_t a, uint32_t b) {
  const uint32_t d = a - b;
  const uint32_t t = d + kP;
  return d < t ? d : t;
}
inline uint32_t m_red64(uint64_t x) {
  const uint64_t y = (x & kP) + (x >> 31);
  const uint32_t r = (uint32_t)(y & kP) + (uint32_t)(y >> 31);
  const uint32_t t = r - kP;
  return r < t ? r : t;
}
struct Q {
  uint32_t w[4];
};
inline Q q_ld(const uint32_t* p) { return Q{{p[0], p[1], p[2], p[3]}}; }
inline void q_st(uint32_t* p, const Q& q) {
  p[0] = q.w[0];
  p[1] = q.w[1];
  p[2] = q.w[2];
  p[3] = q.w[3];
}
inline Q q_add(const Q& x, const Q& y) {
  return Q{{m_add(x.w[0], y.w[0]), m_add(x.w[1], y.w[1]), m_add(x.w[2], y.w[2]), m_add(x.w[3], y.w[3])}};
}
inline Q q_sub(const Q& x, const Q& y) {
  return Q{{m_sub(x.w[0], y.w[0]), m_sub(x.w[1], y.w[1]), m_sub(x.w[2], y.w[2]), m_sub(x.w[3], y.w[3])}};
}
// The product of field.h's qm31_mul: (x_lo + x_hi u)(y_lo + y_hi u) with
// u^2 = 2 + i, one reduction per output word (and two for x_hi y_hi).
inline Q q_mul(const Q& x, const Q& y) {
  const uint64_t a = x.w[0], b = x.w[1], c = x.w[2], d = x.w[3];
  const uint64_t e = y.w[0], f = y.w[1], g = y.w[2], h = y.w[3];
  const uint32_t tr = m_red64(c * g + (kP - d) * h), ti = m_red64(c * h + d * g);
  const uint64_t lo_re = a * e + (kP - b) * f + 2ull * tr + (uint64_t)(kP - ti);
  const uint64_t lo_im = a * f + b * e + (uint64_t)tr + 2ull * ti;
  const uint64_t hi_re = (uint64_t)m_red64(a * g + (kP - b) * h) + c * e + (kP - d) * f;
  const uint64_t hi_im = (uint64_t)m_red64(a * h + b * g) + c * f + d * e;
  return Q{{m_red64(lo_re), m_red64(lo_im), m_red64(hi_re), m_red64(hi_im)}};
}

// ------------------------------------------------------------------ four at a time
struct Q4 {
  __m256i a, b, c, d;
};
inline __m256i v_p() { return _mm256_set1_epi64x(kP); }
inline __m256i v_lo32() { return _mm256_set1_epi64x(0xffffffffll); }
// min(s, s - P) per 32-bit lane; the high halves of the lanes stay 0
inline __m256i v_canon(__m256i s) { return _mm256_min_epu32(s, _mm256_sub_epi32(s, v_p())); }
inline __m256i v_add(__m256i x, __m256i y) { return v_canon(_mm256_add_epi32(x, y)); }
inline __m256i v_sub(__m256i x, __m256i y) {
  const __m256i dd = _mm256_sub_epi32(x, y);
  return _mm256_and_si256(_mm256_min_epu32(dd, _mm256_add_epi32(dd, v_p())), v_lo32());
}
// x < 2^64 per 64-bit lane -> canonical
inline __m256i v_red64(__m256i x) {
  const __m256i p = v_p();
  const __m256i y = _mm256_add_epi64(_mm256_and_si256(x, p), _mm256_srli_epi64(x, 31));
  const __m256i r = _mm256_add_epi64(_mm256_and_si256(y, p), _mm256_srli_epi64(y, 31));
  return v_canon(r);
}
inline __m256i v_mul(__m256i x, __m256i y) { return _mm256_mul_epu32(x, y); }
inline Q4 q4_add(const Q4& x, const Q4& y) {
  return Q4{v_add(x.a, y.a), v_add(x.b, y.b), v_add(x.c, y.c), v_add(x.d, y.d)};
}
inline Q4 q4_sub(const Q4& x, const Q4& y) {
  return Q4{v_sub(x.a, y.a), v_sub(x.b, y.b), v_sub(x.c, y.c), v_sub(x.d, y.d)};
}
inline Q4 q4_mul(const Q4& x, const Q4& y) {
  const __m256i p = v_p();
  const __m256i nb = _mm256_sub_epi64(p, x.b), nd = _mm256_sub_epi64(p, x.d);
  const __m256i tr = v_red64(_mm256_add_epi64(v_mul(x.c, y.c), v_mul(nd, y.d)));
  const __m256i ti = v_red64(_mm256_add_epi64(v_mul(x.c, y.d), v_mul(x.d, y.c)));
  __m256i lo_re = _mm256_add_epi64(v_mul(x.a, y.a), v_mul(nb, y.b));
  lo_re = _mm256_add_epi64(lo_re, _mm256_add_epi64(_mm256_add_epi64(tr, tr), _mm256_sub_epi64(p, ti)));
  __m256i lo_im = _mm256_add_epi64(v_mul(x.a, y.b), v_mul(x.b, y.a));
  lo_im = _mm256_add_epi64(lo_im, _mm256_add_epi64(tr, _mm256_add_epi64(ti, ti)));
  __m256i hi_re = v_red64(_mm256_add_epi64(v_mul(x.a, y.c), v_mul(nb, y.d)));
  hi_re = _mm256_add_epi64(hi_re, _mm256_add_epi64(v_mul(x.c, y.a), v_mul(nd, y.b)));
  __m256i hi_im = v_red64(_mm256_add_epi64(v_mul(x.a, y.d), v_mul(x.b, y.c)));
  hi_im = _mm256_add_epi64(hi_im, _mm256_add_epi64(v_mul(x.c, y.b), v_mul(x.d, y.a)));
  return Q4{v_red64(lo_re), v_red64(lo_im), v_red64(hi_re), v_red64(hi_im)};
}
// four consecutive values p[0..3] (16 words)
inline Q4 q4_ld(const uint32_t* p) {
  const __m256i idx = _mm256_setr_epi32(0, 1, 4, 5, 2, 3, 6, 7);
  const __m256i t0 = _mm256_permutevar8x32_epi32(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(p)), idx);
  const __m256i t1 = _mm256_permutevar8x32_epi32(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(p + 8)), idx);
  const __m256i ab = _mm256_permute2x128_si256(t0, t1, 0x20);  // a b of values 0 1 | 2 3
  const __m256i cd = _mm256_permute2x128_si256(t0, t1, 0x31);
  const __m256i m = v_lo32();
  return Q4{_mm256_and_si256(ab, m), _mm256_srli_epi64(ab, 32), _mm256_and_si256(cd, m), _mm256_srli_epi64(cd, 32)};
}
inline void q4_st(uint32_t* p, const Q4& q) {
  const __m256i idx = _mm256_setr_epi32(0, 1, 4, 5, 2, 3, 6, 7);
  const __m256i ab = _mm256_or_si256(q.a, _mm256_slli_epi64(q.b, 32));
  const __m256i cd = _mm256_or_si256(q.c, _mm256_slli_epi64(q.d, 32));
  _mm256_storeu_si256(reinterpret_cast<__m256i*>(p),
                      _mm256_permutevar8x32_epi32(_mm256_permute2x128_si256(ab, cd, 0x20), idx));
  _mm256_storeu_si256(reinterpret_cast<__m256i*>(p + 8),
                      _mm256_permutevar8x32_epi32(_mm256_permute2x128_si256(ab, cd, 0x31), idx));
}
inline Q4 q4_bcast(const uint32_t* q) {
  return Q4{_mm256_set1_epi64x(q[0]), _mm256_set1_epi64x(q[1]), _mm256_set1_epi64x(q[2]), _mm256_set1_epi64x(q[3])};
}
inline Q4 q4_zero() { return Q4{_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256()}; }
// the sum of the four values
inline Q q4_hsum(const Q4& v) {
  alignas(32) uint64_t w[4][4];
  _mm256_store_si256(reinterpret_cast<__m256i*>(w[0]), v.a);
  _mm256_store_si256(reinterpret_cast<__m256i*>(w[1]), v.b);
  _mm256_store_si256(reinterpret_cast<__m256i*>(w[2]), v.c);
  _mm256_store_si256(reinterpret_cast<__m256i*>(w[3]), v.d);
  Q s{{0, 0, 0, 0}};
  for (int k = 0; k < 4; k++)
    for (int l = 0; l < 4; l++) s.w[k] = m_add(s.w[k], (uint32_t)w[k][l]);
  return s;
}

// ------------------------------------------------------------------ sumcheck rounds
// V (2 half values) <- V[i] + r (V[i + half] - V[i]) for i < half.
inline void fold(uint32_t* V, size_t half, const uint32_t r[4]) {
  size_t i = 0;
  const Q4 r4 = q4_bcast(r);
  for (; i + 4 <= half; i += 4) {
    const Q4 x = q4_ld(V + 4 * i), y = q4_ld(V + 4 * (i + half));
    q4_st(V + 4 * i, q4_add(x, q4_mul(r4, q4_sub(y, x))));
  }
  const Q rq = q_ld(r);
  for (; i < half; i++) {
    const Q x = q_ld(V + 4 * i), y = q_ld(V + 4 * (i + half));
    q_st(V + 4 * i, q_add(x, q_mul(rq, q_sub(y, x))));
  }
}
// A degree-2 product round over A, B (2 half values each): out[t] =
// sum_i a_t(i) b_t(i) at t = 0, 1, 2 (x_2 = 2 x_1 - x_0).
inline void product_round(const uint32_t* A, const uint32_t* B, size_t half, uint32_t out[3][4]) {
  Q4 s0 = q4_zero(), s1 = q4_zero(), s2 = q4_zero();
  size_t i = 0;
  for (; i + 4 <= half; i += 4) {
    const Q4 a0 = q4_ld(A + 4 * i), a1 = q4_ld(A + 4 * (i + half));
    const Q4 b0 = q4_ld(B + 4 * i), b1 = q4_ld(B + 4 * (i + half));
    s0 = q4_add(s0, q4_mul(a0, b0));
    s1 = q4_add(s1, q4_mul(a1, b1));
    s2 = q4_add(s2, q4_mul(q4_sub(q4_add(a1, a1), a0), q4_sub(q4_add(b1, b1), b0)));
  }
  Q t0 = q4_hsum(s0), t1 = q4_hsum(s1), t2 = q4_hsum(s2);
  for (; i < half; i++) {
    const Q a0 = q_ld(A + 4 * i), a1 = q_ld(A + 4 * (i + half)), b0 = q_ld(B + 4 * i), b1 = q_ld(B + 4 * (i + half));
    t0 = q_add(t0, q_mul(a0, b0));
    t1 = q_add(t1, q_mul(a1, b1));
    t2 = q_add(t2, q_mul(q_sub(q_add(a1, a1), a0), q_sub(q_add(b1, b1), b0)));
  }
  q_st(out[0], t0);
  q_st(out[1], t1);
  q_st(out[2], t2);
}
// A degree-3 eq-weighted round over E, W, D (2 half values each): out[t] =
// sum_i e_t(i) w_t(i) d_t(i) at t = 0 .. 3 (x_{t+1} = x_t + (x_1 - x_0)).
inline void eq3_round(const uint32_t* E, const uint32_t* W, const uint32_t* D, size_t half, uint32_t out[4][4]) {
  Q4 s[4] = {q4_zero(), q4_zero(), q4_zero(), q4_zero()};
  size_t i = 0;
  for (; i + 4 <= half; i += 4) {
    Q4 e = q4_ld(E + 4 * i), w = q4_ld(W + 4 * i), d = q4_ld(D + 4 * i);
    const Q4 e1 = q4_ld(E + 4 * (i + half)), w1 = q4_ld(W + 4 * (i + half)), d1 = q4_ld(D + 4 * (i + half));
    const Q4 de = q4_sub(e1, e), dw = q4_sub(w1, w), dd = q4_sub(d1, d);
    for (int t = 0; t < 4; t++) {
      if (t) {
        e = q4_add(e, de);
        w = q4_add(w, dw);
        d = q4_add(d, dd);
      }
      s[t] = q4_add(s[t], q4_mul(q4_mul(e, w), d));
    }
  }
  Q r[4];
  for (int t = 0; t < 4; t++) r[t] = q4_hsum(s[t]);
  for (; i < half; i++) {
    Q e = q_ld(E + 4 * i), w = q_ld(W + 4 * i), d = q_ld(D + 4 * i);
    const Q de = q_sub(q_ld(E + 4 * (i + half)), e), dw = q_sub(q_ld(W + 4 * (i + half)), w),
            dd = q_sub(q_ld(D + 4 * (i + half)), d);
    for (int t = 0; t < 4; t++) {
      if (t) {
        e = q_add(e, de);
        w = q_add(w, dw);
        d = q_add(d, dd);
      }
      r[t] = q_add(r[t], q_mul(q_mul(e, w), d));
    }
  }
  for (int t = 0; t < 4; t++) q_st(out[t], r[t]);
}
// out[0] = sum of V[0 .. half), out[1] = sum of V[half .. 2 half)
inline void halves_sum(const uint32_t* V, size_t half, uint32_t out[2][4]) {
  Q4 s0 = q4_zero(), s1 = q4_zero();
  size_t i = 0;
  for (; i + 4 <= half; i += 4) {
    s0 = q4_add(s0, q4_ld(V + 4 * i));
    s1 = q4_add(s1, q4_ld(V + 4 * (i + half)));
  }
  Q t0 = q4_hsum(s0), t1 = q4_hsum(s1);
  for (; i < half; i++) {
    t0 = q_add(t0, q_ld(V + 4 * i));
    t1 = q_add(t1, q_ld(V + 4 * (i + half)));
  }
  q_st(out[0], t0);
  q_st(out[1], t1);
}

}  // namespace hostfield
