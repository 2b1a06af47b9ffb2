/* Internal helpers of the CPU oracle.  TEST INFRASTRUCTURE ONLY. */
#ifndef GKR_ORACLE_INTERNAL_H
#define GKR_ORACLE_INTERNAL_H
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define ORC_P 0x7fffffffu

/* m31.rs:41-43 partial_reduce: val in [0, 2P) */
static inline uint32_t m31_partial_reduce(uint32_t v) { return v >= ORC_P ? v - ORC_P : v; }
/* m31.rs:58-60 reduce: val in [0, P^2) */
static inline uint32_t m31_reduce(uint64_t v) {
  return (uint32_t)(((((v >> 31) + v + 1) >> 31) + v) & (uint64_t)ORC_P);
}
/* M31::from(u32) */
static inline uint32_t m31_from(uint32_t v) { return (uint32_t)((uint64_t)v % ORC_P); }

typedef struct { uint32_t a, b; } cm;
typedef struct { cm lo, hi; } qm;

cm cm_mul(cm x, cm y);
cm cm_add(cm x, cm y);
cm cm_sub(cm x, cm y);
cm cm_neg(cm x);
cm cm_inv(cm x);
qm q_mul(qm x, qm y);
qm q_add(qm x, qm y);
qm q_sub(qm x, qm y);
qm q_neg(qm x);
qm q_inv(qm x);
qm q_from_m31(uint32_t v);
qm q_zero(void);
qm q_one(void);
int q_eq(qm x, qm y);
qm q_load(const uint32_t* w);
void q_store(uint32_t* w, qm x);
void q_batch_inverse(const qm* col, qm* dst, size_t n);

/* felt252 in Montgomery form (poseidon.c) */
typedef struct { uint64_t v[4]; } fe;
fe fe_from_u64(uint64_t x);
fe fe_from_words(const uint32_t w[8]);
void fe_to_words(fe x, uint32_t w[8]);
fe fe_pack_m31s(const uint32_t* v, int n);
fe fe_hash_many(const fe* in, size_t n);
fe fe_hash2(fe a, fe b);

/* matmul.c helpers shared with logup.c / verify.c */
qm mle_evaluate(const qm* evals, int n_vars, const qm* point); /* copies evals */
void mle_eq_evals(const qm* r, int n, qm* out);

#endif
