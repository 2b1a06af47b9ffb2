/* MLE commitments, restated from engine/src/crypto/mle_opening.rs:630-640
 * (commit_mle_root_only) and engine/src/crypto/poseidon_merkle.rs:255-280
 * (PoseidonMerkleTree::root_only_parallel): leaves securefield_to_felt(v)
 * (poseidon_channel.rs:59-69), padded with zero felts to a power of two (at
 * least 2), internal node = poseidon_hash(left, right).  The weight
 * commitment of a k x n matrix commits to matrix_to_mle_col_major_padded
 * (prover.rs:1021-1023): B[i][j] at index j * pk + i.  TEST INFRASTRUCTURE
 * ONLY. */
#include "oracle_internal.h"

static fe merkle_root(fe* leaves, size_t n_leaves) {
  size_t n = 2;
  while (n < n_leaves) n <<= 1;
  for (size_t i = n_leaves; i < n; i++) memset(&leaves[i], 0, sizeof(fe)); /* FieldElement::ZERO */
  while (n > 1) {
    for (size_t i = 0; i < n / 2; i++) leaves[i] = fe_hash2(leaves[2 * i], leaves[2 * i + 1]);
    n /= 2;
  }
  return leaves[0];
}

void orc_mle_commitment(const uint32_t* evals_qm31, size_t len, uint32_t out[8]) {
  size_t n = 2;
  while (n < len) n <<= 1;
  fe* leaves = (fe*)malloc(n * sizeof(fe));
  for (size_t i = 0; i < len; i++) leaves[i] = fe_pack_m31s(evals_qm31 + 4 * i, 4);
  fe root = merkle_root(leaves, len);
  free(leaves);
  fe_to_words(root, out);
}

void orc_weight_commitment(const uint32_t* B, size_t k, size_t n, uint32_t out[8]) {
  size_t pk = 1, pn = 1;
  while (pk < k) pk <<= 1;
  while (pn < n) pn <<= 1;
  const size_t len = pk * pn;
  uint32_t* q = (uint32_t*)calloc(4 * len, sizeof(uint32_t));
  for (size_t i = 0; i < k; i++)
    for (size_t j = 0; j < n; j++) q[4 * (j * pk + i)] = m31_from(B[i * n + j]);
  orc_mle_commitment(q, len, out);
  free(q);
}
