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

/* All levels of a Poseidon Merkle tree over n leaves (padded with zero felts to
 * a power of two, at least 2): level s holds N >> s nodes at off[s]. */
typedef struct {
  fe* nodes;
  size_t off[64];
  int height;
} orc_tree;

static void tree_build(orc_tree* t, const fe* leaves, size_t n) {
  size_t N = 2;
  while (N < n) N <<= 1;
  t->nodes = (fe*)calloc(2 * N, sizeof(fe));
  memcpy(t->nodes, leaves, n * sizeof(fe));
  t->off[0] = 0;
  t->height = 0;
  size_t len = N, o = 0;
  while (len > 1) {
    const size_t no = o + len;
    for (size_t i = 0; i < len / 2; i++) t->nodes[no + i] = fe_hash2(t->nodes[o + 2 * i], t->nodes[o + 2 * i + 1]);
    o = no;
    len /= 2;
    t->off[++t->height] = o;
  }
}

typedef struct {
  uint32_t* out;
  size_t cap, n;
} felt_sink;
static void sink_u(felt_sink* s, uint64_t v) {
  if (s->n < s->cap) {
    uint32_t* w = s->out + 8 * s->n;
    memset(w, 0, 32);
    w[0] = (uint32_t)v;
    w[1] = (uint32_t)(v >> 32);
  }
  s->n++;
}
static void sink_f(felt_sink* s, fe x) {
  if (s->n < s->cap) fe_to_words(x, s->out + 8 * s->n);
  s->n++;
}
static void sink_q(felt_sink* s, qm x) {
  uint32_t w[4];
  q_store(w, x);
  for (int i = 0; i < 4; i++) sink_u(s, w[i]);
}

/* prove_mle_opening_with_commitment (engine/src/crypto/mle_opening.rs:1654-1915):
 * mix the root of the evaluations; fold on the top variable with each
 * challenge (f'[j] = f[j] + r (f[mid + j] - f[j])), committing and mixing every
 * folded layer longer than 1; draw min(n_queries, len / 2) query pairs
 * (low 64 bits of draw_felt252 mod len / 2, reduced mod max(mid / 2, 1) per
 * round); for each query and round, the pair's values and both Merkle paths.
 * Output: the serialized MleOpeningProof (serialize_mle_opening_proof,
 * cairo_serde.rs:341-369), felt count returned (written up to cap); the
 * initial root goes to commitment. */
size_t orc_mle_opening(const uint32_t* evals, size_t len, const uint32_t* challenges, size_t n_queries_cfg,
                       orc_channel* ch, uint32_t commitment[8], uint32_t* out, size_t cap) {
  int n_vars = 0;
  while (((size_t)1 << n_vars) < len) n_vars++;
  qm** layers = (qm**)calloc((size_t)n_vars + 1, sizeof(qm*));
  orc_tree* trees = (orc_tree*)calloc((size_t)n_vars + 1, sizeof(orc_tree));
  layers[0] = (qm*)malloc(len * sizeof(qm));
  for (size_t i = 0; i < len; i++) layers[0][i] = q_load(evals + 4 * i);
  felt_sink s = {out, cap, 0};
  uint32_t w[8];
  for (int t = 0; t <= n_vars; t++) {
    const size_t L = len >> t;
    if (t == 0 || L > 1) {
      fe* leaves = (fe*)malloc(L * sizeof(fe));
      for (size_t i = 0; i < L; i++) {
        uint32_t q[4];
        q_store(q, layers[t][i]);
        leaves[i] = fe_pack_m31s(q, 4);
      }
      tree_build(&trees[t], leaves, L);
      free(leaves);
      fe_to_words(trees[t].nodes[trees[t].off[trees[t].height]], w);
      orc_mix_felt(ch, w);
      if (t == 0) memcpy(commitment, w, 32);
    }
    if (t == n_vars) break;
    const qm r = q_load(challenges + 4 * t);
    const size_t mid = L / 2;
    layers[t + 1] = (qm*)malloc(mid * sizeof(qm));
    for (size_t j = 0; j < mid; j++)
      layers[t + 1][j] = q_add(layers[t][j], q_mul(r, q_sub(layers[t][mid + j], layers[t][j])));
  }
  /* intermediate roots (layers 1 .. n_vars - 1) */
  sink_u(&s, n_vars > 0 ? (uint64_t)(n_vars - 1) : 0);
  for (int t = 1; t < n_vars; t++) sink_f(&s, trees[t].nodes[trees[t].off[trees[t].height]]);
  const size_t half = len / 2;
  const size_t nq = n_queries_cfg < half ? n_queries_cfg : half;
  sink_u(&s, nq);
  for (size_t q = 0; q < nq; q++) {
    orc_draw_felt252(ch, w);
    const uint64_t raw = (uint64_t)w[0] | ((uint64_t)w[1] << 32);
    size_t idx = (size_t)(raw % half);
    sink_u(&s, idx);
    sink_u(&s, (uint64_t)n_vars);
    for (int t = 0; t < n_vars; t++) {
      const size_t L = len >> t, mid = L / 2;
      const size_t li = idx, ri = mid + idx;
      sink_q(&s, layers[t][li]);
      sink_q(&s, layers[t][ri]);
      const orc_tree* tr = &trees[t];
      for (int side = 0; side < 2; side++) {
        size_t k = side ? ri : li;
        sink_u(&s, (uint64_t)tr->height);
        for (int lv = 0; lv < tr->height; lv++) {
          sink_f(&s, tr->nodes[tr->off[lv] + (k ^ 1)]);
          k >>= 1;
        }
      }
      const size_t next_half = mid / 2 > 1 ? mid / 2 : 1;
      idx %= next_half;
    }
  }
  sink_q(&s, layers[n_vars][0]);
  for (int t = 0; t <= n_vars; t++) {
    free(layers[t]);
    free(trees[t].nodes);
  }
  free(layers);
  free(trees);
  return s.n;
}
