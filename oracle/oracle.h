/*
 * CPU oracle for the GKR matmul / LogUp path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU prover, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker
 * and the timed CPU baseline.  The product library never links or calls it.
 *
 * Each function cites the reference file:line it restates.  Values:
 *   QM31 = 4 x u32 {a, b, c, d} = (a + b i) + (c + d i) u, canonical M31 words
 *   felt = 8 x u32 little-endian words of a canonical felt252
 * Parity pinning: see the table at the end of this comment.
 */
#ifndef GKR_ORACLE_H
#define GKR_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------- fields (field.c) */
uint32_t orc_m31_add(uint32_t a, uint32_t b);
uint32_t orc_m31_sub(uint32_t a, uint32_t b);
uint32_t orc_m31_mul(uint32_t a, uint32_t b);
uint32_t orc_m31_inv(uint32_t a);
void orc_qm31_add(const uint32_t* x, const uint32_t* y, uint32_t* out);
void orc_qm31_sub(const uint32_t* x, const uint32_t* y, uint32_t* out);
void orc_qm31_mul(const uint32_t* x, const uint32_t* y, uint32_t* out);
void orc_qm31_inv(const uint32_t* x, uint32_t* out);

/* ---------------------------------------------------------- Poseidon (poseidon.c) */
typedef struct {
  uint64_t digest[4]; /* Montgomery form */
  uint32_t n_draws;
  uint64_t hash_count;
} orc_channel;

void orc_sha256(const uint8_t* msg, size_t len, uint8_t out[32]);
void orc_hades_constant(int idx, uint32_t out[8]); /* raw round constant idx (canonical) */
void orc_hades(uint32_t state[24]);                 /* 3 felts */
void orc_hash_many(const uint32_t* felts, size_t n, uint32_t out[8]);
void orc_channel_init(orc_channel* ch);
void orc_mix_u64(orc_channel* ch, uint64_t v);
void orc_mix_felt(orc_channel* ch, const uint32_t w[8]);
void orc_mix_secure_field(orc_channel* ch, const uint32_t q[4]);
void orc_mix_felts(orc_channel* ch, const uint32_t* q, size_t n);
void orc_mix_felts_stwo(orc_channel* ch, const uint32_t* q, size_t n);
void orc_trace(const orc_channel* ch, const char* label, long index);
void orc_mix_poly_coeffs(orc_channel* ch, const uint32_t c[12]);
void orc_mix_poly_coeffs_deg3(orc_channel* ch, const uint32_t c[16]);
void orc_draw_felt252(orc_channel* ch, uint32_t out[8]);
void orc_draw_qm31(orc_channel* ch, uint32_t out[4]);
void orc_draw_qm31s(orc_channel* ch, size_t n, uint32_t* out);
void orc_digest(const orc_channel* ch, uint32_t out[8]);
void orc_channel_set_state(orc_channel* ch, const uint32_t st[11]);
size_t orc_channel_size(void);

/* ---------------------------------------------------------- MLE / matmul (matmul.c) */
void orc_evaluate_mle(const uint32_t* evals, int n_vars, const uint32_t* point, uint32_t out[4]);
void orc_inner_product_q(const uint32_t* fa, const uint32_t* fb, size_t n, uint32_t out[4]);
void orc_restrict_mle(const uint32_t* evals, size_t len, const uint32_t* assign, int s, uint32_t* out);
void orc_lagrange_basis(const uint32_t* c, int n, uint32_t* out);
void orc_eq_evals(const uint32_t* r, int n, uint32_t* out);
void orc_matmul_forward(const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n, uint32_t* C);
void orc_matmul_output_claim(const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n,
                             const uint32_t* r_out, int n_vars, uint32_t out[4]);
int orc_reduce_matmul_layer(const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n,
                            const uint32_t* r_i, int n_ri, const uint32_t* r_j, int n_rj, size_t pk,
                            orc_channel* ch, uint32_t* round_polys, uint32_t* challenges, uint32_t* final_a,
                            uint32_t* final_b);
int orc_prove_matmul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                           const uint32_t* A, size_t m, size_t k, const uint32_t* B, size_t n, orc_channel* ch,
                           uint32_t* round_polys, uint32_t* final_a, uint32_t* final_b, uint32_t* next_point,
                           uint32_t* next_value);
void orc_restrict_cols_fused(const uint32_t* B, size_t k, size_t n, const uint32_t* r_j, int n_rj, size_t pk,
                             uint32_t* out);
void orc_restrict_rows_fused(const uint32_t* A, size_t m, size_t k, const uint32_t* r_i, int n_ri, size_t pk,
                             uint32_t* out);
uint32_t orc_synthetic_value(int kind, uint64_t seed, uint64_t i);
void orc_synthetic_fill(uint32_t* out, size_t n, int kind, uint64_t seed);

/* ---------------------------------------------------------- LogUp (logup.c) */
uint32_t orc_activation(uint32_t tag, uint32_t v);
int orc_prove_activation_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                               const uint32_t* X, size_t rows, size_t cols, uint32_t tag, uint32_t table_log,
                               orc_channel* ch, uint32_t* claimed_sum, uint32_t* eq_round_polys,
                               uint32_t* final_evals /* w, in, out */, uint32_t* multiplicities,
                               uint32_t* mult_round_polys, uint32_t* mult_final, uint32_t* mult_sum,
                               uint32_t* input_eval, uint32_t* table_commitment);

/* ---------------------------------------------------------- verifier (verify.c) */
/* MLE commitments (commit.c): Poseidon Merkle root over securefield_to_felt leaves. */
void orc_mle_commitment(const uint32_t* evals_qm31, size_t len, uint32_t out[8]);
void orc_weight_commitment(const uint32_t* B, size_t k, size_t n, uint32_t out[8]);
size_t orc_mle_opening(const uint32_t* evals, size_t len, const uint32_t* challenges, size_t n_queries_cfg,
                       orc_channel* ch, uint32_t commitment[8], uint32_t* out, size_t cap);
/* The product-sumcheck round loop over QM31 vectors of length n (matmul.c). */
int orc_sumcheck_product(const uint32_t* fa, const uint32_t* fb, size_t n, orc_channel* ch, uint32_t* round_polys,
                         uint32_t* challenges, uint32_t* final_a, uint32_t* final_b);
/* Mul layer (mul.c): lhs/rhs n QM31 each; eq_round_polys 4*log2(n) QM31. */
int orc_reduce_mul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                         const uint32_t* lhs, const uint32_t* rhs, size_t n, orc_channel* ch,
                         uint32_t* eq_round_polys, uint32_t* lhs_eval, uint32_t* rhs_eval, uint32_t* alpha_out,
                         uint32_t* next_value);
/* verify_mul_reduction (verify.c); c0c2c3: 3 QM31 per round; writes the next claim value. */
int orc_verify_mul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                         const uint32_t* c0c2c3, int n_rounds, const uint32_t* lhs_eval, const uint32_t* rhs_eval,
                         orc_channel* ch, uint32_t* next_value);
int orc_verify_matmul_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value, size_t m,
                            size_t k, size_t n, const uint32_t* c0c2 /* 8 words per round */, int n_rounds,
                            const uint32_t* final_a, const uint32_t* final_b, orc_channel* ch,
                            uint32_t* next_point, uint32_t* next_value);
int orc_verify_activation_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                                uint32_t tag, uint32_t table_log, const uint32_t* claimed_sum,
                                const uint32_t* c0c2c3 /* 12 words per round */, int n_rounds,
                                const uint32_t* final_evals, const uint32_t* multiplicities,
                                const uint32_t* mult_round_polys, const uint32_t* mult_final,
                                const uint32_t* mult_sum, const uint32_t* input_eval, orc_channel* ch);

/* ---------------------------------------------------------- LayerNorm / RMSNorm (norm.c) */
/* Outputs of reduce_layernorm_layer / reduce_rmsnorm_layer_with_gamma
 * (prover.rs:7944-8395, 8407-8801).  Caller-provided arrays: the three
 * round-polynomial arrays hold 16 words (c0..c3) per round (nv rounds),
 * multiplicities 2^16, mult_round_polys 16 x (c0, c1), row_stats0/1 one word
 * per padded row.  RMSNorm uses mean_eval for rms_sq_eval, sum0 for the
 * square sum, p0_final0 for its final input value, lin_final0/1 for
 * (input_final, scale_final), row_stats0 for the per-row rms_sq; var_eval,
 * sum1, p0_final1, cb_input, cb_mean and row_stats1 are LayerNorm-only. */
typedef struct {
  uint32_t input_eval[4], output_eval[4], mean_eval[4], rsqrt_eval[4], var_eval[4];
  uint32_t n_active;
  uint32_t sum0[4], sum1[4];
  uint32_t* p0_round_polys;
  uint32_t p0_final0[4], p0_final1[4];
  uint32_t* lin_round_polys;
  uint32_t lin_final0[4], lin_final1[4];
  uint32_t cb_input[4], cb_mean[4];
  uint32_t claimed_sum[4];
  uint32_t* logup_round_polys;
  uint32_t w_eval[4], in_eval[4], out_eval[4];
  uint32_t* multiplicities;
  uint32_t* mult_round_polys;
  uint32_t mult_final[4], mult_sum[4];
  uint32_t table_commitment[8];
  uint32_t n_rows;
  uint32_t* row_stats0;
  uint32_t* row_stats1;
  uint32_t gamma_commitment[8], gamma_eval[4];
} orc_norm_out;
uint32_t orc_rsqrt(uint32_t v); /* build_rsqrt_table entry (layernorm.rs:116-135) */
void orc_layernorm_forward(const uint32_t* X, size_t rows, size_t cols, size_t dim, uint32_t* out_padded);
void orc_rmsnorm_forward(const uint32_t* X, size_t rows, size_t cols, size_t dim, const uint32_t* gamma, size_t ng,
                         uint32_t* out_padded);
int orc_prove_layernorm_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value,
                              const uint32_t* X, size_t rows, size_t cols, size_t dim, orc_channel* ch,
                              orc_norm_out* out);
int orc_prove_rmsnorm_layer(const uint32_t* claim_point, int n_point, const uint32_t* claim_value, const uint32_t* X,
                            size_t rows, size_t cols, size_t dim, const uint32_t* gamma, size_t ng, orc_channel* ch,
                            orc_norm_out* out);
int orc_verify_layernorm_layer(const uint32_t* claim_point, int nv, const uint32_t* claim_value, size_t dim,
                               const orc_norm_out* p, orc_channel* ch, uint32_t next_value[4]);
int orc_verify_rmsnorm_layer(const uint32_t* claim_point, int nv, const uint32_t* claim_value, size_t dim,
                             const orc_norm_out* p, orc_channel* ch, uint32_t next_value[4]);

#ifdef __cplusplus
}
#endif

/* STWO LogUp-GKR / grand-product batch (lookup_gkr.c).  kind: 0 grand
 * product (den = the column), 1 LogUp generic (num QM31), 2 LogUp with M31
 * multiplicities (num u32), 3 LogUp singles (numerators 1). */
typedef struct {
  uint32_t kind, n_vars;
  const uint32_t* num;
  const uint32_t* den;
} orc_lookup_layer;
/* Dense proof layout: output_claims / claims_to_verify 2 QM31 per instance;
 * round_polys 4 QM31 per round (layers 0.. n_layers-1, `layer` rounds each)
 * with round_poly_lens the coefficient counts; masks 4 QM31 per (layer,
 * instance), zero where the instance is not active; ood_point n_layers QM31. */
typedef struct {
  uint32_t* output_claims;
  uint32_t* round_polys;
  uint32_t* round_poly_lens;
  uint32_t* masks;
  uint32_t* ood_point;
  uint32_t* claims_to_verify;
  uint32_t n_layers;
} orc_lookup_out;
int orc_prove_lookup_batch(orc_channel* ch, const orc_lookup_layer* inst, size_t n_inst, orc_lookup_out* out);
int orc_verify_lookup_batch(const uint32_t* gates, const uint32_t* n_vars, size_t n_inst, const orc_lookup_out* p,
                            orc_channel* ch, uint32_t* ood_out, uint32_t* claims_out);

#endif
