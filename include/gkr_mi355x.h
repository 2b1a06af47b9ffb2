/*
 * gkr_mi355x.h -- C ABI of the MI355X GKR sumcheck prover (matmul + LogUp layers).
 *
 * Plain C types only: pointers, sizes and the two value structs below.
 * Every function returns GKR_OK (0) on success or a GKR_ERR_* code; the
 * message of the last failure on the calling thread is gkr_last_error().
 * This mirrors the reference's Result<_, String> convention
 * (engine/src/backend.rs:85-107, engine/src/gkr/prover.rs:6017-6022).
 *
 * Value conventions
 *   gkr_qm31  {v0, v1, v2, v3} = (v0 + v1*i) + (v2 + v3*i)*u, each word a
 *             canonical M31 in [0, 2^31 - 1)  (stwo core/fields/qm31.rs:14-33)
 *   gkr_felt  a canonical felt252 (< 2^251 + 17*2^192 + 1) as 8 little-endian
 *             u32 words (engine/src/crypto/poseidon_constants.rs:75-86)
 *   matrices  row-major canonical M31 words (components/matmul.rs:85-107)
 *   MLE index order: the first variable of a point is the most significant
 *             index bit (components/matmul.rs:118-136, 342-355).
 *
 * Threading: a gkr_ctx owns one HIP stream and its device buffers and is not
 * re-entrant; use one context per thread, as the reference uses one
 * executor per thread (engine/src/gpu_sumcheck.rs:1365-1380).
 */
#ifndef GKR_MI355X_H
#define GKR_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  uint32_t v[4];
} gkr_qm31;

typedef struct {
  uint32_t w[8];
} gkr_felt;

enum {
  GKR_OK = 0,
  GKR_ERR_INVALID = 1, /* bad argument or shape */
  GKR_ERR_DEVICE = 2,  /* HIP runtime failure */
  GKR_ERR_LOGUP = 3,   /* LogUp trace/table sums disagree (prover.rs:6488-6495) */
  GKR_ERR_NOMEM = 4,
  GKR_ERR_BUFFER = 5,  /* caller buffer too small */
  GKR_ERR_VERIFY = 6   /* a verifier check failed (reason in gkr_last_error) */
};

/* Message of the last error on this thread (never NULL). */
const char* gkr_last_error(void);
const char* gkr_version(void);

/* ------------------------------------------------------------------ Poseidon
 * Replaces starknet_crypto::poseidon_permute_comp / poseidon_hash /
 * poseidon_hash_many (called at engine/src/crypto/hades.rs:22,
 * poseidon_channel.rs:222, 249, 294).                                        */
int gkr_hades_permute(gkr_felt state[3]);
int gkr_poseidon_hash(const gkr_felt* a, const gkr_felt* b, gkr_felt* out);
int gkr_poseidon_hash_many(const gkr_felt* in, size_t n, gkr_felt* out);

/* ------------------------------------------------------------------ channel
 * Replaces PoseidonChannel (engine/src/crypto/poseidon_channel.rs:83-308).   */
typedef struct gkr_channel gkr_channel;
int gkr_channel_new(gkr_channel** out);                                    /* PoseidonChannel::new, :98-104 */
void gkr_channel_free(gkr_channel* ch);
int gkr_channel_clone(const gkr_channel* ch, gkr_channel** out);           /* #[derive(Clone)], :80 */
int gkr_channel_mix_u64(gkr_channel* ch, uint64_t v);                      /* mix_u64, :140-142 */
int gkr_channel_mix_felt(gkr_channel* ch, const gkr_felt* v);              /* mix_felt, :145-151 */
int gkr_channel_mix_secure_field(gkr_channel* ch, const gkr_qm31* v);      /* gkr/prover.rs:9434-9436 */
int gkr_channel_mix_felts(gkr_channel* ch, const gkr_qm31* v, size_t n);   /* mix_felts, :261-297 */
int gkr_channel_mix_poly_coeffs(gkr_channel* ch, const gkr_qm31 c[3]);     /* mix_poly_coeffs, :213-226 */
int gkr_channel_mix_poly_coeffs_deg3(gkr_channel* ch, const gkr_qm31 c[4]);/* :234-253 */
int gkr_channel_draw_felt252(gkr_channel* ch, gkr_felt* out);              /* draw_felt252, :156-166 */
int gkr_channel_draw_qm31(gkr_channel* ch, gkr_qm31* out);                 /* draw_qm31, :176-200 */
int gkr_channel_draw_qm31s(gkr_channel* ch, size_t n, gkr_qm31* out);      /* draw_qm31s, :203-205 */
int gkr_channel_digest(const gkr_channel* ch, gkr_felt* out);              /* digest(), :300-302 */
uint64_t gkr_channel_hash_count(const gkr_channel* ch);                    /* hash_count(), :108-110 */
/* State as [8 digest words LE, n_draws, hash_count lo, hash_count hi]
 * (to_gpu_state / from_gpu_state, :115-135): lets a Rust caller hand its
 * PoseidonChannel over and take it back around each call.                   */
int gkr_channel_export(const gkr_channel* ch, uint32_t state[11]);
int gkr_channel_import(gkr_channel* ch, const uint32_t state[11]);

/* ------------------------------------------------------------------ device context */
typedef struct gkr_ctx gkr_ctx;
int gkr_ctx_create(int device, gkr_ctx** out);  /* replaces GpuSumcheckExecutor::new/cached, gpu_sumcheck.rs:1309-1380 */
/* A weight matrix whose entries are all int8-range gets an int8 copy on first
 * use and the weight-side restriction reads that copy (one byte per weight,
 * digit sums on the matrix cores); other matrices, and every matrix of a
 * context created with GKR_INT8_WEIGHTS=0 in the environment, are read as
 * u32.  Proofs are identical. */
void gkr_ctx_destroy(gkr_ctx* ctx);
int gkr_ctx_synchronize(gkr_ctx* ctx);
/* Per-kernel timing (HIP events on the context stream), for benchmarks.
 * ids: 0 restrict_cols (weight and activation side of a matmul in one
 * launch), 1 the SIMD layer's weighted activation-side restriction, 2
 * product-sumcheck trip (several
 * rounds per launch), 3 eq-sumcheck or degree-1 trip, 4 logup prepare, 5 eq
 * tables (device kernels: one event pair per launch); 6 host Fiat-Shamir
 * inside the reducers, 7 host wait for results of device kernels, 8 host wait
 * for the hand-over of a sumcheck's last vectors
 * (wall-clock, bytes = 0); 9 Merkle level kernel of the commitments, whose
 * "bytes" count Poseidon hashes instead; 10 host: claim-point draws in the
 * walk, 11 host: time inside kernel-launch calls of the reducers, 12 host:
 * the host-finish rounds' arithmetic (wall-clock, bytes = 0); 13 the norm
 * layers' row statistics and padded-vector kernels (device); 14 the LogUp-GKR
 * batch kernels (device); 15 host: round polynomials derived from a trip's
 * sums; 16 host: proof-record appends; 17 / 18 host: the walk's matmul /
 * activation steps, whole (wall-clock, bytes = 0); 19: walk steps proved a
 * second time because a kernel's bounded wait for the host (about 5.5 s)
 * expired (launches = the count, counted at every timing level); 20:
 * activation layers whose first kernels were launched ahead of their claim
 * point and gamma, beta (launches = the count, at every timing level). */
/* level 0: off; 1: every 8th launch of ids 0 and 4 (the walk's critical
 * path: a timed dispatch waits about 4 us for its events on each side) and
 * every launch of ids 1, 9, 13 and 14, plus the host timers; 2: every launch
 * of every timed kernel.  One-launch scopes (ids 0, 1, 4) carry their events
 * in the kernel's own dispatch (hipExtLaunchKernel); the others are
 * bracketed by event records. */
int gkr_ctx_set_timing(gkr_ctx* ctx, int level);
int gkr_ctx_kernel_time(gkr_ctx* ctx, int kernel_id, double* total_ms, uint64_t* launches, uint64_t* bytes);
/* The same totals split by the bytes one launch moves (launches of one
 * matrix shape share it), in increasing order of bytes: fills the first cap
 * entries and sets *n to the number of distinct sizes.  No counterpart in
 * the reference (benchmark instrumentation, as the totals above). */
int gkr_ctx_kernel_time_by_size(gkr_ctx* ctx, int kernel_id, uint64_t* bytes, double* total_ms, uint64_t* launches,
                                size_t cap, size_t* n);
int gkr_ctx_reset_timing(gkr_ctx* ctx);
/* Test hooks for the failure paths of the hand-over (no counterpart in the
 * reference).  Each applies to the next sumcheck hand-over on the context:
 *   GKR_DEBUG_HANDOVER_CANCEL: the host leaves before posting the last
 *     challenges, as on an error; the call fails with GKR_ERR_DEVICE and the
 *     kernel ends on the cancel code;
 *   GKR_DEBUG_HANDOVER_EXPIRE: the kernel's bounded wait is `arg` polls and
 *     the host posts only after it expired; the call fails with GKR_ERR_DEVICE
 *     (when the last trip has two or more rounds: the kernel folds all of its
 *     levels but the last, which the host folds, so a last trip of one round
 *     waits for nothing and the hook has no effect on it).
 *   GKR_DEBUG_TRIP_EXPIRE: the same for the next wait launched ahead of
 *     its values: a sumcheck trip's challenges, or an activation layer's
 *     gamma and beta when its first kernels were launched ahead (that wait
 *     expires).
 * Every kernel exits normally and the context stays usable.                 */
enum { GKR_DEBUG_HANDOVER_CANCEL = 1, GKR_DEBUG_HANDOVER_EXPIRE = 2, GKR_DEBUG_TRIP_EXPIRE = 3 };
int gkr_ctx_debug(gkr_ctx* ctx, int op, uint64_t arg);

/* ------------------------------------------------------------------ resident matrices
 * The reference re-uploads A and B on every restriction
 * (gpu_sumcheck.rs:2012-2015, 2079-2082); here a matrix is uploaded once
 * and stays in HBM.  Values must be canonical M31 (< 2^31 - 1).              */
typedef struct gkr_matrix gkr_matrix;
int gkr_matrix_upload(gkr_ctx* ctx, const uint32_t* host, uint64_t rows, uint64_t cols, gkr_matrix** out);
/* Borrow device memory the caller owns (e.g. a torch tensor); not freed here.
 * The library derives copies from a matrix's contents on first use and keeps
 * them (the int8 copy of the weight-side restriction, the forward product's
 * digit planes): a caller that writes to the memory afterwards must call
 * gkr_matrix_invalidate before the matrix is used again.                    */
int gkr_matrix_wrap_device(gkr_ctx* ctx, const uint32_t* device_ptr, uint64_t rows, uint64_t cols,
                           gkr_matrix** out);
/* The contents of m changed outside the library (memory of
 * gkr_matrix_wrap_device written by the caller): drops the copies derived
 * from them, which the next use rebuilds.  No counterpart in the reference,
 * which re-uploads its matrices on every call.                              */
int gkr_matrix_invalidate(gkr_ctx* ctx, gkr_matrix* m);
/* Fill a new resident matrix on the device from the documented synthetic
 * generator (counter-mode SplitMix64; kind 0 uniform M31, kind 1 int8-range). */
int gkr_matrix_synthetic(gkr_ctx* ctx, uint64_t rows, uint64_t cols, int kind, uint64_t seed, gkr_matrix** out);
int gkr_matrix_download(gkr_ctx* ctx, const gkr_matrix* m, uint32_t* host);
void gkr_matrix_free(gkr_matrix* m);
/* Host-side copy of the synthetic generator, for callers that need the same
 * values without a device (value i of the row-major stream).               */
uint32_t gkr_synthetic_value(int kind, uint64_t seed, uint64_t i);

/* ------------------------------------------------------------------ ZkmlOps
 * trait ZkmlOps, engine/src/backend.rs:85-107 (CPU impl :110-215, GPU impl
 * gpu_sumcheck.rs:4484-4525).                                                */

/* ZkmlOps::reduce_matmul_layer (backend.rs:87-94).  A is m x k, B is k x n;
 * n_r_i = log2(next_pow2(m)), n_r_j = log2(next_pow2(n)),
 * pk = next_pow2(k).  The transcript (mix_poly_coeffs + draw_qm31 per
 * round) is applied to `ch` inside, as in the reference.  Outputs:
 * round_polys[3*t + {0,1,2}] = (c0, c1, c2) of round t, challenges[t],
 * final_a, final_b; log2(pk) rounds.                                         */
int gkr_reduce_matmul_layer(gkr_ctx* ctx, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_i,
                            uint32_t n_r_i, const gkr_qm31* r_j, uint32_t n_r_j, uint64_t pk, gkr_channel* ch,
                            gkr_qm31* round_polys, gkr_qm31* challenges, gkr_qm31* final_a, gkr_qm31* final_b);
/* ZkmlOps::evaluate_mle_at_point (backend.rs:97-100); len == 2^n_vars. */
int gkr_evaluate_mle_at_point(gkr_ctx* ctx, const gkr_qm31* mle, uint64_t len, const gkr_qm31* point,
                              uint32_t n_vars, gkr_qm31* out);
/* ZkmlOps::restrict_mle (backend.rs:103-106): fixes the first n_assign
 * variables; out has len >> n_assign entries.                                */
int gkr_restrict_mle(gkr_ctx* ctx, const gkr_qm31* mle, uint64_t len, const gkr_qm31* assignments,
                     uint32_t n_assign, gkr_qm31* out);

/* ------------------------------------------------------------------ GKR layer reducers
 * Proof container (GKRProof, engine/src/gkr/types.rs:589-643).  Layer
 * reducers append their LayerProof when given a non-NULL proof.              */
typedef struct gkr_proof gkr_proof;
int gkr_proof_new(gkr_proof** out);
void gkr_proof_free(gkr_proof* p);
size_t gkr_proof_num_layers(const gkr_proof* p);
int gkr_proof_set_input_claim(gkr_proof* p, const gkr_qm31* point, uint32_t n_vars, const gkr_qm31* value);
/* The value of the output claim layer `layer` (proving order) was proved against. */
int gkr_proof_layer_claim_value(const gkr_proof* p, size_t layer, gkr_qm31* value);
int gkr_proof_add_weight_commitment(gkr_proof* p, const gkr_felt* c);
int gkr_proof_set_io_commitment(gkr_proof* p, const gkr_felt* c);
/* serialize_gkr_model_proof (engine/src/cairo_serde.rs:1307-1772) for MatMul
 * (tag 0) and Activation (tag 3) layers, followed by the input claim, the
 * weight commitments, the count of weight openings (0: opening proofs are
 * not produced by this library) and the IO commitment.  Writes up to `cap`
 * felts; *n_out receives the full length (GKR_ERR_BUFFER when cap is short). */
int gkr_proof_serialize(const gkr_proof* p, gkr_felt* out, size_t cap, size_t* n_out);
/* Serialization while proving (no counterpart in the reference, which
 * serializes the finished proof): from this call on, a thread of the proof
 * writes each layer record, as the reducers append it, into out (the layout
 * gkr_proof_serialize writes, layer 0 at felt 1).  gkr_proof_serialize with
 * the same out and cap then writes only the layer count and the tail; with
 * another buffer, or when a layer did not fit in cap, it writes everything
 * itself, as without streaming.  out must stay valid until the proof is
 * freed, serialized or streamed elsewhere; out == NULL ends the streaming.   */
int gkr_proof_stream_to(gkr_proof* p, gkr_felt* out, size_t cap);

/* Proof-generation policy (PolicyConfig, engine/src/policy.rs:48-121): every
 * field is 0 or 1 except weight_binding_mode (0 Individual, 1 Aggregated,
 * 2 TrustlessMode2, 3 TrustlessMode3, policy.rs:30-43).                      */
typedef struct {
  uint8_t allow_missing_norm_proof, allow_logup_activation, allow_missing_segment_binding;
  uint8_t skip_rms_sq_proof, piecewise_activation, skip_batch_tokens, skip_unified_stark;
  uint8_t weight_binding_mode;
  uint8_t aggregated_full_binding, aggregated_rlc_only;
  uint8_t io_packing, packed_proof, double_packed_proof;
  uint8_t validate_decode_chain;
} gkr_policy;
/* The presets PolicyConfig::strict / standard / relaxed (policy.rs:131-203),
 * by name, case-insensitive (from_preset_name, policy.rs:288-295); an
 * unknown name is GKR_ERR_INVALID.                                           */
int gkr_policy_preset(const char* name, gkr_policy* out);
/* PolicyConfig::policy_commitment (policy.rs:236-254): poseidon_hash_many of
 * the domain separator 0x504F4C01 and the 14 fields in declaration order, the
 * value gkr_seed_channel mixes.  A field out of range is GKR_ERR_INVALID.    */
int gkr_policy_commitment(const gkr_policy* policy, gkr_felt* out);

/* GKR driver seeding (gkr/prover.rs:1527-1560): mix_u64(num_layers),
 * mix_u64(in_rows), mix_u64(in_cols), then mix_felt(policy_commitment) when
 * policy != NULL and non-zero (prover.rs:1533-1537).                         */
int gkr_seed_channel(gkr_channel* ch, uint64_t num_layers, uint64_t in_rows, uint64_t in_cols,
                     const gkr_felt* policy_commitment);

/* MLE of C = A*B at r_out = (r_i || r_j), computed as sum_l f_a[l]*f_b[l]
 * from the two restrictions (equal to evaluate_mle(pad(C), r_out) as used
 * by the driver, prover.rs:1543-1553).  The restrictions are kept and reused
 * by a following reduce on the same (a, b, r_i, r_j).                       */
int gkr_matmul_output_claim(gkr_ctx* ctx, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_out,
                            uint32_t n_vars, gkr_qm31* value);

/* reduce_matmul_layer_with_backend (gkr/prover.rs:5959-6070): mixes m, k, n
 * and the claim, runs the backend reduction, mixes final_a and final_b.
 * claim point = r_i || r_j (log2 pm + log2 pn entries).  Outputs the round
 * polys (3 per round), final evals, and the next claim: point r_i ||
 * challenges (n_next_point = log2 pm + log2 pk entries) and value final_a.  */
int gkr_prove_matmul_layer(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                           const gkr_matrix* a, const gkr_matrix* b, gkr_channel* ch, gkr_proof* proof,
                           gkr_qm31* round_polys, gkr_qm31* final_a, gkr_qm31* final_b, gkr_qm31* next_point,
                           gkr_qm31* next_value);

/* reduce_matmul_layer_simd_gpu (gkr/prover.rs:5422-5600): a shared-weight
 * SIMD matmul over n_blocks (1 .. 64) activation blocks a_blocks[b] (all
 * m x k) and one b.  f_a = sum_b block_weights[b] * restrict_rows(A_b, r_i)
 * (combine_blocks, gpu_sumcheck.rs:1123-1146), f_b = restrict_cols(B, r_j);
 * transcript, outputs and proof record as gkr_prove_matmul_layer (a MatMul
 * layer proof).                                                            */
int gkr_prove_matmul_layer_simd(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point,
                                const gkr_qm31* claim_value, const gkr_matrix* const* a_blocks,
                                const gkr_qm31* block_weights, uint32_t n_blocks, const gkr_matrix* b,
                                gkr_channel* ch, gkr_proof* proof, gkr_qm31* round_polys, gkr_qm31* final_a,
                                gkr_qm31* final_b, gkr_qm31* next_point, gkr_qm31* next_value);

/* reduce_matmul_layer_dual_simd_gpu (gkr/prover.rs:5615-5785): n_blocks (a
 * power of two, up to 64) pairs A_b (m x k), B_b (k x n) with weights w_b.
 * Mixes m, k, n, n_blocks and the claim, runs the three-factor sumcheck of
 * sumcheck_3way (gpu_sumcheck.rs:2597-2681) over the block-extended
 * (w_b, restrict_rows(A_b, r_i), restrict_cols(B_b, r_j)) — block variables
 * first — and mixes final_a, final_b.  round_polys: 4 per round (c0..c3),
 * log2(n_blocks) + log2(pk) rounds.  Records a MatMulDualSimd layer.      */
int gkr_prove_matmul_layer_dual_simd(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point,
                                     const gkr_qm31* claim_value, const gkr_matrix* const* a_blocks,
                                     const gkr_matrix* const* b_blocks, const gkr_qm31* block_weights,
                                     uint32_t n_blocks, gkr_channel* ch, gkr_proof* proof, gkr_qm31* round_polys,
                                     gkr_qm31* final_a, gkr_qm31* final_b);

/* Outputs of reduce_activation_layer (gkr/prover.rs:6400-6600).  The caller
 * provides the arrays; sizes: eq_round_polys 4*n_vars, multiplicities
 * 2^table_log_size, mult_round_polys 2*table_log_size.                       */
typedef struct {
  gkr_qm31 claimed_sum;       /* trace-side LogUp sum (LogUpProof::claimed_sum) */
  gkr_qm31* eq_round_polys;   /* [4*t + {0..3}] = c0..c3 of eq round t */
  gkr_qm31 w_eval, in_eval, out_eval;   /* LogUpProof::final_evals */
  uint32_t* multiplicities;
  gkr_qm31* mult_round_polys; /* [2*t + {0,1}] = (c0, c1) of multiplicity round t */
  gkr_qm31 mult_final_eval, mult_claimed_sum;
  gkr_qm31 input_eval, output_eval;
  gkr_felt table_commitment;
  gkr_qm31 gamma, beta;       /* LogUp encoding challenges (not serialized) */
} gkr_logup_out;

/* reduce_activation_layer: input is the rows x cols activation matrix,
 * activation_type the reference type tag (1 ReLU, 2 GELU, 3 Sigmoid,
 * 4 Softmax, 5 SiLU), table_log_size the lookup table size (0 = the
 * reference default: 20 for Softmax, 16 otherwise).  claim_point has
 * log2(next_pow2(rows) * next_pow2(cols)) entries.                           */
int gkr_prove_activation_layer(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point,
                               const gkr_qm31* claim_value, const gkr_matrix* input, uint32_t activation_type,
                               uint32_t table_log_size, gkr_channel* ch, gkr_proof* proof, gkr_logup_out* out);

/* Resident QM31 vectors (AoS, 16 B each) and the product sumcheck alone:
 * the round loop of ZkmlOps::reduce_matmul_layer (engine/src/backend.rs:146-177;
 * GPU twin gpu_sumcheck.rs:2820-2840) over given f_a, f_b of length 2^T:
 * per round s0, s1, s2 -> (c0, c1, c2), mix_poly_coeffs, draw_qm31, fold.
 * No separate reference entry point: this is the part of
 * gkr_reduce_matmul_layer after the restriction, exported for callers that
 * already hold the restricted MLEs.  The vectors are left unchanged.
 * gkr_qvec_synthetic fills n uniform QM31 (four SplitMix64 M31 draws each,
 * the generator of gkr_matrix_synthetic kind 0 at indices 4i..4i+3). */
typedef struct gkr_qvec gkr_qvec;
int gkr_qvec_upload(gkr_ctx* ctx, const gkr_qm31* host, uint64_t n, gkr_qvec** out);
int gkr_qvec_synthetic(gkr_ctx* ctx, uint64_t n, uint64_t seed, gkr_qvec** out);
int gkr_qvec_download(gkr_ctx* ctx, const gkr_qvec* v, gkr_qm31* host);
void gkr_qvec_free(gkr_qvec* v);
/* Device address of a vector's n QM31 (for device-pointer entry points). */
const gkr_qm31* gkr_qvec_device_ptr(const gkr_qvec* v);
int gkr_sumcheck_product(gkr_ctx* ctx, const gkr_qvec* fa, const gkr_qvec* fb, gkr_channel* ch,
                         gkr_qm31* round_polys /* 3T: c0, c1, c2 */, gkr_qm31* challenges /* T */,
                         gkr_qm31* final_a, gkr_qm31* final_b);

/* Allocation-free variant of gkr_sumcheck_product (no counterpart in the
 * reference): for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  fa
 * and fb are device pointers of the context's GPU holding n canonical QM31
 * each (n a power of two, at most 2^20); outputs as gkr_sumcheck_product.
 * Every device buffer the kernels need (fold levels, partial rows, arrival
 * counter) lives in a static 25 MiB device array, one per GPU, held until
 * the process ends; no hipMalloc or hipFree is called.  All calls on one GPU
 * share that array, so they take turns: a call holds a per-GPU lock until its
 * kernels have finished, and a call from another context or thread on the
 * same GPU waits for it.  Longer vectors fail with GKR_ERR_INVALID.       */
int gkr_sumcheck_product_noalloc(gkr_ctx* ctx, const gkr_qm31* fa, const gkr_qm31* fb, uint64_t n, gkr_channel* ch,
                                 gkr_qm31* round_polys /* 3T */, gkr_qm31* challenges /* T */, gkr_qm31* final_a,
                                 gkr_qm31* final_b);

/* Forward-pass matrix product (the witness before the walk): C = A * B mod P
 * for canonical M31 matrices, a new resident matrix (m x n).  Replaces
 * gpu_matmul_m31_full (engine/src/gpu_sumcheck.rs:3104) and its GEMM/GEMV
 * kernels (:418-460); computed on the matrix cores (i8 MFMA on digit planes),
 * exact for any M31 values.                                                  */
int gkr_matmul_forward(gkr_ctx* ctx, const gkr_matrix* a, const gkr_matrix* b, gkr_matrix** out);
/* The same into an existing m x n matrix (no allocation; asynchronous on the
 * context stream, ordered before the next call that uses `out`).  The first
 * product with a given B also builds and keeps B's digit planes (one pass
 * over B plus a host round trip).                                          */
int gkr_matmul_forward_into(gkr_ctx* ctx, const gkr_matrix* a, const gkr_matrix* b, gkr_matrix* out);

/* MLE commitments: Poseidon Merkle roots (engine/src/crypto/poseidon_merkle.rs:255-280,
 * root_only_parallel) over securefield_to_felt leaves (poseidon_channel.rs:59-69),
 * padded with zero felts to a power of two (at least 2); node = poseidon_hash(l, r).
 * Roots are canonical felts (8 little-endian u32 words).
 *
 * gkr_weight_commitment: the weight commitment of the GKR prover,
 * commit_mle_root_only(matrix_to_mle_col_major_padded(B)) (engine/src/gkr/prover.rs:1021-1023,
 * mle_opening.rs:630-641): B[i][j] at index j * next_pow2(rows) + i of the padded grid.
 * gkr_weight_commitments: the same for `count` matrices in one batch (one root each,
 * in order), the role of commit_mle_root_only_batch (mle_opening.rs:791-809).
 * gkr_mle_commitment: commit_mle_root_only over the n QM31 values of `evals`.
 * A weight's root is kept on its resident matrix once computed (the weight
 * phase of every later proof takes it from there) until its contents change
 * (gkr_matrix_invalidate, gkr_matmul_forward_into).                           */
int gkr_weight_commitment(gkr_ctx* ctx, const gkr_matrix* b, gkr_felt* root);
int gkr_weight_commitments(gkr_ctx* ctx, const gkr_matrix* const* mats, size_t count, gkr_felt* roots);
int gkr_mle_commitment(gkr_ctx* ctx, const gkr_qvec* evals, gkr_felt* root);
/* The weight-commitment cache kept on resident matrices, for a caller that
 * persists roots across processes (the reference's WeightCommitmentCache,
 * engine/src/weight_cache.rs:283-327: get_root / insert_root, saved to a file
 * with a content fingerprint, :339-395, :646).
 * gkr_matrix_commitment_cached: *cached = 1 and the root when m holds one.
 * gkr_matrix_set_commitment: m holds `root` from now on (canonical felt); the
 * caller vouches that it is m's weight commitment, as the reference trusts a
 * cache file whose fingerprint matches.                                        */
int gkr_matrix_commitment_cached(const gkr_matrix* m, gkr_felt* root, int* cached);
int gkr_matrix_set_commitment(gkr_ctx* ctx, gkr_matrix* m, const gkr_felt* root);

/* Weight openings: prove_mle_opening_with_commitment (mle_opening.rs:1654-1915)
 * over matrix_to_mle_col_major_padded(B) at eval_point (log2(next_pow2(rows)) +
 * log2(next_pow2(cols)) values, the first folding the top variable): mixes the
 * commitment and the roots of the folded layers, draws 10 query pairs
 * (MLE_N_QUERIES, mle_opening.rs:47; fewer when the MLE has under 20 values)
 * and appends the commitment and the opening (claim point, expected value,
 * MleOpeningProof, laid out as cairo_serde.rs:1759-1767) to `proof`, so that
 * gkr_proof_serialize emits them.  expected_value, when not NULL, must equal
 * the MLE at the point (GKR_ERR_INVALID otherwise).  `commitment` may be NULL.
 *
 * gkr_prove_weight_openings: the sequential weight-opening phase of the GKR
 * prover (prover.rs:2059-2200, main channel, no sub-channels): opens, in
 * proving order, the claim MLE(B)(r_j || sumcheck challenges) = final_b that
 * every MatMul layer proved into `proof` recorded (prover.rs:1465-1483), then
 * forgets the claims.  The weight matrices must still be alive.             */
int gkr_prove_weight_opening(gkr_ctx* ctx, const gkr_matrix* b, const gkr_qm31* eval_point, uint32_t n_point,
                             const gkr_qm31* expected_value, gkr_channel* ch, gkr_proof* proof, gkr_felt* commitment);
int gkr_prove_weight_openings(gkr_ctx* ctx, gkr_channel* ch, gkr_proof* proof);
/* The weight phase in one of the reference's transcript modes (prover.rs:2059-2200),
 * over the claims recorded in `proof`, which are then forgotten:
 *   GKR_WEIGHT_SEQUENTIAL     = gkr_prove_weight_openings (STWO_WEIGHT_BINDING=sequential);
 *   GKR_WEIGHT_AGGREGATED_RLC = the reference default (aggregated oracle sumcheck,
 *     RLC fast path, prover.rs:368-658): the commitment of every claimed weight is
 *     appended to the proof (one GPU batch), then rho = draw_qm31 and
 *     mix_secure_field(sum_i rho^i * value_i); no openings;
 *   GKR_WEIGHT_RLC_DIRECT     = apply_aggregated_rlc_binding (prover.rs:669-699): rho and
 *     the combined value only;
 *   GKR_WEIGHT_AGGREGATED_FULL = STWO_AGGREGATED_FULL_BINDING=1 (prover.rs:1233-1330): the
 *     commitments as in AGGREGATED_RLC, then one gkr_prove_aggregated_binding per group of
 *     4 claims (BINDING_GROUP_SIZE, prover.rs:366) on the channel, in claim order; the
 *     groups' serialized proofs are kept in `proof` (gkr_proof_binding_group).        */
enum { GKR_WEIGHT_SEQUENTIAL = 0, GKR_WEIGHT_AGGREGATED_RLC = 1, GKR_WEIGHT_RLC_DIRECT = 2,
       GKR_WEIGHT_AGGREGATED_FULL = 3 };
int gkr_prove_weight_binding(gkr_ctx* ctx, gkr_channel* ch, gkr_proof* proof, int mode);
size_t gkr_proof_num_binding_groups(const gkr_proof* proof);
/* The serialize_aggregated_binding_proof felts of group g; *n_felts gets the length
 * (GKR_ERR_BUFFER when cap is short). */
int gkr_proof_binding_group(const gkr_proof* proof, size_t g, gkr_felt* out, size_t cap, size_t* n_felts);

/* Mul layer (element-wise product c = lhs * rhs), reduce_mul_layer
 * (engine/src/gkr/prover.rs:6172-6271): mix_u64(0x4D554C), mix the claim
 * value, a degree-3 eq-sumcheck over eq(r[..n_vars], x) * lhs(x) * rhs(x)
 * (4 coefficients per round, mix_poly_coeffs_deg3 + draw), mix lhs_eval and
 * rhs_eval, draw alpha; the next claim is (claim_point, alpha * lhs + (1 -
 * alpha) * rhs).  The claim point may be longer than n_vars; its first n_vars
 * entries are used.  The caller provides eq_round_polys (4 * n_vars).  */
typedef struct {
  gkr_qm31* eq_round_polys;  /* in: caller buffer; out: c0..c3 per round */
  gkr_qm31 lhs_eval, rhs_eval, alpha, next_value;
  uint32_t n_vars;
} gkr_mul_out;
/* lhs/rhs: resident matrices, padded as pad_matrix_pow2 + matrix_to_mle
 * (get_binary_op_intermediates, prover.rs:9563-9595); their padded lengths
 * must agree.  Appends LayerProof::Mul to `proof` when it is non-null. */
int gkr_prove_mul_layer(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                        const gkr_matrix* lhs, const gkr_matrix* rhs, gkr_channel* ch, gkr_proof* proof,
                        gkr_mul_out* out);
/* The reference signature: lhs_vals / rhs_vals are host QM31 slices of length n
 * (a power of two). */
int gkr_reduce_mul_layer(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                         const gkr_qm31* lhs_vals, const gkr_qm31* rhs_vals, uint64_t n, gkr_channel* ch,
                         gkr_proof* proof, gkr_mul_out* out);
/* MLE of the padded element-wise product at `point` (n_point = log2 of the
 * padded length): the Mul layer's output claim value (cf. prover.rs:1543-1560). */
int gkr_mul_output_claim(gkr_ctx* ctx, const gkr_matrix* lhs, const gkr_matrix* rhs, const gkr_qm31* point,
                         uint32_t n_point, gkr_qm31* out);

/* LayerNorm and RMSNorm layers (reduce_layernorm_layer, gkr/prover.rs:7944-8395;
 * reduce_rmsnorm_layer_with_gamma, 8407-8801): Part 0 a plain sumcheck
 * (LayerNorm: eta0 input + eta1 centered^2, tag 0x4D56; RMSNorm: input^2, tag
 * 0x5251), Part 1 the eq-sumcheck of output = centered * rsqrt (LayerNorm, tag
 * 0x4C4E) or input * scale (RMSNorm, tag 0x524E; scale = rsqrt * gamma), Part 2
 * the LogUp of (variance or rms^2, rsqrt) in the 2^16-entry rsqrt table with
 * its multiplicity sumcheck.  dim: the normalized width (the first
 * min(dim, padded cols) columns); the claim point has log2 of the padded size
 * entries.  The caller provides p0/lin/logup_round_polys (4 * n_vars each,
 * c0..c3), multiplicities (2^16), mult_round_polys (2 * 16) and row_stats0/1
 * (next_pow2(rows) each).  RMSNorm reports rms^2 in mean_eval, the square sum
 * in sum0, its Part 0 final input in p0_final0, (input, scale) finals in
 * lin_final0/1 and the per-row rms^2 in row_stats0; var_eval, sum1,
 * p0_final1, cb_input, cb_mean and row_stats1 are LayerNorm's only, and
 * gamma_commitment / gamma_eval RMSNorm's (not mixed, not serialized;
 * gkr_prove_walk does not compute the commitment, a chain of one Poseidon
 * mix per scale entry). */
typedef struct {
  gkr_qm31 input_eval, output_eval, mean_eval, rsqrt_eval, var_eval;
  uint32_t n_active;
  gkr_qm31 sum0, sum1;        /* LayerNorm: input sum, centered^2 sum; RMSNorm: input^2 sum */
  gkr_qm31* p0_round_polys;   /* Part 0 */
  gkr_qm31 p0_final0, p0_final1;
  gkr_qm31* lin_round_polys;  /* Part 1 */
  gkr_qm31 lin_final0, lin_final1;
  gkr_qm31 cb_input, cb_mean; /* LayerNorm centered binding (input - mean = centered) */
  gkr_qm31 claimed_sum;       /* Part 2: LogUp trace sum */
  gkr_qm31* logup_round_polys;
  gkr_qm31 w_eval, in_eval, out_eval;
  uint32_t* multiplicities;
  gkr_qm31* mult_round_polys;
  gkr_qm31 mult_final_eval, mult_claimed_sum;
  gkr_felt table_commitment;  /* hash_many([0x5253, 16]) (prover.rs:8357-8363) */
  uint32_t n_rows;            /* padded rows */
  uint32_t* row_stats0;       /* LayerNorm per-row means, RMSNorm per-row rms^2 */
  uint32_t* row_stats1;       /* LayerNorm per-row variances */
  gkr_felt gamma_commitment;
  gkr_qm31 gamma_eval;
} gkr_norm_out;
int gkr_prove_layernorm_layer(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                              const gkr_matrix* input, uint64_t dim, gkr_channel* ch, gkr_proof* proof,
                              gkr_norm_out* out);
/* gamma: host array of n_gamma canonical M31 (the learned per-column scale), or NULL. */
int gkr_prove_rmsnorm_layer(gkr_ctx* ctx, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                            const gkr_matrix* input, uint64_t dim, const uint32_t* gamma, uint64_t n_gamma,
                            gkr_channel* ch, gkr_proof* proof, gkr_norm_out* out);
/* MLE at `point` of the layer's output as the reducers define it (kind
 * GKR_STEP_LAYERNORM or GKR_STEP_RMSNORM): LayerNorm (x - mean) * rsqrt on
 * every padded entry; RMSNorm x * scale on the active columns, x elsewhere. */
int gkr_norm_output_claim(gkr_ctx* ctx, uint32_t kind, const gkr_matrix* input, uint64_t dim, const uint32_t* gamma,
                          uint64_t n_gamma, const gkr_qm31* point, uint32_t n_point, gkr_qm31* value);

/* ------------------------------------------------------------------ STWO LogUp-GKR batch
 * prove_batch (stwo-gpu/crates/stwo/src/prover/lookups/gkr_prover.rs:396-500)
 * over device columns, with the Poseidon252 channel (the engine calls it from
 * prove_logup_gkr, engine/src/aggregation.rs:3926-4062, after drawing the
 * LogUp alpha).  An instance is one binary-tree circuit over 2^n_vars
 * entries: GKR_LOOKUP_GRAND_PRODUCT (`denominators` holds the column),
 * _LOGUP_GENERIC (QM31 numerators), _LOGUP_MULTIPLICITIES (u32 M31
 * numerators; n_vars >= 2) or _LOGUP_SINGLES (numerators 1).  Columns are
 * device pointers in the reference's Mle order (first variable on the most
 * significant bit of the index).  n_layers = the largest n_vars; the caller
 * provides output_claims and claims_to_verify (2 QM31 per instance; a grand
 * product uses the first), round_polys (4 QM31 per round, n_layers *
 * (n_layers - 1) / 2 rounds: layer 0's, then layer 1's ...), round_poly_lens
 * (one per round: the coefficients the reference keeps, leading zeros
 * dropped), masks (4 QM31 per (layer, instance): instance i of layer l at
 * 4 * (l * n_instances + i), LogUp: num(0), num(1), den(0), den(1), grand
 * product: the two values; zero before the instance joins) and ood_point
 * (n_layers).  The claims are the artifact's claims_to_verify_by_instance:
 * the input columns at the last n_vars coordinates of ood_point. */
enum {
  GKR_LOOKUP_GRAND_PRODUCT = 0,
  GKR_LOOKUP_LOGUP_GENERIC = 1,
  GKR_LOOKUP_LOGUP_MULTIPLICITIES = 2,
  GKR_LOOKUP_LOGUP_SINGLES = 3
};
typedef struct {
  uint32_t kind;
  uint32_t n_vars;
  const void* numerators;         /* device: gkr_qm31 (generic) or uint32_t (multiplicities); else NULL */
  const gkr_qm31* denominators;   /* device */
} gkr_lookup_instance;
typedef struct {
  gkr_qm31* output_claims;
  gkr_qm31* round_polys;
  uint32_t* round_poly_lens;
  gkr_qm31* masks;
  gkr_qm31* ood_point;
  gkr_qm31* claims_to_verify;
  uint32_t n_layers;
} gkr_lookup_batch;
int gkr_prove_lookup_batch(gkr_ctx* ctx, gkr_channel* ch, const gkr_lookup_instance* instances, size_t n_instances,
                           gkr_lookup_batch* out);
/* partially_verify_batch (stwo-gpu/crates/stwo/src/prover/lookups/gkr_verifier.rs:17-157),
 * host only.  gates: 0 grand product, 1 LogUp, per instance; proof as
 * gkr_prove_lookup_batch writes it (n_layers set).  Returns the artifact's
 * OOD point (n_layers) and claims (2 per instance), or GKR_ERR_VERIFY. */
int gkr_verify_lookup_batch(const uint32_t* gates, const uint32_t* n_vars, size_t n_instances,
                            const gkr_lookup_batch* proof, gkr_channel* ch, gkr_qm31* ood_point,
                            gkr_qm31* claims_to_verify);
/* serialize_stwo_gkr_batch_proof (engine/src/cairo_serde.rs:3330-3420).  It
 * indexes each instance's masks by the global layer, so every instance must
 * have n_vars = n_layers (GKR_ERR_INVALID otherwise).  *n_felts receives the
 * full length (GKR_ERR_BUFFER when cap is short). */
int gkr_serialize_lookup_batch(const uint32_t* gates, const uint32_t* n_vars, size_t n_instances,
                               const gkr_lookup_batch* proof, gkr_felt* out, size_t cap, size_t* n_felts);
/* Device address of a matrix's u32 entries (row-major), e.g. multiplicities for a lookup instance. */
const uint32_t* gkr_matrix_device_ptr(const gkr_matrix* m);

/* ------------------------------------------------------------------ aggregated weight binding
 * prove_aggregated_binding_streaming (engine/src/crypto/aggregated_opening.rs:1647-1720),
 * the full binding proof of STWO_AGGREGATED_FULL_BINDING=1 (gkr/prover.rs:1233-1330): one
 * AggregatedWeightBindingProof over up to 8 claims (the prover groups them by 4,
 * BINDING_GROUP_SIZE).  Claim i sits in selector slot i; its weight's MLE is
 * matrix_to_mle_col_major_padded(B) (log2 pk + log2 pn variables = n_point);
 * commitment = that MLE's root (gkr_weight_commitment).  The proof is written as
 * serialize_aggregated_binding_proof (cairo_serde.rs:3885-3920): config, sumcheck
 * round polynomials, oracle value, super root, subtree roots, the opening of the
 * virtual MLE.  *n_felts receives its length (GKR_ERR_BUFFER, channel untouched,
 * when cap is short). */
typedef struct {
  const gkr_matrix* weight;
  const gkr_qm31* eval_point;
  uint32_t n_point;
  gkr_qm31 expected_value;
  gkr_felt commitment;
} gkr_binding_claim;
int gkr_prove_aggregated_binding(gkr_ctx* ctx, gkr_channel* ch, const gkr_binding_claim* claims, size_t n_claims,
                                 gkr_felt* out, size_t cap, size_t* n_felts);

/* GKR walk over a sequence of layers (the layer loop of prove_gkr_with_cache,
 * gkr/prover.rs:1500-1660, for MatMul, Mul, Activation, LayerNorm and RMSNorm
 * layers).  Steps run in order on one channel and append their LayerProof to
 * `proof`.  Each step's output claim is either chained (the previous step's
 * input claim, or init_point/init_value for the first step: the reference's
 * walk) or fresh: a MatMul draws r_out = draw_qm31s(log2 pm + log2 pn), takes
 * value = MLE of A*B at r_out and mixes it (prover.rs:1543-1560); an
 * Activation draws its point (log2 of the padded size) and then its value
 * with draw_qm31; a Mul, LayerNorm or RMSNorm draws its point (log2 of the
 * padded size), takes the MLE of its output there and mixes it.  On return
 * final_point/final_value hold the last input claim (final_point needs room
 * for 64 entries).  A step that fails because a kernel's bounded wait for the
 * host expired (the host thread held up for about 5.5 s) is proved once more
 * from the channel and claim it started from, giving the same proof (timer
 * id 19 counts these).                                                      */
enum { GKR_STEP_MATMUL = 0, GKR_STEP_MUL = 2, GKR_STEP_ACTIVATION = 3, GKR_STEP_LAYERNORM = 4, GKR_STEP_RMSNORM = 8 };
enum { GKR_CLAIM_CHAINED = 0, GKR_CLAIM_FRESH = 1 };
typedef struct {
  uint32_t kind;             /* GKR_STEP_* */
  uint32_t claim;            /* GKR_CLAIM_CHAINED / GKR_CLAIM_FRESH */
  const gkr_matrix* a;       /* MatMul: A (m x k); Mul: lhs; Activation / norms: the input matrix */
  const gkr_matrix* b;       /* MatMul: B (k x n); Mul: rhs; RMSNorm: gamma (1 x n_gamma) or NULL */
  uint32_t activation_type;  /* Activation: reference type tag */
  uint32_t table_log_size;   /* Activation: 0 = reference default */
  uint64_t dim;              /* LayerNorm / RMSNorm: normalized width (0: the input's columns) */
} gkr_step;
int gkr_prove_walk(gkr_ctx* ctx, gkr_channel* ch, const gkr_step* steps, size_t n_steps, const gkr_qm31* init_point,
                   uint32_t n_init, const gkr_qm31* init_value, gkr_proof* proof, gkr_qm31* final_point,
                   uint32_t* n_final, gkr_qm31* final_value);

/* ------------------------------------------------------------------ verifier replay
 * Host-only: each call replays the layer's transcript on `ch` and returns
 * GKR_OK with the claim on the layer's input, or GKR_ERR_VERIFY with the
 * failing check in gkr_last_error. */
/* verify_matmul_reduction (engine/src/gkr/verifier.rs:2675-2788).
 * round_polys: (c0, c1, c2) per round; next_point receives log2(pm) +
 * n_rounds entries (r_i then the challenges); next_value = final_a. */
int gkr_verify_matmul_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value, uint64_t m,
                            uint64_t k, uint64_t n, const gkr_qm31* round_polys, uint32_t n_rounds,
                            const gkr_qm31* final_a, const gkr_qm31* final_b, gkr_channel* ch, gkr_qm31* next_point,
                            uint32_t* n_next, gkr_qm31* next_value);
/* verify_mul_reduction (verifier.rs:2963-3045).  eq_round_polys: (c0..c3)
 * per round; next_value = alpha * lhs + (1 - alpha) * rhs (the point is
 * unchanged). */
int gkr_verify_mul_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                         const gkr_qm31* eq_round_polys, uint32_t n_rounds, const gkr_qm31* lhs_eval,
                         const gkr_qm31* rhs_eval, gkr_channel* ch, gkr_qm31* next_value);
/* verify_activation_reduction, LogUp branch, with verify_multiplicity_sumcheck
 * (verifier.rs:3058-3290, 5818-5842).  `proof` carries the prover's outputs
 * (gkr_logup_out: eq_round_polys 4 x n_eq_rounds, 2^table_log_size
 * multiplicities, 2 x table_log_size multiplicity round polys); next_value =
 * input_eval.  The reference refuses LogUp-only proofs of non-ReLU
 * activations unless STWO_ALLOW_LOGUP_ACTIVATION is set; this replay
 * corresponds to that setting. */
int gkr_verify_activation_layer(const gkr_qm31* claim_point, uint32_t n_point, uint32_t activation_type,
                                uint32_t table_log_size, uint32_t n_eq_rounds, const gkr_logup_out* proof,
                                gkr_channel* ch, gkr_qm31* next_value);
/* verify_layernorm_reduction / verify_rmsnorm_reduction (verifier.rs:4153-4690,
 * 4693-5076), non-SIMD with the Part 0 proof: `proof` as the reducers fill it
 * (round polynomials in full, n_rows padded rows).  The multi-row LayerNorm
 * variance binding is the reference's (rows with equal variances pass). */
int gkr_verify_layernorm_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                               uint64_t dim, const gkr_norm_out* proof, gkr_channel* ch, gkr_qm31* next_value);
int gkr_verify_rmsnorm_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                             uint64_t dim, const gkr_norm_out* proof, gkr_channel* ch, gkr_qm31* next_value);
/* One layer of the circuit a walk is verified against. */
typedef struct {
  uint32_t kind;             /* GKR_STEP_MATMUL / GKR_STEP_MUL / GKR_STEP_ACTIVATION */
  uint64_t rows, cols;       /* MatMul: A is rows x cols (m x k); Mul / Activation: the operand */
  uint64_t cols_b;           /* MatMul: n (B is cols x cols_b) */
  uint32_t activation_type;  /* Activation */
  uint32_t table_log_size;   /* Activation: 0 = reference default */
  uint32_t claim;            /* GKR_CLAIM_CHAINED / GKR_CLAIM_FRESH, as the walk that proved it */
  uint64_t dim;              /* LayerNorm: normalized width (0: cols) */
} gkr_layer_shape;
/* A walk from serialize_gkr_model_proof calldata (the layer section and the
 * input claim that follows it).  A chained layer's claim is the previous
 * layer's input claim, starting from init_point / init_value (the seeded
 * output claim; both may be absent when the first layer is fresh).  A fresh
 * layer replays gkr_prove_walk's rule: its point is drawn from the channel;
 * an Activation draws its value, a MatMul or Mul takes the next of the
 * fresh_values (the values its prover computed from the witness, public to
 * this verifier like the model output; gkr_proof_layer_claim_value) and mixes
 * it.  Round polynomials are compressed (c1 rebuilt from the running sum).
 * The weight commitments, openings and IO commitment after the input claim
 * are not examined; *n_consumed receives the number of felts read. */
int gkr_verify_walk(const gkr_felt* calldata, size_t n_felts, const gkr_layer_shape* layers, size_t n_layers,
                    const gkr_qm31* init_point, uint32_t n_init, const gkr_qm31* init_value,
                    const gkr_qm31* fresh_values, size_t n_fresh, gkr_channel* ch, gkr_qm31* final_point,
                    uint32_t* n_final, gkr_qm31* final_value, size_t* n_consumed);

/* Activation table output column, f(j) for j < 2^log_size (host). */
int gkr_activation_table(uint32_t activation_type, uint32_t log_size, uint32_t* out);

/* Bandwidth reference (no counterpart in the reference): a plain 128-bit
 * device-to-device copy and a read-only stream over `bytes`, `iters` times;
 * reports (bytes read + written) / time and bytes read / time in GB/s.    */
int gkr_bench_copy(gkr_ctx* ctx, uint64_t bytes, int iters, double* copy_gbps, double* read_gbps);

#ifdef __cplusplus
}
#endif
#endif /* GKR_MI355X_H */
