// LayerNorm and RMSNorm layers: reduce_layernorm_layer (engine/src/gkr/
// prover.rs:7944-8395) and reduce_rmsnorm_layer_with_gamma (8407-8801).
//
// Device: the per-row sums of the input (forward statistics), the padded
// vectors (input, centered or scaled, output), the eq-weighted evaluations
// of input and output at the claim point, the plain sumcheck of Part 0
// (LayerNorm: sum eta0 input + eta1 centered^2 as a Gram trip of centered
// plus a plain-sum trip of input; RMSNorm: the product sumcheck of input with
// itself) and the eq-weighted sumcheck of Part 1.  Host: everything that is
// constant per row.  The rsqrt LogUp of Part 2 runs on per-row vectors (its
// w, d and keys do not depend on the column): its row rounds are the
// reference's eq-sumcheck over the padded rows, its column rounds have
// w d = W D constant, so p(X) = W D eq(z_row, s_row) prod eqlin(z, s)
// eqlin(z_t, X) (degree 1); the multiplicity sumcheck runs over the few
// nonzero multiplicities.  Every round polynomial is the unique polynomial
// the reference computes, so coefficients and transcript are identical.
#include "internal.h"
#include "norm.h"

// ------------------------------------------------------------------ kernels
// Per real row r (one workgroup each): sums mod P of x and x^2 over the first
// `active` columns (S1, S2) and over all columns (T1, T2), to out[4r .. 4r+3].
static __global__ void __launch_bounds__(kBlock) k_norm_rows(const uint32_t* __restrict__ X, uint64_t cols,
                                                            uint64_t active, uint32_t* __restrict__ out) {
  const uint32_t* row = X + (uint64_t)blockIdx.x * cols;
  uint64_t s1 = 0, s2 = 0, t1 = 0, t2 = 0;
  for (uint64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const uint32_t x = row[c];
    const uint32_t x2 = m31_mul(x, x);
    t1 += x;
    t2 += x2;
    if (c < active) {
      s1 += x;
      s2 += x2;
    }
  }
  __shared__ uint64_t sh[4][kBlock / 64];
  uint64_t v[4] = {s1, s2, t1, t2};
#pragma unroll
  for (int q = 0; q < 4; q++) {
    for (int m = 32; m >= 1; m >>= 1) v[q] += (uint64_t)__shfl_xor((long long)v[q], m, 64);
    if ((threadIdx.x & 63) == 0) sh[q][threadIdx.x >> 6] = v[q];
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    uint64_t s = 0;
    for (int w = 0; w < kBlock / 64; w++) s += sh[threadIdx.x][w] % P;
    out[4 * (uint64_t)blockIdx.x + threadIdx.x] = (uint32_t)(s % P);
  }
}

// The padded vectors over n = prow * pcol entries (entry p: row p >> log_pcol,
// column p & (pcol - 1); padding entries are 0).  rowv holds (mean or 0,
// rsqrt) per padded row.  LayerNorm: w = x - mean (centered), d = rsqrt,
// in_q = x, out = centered * rsqrt.  RMSNorm: w = x, d = scale = rsqrt *
// gamma[min(col, ng - 1)] on the active columns (rsqrt elsewhere), out = x *
// scale on the active columns (x elsewhere); in_q is not written.
static __global__ void k_norm_prepare(const uint32_t* __restrict__ X, uint64_t rows, uint64_t cols, int log_pcol,
                                      uint64_t n, int layernorm, uint64_t active, const uint32_t* __restrict__ rowv,
                                      const uint32_t* __restrict__ gamma, uint64_t ng, qm31* __restrict__ w,
                                      qm31* __restrict__ d, qm31* __restrict__ in_q, uint32_t* __restrict__ in_u,
                                      uint32_t* __restrict__ out_u) {
  const uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint64_t r = p >> log_pcol, c = p & ((1ull << log_pcol) - 1);
  const uint32_t x = (r < rows && c < cols) ? X[r * cols + c] : 0u;
  const uint32_t mean = rowv[2 * r], rs = rowv[2 * r + 1];
  in_u[p] = x;
  if (layernorm) {
    const uint32_t cen = m31_sub(x, mean);
    st_q(w, p, qm31_from_m31(cen));
    st_q(d, p, qm31_from_m31(rs));
    st_q(in_q, p, qm31_from_m31(x));
    out_u[p] = m31_mul(cen, rs);
  } else {
    const uint32_t sc = (c < active && ng) ? m31_mul(rs, gamma[c < ng - 1 ? c : ng - 1]) : rs;
    st_q(w, p, qm31_from_m31(x));
    st_q(d, p, qm31_from_m31(sc));
    out_u[p] = c < active ? m31_mul(x, sc) : x;
  }
}

// ------------------------------------------------------------------ host side
namespace {

struct NormShape {
  bool ln = true;
  uint64_t rows = 0, cols = 0, prow = 0, pcol = 0, n = 0, active = 0;
  int nv = 0, lr = 0;
  std::vector<uint32_t> key, var, rsq, mean;  // per padded row: key = LN variance / RMS rms^2
  uint32_t t1_total = 0;                      // sum of the input over every entry (LN)
  uint32_t cen_sq_total = 0;                  // sum of centered^2 over every entry (LN)
  uint32_t sq_total = 0;                      // sum of input^2 over every entry (RMS)
};

// sum_r v_r eq(z[0 .. lr), r): the MLE at z of a function constant along the
// columns (the column variables of eq sum to one).
qm31 row_mle(const std::vector<qm31>& v, int lr, const qm31* z) {
  std::vector<qm31> e(v.begin(), v.end());
  size_t len = e.size();
  for (int k = 0; k < lr; k++) {  // fold the most significant variable first
    const size_t h = len / 2;
    for (size_t i = 0; i < h; i++) e[i] = qm31_fold(e[i], e[i + h], z[k]);
    len = h;
  }
  return e[0];
}
std::vector<qm31> as_q(const std::vector<uint32_t>& v) {
  std::vector<qm31> q(v.size());
  for (size_t i = 0; i < v.size(); i++) q[i] = qm31_from_m31(v[i]);
  return q;
}

// Forward statistics of both layers (prover.rs:7968-8020, 8447-8487) from the
// device row sums: LayerNorm mean = S1 / active, variance = (S2 - 2 mean S1 +
// active mean^2) / active masked to the table, rsqrt = table[variance];
// RMSNorm rms^2 = (S2 / active) masked, rsqrt = table[rms^2].  Padding rows
// are zero.  Also the whole-vector sums Part 0 mixes.
int norm_stats(gkr_ctx* c, const gkr_matrix* X, bool ln, uint64_t dim, NormShape* S) {
  S->ln = ln;
  S->rows = X->rows;
  S->cols = X->cols;
  S->prow = next_pow2(X->rows);
  S->pcol = next_pow2(X->cols);
  S->n = S->prow * S->pcol;
  S->nv = log2_exact(S->n);
  S->lr = log2_exact(S->prow);
  S->active = dim < S->pcol ? dim : S->pcol;
  if (S->nv == 0) return fail(GKR_ERR_INVALID, "norm layer over a single entry has no rounds");
  if (dim == 0) return fail(GKR_ERR_INVALID, "norm layer with no active column");
  if (S->nv > kMaxVars) return fail(GKR_ERR_INVALID, "norm layer too large");
  std::vector<uint32_t> sums(4 * X->rows);
  uint32_t* d_sums;
  TRY(ensureT(c, S_NORMSUM, 4 * X->rows, &d_sums));
  const uint64_t act_real = S->active < X->cols ? S->active : X->cols;
  {
    TimedLaunch tl(c, K_NORM, 4 * X->rows * X->cols + 16 * X->rows);
    GKR_LAUNCH(c, k_norm_rows, dim3((unsigned)X->rows), dim3(kBlock), 0, X->dev, X->cols, act_real,
                       d_sums);
  }
  TRY(check_launch(c));
  HIP_TRY(hipMemcpyAsync(sums.data(), d_sums, sums.size() * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
  TRY(sync(c));
  const uint32_t act_m = m31_from_u32((uint32_t)(S->active % P));
  const uint32_t inv_n = S->active ? m31_inv(act_m) : 0u;
  const uint32_t pcol_m = m31_from_u32((uint32_t)(S->pcol % P));
  S->key.assign(S->prow, 0);
  S->var.assign(S->prow, 0);
  S->rsq.assign(S->prow, 0);
  S->mean.assign(S->prow, 0);
  S->t1_total = S->cen_sq_total = S->sq_total = 0;
  for (uint64_t r = 0; r < S->prow; r++) {
    const bool real = r < X->rows;
    const uint32_t s1 = real ? sums[4 * r] : 0u, s2 = real ? sums[4 * r + 1] : 0u;
    const uint32_t t1 = real ? sums[4 * r + 2] : 0u, t2 = real ? sums[4 * r + 3] : 0u;
    if (ln) {
      const uint32_t mean = m31_mul(s1, inv_n);
      // sum over the active columns of (x - mean)^2 = S2 - 2 mean S1 + active mean^2
      const uint32_t m2 = m31_mul(mean, mean);
      const uint32_t vs = m31_add(m31_sub(s2, m31_mul(m31_add(mean, mean), s1)), m31_mul(act_m, m2));
      const uint32_t var = m31_mul(vs, inv_n) & kNormMask;
      S->mean[r] = mean;
      S->var[r] = var;
      S->key[r] = var;
      S->rsq[r] = norm_rsqrt(var);
      // Part 0 totals over the whole padded row: sum x and sum (x - mean)^2 over pcol entries
      S->t1_total = m31_add(S->t1_total, t1);
      const uint32_t row_sq = m31_add(m31_sub(t2, m31_mul(m31_add(mean, mean), t1)), m31_mul(pcol_m, m2));
      S->cen_sq_total = m31_add(S->cen_sq_total, row_sq);
    } else {
      const uint32_t ms = m31_mul(s2, inv_n) & kNormMask;
      S->key[r] = ms;
      S->rsq[r] = norm_rsqrt(ms);
      S->sq_total = m31_add(S->sq_total, t2);
    }
  }
  return GKR_OK;
}

// Builds the padded device vectors: S_W0 (w), S_D0 (d), S_E0 (LayerNorm input
// as QM31), S_MIN (input u32), S_MOUT (output u32).
int norm_prepare(gkr_ctx* c, const gkr_matrix* X, const NormShape& S, const uint32_t* gamma, uint64_t ng) {
  std::vector<uint32_t> rowv(2 * S.prow);
  for (uint64_t r = 0; r < S.prow; r++) {
    rowv[2 * r] = S.ln ? S.mean[r] : 0u;
    rowv[2 * r + 1] = S.rsq[r];
  }
  uint32_t *d_rowv, *d_gamma = nullptr, *in_u, *out_u;
  qm31 *w, *d, *in_q;
  TRY(ensureT(c, S_NORMROW, rowv.size() + (gamma ? ng : 0), &d_rowv));
  if (gamma && ng) d_gamma = d_rowv + rowv.size();
  TRY(ensureT(c, S_W0, S.n, &w));
  TRY(ensureT(c, S_D0, S.n, &d));
  TRY(ensureT(c, S_E0, S.ln ? S.n : 1, &in_q));
  TRY(ensureT(c, S_MIN, S.n, &in_u));
  TRY(ensureT(c, S_MOUT, S.n, &out_u));
  HIP_TRY(hipMemcpyAsync(d_rowv, rowv.data(), rowv.size() * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
  if (d_gamma)
    HIP_TRY(hipMemcpyAsync(d_gamma, gamma, ng * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
  {  // reads X once; writes w, d (and the LayerNorm input) as QM31, input and output as u32
    TimedLaunch tl(c, K_NORM, 4 * S.rows * S.cols + (S.ln ? 56 : 40) * S.n);
    GKR_LAUNCH(c, k_norm_prepare, dim3(grid_for(S.n)), dim3(kBlock), 0, X->dev, S.rows, S.cols,
                       log2_exact(S.pcol), S.n, S.ln ? 1 : 0, S.active, d_rowv, d_gamma, d_gamma ? ng : 0, w, d,
                       in_q, in_u, out_u);
  }
  TRY(check_launch(c));
  // the host copies of rowv / gamma must outlive the copies
  return sync(c);
}

// MLEs of the input (S_MIN) and output (S_MOUT) at z: one eq split, one pass.
int norm_evals(gkr_ctx* c, const NormShape& S, const qm31* z, qm31* in_eval, qm31* out_eval) {
  uint32_t *in_u, *out_u;
  TRY(ensureT(c, S_MIN, S.n, &in_u));
  TRY(ensureT(c, S_MOUT, S.n, &out_u));
  if (S.n != (1ull << S.nv)) return fail(GKR_ERR_DEVICE, "norm vectors of %llu entries over %d variables",
                                         (unsigned long long)S.n, S.nv);
  qm31 io[2];
  TRY(dot2_evals(c, z, S.nv, in_u, out_u, io));
  *in_eval = io[0];
  *out_eval = io[1];
  return GKR_OK;
}

void deg2_coeffs(const qm31 s[3], qm31 cf[4]) {  // Newton form, c3 = 0 (prover.rs:8074-8082)
  const qm31 inv2 = qm31_from_m31(1u << 30);
  const qm31 dd1 = qm31_sub(s[1], s[0]);
  const qm31 dd2 = qm31_mul(qm31_sub(qm31_sub(s[2], s[1]), dd1), inv2);
  cf[0] = s[0];
  cf[1] = qm31_sub(dd1, dd2);
  cf[2] = dd2;
  cf[3] = qm31_zero();
}

// LayerNorm Part 0 (prover.rs:8030-8097): the plain sumcheck of
// eta0 input(x) + eta1 centered(x)^2 over 2^T entries.  Device trips of up to
// 3 rounds: a Gram trip (kind 0) of centered with itself gives the squared
// part, a plain-sum trip (kind 2) of input the linear part, both folded by the
// same challenges; the hand-over brings both vectors to the host for the last
// rounds.  Outputs: 4 coefficients per round (c3 = 0), the challenges, and
// the final values of input and centered.
int mean_var_sumcheck(gkr_ctx* c, PoseidonChannel& ch, int T, const qm31* cen, const qm31* inp, const qm31& eta0,
                      const qm31& eta1, gkr_qm31* polys, qm31* chal, qm31* in_final, qm31* cen_final) {
  const uint64_t n = 1ull << T;
  qm31 *ca1, *ca2, *ia1, *ia2;
  TRY(ensureT(c, S_FA1, n / 2 + 1, &ca1));
  TRY(ensureT(c, S_FA0, n / 4 + 1, &ca2));
  TRY(ensureT(c, S_FB1, n / 2 + 1, &ia1));
  TRY(ensureT(c, S_FB0, n / 4 + 1, &ia2));
  c->mm.valid = false;
  qm31* cb[2] = {ca1, ca2};
  qm31* ib[2] = {ia1, ia2};
  auto absorb = [&](int t, const qm31 s[3]) {
    qm31 cf[4];
    deg2_coeffs(s, cf);
    for (int k = 0; k < 4; k++) polys[4 * t + k] = G(cf[k]);
    HostTimer ht(c, K_HOST_FS);
    ch.mix_poly_coeffs_deg3(cf[0], cf[1], cf[2], cf[3]);
    chal[t] = ch.draw_qm31();
  };
  const std::vector<Trip> trips = plan_trips(T, kHostTailMM, trip_k(n));
  const qm31 xs[3] = {qm31_zero(), qm31_one(), qm31_from_m31(2)};
  HandoverSession ho(c);
  const qm31 *src_c = cen, *src_i = inp, *pend = nullptr;
  int np = 0;
  for (size_t j = 0; j < trips.size(); j++) {
    const Trip& tr = trips[j];
    qm31* dc = j == 0 ? nullptr : cb[(j - 1) & 1];
    qm31* di = j == 0 ? nullptr : ib[(j - 1) & 1];
    RoundSink skq, skl;
    TRY(launch_trip(c, 0, tr.K, src_c, src_c, tr.n, np, pend, dc, nullptr, nullptr, nullptr, 0, 0, &skq));
    TRY(launch_trip(c, 2, tr.K, src_i, nullptr, tr.n, np, pend, di, nullptr, nullptr, nullptr, 0, kSlotMult0, &skl));
    if (j > 0) {
      src_c = dc;
      src_i = di;
    }
    if (j + 1 == trips.size()) TRY(ho.launch<2>(src_c, src_i, tr.n, tr.K));
    qm31 L[8];
    TRY(wait_trip(c, skl, 1 << tr.K, L));  // the Gram sums (earlier on the stream) are in their slot too
    qm31 Gm[kMaxSums];
    const int slot_q = (int)(skq.out - c->h_out);
    for (int q = 0; q < trip_nq(0, tr.K); q++) Gm[q] = c->h_out[slot_q + q];
    TripGram tg(Gm, tr.K, nullptr, qm31_zero());
    for (int i = 0; i < tr.K; i++) {
      qm31 qv[3], lv[2], s[3];
      if (i) tg.fold(chal[tr.t + i - 1]);
      tg.values(3, xs, qv);
      trip_round_sum(L, tr.K, i, chal + tr.t, lv);
      const qm31 l2 = qm31_sub(qm31_add(lv[1], lv[1]), lv[0]);
      s[0] = qm31_add(qm31_mul(eta0, lv[0]), qm31_mul(eta1, qv[0]));
      s[1] = qm31_add(qm31_mul(eta0, lv[1]), qm31_mul(eta1, qv[1]));
      s[2] = qm31_add(qm31_mul(eta0, l2), qm31_mul(eta1, qv[2]));
      absorb(tr.t + i, s);
      if (j + 1 == trips.size()) TRY(ho.post_one(i, chal[tr.t + i]));  // the hand-over folds it while the next is drawn
    }
    np = tr.K;
    pend = chal + tr.t;
  }
  const int t_end = trips.empty() ? 0 : trips.back().t + trips.back().K;
  std::vector<qm31> v[2];
  TRY(ho.post(pend, np));
  TRY(ho.fetch(n >> t_end, 2, v));
  std::vector<qm31>& Cv = v[0];
  std::vector<qm31>& Iv = v[1];
  for (int t = t_end; t < T; t++) {
    const size_t half = Cv.size() / 2;
    qm31 s[3] = {qm31_zero(), qm31_zero(), qm31_zero()};
    {
      HostTimer ht(c, K_HOST_FINISH);
      for (size_t i = 0; i < half; i++) {
        const qm31 c0 = Cv[i], c1 = Cv[i + half], i0 = Iv[i], i1 = Iv[i + half];
        const qm31 c2 = qm31_sub(qm31_add(c1, c1), c0), i2 = qm31_sub(qm31_add(i1, i1), i0);
        s[0] = qm31_add(s[0], qm31_add(qm31_mul(eta0, i0), qm31_mul(eta1, qm31_sqr(c0))));
        s[1] = qm31_add(s[1], qm31_add(qm31_mul(eta0, i1), qm31_mul(eta1, qm31_sqr(c1))));
        s[2] = qm31_add(s[2], qm31_add(qm31_mul(eta0, i2), qm31_mul(eta1, qm31_sqr(c2))));
      }
    }
    absorb(t, s);
    HostTimer ht(c, K_HOST_FINISH);
    for (size_t i = 0; i < half; i++) {
      Cv[i] = qm31_fold(Cv[i], Cv[i + half], chal[t]);
      Iv[i] = qm31_fold(Iv[i], Iv[i + half], chal[t]);
    }
    Cv.resize(half);
    Iv.resize(half);
  }
  *cen_final = Cv[0];
  *in_final = Iv[0];
  return GKR_OK;
}

// The rsqrt LogUp of Part 2 over the per-row keys and rsqrt values (see the
// file comment), the multiplicity sumcheck (prover.rs:9449-9511) over the
// nonzero multiplicities, and the table commitment (prover.rs:8357-8363).
int norm_logup(gkr_ctx* c, PoseidonChannel& C, uint64_t type_tag, const NormShape& S, const qm31* z,
               gkr_norm_out* out) {
  const uint32_t tsize = 1u << kNormTableLog;
  memset(out->multiplicities, 0, tsize * sizeof(uint32_t));
  for (uint64_t r = 0; r < S.prow; r++) out->multiplicities[S.key[r]] += (uint32_t)S.pcol;
  C.mix_u64(0x4C4F47ull);  // "LOG"
  C.mix_u64(type_tag);
  const qm31 gamma = C.draw_qm31(), beta = C.draw_qm31();
  std::vector<qm31> w(S.prow), d(S.prow), e(S.prow);
  qm31 wsum = qm31_zero();
  for (uint64_t r = 0; r < S.prow; r++) {
    d[r] = qm31_sub(qm31_sub(gamma, qm31_from_m31(S.key[r])), qm31_mul(beta, qm31_from_m31(S.rsq[r])));
    w[r] = qm31_inv(d[r]);
    wsum = qm31_add(wsum, w[r]);
  }
  const qm31 trace_sum = qm31_mul_m31(wsum, m31_from_u32((uint32_t)(S.pcol % P)));
  qm31 table_sum = qm31_zero();
  for (uint32_t j = 0; j < tsize; j++)
    if (out->multiplicities[j]) {
      const qm31 dj =
          qm31_sub(qm31_sub(gamma, qm31_from_m31(j)), qm31_mul(beta, qm31_from_m31(norm_rsqrt(j))));
      table_sum = qm31_add(table_sum, qm31_mul_m31(qm31_inv(dj), m31_from_u32(out->multiplicities[j])));
    }
  if (!qm31_eq(trace_sum, table_sum)) return fail(GKR_ERR_LOGUP, "norm rsqrt LogUp sum mismatch");
  C.mix_secure_field(trace_sum);
  out->claimed_sum = G(trace_sum);
  // row rounds: the eq-sumcheck over the padded rows (prover.rs:8270-8319)
  const qm31 two = qm31_from_m31(2), three = qm31_from_m31(3);
  const qm31 inv2 = qm31_from_m31(1u << 30), inv6 = qm31_from_m31(m31_inv(6));
  {
    e[0] = qm31_one();  // eq(z[0 .. lr), r), first coordinate on the most significant bit
    for (int l = 0; l < S.lr; l++) {
      const uint64_t m = 1ull << l;
      for (int64_t u = (int64_t)m - 1; u >= 0; u--) {
        const qm31 eu = e[u];
        e[2 * u + 1] = qm31_mul(eu, z[l]);
        e[2 * u] = qm31_sub(eu, e[2 * u + 1]);
      }
    }
  }
  std::vector<qm31> s(S.nv);
  size_t len = S.prow;
  for (int t = 0; t < S.lr; t++) {
    const size_t mid = len / 2;
    qm31 sk[4];
    for (int k = 0; k < 4; k++) {
      const qm31 x = qm31_from_m31((uint32_t)k), omx = qm31_sub(qm31_one(), x);
      qm31 acc = qm31_zero();
      for (size_t i = 0; i < mid; i++) {
        const qm31 et = qm31_add(qm31_mul(omx, e[i]), qm31_mul(x, e[mid + i]));
        const qm31 wt = qm31_add(qm31_mul(omx, w[i]), qm31_mul(x, w[mid + i]));
        const qm31 dt = qm31_add(qm31_mul(omx, d[i]), qm31_mul(x, d[mid + i]));
        acc = qm31_add(acc, qm31_mul(qm31_mul(et, wt), dt));
      }
      sk[k] = acc;
    }
    const qm31 dd1 = qm31_sub(sk[1], sk[0]);
    const qm31 dd2 = qm31_mul(qm31_add(qm31_sub(qm31_sub(sk[2], sk[1]), sk[1]), sk[0]), inv2);
    const qm31 dd3 = qm31_mul(qm31_sub(qm31_sub(sk[3], sk[0]), qm31_mul(three, qm31_sub(sk[2], sk[1]))), inv6);
    const qm31 cf[4] = {sk[0], qm31_add(qm31_sub(dd1, dd2), qm31_mul(two, dd3)), qm31_sub(dd2, qm31_mul(three, dd3)),
                        dd3};
    for (int k = 0; k < 4; k++) out->logup_round_polys[4 * t + k] = G(cf[k]);
    C.mix_poly_coeffs_deg3(cf[0], cf[1], cf[2], cf[3]);
    s[t] = C.draw_qm31();
    for (size_t i = 0; i < mid; i++) {
      e[i] = qm31_fold(e[i], e[i + mid], s[t]);
      w[i] = qm31_fold(w[i], w[i + mid], s[t]);
      d[i] = qm31_fold(d[i], d[i + mid], s[t]);
    }
    len = mid;
  }
  // column rounds: w d constant, p(X) = K eqlin(z_t, X) with K = e w d prod_{earlier} eqlin(z, s)
  qm31 K = qm31_mul(qm31_mul(e[0], w[0]), d[0]);
  for (int t = S.lr; t < S.nv; t++) {
    const qm31 zt = z[t];
    const qm31 cf[4] = {qm31_mul(K, qm31_sub(qm31_one(), zt)), qm31_mul(K, qm31_sub(qm31_add(zt, zt), qm31_one())),
                        qm31_zero(), qm31_zero()};
    for (int k = 0; k < 4; k++) out->logup_round_polys[4 * t + k] = G(cf[k]);
    C.mix_poly_coeffs_deg3(cf[0], cf[1], cf[2], cf[3]);
    s[t] = C.draw_qm31();
    const qm31 el = qm31_add(qm31_mul(qm31_sub(qm31_one(), zt), qm31_sub(qm31_one(), s[t])), qm31_mul(zt, s[t]));
    K = qm31_mul(K, el);
  }
  out->w_eval = G(w[0]);
  out->in_eval = G(row_mle(as_q(S.key), S.lr, s.data()));
  out->out_eval = G(row_mle(as_q(S.rsq), S.lr, s.data()));
  // multiplicity sumcheck over the 2^16 table, from the nonzero entries
  std::vector<uint32_t> nz;
  for (uint32_t j = 0; j < tsize; j++)
    if (out->multiplicities[j]) nz.push_back(j);
  std::vector<qm31> ew(nz.size(), qm31_one());
  qm31 msum = qm31_zero();
  for (uint32_t j : nz) msum = qm31_add(msum, qm31_from_m31(m31_from_u32(out->multiplicities[j])));
  for (uint32_t t = 0; t < kNormTableLog; t++) {
    qm31 lo = qm31_zero(), hi = qm31_zero();
    const uint32_t bit = kNormTableLog - 1 - t;
    for (size_t q = 0; q < nz.size(); q++) {
      const qm31 v = qm31_mul_m31(ew[q], m31_from_u32(out->multiplicities[nz[q]]));
      if ((nz[q] >> bit) & 1)
        hi = qm31_add(hi, v);
      else
        lo = qm31_add(lo, v);
    }
    const qm31 c0 = lo, c1 = qm31_sub(hi, lo);
    out->mult_round_polys[2 * t] = G(c0);
    out->mult_round_polys[2 * t + 1] = G(c1);
    C.mix_secure_field(c0);
    C.mix_secure_field(c1);
    const qm31 a = C.draw_qm31();
    for (size_t q = 0; q < nz.size(); q++)
      ew[q] = qm31_mul(ew[q], ((nz[q] >> bit) & 1) ? a : qm31_sub(qm31_one(), a));
  }
  qm31 mfin = qm31_zero();
  for (size_t q = 0; q < nz.size(); q++)
    mfin = qm31_add(mfin, qm31_mul_m31(ew[q], m31_from_u32(out->multiplicities[nz[q]])));
  out->mult_final_eval = G(mfin);
  out->mult_claimed_sum = G(msum);
  felt tc_in[2] = {felt_from_u64(kNormTagRS), felt_from_u64(kNormTableLog)};
  out->table_commitment = felt_to_abi(poseidon_hash_many(tc_in, 2));
  return GKR_OK;
}

int norm_check(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
               const gkr_matrix* X, gkr_norm_out* out, std::vector<qm31>* cpt) {
  if (!c || !X || !claim_value || !out || (!claim_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (X->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another context");
  if (!out->p0_round_polys || !out->lin_round_polys || !out->logup_round_polys || !out->multiplicities ||
      !out->mult_round_polys || !out->row_stats0 || !out->row_stats1)
    return fail(GKR_ERR_INVALID, "null output arrays");
  const int nv = log2_exact(next_pow2(X->rows) * next_pow2(X->cols));
  if ((int)n_point != nv) return fail(GKR_ERR_INVALID, "claim point has %u vars, the norm MLE has %d", n_point, nv);
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  cpt->resize(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(claim_point[l])) return fail(GKR_ERR_INVALID, "claim point not canonical");
    (*cpt)[l] = Q(claim_point[l]);
  }
  return GKR_OK;
}

void record_norm(gkr_proof* proof, bool ln, const qm31& claim, const NormShape& S, const gkr_norm_out* o) {
  if (!proof) return;
  LayerRec L;
  L.tag = ln ? 4 : 8;
  L.claim_value = claim;
  NormRec& N = L.norm;
  N.input_eval = Q(o->input_eval);
  N.output_eval = Q(o->output_eval);
  N.mean_eval = Q(o->mean_eval);
  N.rsqrt_eval = Q(o->rsqrt_eval);
  N.var_eval = Q(o->var_eval);
  N.n_active = o->n_active;
  N.sum0 = Q(o->sum0);
  N.sum1 = Q(o->sum1);
  for (int i = 0; i < 4 * S.nv; i++) {
    N.p0.push_back(Q(o->p0_round_polys[i]));
    N.lin.push_back(Q(o->lin_round_polys[i]));
    N.logup.push_back(Q(o->logup_round_polys[i]));
  }
  N.p0_final0 = Q(o->p0_final0);
  N.p0_final1 = Q(o->p0_final1);
  N.lin_final0 = Q(o->lin_final0);
  N.lin_final1 = Q(o->lin_final1);
  N.cb_input = Q(o->cb_input);
  N.cb_mean = Q(o->cb_mean);
  N.claimed_sum = Q(o->claimed_sum);
  N.w_eval = Q(o->w_eval);
  N.in_eval = Q(o->in_eval);
  N.out_eval = Q(o->out_eval);
  N.mults.assign(o->multiplicities, o->multiplicities + (1u << kNormTableLog));
  for (uint32_t i = 0; i < 2 * kNormTableLog; i++) N.mult_rp.push_back(Q(o->mult_round_polys[i]));
  N.mult_final = Q(o->mult_final_eval);
  N.mult_sum = Q(o->mult_claimed_sum);
  N.table_commitment = felt_canon_from_words(o->table_commitment.w);
  N.rows0.assign(o->row_stats0, o->row_stats0 + o->n_rows);
  N.rows1.assign(o->row_stats1, o->row_stats1 + o->n_rows);
  proof_add_layer(proof, std::move(L));
}

}  // namespace

// Both reducers: ln selects LayerNorm (prover.rs:7944-8395) or RMSNorm
// (8407-8801, with the optional per-column gamma).
int prove_norm(gkr_ctx* c, bool ln, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
               const gkr_matrix* X, uint64_t dim, const uint32_t* gamma, uint64_t ng, gkr_channel* ch,
               gkr_proof* proof, gkr_norm_out* out, bool commit_gamma) {
  CH_CHECK(ch);
  std::vector<qm31> z;
  TRY(norm_check(c, claim_point, n_point, claim_value, X, out, &z));
  if (gamma && ng)
    for (uint64_t i = 0; i < ng; i++)
      if (gamma[i] >= P) return fail(GKR_ERR_INVALID, "gamma value %llu not canonical", (unsigned long long)i);
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  TraceScope trace;
  PoseidonChannel& C = ch->ch;
  NormShape S;
  TRY(norm_stats(c, X, ln, dim, &S));
  TRY(norm_prepare(c, X, S, ln ? nullptr : gamma, ln ? 0 : ng));
  const qm31 claim = Q(*claim_value);
  qm31 input_eval, output_eval;
  TRY(norm_evals(c, S, z.data(), &input_eval, &output_eval));
  const qm31 key_eval = row_mle(as_q(S.key), S.lr, z.data());
  const qm31 rsqrt_eval = row_mle(as_q(S.rsq), S.lr, z.data());
  out->input_eval = G(input_eval);
  out->output_eval = G(output_eval);
  out->mean_eval = G(ln ? row_mle(as_q(S.mean), S.lr, z.data()) : key_eval);
  out->rsqrt_eval = G(rsqrt_eval);
  out->var_eval = G(ln ? key_eval : qm31_zero());
  out->n_active = (uint32_t)S.active;
  out->gamma_commitment = felt_to_abi(felt_zero());
  out->gamma_eval = G(qm31_zero());
  if (!ln && gamma && ng) {  // gamma commitment and evaluation (prover.rs:8758-8781), neither mixed nor serialized
    if (commit_gamma) {
      PoseidonChannel g;
      g.mix_u64(kNormTagGamma);
      for (uint64_t i = 0; i < ng; i++) g.mix_secure_field(qm31_from_m31(gamma[i]));
      out->gamma_commitment = felt_to_abi(g.digest);
    }
    std::vector<qm31> gcol(S.pcol);
    for (uint64_t col = 0; col < S.pcol; col++) gcol[col] = col < ng ? qm31_from_m31(gamma[col]) : qm31_one();
    // MLE at z of gamma broadcast over rows: the row variables sum to one
    std::vector<qm31> e(gcol);
    size_t len = e.size();
    for (int k = S.lr; k < S.nv; k++) {
      const size_t h = len / 2;
      for (size_t i = 0; i < h; i++) e[i] = qm31_fold(e[i], e[i + h], z[k]);
      len = h;
    }
    out->gamma_eval = G(e[0]);
  }
  qm31 *w0, *d0, *w1, *d1, *in_q;
  TRY(ensureT(c, S_W0, S.n, &w0));
  TRY(ensureT(c, S_D0, S.n, &d0));
  TRY(ensureT(c, S_E0, ln ? S.n : 1, &in_q));

  std::vector<qm31> chal0(S.nv), chal1(S.nv);
  if (ln) {  // Part 0 (prover.rs:8030-8097)
    const qm31 tin = qm31_from_m31(S.t1_total), tcs = qm31_from_m31(S.cen_sq_total);
    C.mix_u64(kNormTagMV);
    C.mix_u64(S.active);
    C.mix_secure_field(tin);
    C.mix_secure_field(tcs);
    const qm31 eta0 = C.draw_qm31(), eta1 = qm31_mul(eta0, eta0);
    out->sum0 = G(tin);
    out->sum1 = G(tcs);
    qm31 in_f, cen_f;
    TRY(mean_var_sumcheck(c, C, S.nv, w0, in_q, eta0, eta1, out->p0_round_polys, chal0.data(), &in_f, &cen_f));
    const qm31 mean_f = row_mle(as_q(S.mean), S.lr, chal0.data());
    out->p0_final0 = G(in_f);
    out->p0_final1 = G(mean_f);
    C.mix_secure_field(in_f);
    C.mix_secure_field(mean_f);
  } else {  // Part 0 (prover.rs:8497-8540)
    const qm31 tsq = qm31_from_m31(S.sq_total);
    C.mix_u64(kNormTagRQ);
    C.mix_u64(S.active);
    C.mix_secure_field(tsq);
    out->sum0 = G(tsq);
    out->sum1 = G(qm31_zero());
    qm31 *a1, *a2, *b1, *b2;
    TRY(ensureT(c, S_FA1, S.n / 2 + 1, &a1));
    TRY(ensureT(c, S_FB1, S.n / 2 + 1, &b1));
    TRY(ensureT(c, S_FA0, S.n / 4 + 1, &a2));
    TRY(ensureT(c, S_FB0, S.n / 4 + 1, &b2));
    qm31* bufs_a[2] = {a1, a2};
    qm31* bufs_b[2] = {b1, b2};
    const qm31 one = qm31_one();
    std::vector<gkr_qm31> ch0(S.nv);
    gkr_qm31 fa, fb;
    TRY(product_sumcheck(c, C, S.nv, w0, w0, bufs_a, bufs_b, nullptr, 0, out->p0_round_polys, ch0.data(), &fa, &fb,
                         &one));
    out->p0_final0 = fa;
    out->p0_final1 = G(qm31_zero());
    C.mix_secure_field(Q(fa));
  }
  // Part 1: sum_x eq(z, x) w(x) d(x) (prover.rs:8099-8182, 8553-8630)
  C.mix_u64(ln ? kNormTagLN : kNormTagRN);
  C.mix_secure_field(Q(out->mean_eval));
  C.mix_secure_field(rsqrt_eval);
  C.mix_secure_field(claim);
  Eq3Plan epl;
  TRY(eq3_prepare(c, z.data(), S.nv, &epl));
  TRY(ensureT(c, S_W1, S.n / 2 + 1, &w1));
  TRY(ensureT(c, S_D1, S.n / 2 + 1, &d1));
  qm31 fin[3];
  TRY(eq3_sumcheck(c, C, z.data(), epl, w0, d0, w1, d1, out->lin_round_polys, chal1.data(), fin, nullptr));
  out->lin_final0 = G(fin[1]);
  out->lin_final1 = G(fin[2]);
  C.mix_secure_field(fin[1]);
  C.mix_secure_field(fin[2]);
  out->cb_input = out->cb_mean = G(qm31_zero());
  if (ln) {  // centered binding: centered = input - mean on the hypercube, so also as MLEs
    const qm31 cb_mean = row_mle(as_q(S.mean), S.lr, chal1.data());
    const qm31 cb_in = qm31_add(fin[1], cb_mean);
    out->cb_input = G(cb_in);
    out->cb_mean = G(cb_mean);
    C.mix_secure_field(cb_in);
    C.mix_secure_field(cb_mean);
  }
  // Part 2: rsqrt LogUp, multiplicity sumcheck, final mixes
  TRY(norm_logup(c, C, ln ? kNormTagRS : kNormTagRN, S, z.data(), out));
  C.mix_secure_field(input_eval);
  C.mix_secure_field(output_eval);
  trace_point(C, ln ? "layernorm" : "rmsnorm");
  out->n_rows = (uint32_t)S.prow;
  for (uint64_t r = 0; r < S.prow; r++) {
    out->row_stats0[r] = ln ? S.mean[r] : S.key[r];
    out->row_stats1[r] = ln ? S.var[r] : 0u;
  }
  record_norm(proof, ln, claim, S, out);
  return GKR_OK;
}

extern "C" int gkr_prove_layernorm_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                         const gkr_qm31* claim_value, const gkr_matrix* input, uint64_t dim,
                                         gkr_channel* ch, gkr_proof* proof, gkr_norm_out* out) {
  return prove_norm(c, true, claim_point, n_point, claim_value, input, dim, nullptr, 0, ch, proof, out, false);
}
extern "C" int gkr_prove_rmsnorm_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                       const gkr_qm31* claim_value, const gkr_matrix* input, uint64_t dim,
                                       const uint32_t* gamma, uint64_t n_gamma, gkr_channel* ch, gkr_proof* proof,
                                       gkr_norm_out* out) {
  return prove_norm(c, false, claim_point, n_point, claim_value, input, dim, gamma, n_gamma, ch, proof, out, true);
}

// The layer output's MLE at `point` (the value a fresh claim on the layer takes).
extern "C" int gkr_norm_output_claim(gkr_ctx* c, uint32_t kind, const gkr_matrix* input, uint64_t dim,
                                     const uint32_t* gamma, uint64_t n_gamma, const gkr_qm31* point, uint32_t n_point,
                                     gkr_qm31* value) {
  if (!c || !input || !value || (!point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (kind != GKR_STEP_LAYERNORM && kind != GKR_STEP_RMSNORM) return fail(GKR_ERR_INVALID, "kind %u is no norm", kind);
  if (input->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another context");
  const bool ln = kind == GKR_STEP_LAYERNORM;
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  NormShape S;
  TRY(norm_stats(c, input, ln, dim, &S));
  if ((int)n_point != S.nv) return fail(GKR_ERR_INVALID, "point has %u vars, the norm MLE has %d", n_point, S.nv);
  std::vector<qm31> z(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(point[l])) return fail(GKR_ERR_INVALID, "point not canonical");
    z[l] = Q(point[l]);
  }
  TRY(norm_prepare(c, input, S, ln ? nullptr : gamma, ln ? 0 : n_gamma));
  qm31 ie, oe;
  TRY(norm_evals(c, S, z.data(), &ie, &oe));
  *value = G(oe);
  return GKR_OK;
}
