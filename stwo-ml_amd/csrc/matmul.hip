// Matmul layer reduction: the restriction of both operands, the product
// sumcheck, reduce_matmul_layer_with_backend, the SIMD variants, the ZkmlOps
// MLE helpers and the product sumcheck over resident QM31 vectors.
#include "internal.h"

#include <mutex>
// ------------------------------------------------------------------ matmul reduction
// The weight-side restriction leaves f_b as column-chunk partials; the first
// product trip adds them (and stores f_b), or finish_fb does when another
// consumer comes first.
static int finish_fb(gkr_ctx* c) {
  if (!c->fb_pending) return GKR_OK;
  qm31* fb;
  TRY(ensureT(c, S_FB0, c->fb_pk, &fb));
  GKR_LAUNCH(c, k_restrict_cols_finish, dim3(grid_for(c->fb_pk)), dim3(kBlock), 0, (const qm31*)c->buf[S_COLPART], c->fb_rows, c->fb_pk, c->fb_chunks, fb);
  c->fb_pending = false;
  return check_launch(c);
}
// The int8 copy of weight B for the restriction (k_to_int8), on first use:
// one pass over B and a 4-byte read-back of the range flag.  Skipped when
// the context was created with GKR_INT8_WEIGHTS=0 in the environment.
static int prepare_r8(gkr_ctx* c, gkr_matrix* B) {
  if (B->r8_state || !c->int8_weights) return GKR_OK;
  const uint64_t nst = (B->cols + kR8TileCols - 1) / kR8TileCols;
  const uint64_t nrt = (B->rows + kR8TileRows - 1) / kR8TileRows;
  if (B->rows == 0 || nst == 0 || nrt * nst * kR8Tile > (1ull << 40)) {
    B->r8_state = -1;
    return GKR_OK;
  }
  int8_t* r8 = nullptr;
  if (hipMalloc(&r8, nrt * nst * kR8Tile) != hipSuccess) {  // no room: keep the u32 path
    (void)hipGetLastError();
    B->r8_state = -1;
    return GKR_OK;
  }
  uint32_t* bad;
  TRY(ensureT(c, S_R8FLAG, 1, &bad));
  HIP_TRY(hipMemsetAsync(bad, 0, sizeof(uint32_t), c->stream));
  const uint64_t slots = nrt * nst * 64;  // 16-byte lane slots
  const unsigned grid = (unsigned)std::min<uint64_t>((slots + kBlock - 1) / kBlock, 4096);
  GKR_LAUNCH(c, k_to_int8, dim3(grid), dim3(kBlock), 0, B->dev, B->rows, B->cols, nst, slots, (u32x4*)r8, bad);
  TRY(check_launch(c));
  uint32_t flag = 1;
  HIP_TRY(hipMemcpyAsync(c->h_res, bad, sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
  TRY(sync(c));
  memcpy(&flag, c->h_res, sizeof flag);
  if (flag) {
    drain(c);
    (void)hipFree(r8);
    B->r8_state = -1;
  } else {
    B->r8 = r8;
    B->r8_nst = nst;
    B->r8_state = 1;
  }
  return GKR_OK;
}
// Restrict A rows by r_i and B columns by r_j into f_a (S_FA0) and f_b (S_FB0),
// each of length pk (components/matmul.rs:470-565, backend.rs:127-134): one
// launch for both Lagrange tables, one for both restrictions (f_a directly,
// f_b as column-chunk partials in S_COLPART, pending until added).
// weight_only: f_a is left to the caller (the SIMD layer combines its blocks'
// activation sides itself); L_i is still built.
// The launch shape of one restriction, worked out before anything is
// allocated or launched (so a restriction launched ahead of its claim point
// can first check that no buffer has to grow).
#ifndef GKR_RC_TARGET
#define GKR_RC_TARGET 2560
#endif
#ifndef GKR_RC_MIN_CHUNK
#define GKR_RC_MIN_CHUNK 512
#endif
#ifndef GKR_RC_CEIL
#define GKR_RC_CEIL 1
#endif
#ifndef GKR_R8_WGS
#define GKR_R8_WGS 768
#endif
struct RestrictPlan {
  uint64_t m, k, n, pk;
  bool use8;
  uint64_t ldig_bytes;  // int8 digit blocks (use8)
  uint64_t act_blocks;
  uint64_t gr, gc, chunk;  // u32 path: row blocks, column chunks, chunk columns
  uint64_t nst, nrt;       // int8 path: column steps, row tiles (gc chunks of `chunk` steps)
  uint64_t ngroups;        // int8 path: groups of kR8Rows row tiles (gr == ngroups)
};
static int plan_restrict(const gkr_matrix* A, const gkr_matrix* B, uint64_t pk, bool weight_only, RestrictPlan* p) {
  p->m = A->rows;
  p->k = A->cols;
  p->n = B->cols;
  p->pk = pk;
  const uint64_t k = p->k, n = p->n;
  // int32 digit sums stay exact below 2^17 columns; the digits come from the combined eq launch
  p->use8 = B->r8_state == 1 && n < (1ull << 17) &&
            log2_exact(next_pow2(p->m)) + log2_exact(next_pow2(n)) <= kMaxVars;
  p->ldig_bytes = p->use8 ? (n + kR8TileCols - 1) / kR8TileCols * kR8Tile : 0;
  p->act_blocks = weight_only ? 0 : (pk + 63) / 64;  // 64 columns of A per workgroup
  if (p->use8) {
    // row-tile groups x column chunks: as many chunks (at most 8: the first
    // trip adds the chunk partials) as keep the grid within about GKR_R8_WGS
    // workgroups (768: one round of resident workgroups at this kernel's
    // occupancy; on cold weights the Qwen layer's seven restrictions took
    // 68.8 us against 79.8 us for one row tile per workgroup at 2048)
    p->nst = B->r8_nst;
    p->nrt = (k + kR8TileRows - 1) / kR8TileRows;
    p->ngroups = (p->nrt + kR8Rows - 1) / kR8Rows;
    const uint64_t room = GKR_R8_WGS > p->act_blocks + p->ngroups ? GKR_R8_WGS - p->act_blocks : p->ngroups;
    const uint64_t gc8 = std::max<uint64_t>(1, std::min<uint64_t>({8, room / p->ngroups, p->nst}));
    p->chunk = (p->nst + gc8 - 1) / gc8;
    p->gc = (p->nst + p->chunk - 1) / p->chunk;
    p->gr = p->ngroups;
  } else {
    // column chunks: chunks a multiple of one wave sweep (256 columns), at
    // least GKR_RC_MIN_CHUNK columns, and at most GKR_RC_TARGET workgroups in
    // all (GKR_RC_CEIL: at least that many)
    const uint64_t rows_per_block = (uint64_t)kColRows * kColWaves;
    p->gr = (k + rows_per_block - 1) / rows_per_block;
    uint64_t gc = GKR_RC_CEIL ? (GKR_RC_TARGET + p->gr - 1) / p->gr : GKR_RC_TARGET / p->gr;
    if (gc < 1) gc = 1;
    uint64_t chunk = (n + gc - 1) / gc;
    chunk = (chunk + 255) / 256 * 256;
    if (chunk < GKR_RC_MIN_CHUNK) chunk = GKR_RC_MIN_CHUNK;
    p->chunk = chunk;
    p->gc = (n + chunk - 1) / chunk;
  }
  if (p->act_blocks + p->gr * p->gc > 0x7fffffffull) return fail(GKR_ERR_INVALID, "matrix too large for one restriction");
  return GKR_OK;
}
// Device buffers of a restriction: {slot, bytes}.
static void restrict_buffers(const RestrictPlan& p, std::vector<std::pair<Slot, size_t>>* out) {
  out->clear();
  if (p.use8) out->push_back({S_LDIG, p.ldig_bytes});
  out->push_back({S_LI, p.m * sizeof(qm31)});
  out->push_back({S_LJ, p.n * sizeof(qm31)});
  out->push_back({S_FA0, p.pk * sizeof(qm31)});
  out->push_back({S_FB0, p.pk * sizeof(qm31)});
  out->push_back({S_COLPART, p.gc * p.k * sizeof(qm31)});
}
// The claim point of a restriction launched ahead of it: in device memory,
// written by k_point_wait, valid when *status == want.
struct DevicePoint {
  const PointArg* pt;
  const uint32_t* status;
  uint32_t want;
};

// Restrict A rows by r_i and B columns by r_j into f_a (S_FA0) and f_b (S_FB0),
// each of length pk (components/matmul.rs:470-565, backend.rs:127-134): one
// launch for both Lagrange tables, one for both restrictions (f_a directly,
// f_b as column-chunk partials in S_COLPART, pending until added).
// weight_only: f_a is left to the caller (the SIMD layer combines its blocks'
// activation sides itself); L_i is still built.  dp given: the point (n_ri +
// n_rj coordinates) comes from device memory (r_i, r_j unused) and the int8
// copy must already exist or be ruled out (no synchronisation here).
static int restrict_pair(gkr_ctx* c, const gkr_matrix* A, const gkr_matrix* B, const qm31* r_i, int n_ri,
                         const qm31* r_j, int n_rj, uint64_t pk, bool weight_only = false,
                         const DevicePoint* dp = nullptr) {
  if (!dp) TRY(prepare_r8(c, const_cast<gkr_matrix*>(B)));  // the matrix's contents never change; r8 is derived
  HostTimer ht(c, K_HOST_LAUNCH);
  RestrictPlan p;
  TRY(plan_restrict(A, B, pk, weight_only, &p));
  const uint64_t m = p.m, k = p.k, n = p.n;
  if ((p.use8 || dp) && n_ri + n_rj > kMaxVars)
    return fail(GKR_ERR_DEVICE, "the combined eq launch takes at most %d point coordinates", kMaxVars);
  uint8_t* ldig = nullptr;
  if (p.use8) TRY(ensureT(c, S_LDIG, p.ldig_bytes, &ldig));
  qm31 *Li, *Lj, *fa, *fb, *part;
  TRY(ensureT(c, S_LI, m, &Li));
  TRY(ensureT(c, S_LJ, n, &Lj));
  TRY(ensureT(c, S_FA0, pk, &fa));
  TRY(ensureT(c, S_FB0, pk, &fb));
  TRY(ensureT(c, S_COLPART, (size_t)p.gc * k, &part));
  c->fb_pending = false;
  if (n_ri + n_rj <= kMaxVars) {
    PointArg pt;
    if (dp) {
      memset(&pt, 0, sizeof pt);
    } else {
      std::vector<qm31> both(r_i, r_i + n_ri);
      both.insert(both.end(), r_j, r_j + n_rj);
      pt = make_point(both.data(), n_ri + n_rj);
    }
    TimedLaunch tl(c, K_EQ_TABLE, 16 * (m + n));
    const uint64_t threads =
        kEqLanes * (eq_two_lead(m) + (ldig ? (n + kR8TileCols - 1) / kR8TileCols * kR8TileCols : n));
    GKR_LAUNCH(c, k_eq_two, dim3(grid_for(threads)), dim3(kBlock), 0, pt, dp ? dp->pt : nullptr,
               dp ? dp->status : nullptr, dp ? dp->want : 0u, n_ri, m, n, Li, Lj, ldig);
    TRY(check_launch(c));
  } else {
    TRY(eq_table(c, r_i, n_ri, m, Li));
    TRY(eq_table(c, r_j, n_rj, n, Lj));
  }
  // the activation side rides in act_blocks more workgroups (64 columns of A each)
  RowsJob rows{A->dev, m, k, pk, Li, fa};
  if (p.use8) {
    // algorithmic bytes: B as int8 and L_j's digits (weight side), A and L_i (activation side), f_a written
    TimedLaunch t(c, K_RESTRICT_COLS, k * n + 16 * n + (weight_only ? 0 : 4 * m * k + 16 * m + 16 * pk), true);
    GKR_LAUNCH(c, k_restrict_cols8, dim3((unsigned)(p.act_blocks + p.ngroups * p.gc)), dim3(kBlock), 0,
               (const u32x4*)B->r8, k, p.nst, (const u32x4*)ldig, (uint32_t)p.chunk, (uint32_t*)part, rows,
               (uint32_t)p.act_blocks, (uint32_t)p.ngroups);
    TRY(check_launch(c));
  } else {
    // algorithmic bytes: B and L_j (weight side) plus A and L_i (activation side), f_a written
    TimedLaunch t(c, K_RESTRICT_COLS, 4 * k * n + 16 * n + (weight_only ? 0 : 4 * m * k + 16 * m + 16 * pk), true);
    const dim3 grid((unsigned)(p.act_blocks + p.gr * p.gc));
    if (n % 4 == 0 && ((uintptr_t)B->dev & 15) == 0)
      GKR_LAUNCH(c, k_restrict_cols<true>, grid, dim3(kBlock), 0, B->dev, k, n, p.chunk, Lj, (uint32_t*)part, rows,
                 (uint32_t)p.act_blocks, (uint32_t)p.gr);
    else
      GKR_LAUNCH(c, k_restrict_cols<false>, grid, dim3(kBlock), 0, B->dev, k, n, p.chunk, Lj, (uint32_t*)part, rows,
                 (uint32_t)p.act_blocks, (uint32_t)p.gr);
    TRY(check_launch(c));
  }
  c->fb_pending = true;
  c->fb_rows = k;
  c->fb_pk = pk;
  c->fb_chunks = (int)p.gc;
  return GKR_OK;
}

// A walk's next matmul restriction launched ahead of its claim point (at the
// current step's last launch): k_point_wait, then the restriction reading
// the point from device memory.  Launched only when every buffer it needs is
// already large enough and the weight's int8 copy question is settled, since
// growing a buffer or building the copy synchronises with the stream, whose
// earlier kernels wait for the current step's challenges.  *launched reports
// whether it was.
int prelaunch_matmul(gkr_ctx* c, const gkr_matrix* A, const gkr_matrix* B, bool* launched) {
  *launched = false;
  if (c->noalloc || c->pre.active || !A || !B || A->ctx != c || B->ctx != c || A->cols != B->rows) return GKR_OK;
  if (c->int8_weights && B->r8_state == 0) return GKR_OK;
  const uint64_t pk = next_pow2(A->cols);
  const int n_ri = log2_exact(next_pow2(A->rows)), n_rj = log2_exact(next_pow2(B->cols));
  if (log2_exact(pk) == 0 || n_ri + n_rj > kMaxVars) return GKR_OK;
  RestrictPlan p;
  if (plan_restrict(A, B, pk, false, &p) != GKR_OK) return GKR_OK;
  std::vector<std::pair<Slot, size_t>> bufs;
  restrict_buffers(p, &bufs);
  bufs.push_back({S_PTWAIT, kPtWaitBytes});
  for (const auto& sb : bufs)
    if (c->cap[sb.first] < sb.second) return GKR_OK;
  uint8_t* pw;
  TRY(ensureT(c, S_PTWAIT, kPtWaitBytes, &pw));
  DevicePoint dp;
  dp.pt = reinterpret_cast<const PointArg*>(pw + 256);
  dp.status = reinterpret_cast<const uint32_t*>(pw);
  dp.want = alloc_seq(&c->mb_seq, 1);
  {
    HostTimer ht(c, K_HOST_LAUNCH);
    GKR_LAUNCH(c, k_point_wait, dim3(1), dim3(64), 0, c->mailbox, dp.want, kWaitSpinLimit, n_ri + n_rj,
               reinterpret_cast<PointArg*>(pw + 256), reinterpret_cast<uint32_t*>(pw));
    TRY(check_launch(c));
  }
  c->pre.active = true;  // from here on a failure leaves a wait that the walk cancels
  c->pre.act = false;
  c->pre.want = dp.want;
  c->pre.a = A;
  c->pre.b = B;
  c->mm.valid = false;
  c->mm.have_trip0 = false;
  TRY(restrict_pair(c, A, B, nullptr, n_ri, nullptr, n_rj, pk, false, &dp));
  *launched = true;
  return GKR_OK;
}

// First trip of the product sumcheck (rounds 0 .. K-1, K = min(3, log pk)):
// the 4^K cross sums of the restricted vectors f_a, f_b (S_FA0, S_FB0).
static int first_product_trip(gkr_ctx* c, uint64_t pk, int* K, qm31* g) {
  qm31 *fa, *fb;
  TRY(ensureT(c, S_FA0, pk, &fa));
  TRY(ensureT(c, S_FB0, pk, &fb));
  const int T = log2_exact(pk);
  *K = T < trip_k(pk) ? T : trip_k(pk);
  RoundSink sk;
  if (c->fb_pending) {  // add the chunk partials on the fly and store f_b
    TRY(launch_trip(c, 0, *K, fa, (const qm31*)c->buf[S_COLPART], pk, 0, nullptr, nullptr, fb, nullptr, nullptr, 0,
                    0, &sk, c->fb_rows, c->fb_chunks));
    c->fb_pending = false;
  } else {
    TRY(launch_trip(c, 0, *K, fa, fb, pk, 0, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, &sk));
  }
  return wait_trip(c, sk, trip_nq(0, *K), g);
}

static bool cache_matches(const gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_i, int n_ri,
                          const gkr_qm31* r_j, int n_rj) {
  const MatMulCache& mm = c->mm;
  if (!mm.valid || mm.a != a || mm.b != b || (int)mm.r_i.size() != n_ri || (int)mm.r_j.size() != n_rj) return false;
  if (n_ri && memcmp(mm.r_i.data(), r_i, n_ri * sizeof(gkr_qm31))) return false;
  if (n_rj && memcmp(mm.r_j.data(), r_j, n_rj * sizeof(gkr_qm31))) return false;
  return true;
}

static int validate_matmul(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, uint32_t n_ri, uint32_t n_rj) {
  if (!c || !a || !b) return fail(GKR_ERR_INVALID, "null argument");
  if (a->ctx != c || b->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another context");
  if (a->cols != b->rows)
    return fail(GKR_ERR_INVALID, "shape mismatch: A is %llux%llu, B is %llux%llu", (unsigned long long)a->rows,
                (unsigned long long)a->cols, (unsigned long long)b->rows, (unsigned long long)b->cols);
  if ((int)n_ri != log2_exact(next_pow2(a->rows)))
    return fail(GKR_ERR_INVALID, "r_i has %u entries, expected %d", n_ri, log2_exact(next_pow2(a->rows)));
  if ((int)n_rj != log2_exact(next_pow2(b->cols)))
    return fail(GKR_ERR_INVALID, "r_j has %u entries, expected %d", n_rj, log2_exact(next_pow2(b->cols)));
  return GKR_OK;
}

static int ensure_restricted(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_i, uint32_t n_ri,
                             const gkr_qm31* r_j, uint32_t n_rj) {
  if (c->pre.active && !c->pre.act && c->pre.a == a && c->pre.b == b) {  // launched ahead: post the point
    for (uint32_t l = 0; l < n_ri + n_rj; l++) {
      const gkr_qm31& x = l < n_ri ? r_i[l] : r_j[l - n_ri];
      if (!canonical_q(x)) return fail(GKR_ERR_INVALID, "claim point coordinate %u not canonical", l);
    }
    for (uint32_t l = 0; l < n_ri + n_rj; l++) c->mailbox->point[l] = Q(l < n_ri ? r_i[l] : r_j[l - n_ri]);
    __atomic_store_n(&c->mailbox->seq, c->pre.want, __ATOMIC_RELEASE);
    c->point_mb = c->pre.want;  // checked once the first trip's results are in
    c->pre.active = false;
    c->mm.valid = true;
    c->mm.a = a;
    c->mm.b = b;
    c->mm.r_i.assign(r_i, r_i + n_ri);
    c->mm.r_j.assign(r_j, r_j + n_rj);
    c->mm.have_trip0 = false;
    return GKR_OK;
  }
  if (cache_matches(c, a, b, r_i, (int)n_ri, r_j, (int)n_rj)) return GKR_OK;
  std::vector<qm31> ri(n_ri), rj(n_rj);
  for (uint32_t l = 0; l < n_ri; l++) {
    if (!canonical_q(r_i[l])) return fail(GKR_ERR_INVALID, "r_i[%u] not canonical", l);
    ri[l] = Q(r_i[l]);
  }
  for (uint32_t l = 0; l < n_rj; l++) {
    if (!canonical_q(r_j[l])) return fail(GKR_ERR_INVALID, "r_j[%u] not canonical", l);
    rj[l] = Q(r_j[l]);
  }
  c->mm.valid = false;
  const uint64_t pk = next_pow2(a->cols);
  TRY(restrict_pair(c, a, b, ri.data(), (int)n_ri, rj.data(), (int)n_rj, pk));
  c->mm.valid = true;
  c->mm.a = a;
  c->mm.b = b;
  c->mm.r_i.assign(r_i, r_i + n_ri);
  c->mm.r_j.assign(r_j, r_j + n_rj);
  c->mm.have_trip0 = false;
  return GKR_OK;
}


// Degree-2 product sumcheck sum_x f_a(x) f_b(x) over 2^T entries: the round
// loop of reduce_matmul_layer (backend.rs:146-177; gpu_sumcheck.rs:2820-2840),
// as device trips of up to 3 rounds (plan_trips), then the host.  in_a/in_b
// are only read; trip j >= 1 writes its folded vectors to bufs[(j - 1) & 1]
// (bufs[0] holds 2^(T-1) entries, bufs[1] 2^(T-2)).  g0, when given, holds
// the first trip's sums (rounds 0 .. k0 - 1) already computed for these inputs.
// scale3 set: the rounds of a three-factor sumcheck sum w a b whose w is the
// constant *scale3 over these variables: each round polynomial is *scale3
// times the product one, written and mixed as degree 3 (c3 = 0; 4 per round).
int product_sumcheck(gkr_ctx* c, PoseidonChannel& ch, int T, const qm31* in_a, const qm31* in_b,
                            qm31* const bufs_a[2], qm31* const bufs_b[2], const qm31* g0, int k0,
                            gkr_qm31* round_polys, gkr_qm31* challenges, gkr_qm31* final_a, gkr_qm31* final_b,
                            const qm31* scale3, const FirstTrip* ft) {
  const qm31 inv2 = qm31_from_m31(1u << 30);  // 2^-1 mod P
  const uint64_t pk = 1ull << T;
  const std::vector<Trip> trips = plan_trips(T, kHostTailMM, g0 ? k0 : trip_k(1ull << T));
  std::vector<qm31> chal(T);
  auto absorb = [&](int t, const qm31* sums) {
    const qm31 c0 = sums[0];
    const qm31 c2 = qm31_mul(qm31_add(qm31_sub(qm31_sub(sums[2], sums[1]), sums[1]), sums[0]), inv2);
    const qm31 c1 = qm31_sub(qm31_sub(sums[1], sums[0]), c2);
    if (scale3) {
      const qm31 d0 = qm31_mul(*scale3, c0), d1 = qm31_mul(*scale3, c1), d2 = qm31_mul(*scale3, c2);
      round_polys[4 * t + 0] = G(d0);
      round_polys[4 * t + 1] = G(d1);
      round_polys[4 * t + 2] = G(d2);
      round_polys[4 * t + 3] = G(qm31_zero());
      HostTimer ht(c, K_HOST_FS);
      ch.mix_poly_coeffs_deg3(d0, d1, d2, qm31_zero());
      chal[t] = ch.draw_qm31();
      challenges[t] = G(chal[t]);
      return;
    }
    round_polys[3 * t + 0] = G(c0);
    round_polys[3 * t + 1] = G(c1);
    round_polys[3 * t + 2] = G(c2);
    HostTimer ht(c, K_HOST_FS);
    ch.mix_poly_coeffs(c0, c1, c2);
    chal[t] = ch.draw_qm31();
    challenges[t] = G(chal[t]);
  };
  const qm31 xs[3] = {qm31_zero(), qm31_one(), qm31_from_m31(2)};
  HandoverSession ho(c);
  AheadTrips ahead(c);
  const size_t nt = trips.size();
  std::vector<RoundSink> sks(nt);
  std::vector<TripWait> tws(nt);
  // Every trip is launched up front (the first with its inputs, the others
  // ahead of their challenges, which the host posts as it draws them), then
  // the hand-over: no launch sits between a trip's sums and the next trip.
  // Without launches ahead each trip is launched once its challenges are known.
  const bool pre = ahead.enabled();
  const qm31* src_a = in_a;
  const qm31* src_b = in_b;
  // Launched ahead, each trip's rows are added by the next kernel of the chain
  // (the next trip's mailbox wait, or the hand-over) instead of a finisher.
  CarriedFinish carry;
  memset(&carry, 0, sizeof carry);
  auto launch_j = [&](size_t j, const qm31* pend) -> int {
    const Trip& tr = trips[j];
    qm31* da = j == 0 ? nullptr : bufs_a[(j - 1) & 1];
    qm31* db = j == 0 ? nullptr : bufs_b[(j - 1) & 1];
    const int npj = j == 0 ? 0 : trips[j - 1].K;
    const TripWait* tw = nullptr;
    if (j > 0 && pre) {
      TRY(ahead.make(&tws[j]));
      tw = &tws[j];
    }
    const CarriedFinish carry_in = carry;
    CarriedFinish* carry_out = pre ? &carry : nullptr;
    if (j == 0 && ft && ft->b_chunks)  // add the weight-side chunk partials and store f_b (in_b)
      TRY(launch_trip(c, 0, tr.K, src_a, ft->b_partials, tr.n, 0, nullptr, nullptr, const_cast<qm31*>(in_b),
                      nullptr, nullptr, 0, 0, &sks[0], ft->b_rows, ft->b_chunks, nullptr, carry_out));
    else
      TRY(launch_trip(c, 0, tr.K, src_a, src_b, tr.n, npj, pend, da, db, nullptr, nullptr, 0, 0, &sks[j], 0, 0,
                      tw, carry_out, tw ? &carry_in : nullptr));
    if (j > 0) {
      src_a = da;
      src_b = db;
    }
    if (j + 1 == nt) TRY(ho.launch<2>(src_a, src_b, tr.n, tr.K, pre ? &carry : nullptr));
    return GKR_OK;
  };
  if (g0) {
    if (nt == 1) TRY(ho.launch<2>(in_a, in_b, trips[0].n, trips[0].K));
  } else {
    TRY(launch_j(0, nullptr));
  }
  if (pre) {
    for (size_t j = 1; j < nt; j++) TRY(launch_j(j, nullptr));
    TRY(run_prelaunch(c));  // every launch of this sumcheck is queued
  }
  int np = 0;
  const qm31* pend = nullptr;
  for (size_t j = 0; j < nt; j++) {
    const Trip& tr = trips[j];
    qm31 g[kMaxSums];
    if (j > 0 && !pre) TRY(launch_j(j, pend));
    if (j == 0 && g0) {
      for (int q = 0; q < trip_nq(0, tr.K); q++) g[q] = g0[q];
    } else {
      TRY(wait_trip(c, sks[j], trip_nq(0, tr.K), g, j > 0 && pre ? tws[j].want : 0));
    }
    if (j == 0) TRY(check_point_wait(c));
    if (j == 0 && ft && ft->on_sums) TRY(ft->on_sums(g, tr.K));
    TripGram tg(g, tr.K, nullptr, qm31_zero());
    for (int i = 0; i < tr.K; i++) {
      qm31 sums[3];
      {
        HostTimer hg(c, K_HOST_GRAM);
        tg.values(3, xs, sums);
      }
      absorb(tr.t + i, sums);
      if (j + 1 == nt) TRY(ho.post_one(i, chal[tr.t + i]));  // the hand-over folds it while the next is drawn
      if (i + 1 < tr.K) {
        HostTimer hg(c, K_HOST_GRAM);
        tg.fold(chal[tr.t + i]);
      }
    }
    np = tr.K;
    pend = chal.data() + tr.t;
    if (pre && j + 1 < nt) TRY(ahead.post(tws[j + 1], pend, np));
  }
  const int t_end = trips.empty() ? 0 : trips.back().t + trips.back().K;
  const uint64_t hlen = pk >> t_end;
  std::vector<qm31> v[2];
  TRY(ho.post(pend, np));
  TRY(ho.fetch(hlen, 2, v));
  std::vector<qm31>& A = v[0];
  std::vector<qm31>& B = v[1];
  for (int t = t_end; t < T; t++) {
    const size_t half = A.size() / 2;
    qm31 sums[3];
    {
      HostTimer ht(c, K_HOST_FINISH);
      hostfield::product_round(qwords(A.data()), qwords(B.data()), half, reinterpret_cast<uint32_t(*)[4]>(sums));
    }
    absorb(t, sums);
    HostTimer ht(c, K_HOST_FINISH);
    hostfield::fold(qwords(A.data()), half, qwords(&chal[t]));
    hostfield::fold(qwords(B.data()), half, qwords(&chal[t]));
    A.resize(half);
    B.resize(half);
  }
  *final_a = G(A[0]);
  *final_b = G(B[0]);
  return GKR_OK;
}

// on_sums (T > 0 only): called with trip 0's sums before the first round.
static int reduce_matmul_impl(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_i, uint32_t n_ri,
                              const gkr_qm31* r_j, uint32_t n_rj, uint64_t pk, PoseidonChannel& ch,
                              gkr_qm31* round_polys, gkr_qm31* challenges, gkr_qm31* final_a, gkr_qm31* final_b,
                              const std::function<int(const qm31*, int)>* on_sums = nullptr) {
  TRY(validate_matmul(c, a, b, n_ri, n_rj));
  if (pk != next_pow2(a->cols))
    return fail(GKR_ERR_INVALID, "pk=%llu but next_pow2(k)=%llu", (unsigned long long)pk,
                (unsigned long long)next_pow2(a->cols));
  HIP_TRY(hipSetDevice(c->device));
  TRY(ensure_restricted(c, a, b, r_i, n_ri, r_j, n_rj));
  const int T = log2_exact(pk);
  if (on_sums && T == 0) return fail(GKR_ERR_INVALID, "a claim from trip 0's sums needs k > 1");
  qm31 *fa0, *fa1, *fb0, *fb1, *fa2, *fb2;
  TRY(ensureT(c, S_FA0, pk, &fa0));
  TRY(ensureT(c, S_FB0, pk, &fb0));
  TRY(ensureT(c, S_FA1, pk / 2 + 1, &fa1));
  TRY(ensureT(c, S_FB1, pk / 2 + 1, &fb1));
  TRY(ensureT(c, S_FA2, pk / 4 + 1, &fa2));
  TRY(ensureT(c, S_FB2, pk / 4 + 1, &fb2));
  // The trips write only S_FA1/S_FB1 and S_FA2/S_FB2; S_FA0/S_FB0 keep the
  // restricted vectors, so a cached restriction stays valid.
  if (T == 0) {
    TRY(finish_fb(c));  // the sums read f_b from S_FB0
    qm31 v[1];
    TRY(fetch_q(c, fa0, 1, v));
    *final_a = G(v[0]);
    TRY(fetch_q(c, fb0, 1, v));
    *final_b = G(v[0]);
    return GKR_OK;
  }
  qm31* bufs_a[2] = {fa1, fa2};
  qm31* bufs_b[2] = {fb1, fb2};
  const bool have = c->mm.have_trip0;
  c->mm.have_trip0 = false;  // used once: the transcript moves on
  FirstTrip ft;
  if (!have && c->fb_pending) {  // trip 0 adds the weight-side chunk partials and stores f_b (S_FB0)
    ft.b_partials = (const qm31*)c->buf[S_COLPART];
    ft.b_rows = c->fb_rows;
    ft.b_chunks = c->fb_chunks;
    c->fb_pending = false;
  }
  if (on_sums) ft.on_sums = *on_sums;
  return product_sumcheck(c, ch, T, fa0, fb0, bufs_a, bufs_b, have ? c->mm.trip0 : nullptr, c->mm.trip0_k,
                          round_polys, challenges, final_a, final_b, nullptr, &ft);
}

extern "C" int gkr_reduce_matmul_layer(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_i,
                                       uint32_t n_r_i, const gkr_qm31* r_j, uint32_t n_r_j, uint64_t pk,
                                       gkr_channel* ch, gkr_qm31* round_polys, gkr_qm31* challenges,
                                       gkr_qm31* final_a, gkr_qm31* final_b) {
  CH_CHECK(ch);
  if (!final_a || !final_b || ((!round_polys || !challenges) && pk > 1) || (!r_i && n_r_i) || (!r_j && n_r_j))
    return fail(GKR_ERR_INVALID, "null argument");
  return reduce_matmul_impl(c, a, b, r_i, n_r_i, r_j, n_r_j, pk, ch->ch, round_polys, challenges, final_a, final_b);
}

extern "C" int gkr_matmul_output_claim(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_out,
                                       uint32_t n_vars, gkr_qm31* value) {
  if (!c || !a || !b || !value || (!r_out && n_vars)) return fail(GKR_ERR_INVALID, "null argument");
  const uint32_t n_ri = (uint32_t)log2_exact(next_pow2(a->rows));
  if (n_vars < n_ri) return fail(GKR_ERR_INVALID, "point too short");
  TRY(validate_matmul(c, a, b, n_ri, n_vars - n_ri));
  HIP_TRY(hipSetDevice(c->device));
  TRY(ensure_restricted(c, a, b, r_out, n_ri, r_out + n_ri, n_vars - n_ri));
  const uint64_t pk = next_pow2(a->cols);
  if (pk == 1) {
    TRY(finish_fb(c));
    qm31 fa[1], fb[1];
    qm31 *dfa, *dfb;
    TRY(ensureT(c, S_FA0, 1, &dfa));
    TRY(ensureT(c, S_FB0, 1, &dfb));
    TRY(fetch_q(c, dfa, 1, fa));
    TRY(fetch_q(c, dfb, 1, fb));
    *value = G(qm31_mul(fa[0], fb[0]));
    return GKR_OK;
  }
  int K = 0;
  TRY(first_product_trip(c, pk, &K, c->mm.trip0));
  c->mm.trip0_k = K;
  c->mm.have_trip0 = true;
  qm31 v = qm31_zero();  // sum_x f_a(x) f_b(x) = trace of the cross sums
  for (int q = 0; q < (1 << K); q++) v = qm31_add(v, c->mm.trip0[q * ((1 << K) + 1)]);
  *value = G(v);
  return GKR_OK;
}

// The matmul layer proof.  fresh: the claim value is not given but computed
// as the trace of trip 0's sums (gkr_matmul_output_claim's value) once they
// arrive, mixed as the walk mixes a fresh claim, and returned in
// *claim_value; every trip of the sumcheck is then launched before the first
// wait.  The transcript and the proof equal gkr_matmul_output_claim, the
// walk's mix of the value, then gkr_prove_matmul_layer.  Needs k > 1.
static int prove_matmul_impl(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point, gkr_qm31* claim_value,
                             bool fresh, const gkr_matrix* a, const gkr_matrix* b, gkr_channel* ch, gkr_proof* proof,
                             gkr_qm31* round_polys, gkr_qm31* final_a, gkr_qm31* final_b, gkr_qm31* next_point,
                             gkr_qm31* next_value) {
  CH_CHECK(ch);
  if (!c || !a || !b || !claim_value || !final_a || !final_b || !next_value || (!claim_point && n_point))
    return fail(GKR_ERR_INVALID, "null argument");
  if (!fresh && !canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  TraceScope trace;
  const uint64_t pm = next_pow2(a->rows), pk = next_pow2(a->cols), pn = next_pow2(b->cols);
  const uint32_t log_m = (uint32_t)log2_exact(pm), log_n = (uint32_t)log2_exact(pn);
  const int T = log2_exact(pk);
  if (n_point != log_m + log_n)
    return fail(GKR_ERR_INVALID, "output claim has %u vars, expected exactly %u (log_m=%u + log_n=%u)", n_point,
                log_m + log_n, log_m, log_n);
  if (T > 0 && (!round_polys || !next_point)) return fail(GKR_ERR_INVALID, "null output buffer");
  TRY(validate_matmul(c, a, b, log_m, log_n));
  PoseidonChannel& C = ch->ch;
  auto mix_head = [&](const qm31& v) {
    C.mix_u64(a->rows);
    C.mix_u64(a->cols);
    C.mix_u64(b->cols);
    C.mix_secure_field(v);
  };
  std::function<int(const qm31*, int)> claim_from_sums = [&](const qm31* g, int K) -> int {
    qm31 v = qm31_zero();  // sum_x f_a(x) f_b(x) = trace of the cross sums
    for (int q = 0; q < (1 << K); q++) v = qm31_add(v, g[q * ((1 << K) + 1)]);
    *claim_value = G(v);
    C.mix_secure_field(v);  // the walk's mix of a fresh claim
    mix_head(v);
    return GKR_OK;
  };
  if (!fresh) mix_head(Q(*claim_value));
  std::vector<gkr_qm31> chal(T > 0 ? T : 1);
  TRY(reduce_matmul_impl(c, a, b, claim_point, log_m, claim_point + log_m, log_n, pk, C, round_polys, chal.data(),
                         final_a, final_b, fresh ? &claim_from_sums : nullptr));
  trace_point(C, "matmul.rounds");
  C.mix_secure_field(Q(*final_a));
  C.mix_secure_field(Q(*final_b));
  trace_point(C, "matmul");
  if (next_point) {
    for (uint32_t l = 0; l < log_m; l++) next_point[l] = claim_point[l];
    for (int t = 0; t < T; t++) next_point[log_m + t] = chal[t];
  }
  *next_value = *final_a;
  if (proof) {
    HostTimer hp(c, K_HOST_PROOF);
    LayerRec L;
    L.tag = 0;
    L.claim_value = Q(*claim_value);
    for (int t = 0; t < 3 * T; t++) L.rp.push_back(Q(round_polys[t]));
    L.final_a = Q(*final_a);
    L.final_b = Q(*final_b);
    proof_add_layer(proof, std::move(L));
    WeightClaimRec w;
    w.b = b;
    for (uint32_t l = 0; l < log_n; l++) w.point.push_back(Q(claim_point[log_m + l]));
    for (int t = 0; t < T; t++) w.point.push_back(Q(chal[t]));
    w.value = Q(*final_b);
    proof->weight_claims.push_back(std::move(w));
  }
  return GKR_OK;
}

extern "C" int gkr_prove_matmul_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                      const gkr_qm31* claim_value, const gkr_matrix* a, const gkr_matrix* b,
                                      gkr_channel* ch, gkr_proof* proof, gkr_qm31* round_polys, gkr_qm31* final_a,
                                      gkr_qm31* final_b, gkr_qm31* next_point, gkr_qm31* next_value) {
  if (!claim_value) return fail(GKR_ERR_INVALID, "null argument");
  gkr_qm31 v = *claim_value;
  return prove_matmul_impl(c, claim_point, n_point, &v, false, a, b, ch, proof, round_polys, final_a, final_b,
                           next_point, next_value);
}
// The walk's matmul step with a fresh claim at `point` (k > 1): claim value
// and layer proof in one pass (prove_matmul_impl, fresh).
int walk_matmul_fresh(gkr_ctx* c, const gkr_qm31* point, uint32_t n_point, gkr_qm31* value, const gkr_matrix* a,
                      const gkr_matrix* b, gkr_channel* ch, gkr_proof* proof, gkr_qm31* round_polys,
                      gkr_qm31* final_a, gkr_qm31* final_b, gkr_qm31* next_point, gkr_qm31* next_value) {
  return prove_matmul_impl(c, point, n_point, value, true, a, b, ch, proof, round_polys, final_a, final_b, next_point,
                           next_value);
}

// SIMD matmul layer with a shared weight: N activation blocks A_b (all m x k)
// combined with weights w_b against one B (gkr/prover.rs:5422-5600,
// reduce_matmul_layer_simd_gpu).  Same transcript and proof record as
// gkr_prove_matmul_layer with f_a = sum_b w_b restrict_rows(A_b, r_i).
extern "C" int gkr_prove_matmul_layer_simd(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                           const gkr_qm31* claim_value, const gkr_matrix* const* a_blocks,
                                           const gkr_qm31* block_weights, uint32_t n_blocks, const gkr_matrix* b,
                                           gkr_channel* ch, gkr_proof* proof, gkr_qm31* round_polys,
                                           gkr_qm31* final_a, gkr_qm31* final_b, gkr_qm31* next_point,
                                           gkr_qm31* next_value) {
  CH_CHECK(ch);
  if (!c || !a_blocks || !block_weights || !b || !claim_value || !final_a || !final_b || !next_value ||
      (!claim_point && n_point))
    return fail(GKR_ERR_INVALID, "null argument");
  if (n_blocks == 0 || n_blocks > (uint32_t)kSimdMaxBlocks)
    return fail(GKR_ERR_INVALID, "%u blocks (1 .. %d supported)", n_blocks, kSimdMaxBlocks);
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  const gkr_matrix* a = a_blocks[0];
  if (!a) return fail(GKR_ERR_INVALID, "null block");
  SimdBlocks blk;
  memset(&blk, 0, sizeof blk);
  blk.count = (int)n_blocks;
  for (uint32_t i = 0; i < n_blocks; i++) {
    const gkr_matrix* ai = a_blocks[i];
    if (!ai || ai->ctx != c) return fail(GKR_ERR_INVALID, "block %u missing or from another context", i);
    if (ai->rows != a->rows || ai->cols != a->cols)
      return fail(GKR_ERR_INVALID, "block %u is %llux%llu, block 0 %llux%llu", i, (unsigned long long)ai->rows,
                  (unsigned long long)ai->cols, (unsigned long long)a->rows, (unsigned long long)a->cols);
    if (!canonical_q(block_weights[i])) return fail(GKR_ERR_INVALID, "block weight %u not canonical", i);
    blk.a[i] = ai->dev;
    blk.w[i] = Q(block_weights[i]);
  }
  const uint64_t pm = next_pow2(a->rows), pk = next_pow2(a->cols), pn = next_pow2(b->cols);
  const uint32_t log_m = (uint32_t)log2_exact(pm), log_n = (uint32_t)log2_exact(pn);
  const int T = log2_exact(pk);
  if (n_point != log_m + log_n)
    return fail(GKR_ERR_INVALID, "output claim has %u vars, expected exactly %u (log_m=%u + log_n=%u)", n_point,
                log_m + log_n, log_m, log_n);
  if (T > 0 && (!round_polys || !next_point)) return fail(GKR_ERR_INVALID, "null output buffer");
  TRY(validate_matmul(c, a, b, log_m, log_n));
  std::vector<qm31> ri(log_m), rj(log_n);
  for (uint32_t l = 0; l < log_m + log_n; l++)
    if (!canonical_q(claim_point[l])) return fail(GKR_ERR_INVALID, "claim point coordinate %u not canonical", l);
  for (uint32_t l = 0; l < log_m; l++) ri[l] = Q(claim_point[l]);
  for (uint32_t l = 0; l < log_n; l++) rj[l] = Q(claim_point[log_m + l]);
  HIP_TRY(hipSetDevice(c->device));
  PoseidonChannel& C = ch->ch;
  C.mix_u64(a->rows);
  C.mix_u64(a->cols);
  C.mix_u64(b->cols);
  C.mix_secure_field(Q(*claim_value));
  // the restriction scratch (S_FA0 / S_FB0) is rewritten: no cached restriction survives
  c->mm.valid = false;
  c->mm.have_trip0 = false;
  TRY(restrict_pair(c, a, b, ri.data(), (int)log_m, rj.data(), (int)log_n, pk, true));
  {
    HostTimer ht(c, K_HOST_LAUNCH);
    qm31 *Li, *fa;
    TRY(ensureT(c, S_LI, a->rows, &Li));
    TRY(ensureT(c, S_FA0, pk, &fa));
    // algorithmic bytes: the blocks' activations, L_i, f_a written
    TimedLaunch t(c, K_RESTRICT_ROWS, 4ull * n_blocks * a->rows * a->cols + 16 * a->rows + 16 * pk, true);
    GKR_LAUNCH(c, k_restrict_rows_simd, dim3((unsigned)((pk + 63) / 64)), dim3(kSimdWaves * 64), 0, blk,
                       a->rows, a->cols, pk, (const qm31*)Li, fa);
    TRY(check_launch(c));
  }
  TRY(finish_fb(c));
  std::vector<gkr_qm31> chal(T > 0 ? T : 1);
  qm31 *fa0, *fa1, *fb0, *fb1, *fa2, *fb2;
  TRY(ensureT(c, S_FA0, pk, &fa0));
  TRY(ensureT(c, S_FB0, pk, &fb0));
  TRY(ensureT(c, S_FA1, pk / 2 + 1, &fa1));
  TRY(ensureT(c, S_FB1, pk / 2 + 1, &fb1));
  TRY(ensureT(c, S_FA2, pk / 4 + 1, &fa2));
  TRY(ensureT(c, S_FB2, pk / 4 + 1, &fb2));
  if (T == 0) {
    TRY(finish_fb(c));  // the sums read f_b from S_FB0
    qm31 v[1];
    TRY(fetch_q(c, fa0, 1, v));
    *final_a = G(v[0]);
    TRY(fetch_q(c, fb0, 1, v));
    *final_b = G(v[0]);
  } else {
    qm31* bufs_a[2] = {fa1, fa2};
    qm31* bufs_b[2] = {fb1, fb2};
    TRY(product_sumcheck(c, C, T, fa0, fb0, bufs_a, bufs_b, nullptr, 0, round_polys, chal.data(), final_a, final_b));
  }
  C.mix_secure_field(Q(*final_a));
  C.mix_secure_field(Q(*final_b));
  if (next_point) {
    for (uint32_t l = 0; l < log_m; l++) next_point[l] = claim_point[l];
    for (int t = 0; t < T; t++) next_point[log_m + t] = chal[t];
  }
  *next_value = *final_a;
  if (proof) {
    HostTimer hp(c, K_HOST_PROOF);
    LayerRec L;
    L.tag = 0;
    L.claim_value = Q(*claim_value);
    for (int t = 0; t < 3 * T; t++) L.rp.push_back(Q(round_polys[t]));
    L.final_a = Q(*final_a);
    L.final_b = Q(*final_b);
    proof_add_layer(proof, std::move(L));
    WeightClaimRec w;
    w.b = b;
    for (uint32_t l = 0; l < log_n; l++) w.point.push_back(Q(claim_point[log_m + l]));
    for (int t = 0; t < T; t++) w.point.push_back(Q(chal[t]));
    w.value = Q(*final_b);
    proof->weight_claims.push_back(std::move(w));
  }
  return GKR_OK;
}

// Dual-operand SIMD matmul layer (gkr/prover.rs:5615-5785,
// reduce_matmul_layer_dual_simd_gpu): N = 2^nbv blocks A_b (m x k), B_b
// (k x n) with weights w_b; the three-factor sumcheck over the block-extended
// vectors ext_w[b pk + x] = w_b, ext_a = restrict_rows(A_b, r_i),
// ext_b = restrict_cols(B_b, r_j) (sumcheck_3way, gpu_sumcheck.rs:2597-2681).
// ext_w is constant over the k variables, so the nbv block rounds (first, MSB)
// come from the block Gram matrix D[b1][b2] = sum_x fa_b1(x) fb_b2(x) on the
// host, and the log2 pk remaining rounds are the product sumcheck of the
// blocks' combinations by the block challenges, scaled by the folded weight.
extern "C" int gkr_prove_matmul_layer_dual_simd(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                                const gkr_qm31* claim_value, const gkr_matrix* const* a_blocks,
                                                const gkr_matrix* const* b_blocks, const gkr_qm31* block_weights,
                                                uint32_t n_blocks, gkr_channel* ch, gkr_proof* proof,
                                                gkr_qm31* round_polys, gkr_qm31* final_a, gkr_qm31* final_b) {
  CH_CHECK(ch);
  if (!c || !a_blocks || !b_blocks || !block_weights || !claim_value || !final_a || !final_b ||
      (!claim_point && n_point))
    return fail(GKR_ERR_INVALID, "null argument");
  if (n_blocks == 0 || n_blocks > (uint32_t)kSimdMaxBlocks || (n_blocks & (n_blocks - 1)))
    return fail(GKR_ERR_INVALID, "%u blocks (a power of two up to %d)", n_blocks, kSimdMaxBlocks);
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  const gkr_matrix* a = a_blocks[0];
  const gkr_matrix* b = b_blocks[0];
  if (!a || !b) return fail(GKR_ERR_INVALID, "null block");
  std::vector<qm31> W(n_blocks);
  for (uint32_t i = 0; i < n_blocks; i++) {
    const gkr_matrix *ai = a_blocks[i], *bi = b_blocks[i];
    if (!ai || !bi || ai->ctx != c || bi->ctx != c)
      return fail(GKR_ERR_INVALID, "block %u missing or from another context", i);
    if (ai->rows != a->rows || ai->cols != a->cols || bi->rows != b->rows || bi->cols != b->cols)
      return fail(GKR_ERR_INVALID, "block %u shapes differ from block 0", i);
    if (!canonical_q(block_weights[i])) return fail(GKR_ERR_INVALID, "block weight %u not canonical", i);
    W[i] = Q(block_weights[i]);
  }
  const uint64_t pm = next_pow2(a->rows), pk = next_pow2(a->cols), pn = next_pow2(b->cols);
  const uint32_t log_m = (uint32_t)log2_exact(pm), log_n = (uint32_t)log2_exact(pn);
  const int T = log2_exact(pk), nbv = log2_exact(n_blocks);
  if (n_point != log_m + log_n)
    return fail(GKR_ERR_INVALID, "output claim has %u vars, expected exactly %u (log_m=%u + log_n=%u)", n_point,
                log_m + log_n, log_m, log_n);
  if (nbv + T > 0 && !round_polys) return fail(GKR_ERR_INVALID, "null output buffer");
  TRY(validate_matmul(c, a, b, log_m, log_n));
  std::vector<qm31> ri(log_m), rj(log_n);
  for (uint32_t l = 0; l < log_m + log_n; l++)
    if (!canonical_q(claim_point[l])) return fail(GKR_ERR_INVALID, "claim point coordinate %u not canonical", l);
  for (uint32_t l = 0; l < log_m; l++) ri[l] = Q(claim_point[l]);
  for (uint32_t l = 0; l < log_n; l++) rj[l] = Q(claim_point[log_m + l]);
  HIP_TRY(hipSetDevice(c->device));
  PoseidonChannel& C = ch->ch;
  C.mix_u64(a->rows);
  C.mix_u64(a->cols);
  C.mix_u64(b->cols);
  C.mix_u64(n_blocks);
  C.mix_secure_field(Q(*claim_value));
  c->mm.valid = false;
  c->mm.have_trip0 = false;
  // the blocks' restricted vectors, back to back
  qm31 *ea, *eb, *gram;
  TRY(ensureT(c, S_EXTA, n_blocks * pk, &ea));
  TRY(ensureT(c, S_EXTB, n_blocks * pk, &eb));
  TRY(ensureT(c, S_GRAM, (size_t)n_blocks * n_blocks, &gram));
  {
    // the blocks share the claim point: both Lagrange tables once, then each side for all blocks
    HostTimer ht(c, K_HOST_LAUNCH);
    qm31 *Li, *Lj;
    TRY(ensureT(c, S_LI, a->rows, &Li));
    TRY(ensureT(c, S_LJ, b->cols, &Lj));
    TRY(eq_table(c, ri.data(), (int)log_m, a->rows, Li));
    TRY(eq_table(c, rj.data(), (int)log_n, b->cols, Lj));
    BlockPtrs pa, pb;
    memset(&pa, 0, sizeof pa);
    memset(&pb, 0, sizeof pb);
    for (uint32_t i = 0; i < n_blocks; i++) {
      pa.p[i] = a_blocks[i]->dev;
      pb.p[i] = b_blocks[i]->dev;
    }
    GKR_LAUNCH(c, k_restrict_rows_blocks, dim3(grid_for(pk), n_blocks), dim3(kBlock), 0, pa, a->rows,
                       a->cols, pk, (const qm31*)Li, ea);
    GKR_LAUNCH(c, k_restrict_cols_blocks, dim3((unsigned)((pk + kColWaves - 1) / kColWaves), n_blocks),
                       dim3(kBlock), 0, pb, b->rows, b->cols, pk, (const qm31*)Lj, eb);
    TRY(check_launch(c));
  }
  std::vector<qm31> D((size_t)n_blocks * n_blocks);
  if (nbv > 0) {
    GKR_LAUNCH(c, k_block_gram, dim3(n_blocks * n_blocks), dim3(kBlock), 0, (const qm31*)ea,
                       (const qm31*)eb, n_blocks, pk, gram);
    TRY(check_launch(c));
    HIP_TRY(hipMemcpyAsync(D.data(), gram, D.size() * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
    TRY(sync(c));
  }
  // block rounds on the Gram matrix: with the block variables above bound, D is folded to the remaining
  // blocks (D'[x][y] = sum_{v,v'} l(v) l(v') D[v h + x][v' h + y], l(0) = 1 - r, l(1) = r) and so is W;
  // s(t) = sum_{x < h} W_t(x) sum_{v,v'} l_t(v) l_t(v') D[v h + x][v' h + x] with l_t at t = 0..3
  const qm31 inv2 = qm31_from_m31(1u << 30), inv6 = qm31_from_m31(m31_inv(6));
  const qm31 two = qm31_from_m31(2), three = qm31_from_m31(3);
  std::vector<qm31> chal(nbv + T);
  std::vector<qm31> Wc(W);
  size_t N = n_blocks;
  for (int j = 0; j < nbv; j++) {
    const size_t h = N / 2;
    qm31 sv[4];
    for (int t = 0; t < 4; t++) {
      const qm31 l1 = qm31_from_m31((uint32_t)t), l0 = qm31_sub(qm31_one(), l1);
      const qm31 l00 = qm31_mul(l0, l0), l01 = qm31_mul(l0, l1), l11 = qm31_mul(l1, l1);
      qm31 st = qm31_zero();
      for (size_t x = 0; x < h; x++) {
        const qm31 wt = qm31_add(qm31_mul(l0, Wc[x]), qm31_mul(l1, Wc[h + x]));
        const qm31 g = qm31_add(qm31_add(qm31_mul(l00, D[x * N + x]), qm31_mul(l11, D[(h + x) * N + h + x])),
                                qm31_mul(l01, qm31_add(D[x * N + h + x], D[(h + x) * N + x])));
        st = qm31_add(st, qm31_mul(wt, g));
      }
      sv[t] = st;
    }
    // Newton differences to monomial coefficients (gpu_sumcheck.rs:2632-2640)
    const qm31 d1 = qm31_sub(sv[1], sv[0]);
    const qm31 d2 = qm31_mul(qm31_add(qm31_sub(qm31_sub(sv[2], sv[1]), sv[1]), sv[0]), inv2);
    const qm31 d3 = qm31_mul(qm31_sub(qm31_sub(sv[3], sv[0]), qm31_mul(three, qm31_sub(sv[2], sv[1]))), inv6);
    const qm31 c0 = sv[0], c1 = qm31_add(qm31_sub(d1, d2), qm31_mul(two, d3)), c2 = qm31_sub(d2, qm31_mul(three, d3));
    round_polys[4 * j + 0] = G(c0);
    round_polys[4 * j + 1] = G(c1);
    round_polys[4 * j + 2] = G(c2);
    round_polys[4 * j + 3] = G(d3);
    {
      HostTimer ht(c, K_HOST_FS);
      C.mix_poly_coeffs_deg3(c0, c1, c2, d3);
      chal[j] = C.draw_qm31();
    }
    const qm31 r1 = chal[j], r0 = qm31_sub(qm31_one(), r1);
    std::vector<qm31> Dn(h * h), Wn(h);
    for (size_t x = 0; x < h; x++) {
      Wn[x] = qm31_add(qm31_mul(r0, Wc[x]), qm31_mul(r1, Wc[h + x]));
      for (size_t y = 0; y < h; y++) {
        const qm31 top = qm31_add(qm31_mul(r0, D[x * N + y]), qm31_mul(r1, D[x * N + h + y]));
        const qm31 bot = qm31_add(qm31_mul(r0, D[(h + x) * N + y]), qm31_mul(r1, D[(h + x) * N + h + y]));
        Dn[x * h + y] = qm31_add(qm31_mul(r0, top), qm31_mul(r1, bot));
      }
    }
    D.swap(Dn);
    Wc.swap(Wn);
    N = h;
  }
  // the blocks folded by the block challenges: f_a, f_b and the weight
  std::vector<qm31> lam((size_t)n_blocks);
  lagrange_weights(chal.data(), nbv, lam.data());
  qm31 wf = qm31_zero();
  QWeights qw;
  memset(&qw, 0, sizeof qw);
  for (uint32_t i = 0; i < n_blocks; i++) {
    wf = qm31_add(wf, qm31_mul(lam[i], W[i]));
    qw.w[i] = lam[i];
  }
  qm31 *fa0, *fb0, *fa1, *fb1, *fa2, *fb2;
  TRY(ensureT(c, S_FA0, pk, &fa0));
  TRY(ensureT(c, S_FB0, pk, &fb0));
  TRY(ensureT(c, S_FA1, pk / 2 + 1, &fa1));
  TRY(ensureT(c, S_FB1, pk / 2 + 1, &fb1));
  TRY(ensureT(c, S_FA2, pk / 4 + 1, &fa2));
  TRY(ensureT(c, S_FB2, pk / 4 + 1, &fb2));
  const dim3 gq((unsigned)((pk + kColWaves - 1) / kColWaves));  // one wave per entry
  GKR_LAUNCH(c, k_combine_q, gq, dim3(kBlock), 0, (const qm31*)ea, qw, n_blocks, pk, fa0);
  GKR_LAUNCH(c, k_combine_q, gq, dim3(kBlock), 0, (const qm31*)eb, qw, n_blocks, pk, fb0);
  TRY(check_launch(c));
  std::vector<gkr_qm31> kchal(T > 0 ? T : 1);
  if (T == 0) {
    TRY(finish_fb(c));  // the sums read f_b from S_FB0
    qm31 v[1];
    TRY(fetch_q(c, fa0, 1, v));
    *final_a = G(v[0]);
    TRY(fetch_q(c, fb0, 1, v));
    *final_b = G(v[0]);
  } else {
    qm31* bufs_a[2] = {fa1, fa2};
    qm31* bufs_b[2] = {fb1, fb2};
    TRY(product_sumcheck(c, C, T, fa0, fb0, bufs_a, bufs_b, nullptr, 0, round_polys + 4 * nbv, kchal.data(), final_a,
                         final_b, &wf));
  }
  C.mix_secure_field(Q(*final_a));
  C.mix_secure_field(Q(*final_b));
  if (proof) {
    LayerRec L;
    L.tag = 7;
    L.claim_value = Q(*claim_value);
    L.n_block_vars = (uint32_t)nbv;
    for (int t = 0; t < 4 * (nbv + T); t++) L.rp.push_back(Q(round_polys[t]));
    L.final_a = Q(*final_a);
    L.final_b = Q(*final_b);
    proof_add_layer(proof, LayerRec(L));
  }
  return GKR_OK;
}

// ------------------------------------------------------------------ ZkmlOps MLE helpers
extern "C" int gkr_evaluate_mle_at_point(gkr_ctx* c, const gkr_qm31* mle, uint64_t len, const gkr_qm31* point,
                                         uint32_t n_vars, gkr_qm31* out) {
  if (!c || !mle || !out || (!point && n_vars)) return fail(GKR_ERR_INVALID, "null argument");
  if (n_vars >= 64 || len != (1ull << n_vars))
    return fail(GKR_ERR_INVALID, "evals length must be 2^n_vars (len=%llu, n_vars=%u)", (unsigned long long)len, n_vars);
  HIP_TRY(hipSetDevice(c->device));
  std::vector<qm31> pt(n_vars);
  for (uint32_t l = 0; l < n_vars; l++) {
    if (!canonical_q(point[l])) return fail(GKR_ERR_INVALID, "point not canonical");
    pt[l] = Q(point[l]);
  }
  qm31 *dm, *eq;
  TRY(ensureT(c, S_MLE, len, &dm));
  TRY(ensureT(c, S_EQ, len, &eq));
  HIP_TRY(hipMemcpyAsync(dm, mle, len * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
  TRY(eq_table(c, pt.data(), (int)n_vars, len, eq));
  RoundSink sk;
  TRY(make_sink(c, &sk));
  GKR_LAUNCH(c, k_dot_q, dim3(partial_grid(len)), dim3(kBlock), 0, dm, eq, len, sk);
  TRY(launch_finish<1>(c, sk, partial_grid(len)));
  qm31 r[1];
  TRY(wait_sink<1>(c, sk, r));
  *out = G(r[0]);
  return GKR_OK;
}
extern "C" int gkr_restrict_mle(gkr_ctx* c, const gkr_qm31* mle, uint64_t len, const gkr_qm31* assign,
                                uint32_t n_assign, gkr_qm31* out) {
  if (!c || !mle || !out || (!assign && n_assign)) return fail(GKR_ERR_INVALID, "null argument");
  if (len == 0 || (len & (len - 1)) || (n_assign >= 64) || (1ull << n_assign) > len)
    return fail(GKR_ERR_INVALID, "bad MLE length %llu for %u assignments", (unsigned long long)len, n_assign);
  HIP_TRY(hipSetDevice(c->device));
  std::vector<qm31> pt(n_assign);
  for (uint32_t l = 0; l < n_assign; l++) {
    if (!canonical_q(assign[l])) return fail(GKR_ERR_INVALID, "assignment not canonical");
    pt[l] = Q(assign[l]);
  }
  const uint64_t nx = 1ull << n_assign, rest = len >> n_assign;
  qm31 *dm, *eq, *dout;
  TRY(ensureT(c, S_MLE, len, &dm));
  TRY(ensureT(c, S_EQ, nx, &eq));
  TRY(ensureT(c, S_OUT, rest, &dout));
  HIP_TRY(hipMemcpyAsync(dm, mle, len * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
  TRY(eq_table(c, pt.data(), (int)n_assign, nx, eq));
  GKR_LAUNCH(c, k_restrict_q, dim3(grid_for(rest)), dim3(kBlock), 0, dm, eq, nx, rest, dout);
  TRY(check_launch(c));
  HIP_TRY(hipMemcpyAsync(out, dout, rest * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
  return sync(c);
}

// ------------------------------------------------------------------ QM31 vectors, product sumcheck
extern "C" int gkr_qvec_upload(gkr_ctx* c, const gkr_qm31* host, uint64_t n, gkr_qvec** out) {
  if (!c || !out || !host) return fail(GKR_ERR_INVALID, "null argument");
  if (n == 0) return fail(GKR_ERR_INVALID, "empty vector");
  for (uint64_t i = 0; i < n; i++)
    if (!canonical_q(host[i])) return fail(GKR_ERR_INVALID, "vector value %llu not canonical", (unsigned long long)i);
  HIP_TRY(hipSetDevice(c->device));
  qm31* d = nullptr;
  HIP_TRY(hipMalloc(&d, n * sizeof(qm31)));
  drain(c);
  hipError_t e = hipMemcpyAsync(d, host, n * sizeof(qm31), hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return fail(GKR_ERR_DEVICE, "vector upload: %s", hipGetErrorString(e));
  }
  *out = new gkr_qvec{c, d, n};
  c->qvecs.insert(*out);
  return GKR_OK;
}
extern "C" int gkr_qvec_synthetic(gkr_ctx* c, uint64_t n, uint64_t seed, gkr_qvec** out) {
  if (!c || !out) return fail(GKR_ERR_INVALID, "null argument");
  if (n == 0) return fail(GKR_ERR_INVALID, "empty vector");
  HIP_TRY(hipSetDevice(c->device));
  qm31* d = nullptr;
  HIP_TRY(hipMalloc(&d, n * sizeof(qm31)));
  GKR_LAUNCH(c, k_fill_synth_q, dim3(partial_grid(n) * 8), dim3(kBlock), 0, d, n, seed);
  int rc = check_launch(c);
  if (rc == GKR_OK) rc = sync(c);
  if (rc != GKR_OK) {
    drain(c);
    (void)hipFree(d);
    return rc;
  }
  *out = new gkr_qvec{c, d, n};
  c->qvecs.insert(*out);
  return GKR_OK;
}
extern "C" int gkr_qvec_download(gkr_ctx* c, const gkr_qvec* v, gkr_qm31* host) {
  if (!c || !v || !host) return fail(GKR_ERR_INVALID, "null argument");
  if (v->ctx != c) return fail(GKR_ERR_INVALID, "vector belongs to another (or a destroyed) context");
  HIP_TRY(hipMemcpyAsync(host, v->dev, v->n * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
  return sync(c);
}
extern "C" const gkr_qm31* gkr_qvec_device_ptr(const gkr_qvec* v) {
  return v ? reinterpret_cast<const gkr_qm31*>(v->dev) : nullptr;
}
extern "C" void gkr_qvec_free(gkr_qvec* v) {
  if (!v) return;
  if (v->ctx) {
    v->ctx->qvecs.erase(v);
    if (v->dev) {
      drain(v->ctx);
      (void)hipStreamSynchronize(v->ctx->stream);
      (void)hipFree(v->dev);
    }
  }
  delete v;
}
extern "C" int gkr_sumcheck_product(gkr_ctx* c, const gkr_qvec* fa, const gkr_qvec* fb, gkr_channel* ch,
                                    gkr_qm31* round_polys, gkr_qm31* challenges, gkr_qm31* final_a,
                                    gkr_qm31* final_b) {
  CH_CHECK(ch);
  if (!c || !fa || !fb || !final_a || !final_b) return fail(GKR_ERR_INVALID, "null argument");
  if (fa->ctx != c || fb->ctx != c) return fail(GKR_ERR_INVALID, "vector belongs to another context");
  if (fa->n != fb->n) return fail(GKR_ERR_INVALID, "f_a has %llu entries, f_b %llu", (unsigned long long)fa->n,
                                  (unsigned long long)fb->n);
  const uint64_t n = fa->n;
  if (n & (n - 1)) return fail(GKR_ERR_INVALID, "length %llu is not a power of two", (unsigned long long)n);
  const int T = log2_exact(n);
  if (T > 0 && (!round_polys || !challenges)) return fail(GKR_ERR_INVALID, "null output arrays");
  HIP_TRY(hipSetDevice(c->device));
  if (T == 0) {
    qm31 v;
    TRY(fetch_q(c, fa->dev, 1, &v));
    *final_a = G(v);
    TRY(fetch_q(c, fb->dev, 1, &v));
    *final_b = G(v);
    return GKR_OK;
  }
  // scratch: the fold of round 1 (n/2) and of round 2 (n/4); the caller's vectors stay intact
  c->mm.valid = false;
  qm31 *a1, *a2, *b1, *b2;
  TRY(ensureT(c, S_FA1, n / 2 + 1, &a1));
  TRY(ensureT(c, S_FB1, n / 2 + 1, &b1));
  TRY(ensureT(c, S_FA0, n / 4 + 1, &a2));
  TRY(ensureT(c, S_FB0, n / 4 + 1, &b2));
  qm31* bufs_a[2] = {a1, a2};
  qm31* bufs_b[2] = {b1, b2};
  return product_sumcheck(c, ch->ch, T, fa->dev, fb->dev, bufs_a, bufs_b, nullptr, 0, round_polys, challenges,
                          final_a, final_b);
}

// The allocation-free variant: the caller's vectors are device pointers and
// every device buffer comes from the static scratch array.  The arrival
// counter's expected value belongs to the scratch copy, so the context's
// own counter state is set aside for the call and restored afterwards.
// Every call on one GPU shares that GPU's static scratch array, so the calls
// on a device take turns: each holds its device's lock from its first device
// call until its stream has drained.
constexpr int kNoAllocMaxDevices = 64;
static std::mutex g_noalloc_mu[kNoAllocMaxDevices];
extern "C" int gkr_sumcheck_product_noalloc(gkr_ctx* c, const gkr_qm31* fa, const gkr_qm31* fb, uint64_t n,
                                            gkr_channel* ch, gkr_qm31* round_polys, gkr_qm31* challenges,
                                            gkr_qm31* final_a, gkr_qm31* final_b) {
  CH_CHECK(ch);
  if (!c || !fa || !fb || !final_a || !final_b) return fail(GKR_ERR_INVALID, "null argument");
  if (n == 0 || (n & (n - 1))) return fail(GKR_ERR_INVALID, "length %llu is not a power of two", (unsigned long long)n);
  if (n > kNoAllocMaxN)
    return fail(GKR_ERR_INVALID, "length %llu exceeds the allocation-free maximum of %llu entries",
                (unsigned long long)n, (unsigned long long)kNoAllocMaxN);
  const int T = log2_exact(n);
  if (T > 0 && (!round_polys || !challenges)) return fail(GKR_ERR_INVALID, "null output arrays");
  if (c->device >= kNoAllocMaxDevices) return fail(GKR_ERR_INVALID, "device %d beyond the lock table", c->device);
  std::lock_guard<std::mutex> turn(g_noalloc_mu[c->device]);
  HIP_TRY(hipSetDevice(c->device));
  for (const gkr_qm31* p : {fa, fb}) {  // device memory of this context's GPU, or the kernels would fault
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess || at.type != hipMemoryTypeDevice || at.device != c->device) {
      (void)hipGetLastError();
      return fail(GKR_ERR_INVALID, "vector %p is not device memory of device %d", (const void*)p, c->device);
    }
  }
  const qm31* da = reinterpret_cast<const qm31*>(fa);
  const qm31* db = reinterpret_cast<const qm31*>(fb);
  if (T == 0) {
    qm31 v;
    TRY(fetch_q(c, da, 1, &v));
    *final_a = G(v);
    TRY(fetch_q(c, db, 1, &v));
    *final_b = G(v);
    return GKR_OK;
  }
  c->mm.valid = false;
  qm31* bufs_a[2] = {reinterpret_cast<qm31*>(c->scratch_dev + kScratchOffA1),
                     reinterpret_cast<qm31*>(c->scratch_dev + kScratchOffA2)};
  qm31* bufs_b[2] = {reinterpret_cast<qm31*>(c->scratch_dev + kScratchOffB1),
                     reinterpret_cast<qm31*>(c->scratch_dev + kScratchOffB2)};
  const uint32_t saved_count = c->trip_count;
  const bool saved_valid = c->trip_count_valid;
  const int saved_timing = c->timing;  // timing events would be created on demand
  c->noalloc = true;
  c->trip_count_valid = false;  // the scratch counter starts from zero (a fill kernel, queued first)
  c->timing = 0;
  const int rc = product_sumcheck(c, ch->ch, T, da, db, bufs_a, bufs_b, nullptr, 0, round_polys, challenges, final_a,
                                  final_b);
  c->noalloc = false;
  c->trip_count = saved_count;
  c->trip_count_valid = saved_valid;
  c->timing = saved_timing;
  const int rs = sync(c);  // nothing of this call still touches the scratch array when the lock is released
  return rc != GKR_OK ? rc : rs;
}

