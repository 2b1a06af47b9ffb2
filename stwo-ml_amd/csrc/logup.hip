// LogUp activation layer (reduce_activation_layer, gkr/prover.rs:6400-6600):
// tables, the eq-weighted degree-3 sumcheck and the multiplicity sumcheck.
#include "internal.h"
#include "activations.h"
// ------------------------------------------------------------------ LogUp activation layer
extern "C" int gkr_activation_table(uint32_t tag, uint32_t log_size, uint32_t* out) {
  if (!out || !act_valid(tag) || log_size == 0 || log_size > 24) return fail(GKR_ERR_INVALID, "bad argument");
  std::vector<uint32_t> t = act_table(tag, log_size);
  memcpy(out, t.data(), t.size() * sizeof(uint32_t));
  return GKR_OK;
}

const std::vector<uint32_t>& cached_table(gkr_ctx* c, uint32_t tag, uint32_t log_size) {
  const uint64_t key = ((uint64_t)tag << 32) | log_size;
  auto it = c->tables.find(key);
  if (it == c->tables.end()) it = c->tables.emplace(key, act_table(tag, log_size)).first;
  return it->second;
}
// The table's outputs resident on the device, uploaded on first use and kept
// for the context's lifetime (a model alternates between a few tables).
static int device_table(gkr_ctx* c, uint32_t tag, uint32_t log_size, uint32_t** out) {
  const uint64_t key = ((uint64_t)tag << 32) | log_size;
  auto it = c->dev_tables.find(key);
  if (it != c->dev_tables.end()) {
    *out = it->second;
    return GKR_OK;
  }
  const std::vector<uint32_t>& t = cached_table(c, tag, log_size);
  uint32_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, t.size() * sizeof(uint32_t)));
  const hipError_t e = hipMemcpy(d, t.data(), t.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return fail(GKR_ERR_DEVICE, "table upload: %s", hipGetErrorString(e));
  }
  c->dev_tables.emplace(key, d);
  *out = d;
  return GKR_OK;
}

// Eq-weighted degree-3 sumcheck over n = 2^nv entries (the eq-sumcheck of
// reduce_activation_layer, gkr/prover.rs:6501-6556, and of reduce_mul_layer,
// 6197-6245): s_t = sum_x eq_t * w_t * d_t at t = 0..3, Newton differences to
// (c0, c1, c2, c3), mix_poly_coeffs_deg3, draw, fold.
//
// eq(z, x) = prod_l eqlin(z_l, x_l) is kept factored: only w and d are stored
// and folded.  Round t's polynomial is eqlin(z_t, X) times the product of
// eqlin(z_l, r_l) over the earlier rounds times sum_x eq(z_{>t}, x) w d; the
// trips weight their cross sums by the eq part below their variables (two
// small tables per trip, built at the start), and the host finish rebuilds
// the eq vector of the remaining variables.  The polynomials, challenges and
// final values equal those of folding eq like w and d (the polynomial of each
// round is unique).
// Plan the trips of an eq-sumcheck over 2^nv entries and the eq tables they
// read (with_split, also the two halves of eq(z, .), Eq3Plan::split_*): the
// tables' list for k_eq_parts (its point left to the caller), offsets into
// S_EQPARTS.  arg->count == 0: no tables.
static int eq3_plan(int nv, bool with_split, Eq3Plan* pl, EqPartsArg* arg_out, uint32_t* total_out) {
  pl->nv = nv;
  pl->trips = plan_trips(nv, kHostTailEq3, trip_k(1ull << nv));
  pl->hi_off.clear();
  pl->lo_off.clear();
  pl->h.clear();
  EqPartsArg& arg = *arg_out;
  memset(&arg, 0, sizeof arg);
  uint32_t& total = *total_out;
  total = 0;
  if (pl->trips.empty() && !with_split) return GKR_OK;
  auto table = [&](int s0, int m) -> uint32_t {
    for (int i = 0; i < arg.count; i++)
      if (arg.s[i] == s0 && arg.m[i] == m) return arg.off[i];
    const int i = arg.count++;
    arg.s[i] = s0;
    arg.m[i] = m;
    arg.off[i] = total;
    total += 1u << m;
    return arg.off[i];
  };
  for (const Trip& tr : pl->trips) {
    if (arg.count + 2 > kEqPartsMax) return fail(GKR_ERR_DEVICE, "too many eq tables");
    const int m = nv - tr.t - tr.K;  // coordinates below the trip's variables
    const int h = m < kEqLoMax ? m : kEqLoMax;
    pl->hi_off.push_back(table(tr.t + tr.K, m - h));
    pl->lo_off.push_back(table(nv - h, h));
    pl->h.push_back(h);
  }
  if (with_split) {
    if (arg.count + 2 > kEqPartsMax) return fail(GKR_ERR_DEVICE, "too many eq tables");
    pl->split_h = nv / 2;
    pl->split_hi_off = table(0, nv - pl->split_h);
    pl->split_lo_off = table(nv - pl->split_h, pl->split_h);
  }
  return GKR_OK;
}
// The eq tables of a plan (ps.status given: the point from k_point_wait).
static int launch_eq_parts(gkr_ctx* c, const EqPartsArg& arg, uint32_t total, const Posted& ps) {
  HostTimer ht(c, K_HOST_LAUNCH);
  qm31* parts;
  TRY(ensureT(c, S_EQPARTS, total, &parts));
  {
    TimedLaunch tl(c, K_EQ_TABLE, 16ull * total);
    GKR_LAUNCH(c, k_eq_parts, dim3(grid_for(kEqLanes * (uint64_t)total)), dim3(kBlock), 0, arg, total, parts, ps);
  }
  return check_launch(c);
}
// Plan an eq-sumcheck over 2^nv entries for claim point z and launch the
// kernel that builds its eq tables (S_EQPARTS).
int eq3_prepare(gkr_ctx* c, const qm31* z, int nv, Eq3Plan* pl, bool with_split) {
  EqPartsArg arg;
  uint32_t total;
  TRY(eq3_plan(nv, with_split, pl, &arg, &total));
  if (!arg.count) return GKR_OK;
  arg.z = make_point(z, nv);
  Posted ps;
  memset(&ps, 0, sizeof ps);
  return launch_eq_parts(c, arg, total, ps);
}
// Launch trip j of the plan over sources w, d (np pending challenges pend),
// folded vectors to dw, dd when given.
int eq3_launch_trip(gkr_ctx* c, const Eq3Plan& pl, size_t j, const qm31* w, const qm31* d, int np,
                           const qm31* pend, qm31* dw, qm31* dd, int slot, RoundSink* sk, const TripWait* tw,
                           CarriedFinish* carry_out, const CarriedFinish* carry_in) {
  qm31* parts = (qm31*)c->buf[S_EQPARTS];
  const Trip& tr = pl.trips[j];
  return launch_trip(c, 1, tr.K, w, d, tr.n, np, pend, dw, dd, parts + pl.hi_off[j], parts + pl.lo_off[j], pl.h[j],
                     slot, sk, 0, 0, tw, carry_out, carry_in);
}
// The sumcheck for claim point z over w0, d0 (overwritten: the trips' folded
// vectors go to w1/d1 (n/2 entries) and w0/d0 alternately).  pre0: trip 0
// already launched (eq3_launch_trip, any slot).  Writes 4 * nv round
// coefficients, nv challenges and the final (eq, w, d) values.
int eq3_sumcheck(gkr_ctx* c, PoseidonChannel& C, const qm31* z, const Eq3Plan& pl, qm31* w0, qm31* d0,
                        qm31* w1, qm31* d1, gkr_qm31* rp_out, qm31* chal, qm31 fin[3],
                        const RoundSink* pre0, const std::function<int()>* after_last) {
  const int nv = pl.nv;
  if (nv == 0) {
    fin[0] = qm31_one();
    TRY(fetch_q(c, w0, 1, fin + 1));
    return fetch_q(c, d0, 1, fin + 2);
  }
  const qm31 inv2 = qm31_from_m31(1u << 30);
  const qm31 inv6 = qm31_from_m31(m31_inv(6));
  const qm31 two = qm31_from_m31(2), three = qm31_from_m31(3);
  auto absorb3 = [&](int t, const qm31* s) {
    const qm31 dd1 = qm31_sub(s[1], s[0]);
    const qm31 dd2 = qm31_mul(qm31_add(qm31_sub(qm31_sub(s[2], s[1]), s[1]), s[0]), inv2);
    const qm31 dd3 = qm31_mul(qm31_sub(qm31_sub(s[3], s[0]), qm31_mul(three, qm31_sub(s[2], s[1]))), inv6);
    const qm31 c0 = s[0];
    const qm31 c1 = qm31_add(qm31_sub(dd1, dd2), qm31_mul(two, dd3));
    const qm31 c2 = qm31_sub(dd2, qm31_mul(three, dd3));
    const qm31 c3 = dd3;
    rp_out[4 * t + 0] = G(c0);
    rp_out[4 * t + 1] = G(c1);
    rp_out[4 * t + 2] = G(c2);
    rp_out[4 * t + 3] = G(c3);
    HostTimer ht(c, K_HOST_FS);
    C.mix_poly_coeffs_deg3(c0, c1, c2, c3);
    chal[t] = C.draw_qm31();
  };
  const qm31 xs[4] = {qm31_zero(), qm31_one(), two, three};
  qm31* bw[2] = {w1, w0};
  qm31* bd[2] = {d1, d0};
  HandoverSession ho(c);
  AheadTrips ahead(c);
  const size_t nt = pl.trips.size();
  std::vector<RoundSink> sks(nt);
  std::vector<TripWait> tws(nt);
  // One trip ahead: trip j + 1 is launched (behind its mailbox wait, which also
  // adds trip j's rows) while trip j runs, before the host posts trip j's
  // challenges; the hand-over follows the last trip the same way.
  const bool pre = ahead.enabled();
  CarriedFinish carry;
  memset(&carry, 0, sizeof carry);
  const qm31* sw = w0;
  const qm31* sd = d0;
  auto launch_j = [&](size_t j, const qm31* pend_j) -> int {
    const Trip& tr = pl.trips[j];
    qm31* dw = j == 0 ? nullptr : bw[(j - 1) & 1];
    qm31* dd = j == 0 ? nullptr : bd[(j - 1) & 1];
    const TripWait* tw = nullptr;
    if (j > 0 && pre) {
      TRY(ahead.make(&tws[j]));
      tw = &tws[j];
    }
    const CarriedFinish carry_in = carry;
    TRY(eq3_launch_trip(c, pl, j, sw, sd, j == 0 ? 0 : pl.trips[j - 1].K, pend_j, dw, dd, 0, &sks[j], tw,
                        pre ? &carry : nullptr, tw ? &carry_in : nullptr));
    if (j > 0) {
      sw = dw;
      sd = dd;
    }
    if (j + 1 == nt) {
      TRY(ho.launch<2>(sw, sd, tr.n, tr.K, pre ? &carry : nullptr));
      if (after_last) TRY((*after_last)());
    }
    return GKR_OK;
  };
  if (pre0) {  // trip 0 launched earlier, with its own finisher
    sks[0] = *pre0;
    if (nt == 1) {
      TRY(ho.launch<2>(sw, sd, pl.trips[0].n, pl.trips[0].K));
      if (after_last) TRY((*after_last)());
    }
  } else {
    TRY(launch_j(0, nullptr));
  }
  if (pre && nt > 1) TRY(launch_j(1, nullptr));
  int np = 0;
  const qm31* pend = nullptr;
  qm31 cpre = qm31_one();  // prod of eqlin(z_l, r_l) over the rounds done
  for (size_t j = 0; j < nt; j++) {
    const Trip& tr = pl.trips[j];
    qm31 g[kMaxSums];
    if (j > 0 && !pre) TRY(launch_j(j, pend));
    TRY(wait_trip(c, sks[j], trip_nq(1, tr.K), g, j > 0 && pre ? tws[j].want : 0));
    TripGram tg(g, tr.K, z + tr.t, cpre);
    for (int i = 0; i < tr.K; i++) {
      qm31 sums[4];
      {
        HostTimer hg(c, K_HOST_GRAM);
        tg.values(4, xs, sums);
      }
      absorb3(tr.t + i, sums);
      if (j + 1 == nt) TRY(ho.post_one(i, chal[tr.t + i]));  // the hand-over folds it while the next is drawn
      if (i + 1 < tr.K) {
        HostTimer hg(c, K_HOST_GRAM);
        tg.fold(chal[tr.t + i]);
      }
    }
    for (int i = 0; i < tr.K; i++) cpre = qm31_mul(cpre, eqlin(z[tr.t + i], chal[tr.t + i]));
    np = tr.K;
    pend = chal + tr.t;
    if (pre && j + 1 < nt) {
      TRY(ahead.post(tws[j + 1], pend, np));
      if (j + 2 < nt) TRY(launch_j(j + 2, nullptr));  // while trip j + 1 runs
    }
  }
  const int t_end = pl.trips.back().t + pl.trips.back().K;
  const uint64_t hlen = 1ull << (nv - t_end);
  std::vector<qm31> v[2];
  TRY(ho.post(pend, np));
  TRY(ho.fetch(hlen, 2, v));
  std::vector<qm31>& W = v[0];
  std::vector<qm31>& D = v[1];
  // eq of the remaining coordinates, scaled by the factors already fixed
  std::vector<qm31> E(1, cpre);
  for (int l = t_end; l < nv; l++) {
    std::vector<qm31> nE(2 * E.size());
    for (size_t x = 0; x < E.size(); x++) {
      nE[2 * x + 1] = qm31_mul(E[x], z[l]);
      nE[2 * x] = qm31_sub(E[x], nE[2 * x + 1]);
    }
    E.swap(nE);
  }
  for (int t = t_end; t < nv; t++) {
    const size_t half = E.size() / 2;
    qm31 sums[4];
    {
      HostTimer ht(c, K_HOST_FINISH);
      hostfield::eq3_round(qwords(E.data()), qwords(W.data()), qwords(D.data()), half,
                           reinterpret_cast<uint32_t(*)[4]>(sums));
    }
    absorb3(t, sums);
    HostTimer ht(c, K_HOST_FINISH);
    hostfield::fold(qwords(E.data()), half, qwords(&chal[t]));
    hostfield::fold(qwords(W.data()), half, qwords(&chal[t]));
    hostfield::fold(qwords(D.data()), half, qwords(&chal[t]));
    E.resize(half);
    W.resize(half);
    D.resize(half);
  }
  fin[0] = E[0];
  fin[1] = W[0];
  fin[2] = D[0];
  return GKR_OK;
}

// The activation layer's first launches, in the order the host reads their
// results: the table's fractions (one inversion per table entry), the prepare
// pass (trace sum and input MLE at the claim point, slot kSlotPrep) and the
// eq-sumcheck's first trip (slot kSlotEq0).  ps.status given: launched ahead,
// gamma and beta come from k_point_wait's copies.  The buffers exist.
// Rounds of the eq-sumcheck's first trip when the prepare pass computes its
// sums (k_logup_prepare_trip: a long-vector trip of one or two rounds), else
// 0: the prepare pass and the trip are separate kernels, and the pass takes
// the input MLE from the split halves of eq(z, .).
static int prep_trip_k(int nv) {
  if (nv <= 0 || nv > 62) return 0;
  const uint64_t n = 1ull << nv;
  const int K = trip_k(n) < nv ? trip_k(n) : nv;  // plan_trips' first trip
  return K <= 2 && 2 * n > kTripSplitLanes ? K : 0;
}
#ifndef GKR_PREP_TRIP_BLOCKS
#define GKR_PREP_TRIP_BLOCKS 512
#endif
constexpr unsigned kPrepTripMaxBlocks = GKR_PREP_TRIP_BLOCKS;  // partial rows of the fused pass
template <int K>
static int launch_prepare_trip(gkr_ctx* c, const gkr_matrix* input, uint64_t n, const uint32_t* d_table,
                               const qm31* d_inv, uint32_t tsize, qm31 gamma, qm31 beta, const Eq3Plan& epl,
                               uint32_t* d_min, uint32_t* d_mout, qm31* d_d0, qm31* d_w0, uint32_t* d_mult,
                               const Posted& ps, RoundSink* sk) {
  const qm31* parts = (const qm31*)c->buf[S_EQPARTS];
  TRY(make_sink(c, sk, kSlotEq0));
  unsigned grid = partial_grid(n);
  if (grid > kPrepTripMaxBlocks) grid = kPrepTripMaxBlocks;
  {
    // algorithmic bytes: the input, masked input and output written (8 per entry), d and w written
    TimedLaunch tl(c, K_LOGUP_PREP, 4 * input->rows * input->cols + 8 * n + 32 * n, true);
    GKR_LAUNCH(c, k_logup_prepare_trip<K>, dim3(grid), dim3(kBlock), 0, input->dev, input->rows, input->cols,
               log2_exact(next_pow2(input->cols)), n, d_table, d_inv, tsize - 1, gamma, beta, parts + epl.hi_off[0],
               parts + epl.lo_off[0], epl.h[0], d_min, d_mout, d_d0, d_w0, d_mult, *sk, ps);
  }
  TRY(check_launch(c));
  GKR_LAUNCH(c, k_finish_wide<PrepTrip<K>::NQ>, dim3(1), dim3(kFinishBlock), 0, *sk, grid);
  return check_launch(c);
}

static int logup_first_launches(gkr_ctx* c, const gkr_matrix* input, uint64_t n, const uint32_t* d_table,
                                uint32_t table_log, bool lds_hist, qm31 gamma, qm31 beta, const Eq3Plan& epl,
                                const Posted& ps, RoundSink* sk_prep, RoundSink* sk_eq0) {
  const uint64_t tsize = 1ull << table_log;
  const uint64_t pcol = next_pow2(input->cols);
  uint32_t *d_mult, *d_min, *d_mout;
  qm31 *d_d0, *d_w0, *d_inv;
  TRY(ensureT(c, S_MULT, tsize, &d_mult));
  TRY(ensureT(c, S_MIN, n, &d_min));
  TRY(ensureT(c, S_MOUT, n, &d_mout));
  TRY(ensureT(c, S_D0, n, &d_d0));
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_LKINV, tsize, &d_inv));
  const qm31* eq_hi = (const qm31*)c->buf[S_EQPARTS] + epl.split_hi_off;
  const qm31* eq_lo = (const qm31*)c->buf[S_EQPARTS] + epl.split_lo_off;
  HostTimer ht(c, K_HOST_LAUNCH);
  GKR_LAUNCH(c, k_logup_inv_table, dim3(grid_for(tsize)), dim3(kBlock), 0, d_table, tsize, gamma, beta, d_inv, ps);
  TRY(check_launch(c));
  const int fk = prep_trip_k(epl.nv);
  if (fk) {  // one pass and one finisher: the trip's sums first, then the prepare values (one sink)
    uint32_t* mult = lds_hist ? nullptr : d_mult;
    if (fk == 1)
      TRY(launch_prepare_trip<1>(c, input, n, d_table, d_inv, (uint32_t)tsize, gamma, beta, epl, d_min, d_mout, d_d0,
                                 d_w0, mult, ps, sk_eq0));
    else
      TRY(launch_prepare_trip<2>(c, input, n, d_table, d_inv, (uint32_t)tsize, gamma, beta, epl, d_min, d_mout, d_d0,
                                 d_w0, mult, ps, sk_eq0));
    *sk_prep = *sk_eq0;
    sk_prep->out += 1 << (2 * fk);
    return GKR_OK;
  }
  TRY(make_sink(c, sk_prep, kSlotPrep));
  {
    uint32_t* counter;
    uint32_t base;
    const unsigned grid = partial_grid(n);
    TRY(deliver_args(c, grid, &counter, &base));
    // algorithmic bytes: the input, masked input and output written (8 per entry), d and w written
    TimedLaunch tl(c, K_LOGUP_PREP, 4 * input->rows * input->cols + 8 * n + 32 * n, true);
    GKR_LAUNCH(c, k_logup_prepare, dim3(grid), dim3(kBlock), 0, input->dev, input->rows, input->cols,
               log2_exact(pcol), n, d_table, d_inv, (uint32_t)(tsize - 1), gamma, beta, eq_hi, eq_lo, epl.split_h,
               d_min, d_mout, d_d0, d_w0, lds_hist ? nullptr : d_mult, *sk_prep, counter, base, ps);
    TRY(deliver_finish<2>(c, *sk_prep, grid, counter));
  }
  if (epl.nv > 0) TRY(eq3_launch_trip(c, epl, 0, d_w0, d_d0, 0, nullptr, nullptr, nullptr, kSlotEq0, sk_eq0));
  return GKR_OK;
}

// An activation layer's first kernels launched ahead of its claim point and
// gamma, beta: k_point_wait and the eq tables (the point only), then
// k_mailbox_wait on vmailbox, the table's inversion, the prepare pass and the
// eq-sumcheck's first trip, reading the posted values from device memory.
// gkr_prove_activation_layer posts the point as it starts and gamma, beta once
// drawn, so the eq tables are built while the host draws.  Launched only
// when nothing has to be allocated or uploaded on the way (growing a buffer
// synchronises with the stream, whose earlier kernels may wait for the host):
// this context has proved an activation of the same size before (buffers
// only grow), the table is resident and small enough for the LDS
// multiplicities.  *launched reports whether it was.
int prelaunch_activation(gkr_ctx* c, const gkr_matrix* input, uint32_t tag, uint32_t table_log, bool* launched) {
  *launched = false;
  if (c->noalloc || c->pre.active || !input || input->ctx != c || !act_logup_valid(tag)) return GKR_OK;
  if (table_log == 0) table_log = act_default_log_size(tag);
  const uint64_t n = next_pow2(input->rows) * next_pow2(input->cols);
  const int nv = log2_exact(n);
  const uint64_t tsize = 1ull << table_log;
  if (nv == 0 || nv > kMaxVars || table_log > 24 || tsize > (uint64_t)kHistBins || n < 4) return GKR_OK;
  if (!c->act_shapes.count(std::make_pair(nv, table_log))) return GKR_OK;
  const auto it = c->dev_tables.find(((uint64_t)tag << 32) | table_log);
  if (it == c->dev_tables.end()) return GKR_OK;
  if (c->cap[S_PTWAIT] < kPtWaitBytes) return GKR_OK;
  Eq3Plan epl;
  EqPartsArg arg;
  uint32_t total;
  TRY(eq3_plan(nv, prep_trip_k(nv) == 0, &epl, &arg, &total));
  uint8_t* pw;
  TRY(ensureT(c, S_PTWAIT, kPtWaitBytes, &pw));
  Posted pp;  // the point
  memset(&pp, 0, sizeof pp);
  pp.status = reinterpret_cast<const uint32_t*>(pw);
  pp.want = alloc_seq(&c->mb_seq, 1);
  pp.pt = reinterpret_cast<const PointArg*>(pw + 256);
  {
    HostTimer ht(c, K_HOST_LAUNCH);
    GKR_LAUNCH(c, k_point_wait, dim3(1), dim3(64), 0, c->mailbox, pp.want, kWaitSpinLimit, nv,
               reinterpret_cast<PointArg*>(pw + 256), reinterpret_cast<uint32_t*>(pw));
    TRY(check_launch(c));
  }
  c->pre.active = true;  // from here on a failure leaves a wait that the walk cancels
  c->pre.act = true;
  c->pre.want = pp.want;
  c->pre.a = input;
  c->pre.b = nullptr;
  c->pre.tag = tag;
  c->pre.table_log = table_log;
  c->pre.hold_vals = false;
  c->mm.valid = false;
  TRY(launch_eq_parts(c, arg, total, pp));
  TripWait tw;  // gamma and beta, copied to device memory for the kernels behind it
  tw.mb = c->vmailbox;
  tw.want = alloc_seq(&c->mb_seq, 1);
  tw.spin_limit = kWaitSpinLimit;
  if (c->debug_trip_spins) {  // test hook: a short bounded wait that expires before the post
    tw.spin_limit = c->debug_trip_spins;
    c->debug_trip_spins = 0;
    c->pre.hold_vals = true;
  }
  tw.status = reinterpret_cast<uint32_t*>(pw + 64);
  tw.chal = reinterpret_cast<qm31*>(pw + kPtWaitVals);
  c->pre.want_vals = tw.want;
  {
    HostTimer ht(c, K_HOST_LAUNCH);
    CarriedFinish none;
    memset(&none, 0, sizeof none);
    GKR_LAUNCH(c, k_mailbox_wait, dim3(1), dim3(kWaitBlock), 0, tw, none);
    TRY(check_launch(c));
  }
  Posted pv;  // gamma and beta
  memset(&pv, 0, sizeof pv);
  pv.status = tw.status;
  pv.want = tw.want;
  pv.vals = tw.chal;
  TRY(logup_first_launches(c, input, n, it->second, table_log, true, qm31_zero(), qm31_zero(), epl, pv,
                           &c->pre.sk_prep, &c->pre.sk_eq0));
  *launched = true;
  return GKR_OK;
}

extern "C" int gkr_prove_activation_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                          const gkr_qm31* claim_value, const gkr_matrix* input, uint32_t tag,
                                          uint32_t table_log, gkr_channel* ch, gkr_proof* proof, gkr_logup_out* out) {
  if (out && !out->multiplicities) return fail(GKR_ERR_INVALID, "null output arrays");
  return prove_activation(c, claim_point, n_point, claim_value, input, tag, table_log, ch, proof, out);
}
int prove_activation(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                     const gkr_matrix* input, uint32_t tag, uint32_t table_log, gkr_channel* ch, gkr_proof* proof,
                     gkr_logup_out* out) {
  CH_CHECK(ch);
  if (!c || !input || !claim_value || !out || (!claim_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (!act_valid(tag)) return fail(GKR_ERR_INVALID, "unknown activation type %u", tag);
  if (!act_logup_valid(tag))
    return fail(GKR_ERR_INVALID, "activation type %u (ReLU) is proved algebraically, not by LogUp", tag);
  if (table_log == 0) table_log = act_default_log_size(tag);
  if (table_log > 24) return fail(GKR_ERR_INVALID, "table_log_size %u too large", table_log);
  if (input->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another context");
  const uint64_t prow = next_pow2(input->rows), pcol = next_pow2(input->cols);
  const uint64_t n = prow * pcol;
  const int nv = log2_exact(n);
  if ((int)n_point != nv)
    return fail(GKR_ERR_INVALID, "claim point has %u vars, activation MLE has %d", n_point, nv);
  if (nv > kMaxVars) return fail(GKR_ERR_INVALID, "activation too large");
  if (!out->eq_round_polys && nv > 0) return fail(GKR_ERR_INVALID, "null eq_round_polys");
  if (!out->mult_round_polys) return fail(GKR_ERR_INVALID, "null output arrays");
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  std::vector<qm31> cpt(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(claim_point[l])) return fail(GKR_ERR_INVALID, "claim point not canonical");
    cpt[l] = Q(claim_point[l]);
  }
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  TraceScope trace;
  PoseidonChannel& C = ch->ch;
  const uint64_t tsize = 1ull << table_log;

  uint32_t *d_table, *d_mult, *d_min, *d_mout;
  qm31 *d_d0, *d_d1, *d_w0, *d_w1, *m0, *m1, *d_inv;
  TRY(ensureT(c, S_MULT, tsize, &d_mult));
  TRY(ensureT(c, S_MIN, n, &d_min));
  TRY(ensureT(c, S_MOUT, n, &d_mout));
  TRY(ensureT(c, S_D0, n, &d_d0));
  TRY(ensureT(c, S_D1, n / 2 + 1, &d_d1));
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_W1, n / 2 + 1, &d_w1));
  TRY(ensureT(c, S_M0, tsize, &m0));
  TRY(ensureT(c, S_M1, tsize / 2 + 1, &m1));
  TRY(ensureT(c, S_LKINV, tsize, &d_inv));
  {  // the eq halves of the input and output MLEs' pass (dot2_launch), sized
     // now: it is queued behind the multiplicity sumcheck's hand-over, where
     // nothing may allocate
    qm31 *hi, *lo;
    TRY(ensureT(c, S_EQHI, 1ull << (nv - nv / 2), &hi));
    TRY(ensureT(c, S_EQLO, 1ull << (nv / 2), &lo));
  }
  TRY(ensure_host_mult(c, tsize));
  // the layer's multiplicity slot: handed to its proof record, or freed when this call ends
  struct SlotHold {
    std::shared_ptr<MultRing> r;
    int s;
    ~SlotHold() {
      if (r) r->busy[s].store(0, std::memory_order_release);
    }
  } mslot{c->mring, c->h_mult_slot};
  TRY(device_table(c, tag, table_log, &d_table));
  // Multiplicities: tables of up to 2^16 entries are counted in LDS per
  // workgroup (k_logup_hist) and added in the table pass; larger ones with
  // global atomics into S_MULT, which starts from zero (the previous layer's
  // conversion kernel cleared it, or it is cleared here).
  const bool lds_hist = tsize <= (uint64_t)kHistBins && n >= 4;
  if (!lds_hist) {
    if (c->mult_zero_entries < tsize) HIP_TRY(hipMemsetAsync(d_mult, 0, tsize * sizeof(uint32_t), c->stream));
    c->mult_zero_entries = 0;
  }
  // The layer's first kernels (the eq tables, the table's inversion, the
  // prepare pass and the eq-sumcheck's first trip) are launched ahead when
  // they can be: by the walk at the previous step's last launch, or here,
  // before the host draws gamma and beta (the launch calls then overlap the
  // draws); they wait on the device for the claim point and gamma, beta.
  // Otherwise one launch builds the eq tables of the eq-sumcheck trips (and,
  // when the prepare pass runs apart from the first trip, eq(claim point, x)
  // as the product of its high and low halves, for the input MLE at the
  // claim point) while the host draws gamma and beta, and the rest follows
  // the draws.
  bool pre = c->pre.active && c->pre.act && c->pre.a == input && c->pre.tag == tag && c->pre.table_log == table_log;
  if (!pre && !c->pre.active) {  // nothing queued waits for the host: the wait's buffer may be allocated
    uint8_t* pw;
    TRY(ensureT(c, S_PTWAIT, kPtWaitBytes, &pw));
    TRY(prelaunch_activation(c, input, tag, table_log, &pre));
  }
  Eq3Plan epl;
  if (pre) {  // post the claim point: the eq tables are built while the host draws gamma and beta
    Mailbox* mb = c->mailbox;
    for (int l = 0; l < nv; l++) mb->point[l] = cpt[l];
    __atomic_store_n(&mb->seq, c->pre.want, __ATOMIC_RELEASE);
    c->point_mb = c->pre.want;  // checked once the prepare sums are in
    EqPartsArg arg;
    uint32_t total;
    TRY(eq3_plan(nv, prep_trip_k(nv) == 0, &epl, &arg, &total));
  } else {
    TRY(eq3_prepare(c, cpt.data(), nv, &epl, prep_trip_k(nv) == 0));
  }

  // Fiat-Shamir: LOG tag, type tag, gamma, beta (prover.rs:6451-6454)
  C.mix_u64(0x4C4F47ull);
  C.mix_u64(tag);
  qm31 gb[2];
  C.draw_qm31s(gb, 2);
  const qm31 gamma = gb[0], beta = gb[1];
  trace_point(C, "logup.gamma_beta");
  out->gamma = G(gamma);
  out->beta = G(beta);

  // Launched back to back, read when needed (each result in its own slot), in
  // the order the host needs them:
  //   prepare -> (trace sum, input MLE at the claim point)      kSlotPrep
  //   eq-sumcheck trip 0                                         kSlotEq0
  //   (over more than 2^16 entries one fused pass delivers both to kSlotEq0:
  //   the trip's sums, the trace sum, the input MLE per top sub-vector)
  //   table-side sum over the multiplicities                     kSlotTable
  //   multiplicities -> pinned host copy
  //   multiplicity sumcheck trip 0 (no challenge needed)         kSlotMult0
  RoundSink sk_prep, sk_table, sk_mult0, sk_eq0;
  const bool eq_pre = nv > 0;
  if (pre) {  // post gamma and beta
    Mailbox* vmb = c->vmailbox;
    const uint32_t want = c->pre.want_vals;
    if (c->pre.hold_vals) {  // test hook: post only after the bounded wait gave up
      const auto t0 = std::chrono::steady_clock::now();
      volatile uint32_t* expired = &vmb->expired;
      while (*expired != want && std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < 10.0) {
      }
      c->pre.hold_vals = false;
    }
    vmb->alpha[0] = gamma;
    vmb->alpha[1] = beta;
    __atomic_store_n(&vmb->seq, want, __ATOMIC_RELEASE);
    c->vals_mb = want;  // checked once the prepare sums are in
    sk_prep = c->pre.sk_prep;
    sk_eq0 = c->pre.sk_eq0;
    c->pre.active = false;
    c->pre.act = false;
    c->stats[K_ACT_AHEAD].launches++;
  } else {
    Posted ps;
    memset(&ps, 0, sizeof ps);
    TRY(logup_first_launches(c, input, n, d_table, table_log, lds_hist, gamma, beta, epl, ps, &sk_prep, &sk_eq0));
  }
  // The table side (multiplicities, their copies, the table-side sum) and the
  // multiplicity sumcheck's first trip are needed only after the eq-sumcheck:
  // they are queued behind its last launch (the hand-over), so they run while
  // the host finishes the eq-sumcheck's last rounds instead of between its
  // trips.  Their buffers are set up here: nothing queued after the
  // eq-sumcheck's trips may allocate (a free would wait for those trips, which
  // wait for the host).
  const uint64_t hgroups = (n + kHistPerGroup - 1) / kHistPerGroup;
  uint32_t* hist = nullptr;
  if (lds_hist) TRY(ensureT(c, S_LKHIST, hgroups * (kHistBins / 2), &hist));
  const std::vector<Trip> mtrips = plan_trips((int)table_log, kHostTailSum, kTripMaxK);
  bool table_side_done = false;
  std::function<int()> table_side = [&]() -> int {
    table_side_done = true;
    HostTimer ht(c, K_HOST_LAUNCH);
    // the sink's sequence number is taken now: deliveries publish increasing
    // numbers in stream order, and a wait takes any later number as proof
    TRY(make_sink(c, &sk_table, kSlotTable));
    uint32_t* counter;
    uint32_t base;
    if (lds_hist) {
      // counts of the masked input (the padding added to bin 0 afterwards),
      // then one pass over the bins: multiplicities, their QM31 and host
      // copies, table sum
      GKR_LAUNCH(c, k_logup_hist, dim3((unsigned)hgroups), dim3(kHistBlock), 0, d_min, n, input->rows,
                 input->cols, log2_exact(pcol), hist);
      TRY(check_launch(c));
      const unsigned grid = partial_grid(tsize / 2);
      TRY(deliver_args(c, grid, &counter, &base));
      GKR_LAUNCH(c, k_logup_table_pass, dim3(grid), dim3(kBlock), 0, hist, (int)hgroups,
                 (uint32_t)(n - input->rows * input->cols), d_inv, tsize, m0, c->h_mult, sk_table, counter, base);
      TRY(deliver_finish<1>(c, sk_table, grid, counter));
    } else {
      const unsigned grid = partial_grid(tsize);
      TRY(deliver_args(c, grid, &counter, &base));
      GKR_LAUNCH(c, k_logup_table_sum, dim3(grid), dim3(kBlock), 0, d_inv, d_mult, tsize, sk_table, counter, base);
      TRY(deliver_finish<1>(c, sk_table, grid, counter));
      // the multiplicities as QM31 for the sumcheck, and to the pinned host copy
      GKR_LAUNCH(c, k_u32_to_q, dim3(grid_for(tsize)), dim3(kBlock), 0, d_mult, tsize, m0, c->h_mult, 1);
      TRY(check_launch(c));
      c->mult_zero_entries = tsize;
    }
    return launch_trip(c, 2, mtrips[0].K, m0, nullptr, tsize, 0, nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                       kSlotMult0, &sk_mult0);
  };

  // The trace sum goes into the transcript now; the table-side sum it must
  // equal is checked before the multiplicity sumcheck, so the histogram and
  // table pass run on the device while the host works through the first
  // eq-sumcheck rounds.
  qm31 prep[2];
  if (const int fk = prep_trip_k(nv)) {
    // the trace sum, then the input MLE per top sub-vector c, weighted here by
    // eq(z_0 .. z_(fk-1), c) (z_0 on the most significant bit of c)
    qm31 v[1 + (1 << kTripMaxK)];
    TRY(wait_result<0>(c, sk_prep.seq, nullptr, K_HOST_WAIT));
    const int slot = (int)(sk_prep.out - c->h_out);
    for (int q = 0; q <= (1 << fk); q++) v[q] = c->h_out[slot + q];
    prep[0] = v[0];
    prep[1] = qm31_zero();
    for (int cc = 0; cc < (1 << fk); cc++) {
      qm31 e = qm31_one();
      for (int l = 0; l < fk; l++) e = qm31_mul(e, eqlin(cpt[l], ((cc >> (fk - 1 - l)) & 1) ? qm31_one() : qm31_zero()));
      prep[1] = qm31_add(prep[1], qm31_mul(e, v[1 + cc]));
    }
  } else {
    TRY(wait_sink<2>(c, sk_prep, prep));
  }
  TRY(check_point_wait(c));
  const qm31 trace_sum = prep[0], input_eval = prep[1];
  C.mix_secure_field(trace_sum);
  out->claimed_sum = G(trace_sum);

  // eq-sumcheck: sum eq(r, x) w(x) d(x) = 1 over the hypercube
  std::vector<qm31> chal(nv);
  qm31 fin[3];
  TRY(eq3_sumcheck(c, C, cpt.data(), epl, d_w0, d_d0, d_w1, d_d1, out->eq_round_polys, chal.data(), fin,
                   eq_pre ? &sk_eq0 : nullptr, &table_side));
  trace_point(C, "logup.eq");
  if (!table_side_done) TRY(table_side());
  const qm31 w_eval = fin[1];
  // MLE(masked_in), MLE(masked_out) at the eq-sumcheck challenges, one pass;
  // the transcript does not use them before the multiplicity sumcheck, so the
  // pass is queued behind that sumcheck's hand-over (it runs while the host
  // finishes the last rounds; queued earlier it would delay the trips the
  // host waits for) and read after it
  RoundSink sk_io;
  bool io_launched = false;
  auto launch_io = [&]() -> int {
    io_launched = true;
    return dot2_launch(c, chal.data(), nv, d_min, d_mout, kSlotIO, &sk_io);
  };
  out->w_eval = G(w_eval);

  qm31 tsum[1];
  TRY(wait_sink<1>(c, sk_table, tsum));
  const qm31 table_sum = tsum[0];
  if (!qm31_eq(trace_sum, table_sum))
    return fail(GKR_ERR_LOGUP, "Activation LogUp sum mismatch: trace=(%u,%u,%u,%u) table=(%u,%u,%u,%u)", trace_sum.a,
                trace_sum.b, trace_sum.c, trace_sum.d, table_sum.a, table_sum.b, table_sum.c, table_sum.d);

  // Multiplicity sumcheck (prover.rs:9449-9511): degree-1 rounds over
  // 2^table_log entries.  The multiplicities count every padded input once,
  // so their sum is n.
  const qm31 mult_sum = qm31_from_m31(m31_reduce64(n));
  qm31* bm[2] = {m1, m0};
  qm31 alpha = qm31_zero();
  auto absorb1 = [&](uint32_t t, const qm31* s) {
    const qm31 c0 = s[0];
    const qm31 c1 = qm31_sub(s[1], s[0]);
    out->mult_round_polys[2 * t] = G(c0);
    out->mult_round_polys[2 * t + 1] = G(c1);
    HostTimer ht(c, K_HOST_FS);
    C.mix_secure_field(c0);
    C.mix_secure_field(c1);
    alpha = C.draw_qm31();
  };
  qm31 mfin[1];
  {
    // trips of up to 3 rounds (the first launched ahead above), then the host
    HandoverSession ho(c);
    AheadTrips ahead(c);
    const size_t nt = mtrips.size();
    std::vector<RoundSink> sks(nt);
    std::vector<TripWait> tws(nt);
    sks[0] = sk_mult0;  // launched above, with its own finisher
    // one trip ahead, as in the eq-sumcheck
    const bool pre = ahead.enabled();
    CarriedFinish carry;
    memset(&carry, 0, sizeof carry);
    const qm31* src = m0;
    auto launch_j = [&](size_t j, const qm31* pend_j) -> int {  // j >= 1
      const Trip& tr = mtrips[j];
      qm31* dst = bm[(j - 1) & 1];
      const TripWait* tw = nullptr;
      if (pre) {
        TRY(ahead.make(&tws[j]));
        tw = &tws[j];
      }
      const CarriedFinish carry_in = carry;
      TRY(launch_trip(c, 2, tr.K, src, nullptr, tr.n, mtrips[j - 1].K, pend_j, dst, nullptr, nullptr, nullptr, 0, 0,
                      &sks[j], 0, 0, tw, pre ? &carry : nullptr, tw ? &carry_in : nullptr));
      src = dst;
      if (j + 1 == nt) {
        TRY(ho.launch<1>(src, nullptr, tr.n, tr.K, pre ? &carry : nullptr));
        TRY(launch_io());
        TRY(run_prelaunch(c));  // the activation step's last launch
      }
      return GKR_OK;
    };
    if (nt == 1) {
      TRY(ho.launch<1>(src, nullptr, mtrips[0].n, mtrips[0].K));
      TRY(launch_io());
      TRY(run_prelaunch(c));
    }
    if (pre && nt > 1) TRY(launch_j(1, nullptr));
    int np = 0;
    const qm31* pend = nullptr;
    std::vector<qm31> mchal(table_log);
    for (size_t j = 0; j < nt; j++) {
      const Trip& tr = mtrips[j];
      if (j > 0 && !pre) TRY(launch_j(j, pend));
      qm31 g[kMaxSums];
      TRY(wait_trip(c, sks[j], trip_nq(2, tr.K), g, j > 0 && pre ? tws[j].want : 0));
      for (int i = 0; i < tr.K; i++) {
        qm31 sums[2];
        {
          HostTimer hg(c, K_HOST_GRAM);
          trip_round_sum(g, tr.K, i, mchal.data() + tr.t, sums);
        }
        absorb1((uint32_t)(tr.t + i), sums);
        mchal[tr.t + i] = alpha;
        if (j + 1 == nt) TRY(ho.post_one(i, alpha));  // the hand-over folds it while the next is drawn
      }
      np = tr.K;
      pend = mchal.data() + tr.t;
      if (pre && j + 1 < nt) {
        TRY(ahead.post(tws[j + 1], pend, np));
        if (j + 2 < nt) TRY(launch_j(j + 2, nullptr));  // while trip j + 1 runs
      }
    }
    const int t_end = mtrips.back().t + mtrips.back().K;
    std::vector<qm31> v[1];
    TRY(ho.post(pend, np));
    TRY(ho.fetch(tsize >> t_end, 1, v));
    std::vector<qm31>& V = v[0];
    for (int t = t_end; t < (int)table_log; t++) {
      const size_t half = V.size() / 2;
      qm31 sums[2];
      {
        HostTimer ht(c, K_HOST_FINISH);
        hostfield::halves_sum(qwords(V.data()), half, reinterpret_cast<uint32_t(*)[4]>(sums));
      }
      absorb1((uint32_t)t, sums);
      HostTimer ht(c, K_HOST_FINISH);
      hostfield::fold(qwords(V.data()), half, qwords(&alpha));
      V.resize(half);
    }
    mfin[0] = V[0];
  }
  trace_point(C, "logup.mult");
  // the kernels whose results were waited for in the multiplicity sumcheck
  // were queued after the one writing the multiplicities' pinned copy
  if (out->multiplicities) memcpy(out->multiplicities, c->h_mult, tsize * sizeof(uint32_t));
  if (!io_launched) TRY(launch_io());
  qm31 io[2];
  TRY(wait_sink<2>(c, sk_io, io));
  const qm31 in_eval = io[0], out_eval = io[1];
  out->in_eval = G(in_eval);
  out->out_eval = G(out_eval);
  out->mult_final_eval = G(mfin[0]);
  out->mult_claimed_sum = G(mult_sum);

  // Table commitment = poseidon_hash_many([type_tag, log_size]) (prover.rs:8365-8373), a
  // function of the table alone: hashed once per context and table
  const uint64_t tkey = ((uint64_t)tag << 32) | table_log;
  auto tci = c->table_commitments.find(tkey);
  if (tci == c->table_commitments.end()) {
    felt tc_in[2] = {felt_from_u64(tag), felt_from_u64(table_log)};
    tci = c->table_commitments.emplace(tkey, poseidon_hash_many(tc_in, 2)).first;
  }
  const felt tc = tci->second;
  out->table_commitment = felt_to_abi(tc);
  C.mix_secure_field(input_eval);
  C.mix_secure_field(Q(*claim_value));
  trace_point(C, "logup");
  out->input_eval = G(input_eval);
  out->output_eval = *claim_value;

  if (proof) {
    HostTimer hp(c, K_HOST_PROOF);
    LayerRec L;
    L.tag = 3;
    L.act_type = tag;
    for (int t = 0; t < 4 * nv; t++) L.rp.push_back(Q(out->eq_round_polys[t]));
    L.input_eval = input_eval;
    L.output_eval = Q(*claim_value);
    L.claim_value = Q(*claim_value);
    L.table_commitment = felt_from_mont(tc);
    L.claimed_sum = trace_sum;
    L.w_eval = w_eval;
    L.in_eval = in_eval;
    L.out_eval = out_eval;
    L.mult_ring = std::move(mslot.r);  // copied by layer_take_mults (the proof stream's thread)
    L.mult_slot = mslot.s;
    L.mult_count = tsize;
    for (uint32_t t = 0; t < 2 * table_log; t++) L.mult_rp.push_back(Q(out->mult_round_polys[t]));
    L.mult_final = mfin[0];
    L.mult_sum = mult_sum;
    proof_add_layer(proof, std::move(L));
  }
  c->act_shapes.insert(std::make_pair(nv, table_log));
  return GKR_OK;
}

