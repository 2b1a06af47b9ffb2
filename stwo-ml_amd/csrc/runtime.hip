// Device context, resident matrices, scratch buffers, result sinks and the
// multi-round trip launcher shared by the layer reducers; the bandwidth
// reference kernels.
#include "internal.h"

// ------------------------------------------------------------------ errors, version
thread_local std::string g_err = "";
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
extern "C" const char* gkr_last_error(void) { return g_err.c_str(); }
extern "C" const char* gkr_version(void) { return "gkr_mi355x 0.1 (gfx950)"; }

static __device__ __align__(256) uint8_t scratch[kScratchBytes];
int ensure(gkr_ctx* c, Slot s, size_t bytes, void** out) {
  if (bytes == 0) bytes = 16;
  if (c->noalloc) {
    if (s == S_PART && bytes <= kScratchPartBytes) {
      *out = c->scratch_dev + kScratchOffPart;
      return GKR_OK;
    }
    if (s == S_TRIPCNT && bytes <= 256) {
      *out = c->scratch_dev + kScratchOffCount;
      return GKR_OK;
    }
    return fail(GKR_ERR_NOMEM, "the allocation-free entry point needs device buffer %d (%zu bytes)", (int)s, bytes);
  }
  if (c->cap[s] < bytes) {
    if (s == S_TRIPCNT) c->trip_count_valid = false;  // fresh memory must be zeroed
    if (s == S_MULT) c->mult_zero_entries = 0;
    if (s == S_TRIPMB) c->tripmb_valid = false;
    if (c->buf[s]) HIP_TRY(hipFree(c->buf[s]));
    c->buf[s] = nullptr;
    c->cap[s] = 0;
    size_t want = bytes < 4096 ? 4096 : bytes;
    HIP_TRY(hipMalloc(&c->buf[s], want));
    c->cap[s] = want;
  }
  *out = c->buf[s];
  return GKR_OK;
}

int ensure_host_mult(gkr_ctx* c, uint64_t n) {
  c->h_mult = nullptr;
  c->h_mult_slot = -1;
  if (!c->mring || c->mring->cap < n) {
    // a larger ring; records still holding the old one keep it until they copied their slots
    HIP_TRY(hipStreamSynchronize(c->stream));
    auto r = std::make_shared<MultRing>();
    for (int i = 0; i < MultRing::kSlots; i++)
      HIP_TRY(hipHostMalloc((void**)&r->buf[i], n * sizeof(uint32_t), hipHostMallocCoherent | hipHostMallocMapped));
    r->cap = n;
    c->mring = std::move(r);
  }
  MultRing& r = *c->mring;
  const int s = r.next;
  // the slot's last record copies it as the proof stream writes that record,
  // normally long before the ring comes round again
  const auto t0 = std::chrono::steady_clock::now();
  for (uint32_t i = 0; r.busy[s].load(std::memory_order_acquire); i++)
    if ((i & 1023) == 1023 && std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > 60.0)
      return fail(GKR_ERR_DEVICE, "multiplicity slot %d still held by an unwritten proof record after 60 s", s);
  r.busy[s].store(1, std::memory_order_relaxed);
  r.next = (s + 1) % MultRing::kSlots;
  c->h_mult = r.buf[s];
  c->h_mult_slot = s;
  return GKR_OK;
}

hipEvent_t get_event(gkr_ctx* c) {
  if (!c->free_events.empty()) {
    hipEvent_t e = c->free_events.back();
    c->free_events.pop_back();
    return e;
  }
  // timing-only events: no system-scope fence (cache writeback) when they are
  // recorded, so the pair brackets the kernel and not the cache maintenance
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}
void collect_timing(gkr_ctx* c) {
  for (auto& p : c->pending) {
    float ms = 0;
    if (hipEventElapsedTime(&ms, p.e0, p.e1) == hipSuccess) {
      c->stats[p.kid].ms += ms;
      c->stats[p.kid].launches++;
      c->stats[p.kid].bytes += p.bytes;
      KernelStat& z = c->size_stats[{p.kid, p.bytes}];
      z.ms += ms;
      z.launches++;
      z.bytes += p.bytes;
    }
    c->free_events.push_back(p.e0);
    c->free_events.push_back(p.e1);
  }
  c->pending.clear();
}
int sync(gkr_ctx* c) {
  HIP_TRY(hipStreamSynchronize(c->stream));
  if (c->timing) collect_timing(c);
  return GKR_OK;
}

PointArg make_point(const qm31* r, int n) {
  PointArg p;
  memset(&p, 0, sizeof p);
  p.n = n;
  for (int l = 0; l < n; l++) {
    p.r[l] = r[l];
    p.omr[l] = qm31_sub(qm31_one(), r[l]);
  }
  return p;
}
int eq_table(gkr_ctx* c, const qm31* r, int n, uint64_t count, qm31* out) {
  if (n > kMaxVars) return fail(GKR_ERR_INVALID, "eq table: %d variables exceeds %d", n, kMaxVars);
  PointArg pt = make_point(r, n);
  TimedLaunch t(c, K_EQ_TABLE, 16 * count);
  if (n <= 10) {
    GKR_LAUNCH(c, k_eq_direct, dim3(grid_for(kEqLanes * count)), dim3(kBlock), 0, pt, count, out);
    return check_launch(c);
  }
  const int h = n / 2;
  qm31 *hi, *lo;
  TRY(ensureT(c, S_EQHI, 1ull << (n - h), &hi));
  TRY(ensureT(c, S_EQLO, 1ull << h, &lo));
  GKR_LAUNCH(c, k_eq_tables, dim3(grid_for(kEqLanes * ((1ull << (n - h)) + (1ull << h)))), dim3(kBlock), 0, pt, h,
                     hi, lo);
  TRY(check_launch(c));
  GKR_LAUNCH(c, k_eq_combine, dim3(grid_for(count)), dim3(kBlock), 0, hi, lo, h, count, out);
  return check_launch(c);
}
// The high / low factor tables of eq(r, .) over n coordinates (S_EQHI over
// the first n - h, S_EQLO over the last h = n / 2), one launch.
int eq_split(gkr_ctx* c, const qm31* r, int n, qm31** hi, qm31** lo, int* h) {
  if (n > kMaxVars) return fail(GKR_ERR_INVALID, "eq table: %d variables exceeds %d", n, kMaxVars);
  *h = n / 2;
  const uint64_t n_hi = 1ull << (n - *h), n_lo = 1ull << *h;
  TRY(ensureT(c, S_EQHI, n_hi, hi));
  TRY(ensureT(c, S_EQLO, n_lo, lo));
  PointArg pt = make_point(r, n);
  TimedLaunch t(c, K_EQ_TABLE, 16 * (n_hi + n_lo));
  GKR_LAUNCH(c, k_eq_tables, dim3(grid_for(kEqLanes * (n_hi + n_lo))), dim3(kBlock), 0, pt, *h, *hi, *lo);
  return check_launch(c);
}
// The arrival counter of kernels that deliver their own results
// (sink_finish_counted, fused trips): the base value for a launch of `grid`
// workgroups, zeroing the counter first when its value is unknown.
int arrival_counter(gkr_ctx* c, unsigned grid, uint32_t** counter, uint32_t* base) {
  TRY(ensureT(c, S_TRIPCNT, 1, counter));
  if (!c->trip_count_valid) {
    GKR_LAUNCH(c, k_zero_u32, dim3(1), dim3(64), 0, *counter, 1u);
    TRY(check_launch(c));
    c->trip_count = 0;
    c->trip_count_valid = true;
  }
  *base = c->trip_count;
  c->trip_count += grid;
  return GKR_OK;
}
// Delivery of a reducing kernel's sums: by k_finish launched behind it
// (deliver_finish), or, with GKR_TRIP_FUSED=1 and grids of at most
// kTripFusedMax workgroups, by the kernel itself (an arrival counter).
int deliver_args(gkr_ctx* c, unsigned grid, uint32_t** counter, uint32_t* base) {
  *counter = nullptr;
  *base = 0;
  if (!GKR_TRIP_FUSED || grid > kTripFusedMax) return GKR_OK;
  return arrival_counter(c, grid, counter, base);
}
// MLEs of two M31 vectors of n = 2^nv entries at z (one eq split, one pass).
int dot2_launch(gkr_ctx* c, const qm31* z, int nv, const uint32_t* v0, const uint32_t* v1, int slot, RoundSink* sk) {
  const uint64_t n = 1ull << nv;
  qm31 *hi, *lo;
  int h;
  TRY(eq_split(c, z, nv, &hi, &lo, &h));
  TRY(make_sink(c, sk, slot));
  const unsigned grid = partial_grid(n);
  uint32_t* counter;
  uint32_t base;
  TRY(deliver_args(c, grid, &counter, &base));
  GKR_LAUNCH(c, k_dot2_m31, dim3(grid), dim3(kBlock), 0, v0, v1, hi, lo, h, n, *sk, counter, base);
  return deliver_finish<2>(c, *sk, grid, counter);
}
int dot2_evals(gkr_ctx* c, const qm31* z, int nv, const uint32_t* v0, const uint32_t* v1, qm31 out[2]) {
  RoundSink sk;
  TRY(dot2_launch(c, z, nv, v0, v1, 0, &sk));
  return wait_sink<2>(c, sk, out);
}
int make_sink(gkr_ctx* c, RoundSink* sk, int slot) {
  qm31* part;
  TRY(ensureT(c, S_PART, (size_t)kMaxSums * kMaxPartialBlocks, &part));
  sk->partials = part;
  sk->out = c->h_out + slot;
  sk->flag = c->h_flag;
  sk->seq = alloc_seq(&c->seq, 1);
  return GKR_OK;
}
std::vector<Trip> plan_trips(int T, uint64_t host_len, int k0) {
  std::vector<Trip> v;
  if (T <= 0) return v;
  int t = k0 < T ? k0 : T;
  v.push_back({0, t, 1ull << T});
  while (t < T && (1ull << (T - t)) > host_len) {
    const uint64_t n = 1ull << (T - t);
    int k = trip_k(n);
    if (k > T - t) k = T - t;
    v.push_back({t, k, n});
    t += k;
  }
  return v;
}
void lagrange_weights(const qm31* r, int j, qm31* E) {
  E[0] = qm31_one();
  for (int i = 0; i < j; i++) {
    const int m = 1 << i;
    for (int u = m - 1; u >= 0; u--) {
      const qm31 e = E[u];
      E[2 * u + 1] = qm31_mul(e, r[i]);
      E[2 * u] = qm31_sub(e, E[2 * u + 1]);
    }
  }
}
void trip_round_sum(const qm31* S, int K, int j, const qm31* r, qm31* out) {
  qm31 E[8];
  lagrange_weights(r, j, E);
  out[0] = out[1] = qm31_zero();
  for (int c = 0; c < (1 << K); c++) {
    const int u = c >> (K - j), b = (c >> (K - j - 1)) & 1;
    out[b] = qm31_add(out[b], qm31_mul(E[u], S[c]));
  }
}
// Launch k_trip<KIND, K> over sources sa (, sb) of length n << np with the
// np pending challenges `pend`; folded vectors to da (, db) when given; eq
// weights (KIND 1) from hi/lo; then the finisher into sink slot `slot`.
template <int KIND, int K, bool SPLIT>
static int launch_trip_k(gkr_ctx* c, const qm31* sa, const qm31* sb, uint64_t n, int np, const TripChal& al,
                         qm31* da, qm31* db, const qm31* hi, const qm31* lo, int h, const RoundSink& sk,
                         unsigned grid, uint64_t b_rows, int b_chunks, const TripWait& tw, CarriedFinish* carry_out,
                         const CarriedFinish* carry_in) {
  constexpr int NQ = TripShape<KIND, K, SPLIT>::NQ;
  uint32_t* counter = nullptr;
  uint32_t base = 0;
  if (!carry_out && GKR_TRIP_FUSED && grid <= kTripFusedMax)  // one launch: the last workgroup finishes
    TRY(arrival_counter(c, grid, &counter, &base));
  if (tw.chal) {  // launched ahead: the challenges arrive through the mailbox
    CarriedFinish none;
    memset(&none, 0, sizeof none);
    GKR_LAUNCH(c, k_mailbox_wait, dim3(1), dim3(kWaitBlock), 0, tw, carry_in ? *carry_in : none);
    TRY(check_launch(c));
  }
  GKR_LAUNCH(c, (k_trip<KIND, K, SPLIT>), dim3(grid), dim3(kBlock), 0, sa, sb, n, np, al, da, db, hi, lo, h,
                     sk, counter, base, b_rows, b_chunks, tw);
  TRY(check_launch(c));
  if (counter) return GKR_OK;
  if (carry_out) {  // the next kernel of the chain adds the rows
    carry_out->sk = sk;
    carry_out->nblocks = grid;
    carry_out->nq = NQ;
    carry_out->status = tw.chal ? tw.status : nullptr;
    carry_out->want = tw.want;
    return GKR_OK;
  }
  GKR_LAUNCH(c, k_finish_wide<NQ>, dim3(1), dim3(kFinishBlock), 0, sk, grid);
  return check_launch(c);
}
int launch_trip(gkr_ctx* c, int kind, int K, const qm31* sa, const qm31* sb, uint64_t n, int np,
                       const qm31* pend, qm31* da, qm31* db, const qm31* hi, const qm31* lo, int h, int slot,
                       RoundSink* sk, uint64_t b_rows, int b_chunks, const TripWait* tw, CarriedFinish* carry_out,
                       const CarriedFinish* carry_in) {
  if (carry_in && carry_in->nblocks && !tw)
    return fail(GKR_ERR_DEVICE, "a carried finish needs a trip launched ahead");
  if (np < 0 || np > kTripMaxK || K < 0 || K > kTripMaxK || (n >> K) == 0 || (kind == 1) != (hi != nullptr) ||
      (b_chunks && (kind != 0 || np != 0 || b_rows > n)))
    return fail(GKR_ERR_DEVICE, "bad trip (kind %d, K %d, np %d, n %llu)", kind, K, np, (unsigned long long)n);
  HostTimer ht(c, K_HOST_LAUNCH);
  TripChal al;
  memset(&al, 0, sizeof al);
  TripWait w;
  memset(&w, 0, sizeof w);
  if (tw)
    w = *tw;
  else
    for (int i = 0; i < np; i++) al.c[i] = pend[i];
  TRY(make_sink(c, sk, slot));
  // short vectors: one lane per entry and vector (KIND 0 / 1: 2n lanes, the
  // split layout of k_trip); long ones one lane per entry; up to
  // kTripMaxBlocks workgroups
  const bool split = kind != 2 && 2 * n <= kTripSplitLanes;
  unsigned grid = partial_grid(split ? 2 * n : n);
  const unsigned max_blocks = K <= 2 ? kTripMaxBlocksShort : kTripMaxBlocks;
  if (grid > max_blocks) grid = max_blocks;
  if (GKR_TRIP_FUSED && grid <= kTripFusedGrid) grid = grid < kTripFusedMax ? grid : kTripFusedMax;
  const int nvec = kind == 2 ? 1 : 2;
  TimedLaunch tl(c, kind == 0 ? K_MM_ROUND : K_EQ3_ROUND,
                 16ull * nvec * ((n << np) + (da ? n : 0)));
#define GKR_TRIP_CASE(KI, KK)                                                                                 \
  if (kind == KI && K == KK)                                                                                  \
    return split ? launch_trip_k<KI, KK, true>(c, sa, sb, n, np, al, da, db, hi, lo, h, *sk, grid, b_rows, b_chunks, w, \
                                               carry_out, carry_in)                                              \
                 : launch_trip_k<KI, KK, false>(c, sa, sb, n, np, al, da, db, hi, lo, h, *sk, grid, b_rows, b_chunks, w, \
                                                carry_out, carry_in);
  GKR_TRIP_CASE(0, 1) GKR_TRIP_CASE(0, 2) GKR_TRIP_CASE(0, 3)
  GKR_TRIP_CASE(1, 0) GKR_TRIP_CASE(1, 1) GKR_TRIP_CASE(1, 2) GKR_TRIP_CASE(1, 3)
  GKR_TRIP_CASE(2, 1) GKR_TRIP_CASE(2, 2) GKR_TRIP_CASE(2, 3)
#undef GKR_TRIP_CASE
  return fail(GKR_ERR_DEVICE, "no trip kernel for kind %d, K %d", kind, K);
}
int wait_trip(gkr_ctx* c, const RoundSink& sk, int nq, qm31* out, uint32_t want) {
  TRY(wait_result<0>(c, sk.seq, nullptr, K_HOST_WAIT, 0, want));
  const int slot = (int)(sk.out - c->h_out);
  for (int q = 0; q < nq; q++) out[q] = c->h_out[slot + q];
  return GKR_OK;
}

int fetch_q(gkr_ctx* c, const qm31* dev, int count, qm31* host_out) {
  HIP_TRY(hipMemcpyAsync(c->h_res, dev, count * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
  TRY(sync(c));
  for (int q = 0; q < count; q++) host_out[q] = c->h_res[q];
  return GKR_OK;
}
int dot_m31(gkr_ctx* c, const uint32_t* v, const qm31* eq, uint64_t n, qm31* out) {
  RoundSink sk;
  TRY(make_sink(c, &sk));
  GKR_LAUNCH(c, k_dot_m31, dim3(partial_grid(n)), dim3(kBlock), 0, v, eq, n, sk);
  TRY(launch_finish<1>(c, sk, partial_grid(n)));
  return wait_sink<1>(c, sk, out);
}
// ------------------------------------------------------------------ context ABI
extern "C" void gkr_ctx_destroy(gkr_ctx* c);
extern "C" int gkr_ctx_create(int device, gkr_ctx** out) {
  if (!out) return fail(GKR_ERR_INVALID, "null out");
  int n = 0;
  HIP_CHECK(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(GKR_ERR_INVALID, "device %d not present (%d devices)", device, n);
  HIP_CHECK(hipSetDevice(device));
  gkr_ctx* c = new gkr_ctx();
  c->device = device;
  const char* i8 = getenv("GKR_INT8_WEIGHTS");
  c->int8_weights = !(i8 && i8[0] == '0' && i8[1] == 0);  // default on; GKR_INT8_WEIGHTS=0: u32 restriction
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(GKR_ERR_DEVICE, "hipStreamCreate failed");
  }
  if (hipHostMalloc((void**)&c->h_res, 64 * sizeof(qm31), hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&c->h_out, kOutSlots * sizeof(qm31) + 128 + 2 * sizeof(Mailbox),
                    hipHostMallocCoherent | hipHostMallocMapped) !=
          hipSuccess) {
    gkr_ctx_destroy(c);
    return fail(GKR_ERR_DEVICE, "context buffer allocation failed");
  }
  if (hipHostMalloc((void**)&c->h_vec, 2 * kHandMax * sizeof(qm31), hipHostMallocCoherent | hipHostMallocMapped) !=
      hipSuccess) {
    gkr_ctx_destroy(c);
    return fail(GKR_ERR_DEVICE, "context buffer allocation failed");
  }
  {  // this device's copy of the static scratch array (gkr_sumcheck_product_noalloc)
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      gkr_ctx_destroy(c);
      return fail(GKR_ERR_DEVICE, "scratch address on device %d: %s", device, hipGetErrorString(e));
    }
    c->scratch_dev = static_cast<uint8_t*>(p);
  }
  c->h_flag = reinterpret_cast<uint32_t*>(c->h_out + kOutSlots);
  *c->h_flag = 0;
  c->mailbox = reinterpret_cast<Mailbox*>(reinterpret_cast<char*>(c->h_out) + kOutSlots * sizeof(qm31) + 128);
  c->mailbox->seq = 0;
  c->mailbox->expired = 0;
  c->vmailbox = c->mailbox + 1;
  c->vmailbox->seq = 0;
  c->vmailbox->expired = 0;
  // Launches are issued by a thread of their own unless GKR_ASYNC_LAUNCH=0
  // (the launch cost then falls on the caller's thread).
  const char* al = getenv("GKR_ASYNC_LAUNCH");
  if (!(al && al[0] == '0' && al[1] == 0)) c->launcher.reset(new Launcher(device));
  *out = c;
  return GKR_OK;
}
extern "C" void gkr_ctx_destroy(gkr_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->launcher) {  // issue what is queued, then stop the thread
    c->launcher->drain();
    c->launcher.reset();
  }
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  for (auto& p : c->pending) {
    (void)hipEventDestroy(p.e0);
    (void)hipEventDestroy(p.e1);
  }
  for (auto e : c->free_events) (void)hipEventDestroy(e);
  for (gkr_matrix* m : c->matrices) {  // matrices outliving their context keep only the handle
    if (m->owned && m->dev) (void)hipFree(m->dev);
    if (m->bplanes) (void)hipFree(m->bplanes);
    if (m->r8) (void)hipFree(m->r8);
    m->bplanes = nullptr;
    m->r8 = nullptr;
    m->dev = nullptr;
    m->ctx = nullptr;
  }
  for (gkr_qvec* v : c->qvecs) {
    if (v->dev) (void)hipFree(v->dev);
    v->dev = nullptr;
    v->ctx = nullptr;
  }
  for (int s = 0; s < S_NSLOTS; s++)
    if (c->buf[s]) (void)hipFree(c->buf[s]);
  for (auto& t : c->dev_tables) (void)hipFree(t.second);
  if (c->merkle_consts) (void)hipFree(c->merkle_consts);
  if (c->h_res) (void)hipHostFree(c->h_res);
  c->mring.reset();  // freed with the last proof record still holding a slot
  for (int s = 0; s < H_NSLOTS; s++)
    if (c->hbuf[s]) (void)hipHostFree(c->hbuf[s]);
  if (c->h_vec) (void)hipHostFree(c->h_vec);
  if (c->h_out) (void)hipHostFree(c->h_out);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}
extern "C" int gkr_ctx_debug(gkr_ctx* c, int op, uint64_t arg) {
  if (!c) return fail(GKR_ERR_INVALID, "null ctx");
  switch (op) {
    case GKR_DEBUG_HANDOVER_CANCEL: c->debug_handover_cancel = true; return GKR_OK;
    case GKR_DEBUG_HANDOVER_EXPIRE:
      if (arg == 0 || arg > kWaitSpinLimit) return fail(GKR_ERR_INVALID, "spin limit %llu", (unsigned long long)arg);
      c->debug_handover_spins = (uint32_t)arg;
      return GKR_OK;
    case GKR_DEBUG_TRIP_EXPIRE:
      if (arg == 0 || arg > kWaitSpinLimit) return fail(GKR_ERR_INVALID, "spin limit %llu", (unsigned long long)arg);
      c->debug_trip_spins = (uint32_t)arg;
      return GKR_OK;
    default: return fail(GKR_ERR_INVALID, "unknown debug op %d", op);
  }
}
extern "C" int gkr_ctx_synchronize(gkr_ctx* c) {
  if (!c) return fail(GKR_ERR_INVALID, "null ctx");
  return sync(c);
}
extern "C" int gkr_ctx_set_timing(gkr_ctx* c, int level) {
  const int enabled = level;
  if (!c) return fail(GKR_ERR_INVALID, "null ctx");
  TRY(sync(c));
  c->timing = enabled < 0 ? 0 : (enabled > 2 ? 2 : enabled);
  return GKR_OK;
}
extern "C" int gkr_ctx_kernel_time(gkr_ctx* c, int kid, double* total_ms, uint64_t* launches, uint64_t* bytes) {
  if (!c || kid < 0 || kid >= K_NKERNELS) return fail(GKR_ERR_INVALID, "bad ctx or kernel id");
  TRY(sync(c));
  if (total_ms) *total_ms = c->stats[kid].ms;
  if (launches) *launches = c->stats[kid].launches;
  if (bytes) *bytes = c->stats[kid].bytes;
  return GKR_OK;
}
extern "C" int gkr_ctx_kernel_time_by_size(gkr_ctx* c, int kid, uint64_t* bytes, double* total_ms,
                                           uint64_t* launches, size_t cap, size_t* n) {
  if (!c || kid < 0 || kid >= K_NKERNELS || !n || (cap && (!bytes || !total_ms || !launches)))
    return fail(GKR_ERR_INVALID, "bad ctx, kernel id or output");
  TRY(sync(c));
  size_t k = 0;
  for (const auto& e : c->size_stats) {  // ordered by (id, bytes)
    if (e.first.first != kid) continue;
    if (k < cap) {
      bytes[k] = e.first.second;
      total_ms[k] = e.second.ms;
      launches[k] = e.second.launches;
    }
    k++;
  }
  *n = k;
  return GKR_OK;
}
extern "C" int gkr_ctx_reset_timing(gkr_ctx* c) {
  if (!c) return fail(GKR_ERR_INVALID, "null ctx");
  TRY(sync(c));
  for (auto& s : c->stats) s = KernelStat();
  c->size_stats.clear();
  for (auto& e : c->event_seq) e = 0;
  return GKR_OK;
}

// ------------------------------------------------------------------ matrices
gkr_matrix* new_matrix(gkr_ctx* c, uint32_t* dev, uint64_t rows, uint64_t cols, bool owned);
extern "C" int gkr_matrix_upload(gkr_ctx* c, const uint32_t* host, uint64_t rows, uint64_t cols, gkr_matrix** out) {
  if (!c || !out || (!host && rows * cols)) return fail(GKR_ERR_INVALID, "null argument");
  if (rows == 0 || cols == 0) return fail(GKR_ERR_INVALID, "empty matrix %llux%llu", (unsigned long long)rows,
                                          (unsigned long long)cols);
  const uint64_t n = rows * cols;
  for (uint64_t i = 0; i < n; i++)
    if (host[i] >= P) return fail(GKR_ERR_INVALID, "matrix value %u at %llu is not a canonical M31", host[i],
                                  (unsigned long long)i);
  uint32_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, n * sizeof(uint32_t)));
  drain(c);
  hipError_t e = hipMemcpyAsync(d, host, n * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return fail(GKR_ERR_DEVICE, "matrix upload: %s", hipGetErrorString(e));
  }
  *out = new_matrix(c, d, rows, cols, true);
  return GKR_OK;
}
extern "C" int gkr_matrix_wrap_device(gkr_ctx* c, const uint32_t* dev, uint64_t rows, uint64_t cols, gkr_matrix** out) {
  if (!c || !out || !dev) return fail(GKR_ERR_INVALID, "null argument");
  if (rows == 0 || cols == 0) return fail(GKR_ERR_INVALID, "empty matrix");
  *out = new_matrix(c, const_cast<uint32_t*>(dev), rows, cols, false);
  return GKR_OK;
}
extern "C" int gkr_matrix_synthetic(gkr_ctx* c, uint64_t rows, uint64_t cols, int kind, uint64_t seed,
                                    gkr_matrix** out) {
  if (!c || !out) return fail(GKR_ERR_INVALID, "null argument");
  if (rows == 0 || cols == 0) return fail(GKR_ERR_INVALID, "empty matrix");
  if (kind != 0 && kind != 1) return fail(GKR_ERR_INVALID, "unknown synthetic kind %d", kind);
  const uint64_t n = rows * cols;
  uint32_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, n * sizeof(uint32_t)));
  GKR_LAUNCH(c, k_fill_synth, dim3(partial_grid(n) * 8), dim3(kBlock), 0, d, n, kind, seed);
  int rc = check_launch(c);
  if (rc == GKR_OK) rc = sync(c);
  if (rc != GKR_OK) {
    drain(c);
    (void)hipFree(d);
    return rc;
  }
  *out = new_matrix(c, d, rows, cols, true);
  return GKR_OK;
}
extern "C" int gkr_matrix_download(gkr_ctx* c, const gkr_matrix* m, uint32_t* host) {
  if (!c || !m || !host) return fail(GKR_ERR_INVALID, "null argument");
  if (m->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another (or a destroyed) context");
  HIP_TRY(hipMemcpyAsync(host, m->dev, m->rows * m->cols * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
  return sync(c);
}
extern "C" void gkr_matrix_free(gkr_matrix* m) {
  if (!m) return;
  if (m->ctx) {
    if (m->ctx->mm.a == m || m->ctx->mm.b == m) m->ctx->mm.valid = false;
    m->ctx->matrices.erase(m);
    drain(m->ctx);
    if ((m->owned && m->dev) || m->bplanes || m->r8) (void)hipStreamSynchronize(m->ctx->stream);
    if (m->owned && m->dev) (void)hipFree(m->dev);
    if (m->bplanes) (void)hipFree(m->bplanes);
    if (m->r8) (void)hipFree(m->r8);
  }
  delete m;
}
int drop_derived(gkr_ctx* c, gkr_matrix* m) {
  if (c->mm.a == m || c->mm.b == m) c->mm.valid = false;
  if (m->bplanes || m->r8) {
    HIP_TRY(hipStreamSynchronize(c->stream));  // no queued kernel still reads them
    if (m->bplanes) (void)hipFree(m->bplanes);
    if (m->r8) (void)hipFree(m->r8);
  }
  m->bplanes = nullptr;
  m->bnplanes = 0;
  m->r8 = nullptr;
  m->r8_nst = 0;
  m->r8_state = 0;
  m->have_root = false;
  return GKR_OK;
}
extern "C" int gkr_matrix_invalidate(gkr_ctx* c, gkr_matrix* m) {
  if (!c || !m) return fail(GKR_ERR_INVALID, "null argument");
  if (m->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another (or a destroyed) context");
  HIP_TRY(hipSetDevice(c->device));
  return drop_derived(c, m);
}
gkr_matrix* new_matrix(gkr_ctx* c, uint32_t* dev, uint64_t rows, uint64_t cols, bool owned) {
  gkr_matrix* m = new gkr_matrix{c, dev, rows, cols, owned};
  c->matrices.insert(m);
  return m;
}
extern "C" uint32_t gkr_synthetic_value(int kind, uint64_t seed, uint64_t i) { return synth_value(kind, seed, i); }

// ------------------------------------------------------------------ bandwidth reference
extern "C" int gkr_bench_copy(gkr_ctx* c, uint64_t bytes, int iters, double* copy_gbps, double* read_gbps) {
  if (!c || !copy_gbps || !read_gbps || bytes < 16 || iters < 1) return fail(GKR_ERR_INVALID, "bad argument");
  HIP_TRY(hipSetDevice(c->device));
  const uint64_t n = bytes / 16;
  uint4 *src = nullptr, *dst = nullptr;
  HIP_TRY(hipMalloc(&src, n * 16));
  if (hipMalloc(&dst, n * 16) != hipSuccess) {
    (void)hipFree(src);
    return fail(GKR_ERR_NOMEM, "copy buffers");
  }
  int rc = GKR_OK;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float ms = 0;
  const unsigned g = 256 * 8;  // 8 workgroups per CU, grid-stride
  drain(c);
  if (hipMemsetAsync(src, 1, n * 16, c->stream) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess) {
    rc = fail(GKR_ERR_DEVICE, "copy setup");
  } else {
    GKR_LAUNCH(c, k_copy16, dim3(g), dim3(kBlock), 0, src, dst, n);  // warm-up
    record_event(c, e0);
    for (int i = 0; i < iters; i++) GKR_LAUNCH(c, k_copy16, dim3(g), dim3(kBlock), 0, src, dst, n);
    record_event(c, e1);
    drain(c);
    (void)hipEventSynchronize(e1);
    (void)hipEventElapsedTime(&ms, e0, e1);
    *copy_gbps = 2.0 * n * 16 * iters / (ms * 1e-3) / 1e9;
    record_event(c, e0);
    for (int i = 0; i < iters; i++)
      GKR_LAUNCH(c, k_read16, dim3(g), dim3(kBlock), 0, src, n, (uint32_t*)dst);
    record_event(c, e1);
    drain(c);
    (void)hipEventSynchronize(e1);
    (void)hipEventElapsedTime(&ms, e0, e1);
    *read_gbps = (double)n * 16 * iters / (ms * 1e-3) / 1e9;
    if (check_launch(c) != GKR_OK) rc = fail(GKR_ERR_DEVICE, "copy kernels failed");
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(src);
  (void)hipFree(dst);
  return rc;
}



