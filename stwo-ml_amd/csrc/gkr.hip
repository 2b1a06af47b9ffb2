// Host side of the MI355X GKR prover: C ABI (include/gkr_mi355x.h), device
// context and buffers, the per-round sumcheck loop with the host Poseidon
// transcript, the LogUp activation reducer and the proof serializer.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <chrono>

#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/gkr_mi355x.h"
#include "activations.h"
#include "field.h"
#include "gemm.h"
#include "kernels.h"
#include "merkle.h"
#include "poseidon.h"
#include "poseidon9_host.h"
#include "verifier.h"

using namespace gkr;

// ------------------------------------------------------------------ errors
static thread_local std::string g_err = "";
static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
#define HIP_TRY(expr)                                                                       \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess) return fail(GKR_ERR_DEVICE, "%s: %s (%s:%d)", #expr,              \
                                      hipGetErrorString(e_), __FILE__, __LINE__);           \
  } while (0)
#define TRY(expr)             \
  do {                        \
    int rc_ = (expr);         \
    if (rc_ != GKR_OK) return rc_; \
  } while (0)

static inline qm31 Q(const gkr_qm31& x) { return qm31{x.v[0], x.v[1], x.v[2], x.v[3]}; }
static inline gkr_qm31 G(const qm31& x) {
  gkr_qm31 r;
  r.v[0] = x.a; r.v[1] = x.b; r.v[2] = x.c; r.v[3] = x.d;
  return r;
}
static inline bool canonical_q(const gkr_qm31& x) {
  return x.v[0] < P && x.v[1] < P && x.v[2] < P && x.v[3] < P;
}
static inline uint64_t next_pow2(uint64_t v) {
  uint64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}
static inline int log2_exact(uint64_t v) {
  int l = 0;
  while ((1ull << l) < v) l++;
  return l;
}
static inline felt felt_from_abi(const gkr_felt& f) { return felt_to_mont(felt_canon_from_words(f.w)); }
static inline gkr_felt felt_to_abi(const felt& m) {
  gkr_felt r;
  felt_canon_to_words(felt_from_mont(m), r.w);
  return r;
}
static bool felt_abi_canonical(const gkr_felt& f) {
  felt c = felt_canon_from_words(f.w);
  return !felt_detail::geq_p(c.l);
}

// ------------------------------------------------------------------ context
enum Slot {
  S_LI, S_LJ, S_FA0, S_FA1, S_FB0, S_FB1, S_PART, S_RES, S_EQHI, S_EQLO, S_MLE, S_EQ, S_OUT,
  S_TABLE, S_MULT, S_MIN, S_MOUT, S_D0, S_D1, S_W0, S_W1, S_E0, S_M0, S_M1, S_COLPART,
  S_MK0, S_MK1, S_MKSTEP, S_MKROOT, S_OPL, S_OPI, S_GEMMA, S_GEMMB, S_GEMMP, S_FA2, S_FB2, S_EQPARTS, S_TRIPCNT, S_LDIG, S_R8FLAG, S_EXTA, S_EXTB, S_GRAM, S_NSLOTS
};
// Timer ids: device kernels (HIP events) and host-side phases (Fiat-Shamir
// hashing inside the reducers, waiting for trip results, waiting for the
// hand-over of the last vectors).
enum KernelId { K_RESTRICT_COLS = 0, K_RESTRICT_ROWS = 1, K_MM_ROUND = 2, K_EQ3_ROUND = 3, K_LOGUP_PREP = 4,
                K_EQ_TABLE = 5, K_HOST_FS = 6, K_HOST_WAIT = 7, K_HOST_WAIT_TAIL = 8, K_MERKLE = 9,
                K_HOST_DRAW = 10, K_HOST_LAUNCH = 11, K_HOST_FINISH = 12, K_NKERNELS = 13 };
constexpr int kMaxPartialBlocks = 1024;
constexpr int kMaxSums = 64;  // values per partial row (a 3-round trip's 4^3 cross sums)
// Result slots in the coherent host area (h_out): 0 .. 63 serve the result in
// flight; results launched ahead of time and read later have their own.
constexpr int kSlotEq0 = 64;     // eq-sumcheck trip 0 (up to 64 values)
constexpr int kSlotPrep = 128;   // LogUp prepare: trace sum, input MLE
constexpr int kSlotTable = 130;  // LogUp table-side sum
constexpr int kSlotMult0 = 136;  // multiplicity sumcheck trip 0 (up to 8 values)
constexpr int kOutSlots = 192;

struct KernelStat {
  double ms = 0;
  uint64_t launches = 0;
  uint64_t bytes = 0;
};
struct PendingTiming {
  int kid;
  hipEvent_t e0, e1;
  uint64_t bytes;
};

struct MatMulCache {
  bool valid = false;
  const gkr_matrix* a = nullptr;
  const gkr_matrix* b = nullptr;
  std::vector<gkr_qm31> r_i, r_j;
  // sums of the product sumcheck's first trip over the restricted vectors
  // (rounds 0 .. trip0_k - 1), computed with the output claim
  bool have_trip0 = false;
  int trip0_k = 0;
  qm31 trip0[kMaxSums];
};

struct gkr_matrix {
  gkr_ctx* ctx;
  uint32_t* dev;
  uint64_t rows, cols;
  bool owned;
  // digit planes of the matrix as the B operand of the forward product
  // (gemm.h), built on first use; the contents of a matrix never change
  int8_t* bplanes = nullptr;
  int bnplanes = 0;
  // int8 copy for the weight-side restriction (rows of kR8Block-byte
  // blocks in k_restrict_cols8's permuted order, padded to r8_stride bytes),
  // built on first use when every entry is int8-range;
  // r8_state: 0 not yet checked, 1 copy present, -1 not int8-range
  int8_t* r8 = nullptr;
  uint64_t r8_stride = 0;
  int r8_state = 0;
};

struct gkr_qvec {
  gkr_ctx* ctx;
  qm31* dev;
  uint64_t n;
};

struct gkr_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  void* buf[S_NSLOTS] = {};
  size_t cap[S_NSLOTS] = {};
  qm31* h_res = nullptr;  // pinned result staging (64 QM31)
  uint32_t* h_mult = nullptr;  // pinned copy of the LogUp multiplicities
  qm31* h_vec = nullptr;       // coherent pinned: vectors handed over by k_handover (2 x kHandMax)
  size_t h_mult_cap = 0;
  qm31* h_out = nullptr;      // coherent pinned: results delivered by kernels (RoundSink)
  uint32_t* h_flag = nullptr; // coherent pinned: sequence number of the last delivery
  Mailbox* mailbox = nullptr;  // coherent pinned: challenges posted to persistent tail kernels
  uint32_t seq = 0;            // last result sequence number handed out
  uint32_t mb_seq = 0;         // last mailbox sequence number handed out
  int timing = 0;  // 0 off; 1: k_restrict_cols events + host timers; 2: events on every timed kernel
  KernelStat stats[K_NKERNELS];
  std::vector<PendingTiming> pending;
  std::vector<hipEvent_t> free_events;
  MatMulCache mm;
  std::map<uint64_t, std::vector<uint32_t>> tables;  // (tag << 32 | log) -> table outputs
  std::set<gkr_matrix*> matrices;  // live matrices; detached when the context is destroyed
  std::set<gkr_qvec*> qvecs;       // live QM31 vectors; detached likewise
  uint64_t table_on_device = 0;    // (tag << 32 | log) of the table held in S_TABLE, 0 = none
  MerkleConsts* merkle_consts = nullptr;  // device copy, built on first use
  bool fb_pending = false;  // f_b of the last restriction still as column-chunk partials (S_COLPART)
  uint64_t fb_rows = 0, fb_pk = 0;
  int fb_chunks = 0;
  uint32_t trip_count = 0;         // value of the fused trips' arrival counter (S_TRIPCNT) after the queued launches
  bool trip_count_valid = false;   // false: zero the counter before the next fused trip
  bool int8_weights = false;       // GKR_INT8_WEIGHTS=1 at creation: int8 weight-side restriction
  // allocation-free mode (gkr_sumcheck_product_noalloc): ensure() hands out
  // the partial rows and the arrival counter from the device's static
  // scratch array (scratch_dev: its address on this context's device) and
  // refuses every other slot
  uint8_t* scratch_dev = nullptr;
  bool noalloc = false;
  // test hooks (gkr_ctx_debug), each consumed by the next hand-over
  bool debug_handover_cancel = false;  // the host leaves before posting the challenges
  uint32_t debug_handover_spins = 0;   // nonzero: the kernel's bounded wait, posted only after it expired
};

// ------------------------------------------------------------------ static scratch (allocation-free entry point)
// Device memory of gkr_sumcheck_product_noalloc, one copy per GPU for the
// life of the process: the two fold levels of each vector (n/2 and n/4
// entries), the trips' partial rows and their arrival counter.  Host code
// never uses the array's name as an address: gkr_ctx_create looks up its
// address on the context's device (hipGetSymbolAddress) and everything
// else goes through gkr_ctx::scratch_dev.
constexpr uint64_t kNoAllocMaxN = 1ull << 20;  // longest vectors of the allocation-free sumcheck
constexpr size_t kScratchFold1 = (kNoAllocMaxN / 2) * sizeof(qm31);
constexpr size_t kScratchFold2 = (kNoAllocMaxN / 4) * sizeof(qm31);
constexpr size_t kScratchOffA1 = 0, kScratchOffB1 = kScratchFold1, kScratchOffA2 = 2 * kScratchFold1,
                 kScratchOffB2 = 2 * kScratchFold1 + kScratchFold2, kScratchOffPart = 2 * kScratchFold1 + 2 * kScratchFold2;
constexpr size_t kScratchPartBytes = (size_t)kMaxSums * kMaxPartialBlocks * sizeof(qm31);
constexpr size_t kScratchOffCount = kScratchOffPart + kScratchPartBytes;
constexpr size_t kScratchBytes = kScratchOffCount + 256;  // 25 MiB + 256 B
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

static int ensure(gkr_ctx* c, Slot s, size_t bytes, void** out) {
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
    if (s == S_TABLE) c->table_on_device = 0;
    if (s == S_TRIPCNT) c->trip_count_valid = false;  // fresh memory must be zeroed
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
template <typename T>
static int ensureT(gkr_ctx* c, Slot s, size_t count, T** out) {
  void* p;
  TRY(ensure(c, s, count * sizeof(T), &p));
  *out = (T*)p;
  return GKR_OK;
}

static int ensure_host_mult(gkr_ctx* c, uint64_t n) {
  if (c->h_mult_cap >= n) return GKR_OK;
  if (c->h_mult) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    (void)hipHostFree(c->h_mult);
    c->h_mult = nullptr;
    c->h_mult_cap = 0;
  }
  HIP_TRY(hipHostMalloc((void**)&c->h_mult, n * sizeof(uint32_t), hipHostMallocDefault));
  c->h_mult_cap = n;
  return GKR_OK;
}

static hipEvent_t get_event(gkr_ctx* c) {
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
struct TimedLaunch {
  gkr_ctx* c;
  int kid;
  uint64_t bytes;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  TimedLaunch(gkr_ctx* c_, int kid_, uint64_t bytes_) : c(c_), kid(kid_), bytes(bytes_) {
    if (c->timing >= 2 || (c->timing == 1 && (kid == K_RESTRICT_COLS || kid == K_RESTRICT_ROWS || kid == K_MERKLE))) {
      e0 = get_event(c);
      e1 = get_event(c);
      if (e0) (void)hipEventRecord(e0, c->stream);
    }
  }
  ~TimedLaunch() {
    if (e0 && e1) {
      (void)hipEventRecord(e1, c->stream);
      c->pending.push_back({kid, e0, e1, bytes});
    }
  }
};
struct HostTimer {
  gkr_ctx* c;
  int kid;
  std::chrono::steady_clock::time_point t0;
  HostTimer(gkr_ctx* c_, int kid_) : c(c_), kid(kid_) {
    if (c->timing) t0 = std::chrono::steady_clock::now();
  }
  ~HostTimer() {
    if (c->timing) {
      c->stats[kid].ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
      c->stats[kid].launches++;
    }
  }
};
static void collect_timing(gkr_ctx* c) {
  for (auto& p : c->pending) {
    float ms = 0;
    if (hipEventElapsedTime(&ms, p.e0, p.e1) == hipSuccess) {
      c->stats[p.kid].ms += ms;
      c->stats[p.kid].launches++;
      c->stats[p.kid].bytes += p.bytes;
    }
    c->free_events.push_back(p.e0);
    c->free_events.push_back(p.e1);
  }
  c->pending.clear();
}
static int sync(gkr_ctx* c) {
  HIP_TRY(hipStreamSynchronize(c->stream));
  if (c->timing) collect_timing(c);
  return GKR_OK;
}
static int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GKR_ERR_DEVICE, "kernel launch: %s", hipGetErrorString(e));
  return GKR_OK;
}
static inline unsigned grid_for(uint64_t n, uint64_t per_block = kBlock) {
  uint64_t g = (n + per_block - 1) / per_block;
  return (unsigned)(g == 0 ? 1 : g);
}
static inline unsigned partial_grid(uint64_t n) {
  uint64_t g = (n + kBlock - 1) / kBlock;
  if (g > kMaxPartialBlocks) g = kMaxPartialBlocks;
  return (unsigned)(g == 0 ? 1 : g);
}

static PointArg make_point(const qm31* r, int n) {
  PointArg p;
  memset(&p, 0, sizeof p);
  p.n = n;
  for (int l = 0; l < n; l++) {
    p.r[l] = r[l];
    p.omr[l] = qm31_sub(qm31_one(), r[l]);
  }
  return p;
}

// eq(r, x) for x < count (r[0] on the most significant bit of x).
static int eq_table(gkr_ctx* c, const qm31* r, int n, uint64_t count, qm31* out) {
  if (n > kMaxVars) return fail(GKR_ERR_INVALID, "eq table: %d variables exceeds %d", n, kMaxVars);
  PointArg pt = make_point(r, n);
  TimedLaunch t(c, K_EQ_TABLE, 16 * count);
  if (n <= 10) {
    hipLaunchKernelGGL(k_eq_direct, dim3(grid_for(count)), dim3(kBlock), 0, c->stream, pt, count, out);
    return check_launch();
  }
  const int h = n / 2;
  qm31 *hi, *lo;
  TRY(ensureT(c, S_EQHI, 1ull << (n - h), &hi));
  TRY(ensureT(c, S_EQLO, 1ull << h, &lo));
  hipLaunchKernelGGL(k_eq_tables, dim3(grid_for((1ull << (n - h)) + (1ull << h))), dim3(kBlock), 0, c->stream, pt, h,
                     hi, lo);
  TRY(check_launch());
  hipLaunchKernelGGL(k_eq_combine, dim3(grid_for(count)), dim3(kBlock), 0, c->stream, hi, lo, h, count, out);
  return check_launch();
}

// Result and mailbox sequence numbers come in consecutive ranges and restart
// at 1 before they reach the cancel code reserved at the top of the u32 range
// (kWaitCancel); waits compare them modulo 2^32.
constexpr uint32_t kSeqLimit = 0xFFFFFF00u;
static uint32_t alloc_seq(uint32_t* counter, uint32_t n) {
  if (*counter >= kSeqLimit - n) *counter = 0;
  const uint32_t base = *counter + 1;
  *counter += n;
  return base;
}
// Partial rows for a reducing kernel.  `slot` selects where in the coherent
// host buffer the finisher writes its NQ results: slots 0-3 serve the round
// in flight, higher slots hold results launched ahead of time and read
// later.  The partial rows are shared: each finisher consumes them before the
// next reducing kernel on the stream overwrites them.
static int make_sink(gkr_ctx* c, RoundSink* sk, int slot = 0) {
  qm31* part;
  TRY(ensureT(c, S_PART, (size_t)kMaxSums * kMaxPartialBlocks, &part));
  sk->partials = part;
  sk->out = c->h_out + slot;
  sk->flag = c->h_flag;
  sk->seq = alloc_seq(&c->seq, 1);
  return GKR_OK;
}
// Launch the one-workgroup finisher that adds `nblocks` partial rows and
// delivers the NQ results (after a multi-workgroup reducing kernel).
template <int NQ>
static int launch_finish(gkr_ctx* c, const RoundSink& sk, unsigned nblocks) {
  TRY(check_launch());
  hipLaunchKernelGGL(k_finish<NQ>, dim3(1), dim3(kBlock), 0, c->stream, sk, (uint32_t)nblocks);
  return check_launch();
}
// Wait until result `seq` has been published and copy NQ values.  The wait
// spins on the coherent flag and never blocks on the stream (a hand-over
// kernel queued behind the result may be waiting for the host): from time to
// time it queries the stream, so a device error, or a drained stream without
// the result, is reported; after kWaitWallSeconds it gives up.  hand_mb != 0:
// the result comes from the hand-over waiting for mailbox sequence hand_mb,
// whose expiry is reported at once.
constexpr double kWaitWallSeconds = 60.0;
template <int NQ>
static int wait_result(gkr_ctx* c, uint32_t seq, qm31* host_out, int timer = K_HOST_WAIT_TAIL, int slot = 0,
                       uint32_t hand_mb = 0) {
  TRY(check_launch());
  HostTimer ht(c, timer);
  volatile uint32_t* flag = c->h_flag;
  volatile uint32_t* expired = &c->mailbox->expired;
  std::chrono::steady_clock::time_point t0;
  // the flag only moves forward (mod 2^32): a later delivery implies this one
  for (uint64_t spins = 0; (int32_t)(*flag - seq) < 0; spins++) {
    if (hand_mb && *expired == hand_mb)
      return fail(GKR_ERR_DEVICE, "hand-over kernel stopped waiting for the challenges (mailbox %u)", hand_mb);
    if ((spins & 0xFFFF) != 0xFFFF) continue;
    if (spins == 0xFFFF) t0 = std::chrono::steady_clock::now();
    const hipError_t e = hipStreamQuery(c->stream);
    if (e == hipSuccess) {
      if ((int32_t)(*flag - seq) >= 0) break;
      return fail(GKR_ERR_DEVICE, "device result %u not delivered (stream drained)", seq);
    }
    if (e != hipErrorNotReady) return fail(GKR_ERR_DEVICE, "waiting for device result %u: %s", seq, hipGetErrorString(e));
    if (std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kWaitWallSeconds)
      return fail(GKR_ERR_DEVICE, "device result %u not delivered after %.0f s", seq, kWaitWallSeconds);
  }
  __atomic_thread_fence(__ATOMIC_ACQUIRE);
  for (int q = 0; q < NQ; q++) host_out[q] = c->h_out[slot + q];
  return GKR_OK;
}
template <int NQ>
static int wait_sink(gkr_ctx* c, const RoundSink& sk, qm31* host_out) {
  return wait_result<NQ>(c, sk.seq, host_out, K_HOST_WAIT, (int)(sk.out - c->h_out));
}
// Host side of a k_handover launch: posts the last trip's challenges into
// the mailbox and receives the folded vectors.  If the host leaves before
// posting (an error), the guard posts the cancel code so the kernel stops
// waiting at once, drains the stream, and clears the mailbox so that the
// next hand-over does not read the cancel code.
struct HandoverSession {
  gkr_ctx* c;
  uint32_t res_seq = 0, mb_seq = 0;
  bool launched = false, done = false;
  bool cancel_before_post = false;  // test hook (gkr_ctx_debug): leave without posting
  bool hold_post = false;           // test hook (gkr_ctx_debug): post only after the kernel's wait expired
  explicit HandoverSession(gkr_ctx* c_) : c(c_) {}
  // Launch k_handover<NV> over the vectors a (, b) of length len, to be folded by k challenges.
  template <int NV>
  int launch(const qm31* a, const qm31* b, uint64_t len, int k) {
    HostTimer ht(c, K_HOST_LAUNCH);
    if (len > (uint64_t)kHandMax || k < 0 || k > kTripMaxK || (len >> k) == 0)
      return fail(GKR_ERR_DEVICE, "hand-over of %llu entries folded %d times", (unsigned long long)len, k);
    res_seq = alloc_seq(&c->seq, 1);
    mb_seq = alloc_seq(&c->mb_seq, 1);
    uint32_t spin_limit = kWaitSpinLimit;
    if (c->debug_handover_spins) {  // test hook: a short bounded wait that expires before the post
      spin_limit = c->debug_handover_spins;
      c->debug_handover_spins = 0;
      hold_post = true;
    }
    if (c->debug_handover_cancel) {
      cancel_before_post = true;
      c->debug_handover_cancel = false;
    }
    hipLaunchKernelGGL(k_handover<NV>, dim3(1), dim3(kBlock), 0, c->stream, a, b, (uint32_t)len, k, c->mailbox,
                       mb_seq, spin_limit, c->h_vec, c->h_flag, res_seq);
    launched = true;
    return check_launch();
  }
  int post(const qm31* chal, int k) {
    if (cancel_before_post) return fail(GKR_ERR_DEVICE, "hand-over cancelled before the challenges were posted");
    if (hold_post) {
      const auto t0 = std::chrono::steady_clock::now();
      volatile uint32_t* expired = &c->mailbox->expired;
      while (*expired != mb_seq && std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < 10.0) {
      }
    }
    for (int r = 0; r < k; r++) c->mailbox->alpha[r] = chal[r];
    __atomic_store_n(&c->mailbox->seq, mb_seq, __ATOMIC_RELEASE);
    return GKR_OK;
  }
  // Wait for the folded vectors: count vectors of len entries each.
  int fetch(uint64_t len, int count, std::vector<qm31>* out) {
    TRY(wait_result<0>(c, res_seq, nullptr, K_HOST_WAIT_TAIL, 0, mb_seq));
    for (int v = 0; v < count; v++) out[v].assign(c->h_vec + v * len, c->h_vec + (v + 1) * len);
    done = true;
    return GKR_OK;
  }
  ~HandoverSession() {
    if (launched && !done) {
      __atomic_store_n(&c->mailbox->seq, kWaitCancel, __ATOMIC_RELEASE);
      (void)hipStreamSynchronize(c->stream);
      __atomic_store_n(&c->mailbox->seq, 0u, __ATOMIC_RELEASE);  // 0 is never a wanted sequence
    }
  }
};

// ------------------------------------------------------------------ multi-round trips (host side)
// A sumcheck over 2^T entries runs as a few device trips of K <= 3 rounds
// each (k_trip: one launch plus the finisher per trip), then k_handover
// folds the last trip's vectors and the host finishes the rounds on vectors
// of at most host_len entries.  The first trip covers min(k0, T) rounds;
// later trips cover trip_k(n) rounds: a trip's sums cost 2^K products per
// entry, so trips over long vectors (bound by HBM and VALU, not by launch
// latency) take fewer rounds each.  The loop ends once the next trip's
// vectors would fit the host, so the last trip's vectors have at most
// host_len * 2^K <= kHandMax entries (host_len <= 256).
struct Trip {
  int t, K;    // rounds t .. t + K - 1
  uint64_t n;  // vector length at round t
};
#ifndef GKR_TRIP_BIG
#define GKR_TRIP_BIG (1ull << 16)
#endif
constexpr uint64_t kTripBig = GKR_TRIP_BIG;
#ifndef GKR_TRIP_HUGE
#define GKR_TRIP_HUGE (1ull << 20)
#endif
constexpr uint64_t kTripHuge = GKR_TRIP_HUGE;
// Rounds per trip over a vector of n entries: 3 up to kTripBig, 2 up to kTripHuge, then 1.
static inline int trip_k(uint64_t n) { return n > kTripHuge ? 1 : n > kTripBig ? 2 : 3; }
#ifndef GKR_TRIP_MAX_BLOCKS
#define GKR_TRIP_MAX_BLOCKS 512
#endif
constexpr unsigned kTripMaxBlocks = GKR_TRIP_MAX_BLOCKS;  // partial rows per trip (the finisher adds them)
#ifndef GKR_TRIP_MAX_BLOCKS_SHORT
#define GKR_TRIP_MAX_BLOCKS_SHORT 1024
#endif
constexpr unsigned kTripMaxBlocksShort = GKR_TRIP_MAX_BLOCKS_SHORT;  // the same for trips of at most 2 rounds
static_assert(GKR_TRIP_MAX_BLOCKS_SHORT <= kMaxPartialBlocks && GKR_TRIP_MAX_BLOCKS <= kMaxPartialBlocks,
              "trip partial rows exceed the partial buffer");
// Trips whose one-entry-per-thread grid is at most kTripFusedGrid workgroups
// run on at most kTripFusedMax workgroups and finish in the kernel itself.
#ifndef GKR_TRIP_FUSED
#define GKR_TRIP_FUSED 1
#endif
#ifndef GKR_TRIP_FUSED_GRID
#define GKR_TRIP_FUSED_GRID 256
#endif
constexpr unsigned kTripFusedGrid = GKR_TRIP_FUSED_GRID;
static std::vector<Trip> plan_trips(int T, uint64_t host_len, int k0) {
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
static inline int trip_nq(int kind, int K) { return kind == 2 ? (1 << K) : (1 << (2 * K)); }
// eqlin(z, X) = (1 - z)(1 - X) + z X, the multilinear eq factor of one coordinate.
static inline qm31 eqlin(const qm31& z, const qm31& x) {
  const qm31 one = qm31_one();
  return qm31_add(qm31_mul(qm31_sub(one, z), qm31_sub(one, x)), qm31_mul(z, x));
}
// Lagrange weights E[u] (u < 2^j, first challenge on the MSB) of r[0..j).
static void lagrange_weights(const qm31* r, int j, qm31* E) {
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
// Round j (0-based within the trip) of a product-type trip from its cross sums
// G (4^K, row-major over sub-vectors c, c'), evaluated at the nx points xs:
//   p(X) = sum_v sum_{u,u',b,b'} E[u] E[u'] eqlin(X,b) eqlin(X,b') G[(u,b,v)][(u',b',v)]
// with E the Lagrange weights of the trip's challenges r[0..j) and v running
// over the trip's later variables.  For the eq-sumcheck (zt given: the claim
// coordinates of the trip's variables; cpre: prod of eqlin(z_l, r_l) over all
// earlier rounds) the eq factors are applied:
//   p(X) *= cpre * prod_{i<j} eqlin(zt_i, r_i) * eqlin(zt_j, X),  v weighted by eqlin(zt, v).
static void trip_round_gram(const qm31* G, int K, int j, const qm31* r, int nx, const qm31* xs, qm31* out,
                            const qm31* zt, const qm31& cpre) {
  const int nu = 1 << j, nv = 1 << (K - j - 1), sh_b = K - j - 1, dim = 1 << K;
  qm31 E[8];
  lagrange_weights(r, j, E);
  qm31 H[2][2] = {{qm31_zero(), qm31_zero()}, {qm31_zero(), qm31_zero()}};
  for (int v = 0; v < nv; v++) {
    qm31 ez = qm31_one();
    if (zt)
      for (int i = 0; i < K - j - 1; i++)
        ez = qm31_mul(ez, ((v >> (K - j - 2 - i)) & 1) ? zt[j + 1 + i] : qm31_sub(qm31_one(), zt[j + 1 + i]));
    for (int b = 0; b < 2; b++)
      for (int b2 = 0; b2 < 2; b2++) {
        qm31 acc = qm31_zero();
        for (int u = 0; u < nu; u++) {
          const int row = (u << (K - j)) | (b << sh_b) | v;
          qm31 inner = qm31_zero();
          for (int u2 = 0; u2 < nu; u2++) {
            const int col = (u2 << (K - j)) | (b2 << sh_b) | v;
            inner = qm31_add(inner, qm31_mul(E[u2], G[row * dim + col]));
          }
          acc = qm31_add(acc, qm31_mul(E[u], inner));
        }
        H[b][b2] = qm31_add(H[b][b2], zt ? qm31_mul(ez, acc) : acc);
      }
  }
  qm31 pre = cpre;
  if (zt)
    for (int i = 0; i < j; i++) pre = qm31_mul(pre, eqlin(zt[i], r[i]));
  for (int k = 0; k < nx; k++) {
    const qm31 x = xs[k];
    const qm31 e0 = qm31_sub(qm31_one(), x), e1 = x;
    qm31 p = qm31_add(qm31_mul(qm31_mul(e0, e0), H[0][0]),
                      qm31_add(qm31_mul(qm31_mul(e0, e1), qm31_add(H[0][1], H[1][0])), qm31_mul(qm31_mul(e1, e1), H[1][1])));
    if (zt) p = qm31_mul(p, qm31_mul(pre, eqlin(zt[j], x)));
    out[k] = p;
  }
}
// Round j of a degree-1 trip from its 2^K sums S: p(0), p(1).
static void trip_round_sum(const qm31* S, int K, int j, const qm31* r, qm31* out) {
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
                         unsigned grid, uint64_t b_rows, int b_chunks) {
  uint32_t* counter = nullptr;
  uint32_t base = 0;
  if (GKR_TRIP_FUSED && grid <= kTripFusedMax) {  // one launch: the last workgroup finishes
    TRY(ensureT(c, S_TRIPCNT, 1, &counter));
    if (!c->trip_count_valid) {
      hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(64), 0, c->stream, counter, 1u);
      TRY(check_launch());
      c->trip_count = 0;
      c->trip_count_valid = true;
    }
    base = c->trip_count;
    c->trip_count += grid;
  }
  hipLaunchKernelGGL((k_trip<KIND, K, SPLIT>), dim3(grid), dim3(kBlock), 0, c->stream, sa, sb, n, np, al, da, db, hi, lo, h,
                     sk, counter, base, b_rows, b_chunks);
  TRY(check_launch());
  if (counter) return GKR_OK;
  constexpr int NQ = TripShape<KIND, K, SPLIT>::NQ;
  hipLaunchKernelGGL(k_finish_wide<NQ>, dim3(1), dim3(kFinishBlock), 0, c->stream, sk, grid);
  return check_launch();
}
static int launch_trip(gkr_ctx* c, int kind, int K, const qm31* sa, const qm31* sb, uint64_t n, int np,
                       const qm31* pend, qm31* da, qm31* db, const qm31* hi, const qm31* lo, int h, int slot,
                       RoundSink* sk, uint64_t b_rows = 0, int b_chunks = 0) {
  if (np < 0 || np > kTripMaxK || K < 0 || K > kTripMaxK || (n >> K) == 0 || (kind == 1) != (hi != nullptr) ||
      (b_chunks && (kind != 0 || np != 0 || b_rows > n)))
    return fail(GKR_ERR_DEVICE, "bad trip (kind %d, K %d, np %d, n %llu)", kind, K, np, (unsigned long long)n);
  HostTimer ht(c, K_HOST_LAUNCH);
  TripChal al;
  memset(&al, 0, sizeof al);
  for (int i = 0; i < np; i++) al.c[i] = pend[i];
  TRY(make_sink(c, sk, slot));
  // short vectors: one lane per entry and vector (KIND 0 / 1: 2n lanes, the
  // split layout of k_trip); long ones one lane per entry; up to
  // kTripMaxBlocks workgroups
  const bool split = kind != 2 && 2 * n <= (uint64_t)kTripFusedGrid * kBlock;
  unsigned grid = partial_grid(split ? 2 * n : n);
  const unsigned max_blocks = K <= 2 ? kTripMaxBlocksShort : kTripMaxBlocks;
  if (grid > max_blocks) grid = max_blocks;
  if (GKR_TRIP_FUSED && grid <= kTripFusedGrid) grid = grid < kTripFusedMax ? grid : kTripFusedMax;
  const int nvec = kind == 2 ? 1 : 2;
  TimedLaunch tl(c, kind == 0 ? K_MM_ROUND : K_EQ3_ROUND,
                 16ull * nvec * ((n << np) + (da ? n : 0)));
#define GKR_TRIP_CASE(KI, KK)                                                                                 \
  if (kind == KI && K == KK)                                                                                  \
    return split ? launch_trip_k<KI, KK, true>(c, sa, sb, n, np, al, da, db, hi, lo, h, *sk, grid, b_rows, b_chunks) \
                 : launch_trip_k<KI, KK, false>(c, sa, sb, n, np, al, da, db, hi, lo, h, *sk, grid, b_rows, b_chunks);
  GKR_TRIP_CASE(0, 1) GKR_TRIP_CASE(0, 2) GKR_TRIP_CASE(0, 3)
  GKR_TRIP_CASE(1, 0) GKR_TRIP_CASE(1, 1) GKR_TRIP_CASE(1, 2) GKR_TRIP_CASE(1, 3)
  GKR_TRIP_CASE(2, 1) GKR_TRIP_CASE(2, 2) GKR_TRIP_CASE(2, 3)
#undef GKR_TRIP_CASE
  return fail(GKR_ERR_DEVICE, "no trip kernel for kind %d, K %d", kind, K);
}
// Wait for a trip's nq sums.
static int wait_trip(gkr_ctx* c, const RoundSink& sk, int nq, qm31* out) {
  TRY(wait_result<0>(c, sk.seq, nullptr, K_HOST_WAIT, 0));
  const int slot = (int)(sk.out - c->h_out);
  for (int q = 0; q < nq; q++) out[q] = c->h_out[slot + q];
  return GKR_OK;
}

static int fetch_q(gkr_ctx* c, const qm31* dev, int count, qm31* host_out) {
  HIP_TRY(hipMemcpyAsync(c->h_res, dev, count * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
  TRY(sync(c));
  for (int q = 0; q < count; q++) host_out[q] = c->h_res[q];
  return GKR_OK;
}

// sum_i v[i] * eq[i] (v M31-valued, length n).
static int dot_m31(gkr_ctx* c, const uint32_t* v, const qm31* eq, uint64_t n, qm31* out) {
  RoundSink sk;
  TRY(make_sink(c, &sk));
  hipLaunchKernelGGL(k_dot_m31, dim3(partial_grid(n)), dim3(kBlock), 0, c->stream, v, eq, n, sk);
  TRY(launch_finish<1>(c, sk, partial_grid(n)));
  return wait_sink<1>(c, sk, out);
}

// ------------------------------------------------------------------ error / version
extern "C" const char* gkr_last_error(void) { return g_err.c_str(); }
extern "C" const char* gkr_version(void) { return "gkr_mi355x 0.1 (gfx950)"; }

// ------------------------------------------------------------------ Poseidon ABI
extern "C" int gkr_hades_permute(gkr_felt state[3]) {
  if (!state) return fail(GKR_ERR_INVALID, "null state");
  felt s[3];
  for (int i = 0; i < 3; i++) {
    if (!felt_abi_canonical(state[i])) return fail(GKR_ERR_INVALID, "non-canonical felt");
    s[i] = felt_from_abi(state[i]);
  }
  hades_permute(s);
  for (int i = 0; i < 3; i++) state[i] = felt_to_abi(s[i]);
  return GKR_OK;
}
extern "C" int gkr_poseidon_hash(const gkr_felt* a, const gkr_felt* b, gkr_felt* out) {
  if (!a || !b || !out) return fail(GKR_ERR_INVALID, "null argument");
  if (!felt_abi_canonical(*a) || !felt_abi_canonical(*b)) return fail(GKR_ERR_INVALID, "non-canonical felt");
  *out = felt_to_abi(poseidon_hash(felt_from_abi(*a), felt_from_abi(*b)));
  return GKR_OK;
}
extern "C" int gkr_poseidon_hash_many(const gkr_felt* in, size_t n, gkr_felt* out) {
  if ((!in && n) || !out) return fail(GKR_ERR_INVALID, "null argument");
  std::vector<felt> v(n);
  for (size_t i = 0; i < n; i++) {
    if (!felt_abi_canonical(in[i])) return fail(GKR_ERR_INVALID, "non-canonical felt at %zu", i);
    v[i] = felt_from_abi(in[i]);
  }
  *out = felt_to_abi(poseidon_hash_many(v.data(), (int)n));
  return GKR_OK;
}

// ------------------------------------------------------------------ channel ABI
struct gkr_channel {
  PoseidonChannel ch;
};
extern "C" int gkr_channel_new(gkr_channel** out) {
  if (!out) return fail(GKR_ERR_INVALID, "null out");
  *out = new gkr_channel();
  return GKR_OK;
}
extern "C" void gkr_channel_free(gkr_channel* ch) { delete ch; }
extern "C" int gkr_channel_clone(const gkr_channel* ch, gkr_channel** out) {
  if (!ch || !out) return fail(GKR_ERR_INVALID, "null argument");
  *out = new gkr_channel(*ch);
  return GKR_OK;
}
#define CH_CHECK(ch) \
  if (!(ch)) return fail(GKR_ERR_INVALID, "null channel")
extern "C" int gkr_channel_mix_u64(gkr_channel* ch, uint64_t v) {
  CH_CHECK(ch);
  ch->ch.mix_u64(v);
  return GKR_OK;
}
extern "C" int gkr_channel_mix_felt(gkr_channel* ch, const gkr_felt* v) {
  CH_CHECK(ch);
  if (!v || !felt_abi_canonical(*v)) return fail(GKR_ERR_INVALID, "felt252 value not canonical (must be < p)");
  ch->ch.mix_felt(felt_from_abi(*v));
  return GKR_OK;
}
extern "C" int gkr_channel_mix_secure_field(gkr_channel* ch, const gkr_qm31* v) {
  CH_CHECK(ch);
  if (!v || !canonical_q(*v)) return fail(GKR_ERR_INVALID, "qm31 value not canonical (each word must be < 2^31 - 1)");
  ch->ch.mix_secure_field(Q(*v));
  return GKR_OK;
}
extern "C" int gkr_channel_mix_felts(gkr_channel* ch, const gkr_qm31* v, size_t n) {
  CH_CHECK(ch);
  if (!v && n) return fail(GKR_ERR_INVALID, "null values");
  std::vector<qm31> q(n);
  for (size_t i = 0; i < n; i++) {
    if (!canonical_q(v[i])) return fail(GKR_ERR_INVALID, "non-canonical qm31 at %zu", i);
    q[i] = Q(v[i]);
  }
  ch->ch.mix_felts(q.data(), (int)n);
  return GKR_OK;
}
extern "C" int gkr_channel_mix_poly_coeffs(gkr_channel* ch, const gkr_qm31 c[3]) {
  CH_CHECK(ch);
  if (!c) return fail(GKR_ERR_INVALID, "null coefficients");
  for (int i = 0; i < 3; i++)
    if (!canonical_q(c[i])) return fail(GKR_ERR_INVALID, "non-canonical coefficient");
  ch->ch.mix_poly_coeffs(Q(c[0]), Q(c[1]), Q(c[2]));
  return GKR_OK;
}
extern "C" int gkr_channel_mix_poly_coeffs_deg3(gkr_channel* ch, const gkr_qm31 c[4]) {
  CH_CHECK(ch);
  if (!c) return fail(GKR_ERR_INVALID, "null coefficients");
  for (int i = 0; i < 4; i++)
    if (!canonical_q(c[i])) return fail(GKR_ERR_INVALID, "non-canonical coefficient");
  ch->ch.mix_poly_coeffs_deg3(Q(c[0]), Q(c[1]), Q(c[2]), Q(c[3]));
  return GKR_OK;
}
extern "C" int gkr_channel_draw_felt252(gkr_channel* ch, gkr_felt* out) {
  CH_CHECK(ch);
  if (!out) return fail(GKR_ERR_INVALID, "null out");
  *out = felt_to_abi(ch->ch.draw_felt252());
  return GKR_OK;
}
extern "C" int gkr_channel_draw_qm31(gkr_channel* ch, gkr_qm31* out) {
  CH_CHECK(ch);
  if (!out) return fail(GKR_ERR_INVALID, "null out");
  *out = G(ch->ch.draw_qm31());
  return GKR_OK;
}
extern "C" int gkr_channel_draw_qm31s(gkr_channel* ch, size_t n, gkr_qm31* out) {
  CH_CHECK(ch);
  if (!out && n) return fail(GKR_ERR_INVALID, "null out");
  std::vector<qm31> q(n);
  ch->ch.draw_qm31s(q.data(), n);
  for (size_t i = 0; i < n; i++) out[i] = G(q[i]);
  return GKR_OK;
}
extern "C" int gkr_channel_digest(const gkr_channel* ch, gkr_felt* out) {
  CH_CHECK(ch);
  if (!out) return fail(GKR_ERR_INVALID, "null out");
  *out = felt_to_abi(ch->ch.digest);
  return GKR_OK;
}
extern "C" uint64_t gkr_channel_hash_count(const gkr_channel* ch) { return ch ? ch->ch.hash_count : 0; }
extern "C" int gkr_channel_export(const gkr_channel* ch, uint32_t state[11]) {
  CH_CHECK(ch);
  if (!state) return fail(GKR_ERR_INVALID, "null state");
  ch->ch.export_state(state);
  return GKR_OK;
}
extern "C" int gkr_channel_import(gkr_channel* ch, const uint32_t state[11]) {
  CH_CHECK(ch);
  if (!state) return fail(GKR_ERR_INVALID, "null state");
  gkr_felt f;
  memcpy(f.w, state, sizeof f.w);
  if (!felt_abi_canonical(f)) return fail(GKR_ERR_INVALID, "non-canonical digest");
  ch->ch.import_state(state);
  return GKR_OK;
}
extern "C" int gkr_seed_channel(gkr_channel* ch, uint64_t num_layers, uint64_t in_rows, uint64_t in_cols,
                                const gkr_felt* policy_commitment) {
  CH_CHECK(ch);
  ch->ch.mix_u64(num_layers);
  ch->ch.mix_u64(in_rows);
  ch->ch.mix_u64(in_cols);
  if (policy_commitment) {
    if (!felt_abi_canonical(*policy_commitment)) return fail(GKR_ERR_INVALID, "non-canonical policy commitment");
    bool zero = true;
    for (int i = 0; i < 8; i++) zero = zero && policy_commitment->w[i] == 0;
    if (!zero) ch->ch.mix_felt(felt_from_abi(*policy_commitment));
  }
  return GKR_OK;
}

// ------------------------------------------------------------------ context ABI
extern "C" void gkr_ctx_destroy(gkr_ctx* c);
extern "C" int gkr_ctx_create(int device, gkr_ctx** out) {
  if (!out) return fail(GKR_ERR_INVALID, "null out");
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(GKR_ERR_INVALID, "device %d not present (%d devices)", device, n);
  HIP_TRY(hipSetDevice(device));
  gkr_ctx* c = new gkr_ctx();
  c->device = device;
  const char* i8 = getenv("GKR_INT8_WEIGHTS");
  c->int8_weights = i8 && i8[0] == '1' && i8[1] == 0;
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(GKR_ERR_DEVICE, "hipStreamCreate failed");
  }
  if (hipHostMalloc((void**)&c->h_res, 64 * sizeof(qm31), hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&c->h_out, kOutSlots * sizeof(qm31) + 256, hipHostMallocCoherent | hipHostMallocMapped) !=
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
  *out = c;
  return GKR_OK;
}
extern "C" void gkr_ctx_destroy(gkr_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
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
  if (c->merkle_consts) (void)hipFree(c->merkle_consts);
  if (c->h_res) (void)hipHostFree(c->h_res);
  if (c->h_mult) (void)hipHostFree(c->h_mult);
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
extern "C" int gkr_ctx_reset_timing(gkr_ctx* c) {
  if (!c) return fail(GKR_ERR_INVALID, "null ctx");
  TRY(sync(c));
  for (auto& s : c->stats) s = KernelStat();
  return GKR_OK;
}

// ------------------------------------------------------------------ matrices
static gkr_matrix* new_matrix(gkr_ctx* c, uint32_t* dev, uint64_t rows, uint64_t cols, bool owned);
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
  hipLaunchKernelGGL(k_fill_synth, dim3(partial_grid(n) * 8), dim3(kBlock), 0, c->stream, d, n, kind, seed);
  int rc = check_launch();
  if (rc == GKR_OK) rc = sync(c);
  if (rc != GKR_OK) {
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
    if ((m->owned && m->dev) || m->bplanes || m->r8) (void)hipStreamSynchronize(m->ctx->stream);
    if (m->owned && m->dev) (void)hipFree(m->dev);
    if (m->bplanes) (void)hipFree(m->bplanes);
    if (m->r8) (void)hipFree(m->r8);
  }
  delete m;
}
static gkr_matrix* new_matrix(gkr_ctx* c, uint32_t* dev, uint64_t rows, uint64_t cols, bool owned) {
  gkr_matrix* m = new gkr_matrix{c, dev, rows, cols, owned};
  c->matrices.insert(m);
  return m;
}
extern "C" uint32_t gkr_synthetic_value(int kind, uint64_t seed, uint64_t i) { return synth_value(kind, seed, i); }

// ------------------------------------------------------------------ matmul reduction
// The weight-side restriction leaves f_b as column-chunk partials; the first
// product trip adds them (and stores f_b), or finish_fb does when another
// consumer comes first.
static int finish_fb(gkr_ctx* c) {
  if (!c->fb_pending) return GKR_OK;
  qm31* fb;
  TRY(ensureT(c, S_FB0, c->fb_pk, &fb));
  hipLaunchKernelGGL(k_restrict_cols_finish, dim3(grid_for(c->fb_pk)), dim3(kBlock), 0, c->stream,
                     (const qm31*)c->buf[S_COLPART], c->fb_rows, c->fb_pk, c->fb_chunks, fb);
  c->fb_pending = false;
  return check_launch();
}
// The int8 copy of weight B for the restriction (k_to_int8), on first use:
// one pass over B and a 4-byte read-back of the range flag.  Used only when
// the context was created with GKR_INT8_WEIGHTS=1 in the environment: the
// int8 restriction moves a quarter of the bytes but is bound by v_dot4 issue
// (about 2.8 TB/s of int8 weights on the config shapes), the u32 one by HBM.
static int prepare_r8(gkr_ctx* c, gkr_matrix* B) {
  if (B->r8_state || !c->int8_weights) return GKR_OK;
  const uint64_t stride = (B->cols + kR8Block - 1) / kR8Block * kR8Block;
  if (B->rows == 0 || stride == 0 || B->rows * stride > (1ull << 40)) {
    B->r8_state = -1;
    return GKR_OK;
  }
  int8_t* r8 = nullptr;
  if (hipMalloc(&r8, B->rows * stride) != hipSuccess) {  // no room: keep the u32 path
    (void)hipGetLastError();
    B->r8_state = -1;
    return GKR_OK;
  }
  uint32_t* bad;
  TRY(ensureT(c, S_R8FLAG, 1, &bad));
  HIP_TRY(hipMemsetAsync(bad, 0, sizeof(uint32_t), c->stream));
  const uint64_t words = B->rows * stride / 4;
  const unsigned grid = (unsigned)std::min<uint64_t>((words + kBlock - 1) / kBlock, 4096);
  hipLaunchKernelGGL(k_to_int8, dim3(grid), dim3(kBlock), 0, c->stream, B->dev, B->rows, B->cols, stride,
                     (uint32_t*)r8, bad);
  TRY(check_launch());
  uint32_t flag = 1;
  HIP_TRY(hipMemcpyAsync(c->h_res, bad, sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
  TRY(sync(c));
  memcpy(&flag, c->h_res, sizeof flag);
  if (flag) {
    (void)hipFree(r8);
    B->r8_state = -1;
  } else {
    B->r8 = r8;
    B->r8_stride = stride;
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
static int restrict_pair(gkr_ctx* c, const gkr_matrix* A, const gkr_matrix* B, const qm31* r_i, int n_ri,
                         const qm31* r_j, int n_rj, uint64_t pk, bool weight_only = false) {
  TRY(prepare_r8(c, const_cast<gkr_matrix*>(B)));  // the matrix's contents never change; r8 is derived
  HostTimer ht(c, K_HOST_LAUNCH);
  const uint64_t m = A->rows, k = A->cols, n = B->cols;
  const bool use8 = B->r8_state == 1 && n < (1ull << 17);  // int32 digit sums stay exact below 2^17 columns
  uint8_t* ldig = nullptr;
  if (use8) TRY(ensureT(c, S_LDIG, ((n + 3) / 4) * 64, &ldig));
  qm31 *Li, *Lj, *fa, *fb;
  TRY(ensureT(c, S_LI, m, &Li));
  TRY(ensureT(c, S_LJ, n, &Lj));
  TRY(ensureT(c, S_FA0, pk, &fa));
  TRY(ensureT(c, S_FB0, pk, &fb));
  c->fb_pending = false;
  if (n_ri + n_rj <= kMaxVars) {
    std::vector<qm31> both(r_i, r_i + n_ri);
    both.insert(both.end(), r_j, r_j + n_rj);
    PointArg pt = make_point(both.data(), n_ri + n_rj);
    TimedLaunch tl(c, K_EQ_TABLE, 16 * (m + n));
    hipLaunchKernelGGL(k_eq_two, dim3(grid_for(m + n)), dim3(kBlock), 0, c->stream, pt, n_ri, m, n, Li, Lj, ldig);
    TRY(check_launch());
  } else {
    if (use8) return fail(GKR_ERR_DEVICE, "int8 restriction needs the combined eq launch");
    TRY(eq_table(c, r_i, n_ri, m, Li));
    TRY(eq_table(c, r_j, n_rj, n, Lj));
  }
  {
    // column chunks: chunks a multiple of one wave sweep (256 columns), at
    // least GKR_RC_MIN_CHUNK columns, and at most GKR_RC_TARGET workgroups in
    // all (GKR_RC_CEIL: at least that many)
#ifndef GKR_RC_TARGET
#define GKR_RC_TARGET 2560
#endif
#ifndef GKR_RC_MIN_CHUNK
#define GKR_RC_MIN_CHUNK 512
#endif
#ifndef GKR_RC_CEIL
#define GKR_RC_CEIL 1
#endif
    const uint64_t rows_per_block = (uint64_t)kColRows * kColWaves;
    const uint64_t gr = (k + rows_per_block - 1) / rows_per_block;
    uint64_t gc = GKR_RC_CEIL ? (GKR_RC_TARGET + gr - 1) / gr : GKR_RC_TARGET / gr;
    if (gc < 1) gc = 1;
    uint64_t chunk = (n + gc - 1) / gc;
    chunk = (chunk + 255) / 256 * 256;
    if (chunk < GKR_RC_MIN_CHUNK) chunk = GKR_RC_MIN_CHUNK;
    gc = (n + chunk - 1) / chunk;
    qm31* part;
    TRY(ensureT(c, S_COLPART, (size_t)gc * k, &part));
    // the activation side rides in one more column-chunk slice (one column per thread)
    RowsJob rows{A->dev, m, k, pk, Li, fa};
    const uint64_t act_blocks = weight_only ? 0 : (pk + 63) / 64;  // 64 columns of A per workgroup
    if (act_blocks + gr * gc > 0x7fffffffull) return fail(GKR_ERR_INVALID, "matrix too large for one restriction");
    const dim3 grid((unsigned)(act_blocks + gr * gc));
    if (use8) {
      // column chunks of kR8ChunkBlocks blocks; passes per wave chosen for
      // about 512 weight-side workgroups (measured best on the config shapes)
      const uint64_t nblocks = B->r8_stride / kR8Block;
      const uint64_t gc8 = (nblocks + kR8ChunkBlocks - 1) / kR8ChunkBlocks;
      const uint64_t groups = (k + kColWaves * kR8Rows - 1) / (kColWaves * kR8Rows);
      const int passes = (int)std::max<uint64_t>(1, std::min<uint64_t>(kR8MaxPasses, groups * gc8 / 512));
      const uint64_t gr8 = (k + (uint64_t)kColWaves * kR8Rows * passes - 1) / ((uint64_t)kColWaves * kR8Rows * passes);
      if (gc8 > gc) TRY(ensureT(c, S_COLPART, (size_t)gc8 * k, &part));
      gc = gc8;
      if (act_blocks + gr8 * gc8 > 0x7fffffffull) return fail(GKR_ERR_INVALID, "matrix too large for one restriction");
      // algorithmic bytes: B as int8 and L_j's digits (weight side), A and L_i (activation side), f_a written
      TimedLaunch t(c, K_RESTRICT_COLS, k * n + 16 * n + (weight_only ? 0 : 4 * m * k + 16 * m + 16 * pk));
      hipLaunchKernelGGL(k_restrict_cols8, dim3((unsigned)(act_blocks + gr8 * gc8)), dim3(kBlock), 0, c->stream,
                         B->r8, B->r8_stride, k, (const u32x4*)ldig, (n + 3) / 4, passes, (uint32_t*)part, rows,
                         (uint32_t)act_blocks, (uint32_t)gr8);
      TRY(check_launch());
    } else {
      // algorithmic bytes: B and L_j (weight side) plus A and L_i (activation side), f_a written
      TimedLaunch t(c, K_RESTRICT_COLS, 4 * k * n + 16 * n + (weight_only ? 0 : 4 * m * k + 16 * m + 16 * pk));
      if (n % 4 == 0 && ((uintptr_t)B->dev & 15) == 0)
        hipLaunchKernelGGL(k_restrict_cols<true>, grid, dim3(kBlock), 0, c->stream, B->dev, k, n, chunk, Lj,
                           (uint32_t*)part, rows, (uint32_t)act_blocks, (uint32_t)gr);
      else
        hipLaunchKernelGGL(k_restrict_cols<false>, grid, dim3(kBlock), 0, c->stream, B->dev, k, n, chunk, Lj,
                           (uint32_t*)part, rows, (uint32_t)act_blocks, (uint32_t)gr);
      TRY(check_launch());
    }
    c->fb_pending = true;
    c->fb_rows = k;
    c->fb_pk = pk;
    c->fb_chunks = (int)gc;
  }
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

// The last rounds of each sumcheck run on the host once the vectors are this
// short (the device trips stop there; k_handover folds the last trip's
// vectors and hands them over).
#ifndef GKR_HOST_TAIL_MM
#define GKR_HOST_TAIL_MM 256   // product sumcheck: 5 QM31 products per pair
#endif
#ifndef GKR_HOST_TAIL_EQ3
#define GKR_HOST_TAIL_EQ3 256  // eq-sumcheck: 11 products per pair
#endif
#ifndef GKR_HOST_TAIL_SUM
#define GKR_HOST_TAIL_SUM 256  // multiplicity sumcheck: 1 product per pair
#endif
constexpr uint64_t kHostTailMM = GKR_HOST_TAIL_MM;
constexpr uint64_t kHostTailEq3 = GKR_HOST_TAIL_EQ3;
constexpr uint64_t kHostTailSum = GKR_HOST_TAIL_SUM;
static_assert(kHostTailMM * 8 <= (uint64_t)kHandMax && kHostTailEq3 * 8 <= (uint64_t)kHandMax &&
                  kHostTailSum * 8 <= (uint64_t)kHandMax,
              "the last trip's vectors must fit k_handover");

// Degree-2 product sumcheck sum_x f_a(x) f_b(x) over 2^T entries: the round
// loop of reduce_matmul_layer (backend.rs:146-177; gpu_sumcheck.rs:2820-2840),
// as device trips of up to 3 rounds (plan_trips), then the host.  in_a/in_b
// are only read; trip j >= 1 writes its folded vectors to bufs[(j - 1) & 1]
// (bufs[0] holds 2^(T-1) entries, bufs[1] 2^(T-2)).  g0, when given, holds
// the first trip's sums (rounds 0 .. k0 - 1) already computed for these inputs.
// scale3 set: the rounds of a three-factor sumcheck sum w a b whose w is the
// constant *scale3 over these variables: each round polynomial is *scale3
// times the product one, written and mixed as degree 3 (c3 = 0; 4 per round).
static int product_sumcheck(gkr_ctx* c, PoseidonChannel& ch, int T, const qm31* in_a, const qm31* in_b,
                            qm31* const bufs_a[2], qm31* const bufs_b[2], const qm31* g0, int k0,
                            gkr_qm31* round_polys, gkr_qm31* challenges, gkr_qm31* final_a, gkr_qm31* final_b,
                            const qm31* scale3 = nullptr) {
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
  const qm31* src_a = in_a;
  const qm31* src_b = in_b;
  int np = 0;
  const qm31* pend = nullptr;
  for (size_t j = 0; j < trips.size(); j++) {
    const Trip& tr = trips[j];
    const bool last = j + 1 == trips.size();
    qm31 g[kMaxSums];
    if (j == 0 && g0) {
      for (int q = 0; q < trip_nq(0, tr.K); q++) g[q] = g0[q];
      if (last) TRY(ho.launch<2>(in_a, in_b, tr.n, tr.K));
    } else {
      qm31* da = j == 0 ? nullptr : bufs_a[(j - 1) & 1];
      qm31* db = j == 0 ? nullptr : bufs_b[(j - 1) & 1];
      RoundSink sk;
      TRY(launch_trip(c, 0, tr.K, src_a, src_b, tr.n, np, pend, da, db, nullptr, nullptr, 0, 0, &sk));
      if (j > 0) {
        src_a = da;
        src_b = db;
      }
      if (last) TRY(ho.launch<2>(src_a, src_b, tr.n, tr.K));
      TRY(wait_trip(c, sk, trip_nq(0, tr.K), g));
    }
    for (int i = 0; i < tr.K; i++) {
      qm31 sums[3];
      trip_round_gram(g, tr.K, i, chal.data() + tr.t, 3, xs, sums, nullptr, qm31_zero());
      absorb(tr.t + i, sums);
    }
    np = tr.K;
    pend = chal.data() + tr.t;
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
    qm31 sums[3] = {qm31_zero(), qm31_zero(), qm31_zero()};
    {
      HostTimer ht(c, K_HOST_FINISH);
      for (size_t i = 0; i < half; i++) {
        const qm31 a0 = A[i], a1 = A[i + half], b0 = B[i], b1 = B[i + half];
        sums[0] = qm31_add(sums[0], qm31_mul(a0, b0));
        sums[1] = qm31_add(sums[1], qm31_mul(a1, b1));
        sums[2] = qm31_add(sums[2], qm31_mul(qm31_sub(qm31_add(a1, a1), a0), qm31_sub(qm31_add(b1, b1), b0)));
      }
    }
    absorb(t, sums);
    HostTimer ht(c, K_HOST_FINISH);
    for (size_t i = 0; i < half; i++) {
      A[i] = qm31_fold(A[i], A[i + half], chal[t]);
      B[i] = qm31_fold(B[i], B[i + half], chal[t]);
    }
    A.resize(half);
    B.resize(half);
  }
  *final_a = G(A[0]);
  *final_b = G(B[0]);
  return GKR_OK;
}

static int reduce_matmul_impl(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, const gkr_qm31* r_i, uint32_t n_ri,
                              const gkr_qm31* r_j, uint32_t n_rj, uint64_t pk, PoseidonChannel& ch,
                              gkr_qm31* round_polys, gkr_qm31* challenges, gkr_qm31* final_a, gkr_qm31* final_b) {
  TRY(validate_matmul(c, a, b, n_ri, n_rj));
  if (pk != next_pow2(a->cols))
    return fail(GKR_ERR_INVALID, "pk=%llu but next_pow2(k)=%llu", (unsigned long long)pk,
                (unsigned long long)next_pow2(a->cols));
  HIP_TRY(hipSetDevice(c->device));
  TRY(ensure_restricted(c, a, b, r_i, n_ri, r_j, n_rj));
  if (!c->mm.have_trip0) TRY(finish_fb(c));  // the sumcheck reads f_b from S_FB0
  const int T = log2_exact(pk);
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
  return product_sumcheck(c, ch, T, fa0, fb0, bufs_a, bufs_b, have ? c->mm.trip0 : nullptr, c->mm.trip0_k,
                          round_polys, challenges, final_a, final_b);
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

// ------------------------------------------------------------------ proof container
struct LayerRec {
  uint32_t tag;  // 0 MatMul, 2 Mul, 3 Activation, 7 MatMulDualSimd (rp: c0..c3 per round)
  uint32_t n_block_vars = 0;  // MatMulDualSimd
  qm31 claim_value = {0, 0, 0, 0};  // the output claim's value the layer was proved against
  std::vector<qm31> rp;  // MatMul: c0,c1,c2 per round; Mul, Activation: eq c0..c3 per round
  qm31 final_a, final_b;  // MatMul: final a/b evals; Mul: lhs/rhs evals
  uint32_t act_type = 0;
  qm31 input_eval, output_eval;
  felt table_commitment;
  qm31 claimed_sum, w_eval, in_eval, out_eval;
  std::vector<uint32_t> mults;
  std::vector<qm31> mult_rp;  // c0,c1 per round
  qm31 mult_final, mult_sum;
};
// A MatMul layer's claim on its weight: MLE(B)(r_j || sumcheck challenges) =
// final_b (push_matmul_weight_data, prover.rs:1465-1483).
struct WeightClaimRec {
  const gkr_matrix* b;
  std::vector<qm31> point;
  qm31 value;
};
struct gkr_proof {
  std::vector<LayerRec> layers;
  std::vector<qm31> in_point;
  qm31 in_value = {0, 0, 0, 0};
  std::vector<felt> weight_commitments;
  std::vector<WeightClaimRec> weight_claims;      // recorded by the MatMul layers, in proving order
  std::vector<std::vector<felt>> weight_openings;  // serialized opening records (claim + MleOpeningProof)
  felt io_commitment = {{0, 0, 0, 0}};
};
extern "C" int gkr_proof_new(gkr_proof** out) {
  if (!out) return fail(GKR_ERR_INVALID, "null out");
  *out = new gkr_proof();
  return GKR_OK;
}
extern "C" void gkr_proof_free(gkr_proof* p) { delete p; }
extern "C" size_t gkr_proof_num_layers(const gkr_proof* p) { return p ? p->layers.size() : 0; }
extern "C" int gkr_proof_layer_claim_value(const gkr_proof* p, size_t layer, gkr_qm31* value) {
  if (!p || !value) return fail(GKR_ERR_INVALID, "null argument");
  if (layer >= p->layers.size()) return fail(GKR_ERR_INVALID, "layer %zu of %zu", layer, p->layers.size());
  *value = G(p->layers[layer].claim_value);
  return GKR_OK;
}
extern "C" int gkr_proof_set_input_claim(gkr_proof* p, const gkr_qm31* point, uint32_t n, const gkr_qm31* value) {
  if (!p || !value || (!point && n)) return fail(GKR_ERR_INVALID, "null argument");
  p->in_point.clear();
  for (uint32_t i = 0; i < n; i++) p->in_point.push_back(Q(point[i]));
  p->in_value = Q(*value);
  return GKR_OK;
}
extern "C" int gkr_proof_add_weight_commitment(gkr_proof* p, const gkr_felt* cm) {
  if (!p || !cm || !felt_abi_canonical(*cm)) return fail(GKR_ERR_INVALID, "bad argument");
  p->weight_commitments.push_back(felt_canon_from_words(cm->w));
  return GKR_OK;
}
extern "C" int gkr_proof_set_io_commitment(gkr_proof* p, const gkr_felt* cm) {
  if (!p || !cm || !felt_abi_canonical(*cm)) return fail(GKR_ERR_INVALID, "bad argument");
  p->io_commitment = felt_canon_from_words(cm->w);
  return GKR_OK;
}

// serialize_gkr_model_proof (cairo_serde.rs:1307-1772); felts kept canonical.
// Two passes over the proof: the first counts, the second writes straight
// into the caller's buffer (no intermediate copy of the felt stream).
struct Ser {
  gkr_felt* out;  // nullptr: count only
  size_t n = 0;
  void u(uint64_t v) {
    if (out) {
      gkr_felt& f = out[n];
      f.w[0] = (uint32_t)v;
      f.w[1] = (uint32_t)(v >> 32);
      for (int i = 2; i < 8; i++) f.w[i] = 0;
    }
    n++;
  }
  void q(const qm31& x) { u(x.a); u(x.b); u(x.c); u(x.d); }
  void f(const felt& canon) {
    if (out) felt_canon_to_words(canon, out[n].w);
    n++;
  }
};
static void serialize_proof(const gkr_proof* p, Ser& s) {
  s.u(p->layers.size());
  for (const LayerRec& L : p->layers) {
    if (L.tag == 0) {
      s.u(0);
      const size_t nr = L.rp.size() / 3;
      s.u(nr);
      for (size_t r = 0; r < nr; r++) {  // c1 omitted (cairo_serde.rs:1327-1331)
        s.q(L.rp[3 * r]);
        s.q(L.rp[3 * r + 2]);
      }
      s.q(L.final_a);
      s.q(L.final_b);
    } else if (L.tag == 7) {
      // LayerProof::MatMulDualSimd (cairo_serde.rs:1629-1646): c1 omitted
      s.u(7);
      s.u(L.n_block_vars);
      const size_t nr = L.rp.size() / 4;
      s.u(nr);
      for (size_t r = 0; r < nr; r++) {
        s.q(L.rp[4 * r]);
        s.q(L.rp[4 * r + 2]);
        s.q(L.rp[4 * r + 3]);
      }
      s.q(L.final_a);
      s.q(L.final_b);
    } else if (L.tag == 2) {
      // LayerProof::Mul (cairo_serde.rs:1339-1354): c1 omitted
      s.u(2);
      const size_t nr = L.rp.size() / 4;
      s.u(nr);
      for (size_t r = 0; r < nr; r++) {
        s.q(L.rp[4 * r]);
        s.q(L.rp[4 * r + 2]);
        s.q(L.rp[4 * r + 3]);
      }
      s.q(L.final_a);
      s.q(L.final_b);
    } else {
      s.u(3);
      s.u(L.act_type);
      s.q(L.input_eval);
      s.q(L.output_eval);
      s.f(L.table_commitment);
      s.u(1);  // has LogUp proof
      // serialize_logup_proof_inner with multiplicities (cairo_serde.rs:1080-1105)
      s.q(L.claimed_sum);
      const size_t nr = L.rp.size() / 4;
      s.u(nr);
      for (size_t r = 0; r < nr; r++) {
        s.q(L.rp[4 * r]);
        s.q(L.rp[4 * r + 2]);
        s.q(L.rp[4 * r + 3]);
      }
      s.q(L.w_eval);
      s.q(L.in_eval);
      s.q(L.out_eval);
      s.u(L.mults.size());
      for (uint32_t m : L.mults) s.u(m);
      // serialize_multiplicity_sumcheck (cairo_serde.rs:1138-1156)
      s.u(1);
      const size_t nm = L.mult_rp.size() / 2;
      s.u(nm);
      for (size_t r = 0; r < nm; r++) {
        s.q(L.mult_rp[2 * r]);
        s.q(L.mult_rp[2 * r + 1]);
      }
      s.q(L.mult_final);
      s.q(L.mult_sum);
      s.u(0);  // no activation product proof
      s.u(0);  // no piecewise proof
    }
  }
  s.u(p->in_point.size());
  for (const qm31& x : p->in_point) s.q(x);
  s.q(p->in_value);
  s.u(p->weight_commitments.size());
  for (const felt& w : p->weight_commitments) s.f(w);
  s.u(p->weight_openings.size());  // cairo_serde.rs:1756-1767
  for (const auto& rec : p->weight_openings)
    for (const felt& f : rec) s.f(f);
  s.f(p->io_commitment);
}
extern "C" int gkr_proof_serialize(const gkr_proof* p, gkr_felt* out, size_t cap, size_t* n_out) {
  if (!p || !n_out || (!out && cap)) return fail(GKR_ERR_INVALID, "null argument");
  Ser count{nullptr};
  serialize_proof(p, count);
  *n_out = count.n;
  if (cap < count.n) return fail(GKR_ERR_BUFFER, "need %zu felts, have %zu", count.n, cap);
  Ser write{out};
  serialize_proof(p, write);
  return GKR_OK;
}

extern "C" int gkr_prove_matmul_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                      const gkr_qm31* claim_value, const gkr_matrix* a, const gkr_matrix* b,
                                      gkr_channel* ch, gkr_proof* proof, gkr_qm31* round_polys, gkr_qm31* final_a,
                                      gkr_qm31* final_b, gkr_qm31* next_point, gkr_qm31* next_value) {
  CH_CHECK(ch);
  if (!c || !a || !b || !claim_value || !final_a || !final_b || !next_value || (!claim_point && n_point))
    return fail(GKR_ERR_INVALID, "null argument");
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  const uint64_t pm = next_pow2(a->rows), pk = next_pow2(a->cols), pn = next_pow2(b->cols);
  const uint32_t log_m = (uint32_t)log2_exact(pm), log_n = (uint32_t)log2_exact(pn);
  const int T = log2_exact(pk);
  if (n_point != log_m + log_n)
    return fail(GKR_ERR_INVALID, "output claim has %u vars, expected exactly %u (log_m=%u + log_n=%u)", n_point,
                log_m + log_n, log_m, log_n);
  if (T > 0 && (!round_polys || !next_point)) return fail(GKR_ERR_INVALID, "null output buffer");
  TRY(validate_matmul(c, a, b, log_m, log_n));
  PoseidonChannel& C = ch->ch;
  C.mix_u64(a->rows);
  C.mix_u64(a->cols);
  C.mix_u64(b->cols);
  C.mix_secure_field(Q(*claim_value));
  std::vector<gkr_qm31> chal(T > 0 ? T : 1);
  TRY(reduce_matmul_impl(c, a, b, claim_point, log_m, claim_point + log_m, log_n, pk, C, round_polys, chal.data(),
                         final_a, final_b));
  C.mix_secure_field(Q(*final_a));
  C.mix_secure_field(Q(*final_b));
  if (next_point) {
    for (uint32_t l = 0; l < log_m; l++) next_point[l] = claim_point[l];
    for (int t = 0; t < T; t++) next_point[log_m + t] = chal[t];
  }
  *next_value = *final_a;
  if (proof) {
    LayerRec L;
    L.tag = 0;
    L.claim_value = Q(*claim_value);
    for (int t = 0; t < 3 * T; t++) L.rp.push_back(Q(round_polys[t]));
    L.final_a = Q(*final_a);
    L.final_b = Q(*final_b);
    proof->layers.push_back(L);
    WeightClaimRec w;
    w.b = b;
    for (uint32_t l = 0; l < log_n; l++) w.point.push_back(Q(claim_point[log_m + l]));
    for (int t = 0; t < T; t++) w.point.push_back(Q(chal[t]));
    w.value = Q(*final_b);
    proof->weight_claims.push_back(std::move(w));
  }
  return GKR_OK;
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
    TimedLaunch t(c, K_RESTRICT_ROWS, 4ull * n_blocks * a->rows * a->cols + 16 * a->rows + 16 * pk);
    hipLaunchKernelGGL(k_restrict_rows_simd, dim3((unsigned)((pk + 63) / 64)), dim3(kSimdWaves * 64), 0, c->stream, blk,
                       a->rows, a->cols, pk, (const qm31*)Li, fa);
    TRY(check_launch());
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
    LayerRec L;
    L.tag = 0;
    L.claim_value = Q(*claim_value);
    for (int t = 0; t < 3 * T; t++) L.rp.push_back(Q(round_polys[t]));
    L.final_a = Q(*final_a);
    L.final_b = Q(*final_b);
    proof->layers.push_back(L);
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
    hipLaunchKernelGGL(k_restrict_rows_blocks, dim3(grid_for(pk), n_blocks), dim3(kBlock), 0, c->stream, pa, a->rows,
                       a->cols, pk, (const qm31*)Li, ea);
    hipLaunchKernelGGL(k_restrict_cols_blocks, dim3((unsigned)((pk + kColWaves - 1) / kColWaves), n_blocks),
                       dim3(kBlock), 0, c->stream, pb, b->rows, b->cols, pk, (const qm31*)Lj, eb);
    TRY(check_launch());
  }
  std::vector<qm31> D((size_t)n_blocks * n_blocks);
  if (nbv > 0) {
    hipLaunchKernelGGL(k_block_gram, dim3(n_blocks * n_blocks), dim3(kBlock), 0, c->stream, (const qm31*)ea,
                       (const qm31*)eb, n_blocks, pk, gram);
    TRY(check_launch());
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
  hipLaunchKernelGGL(k_combine_q, gq, dim3(kBlock), 0, c->stream, (const qm31*)ea, qw, n_blocks, pk, fa0);
  hipLaunchKernelGGL(k_combine_q, gq, dim3(kBlock), 0, c->stream, (const qm31*)eb, qw, n_blocks, pk, fb0);
  TRY(check_launch());
  std::vector<gkr_qm31> kchal(T > 0 ? T : 1);
  if (T == 0) {
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
    proof->layers.push_back(L);
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
  hipLaunchKernelGGL(k_dot_q, dim3(partial_grid(len)), dim3(kBlock), 0, c->stream, dm, eq, len, sk);
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
  hipLaunchKernelGGL(k_restrict_q, dim3(grid_for(rest)), dim3(kBlock), 0, c->stream, dm, eq, nx, rest, dout);
  TRY(check_launch());
  HIP_TRY(hipMemcpyAsync(out, dout, rest * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
  return sync(c);
}

// ------------------------------------------------------------------ LogUp activation layer
extern "C" int gkr_activation_table(uint32_t tag, uint32_t log_size, uint32_t* out) {
  if (!out || !act_valid(tag) || log_size == 0 || log_size > 24) return fail(GKR_ERR_INVALID, "bad argument");
  std::vector<uint32_t> t = act_table(tag, log_size);
  memcpy(out, t.data(), t.size() * sizeof(uint32_t));
  return GKR_OK;
}

static const std::vector<uint32_t>& cached_table(gkr_ctx* c, uint32_t tag, uint32_t log_size) {
  const uint64_t key = ((uint64_t)tag << 32) | log_size;
  auto it = c->tables.find(key);
  if (it == c->tables.end()) it = c->tables.emplace(key, act_table(tag, log_size)).first;
  return it->second;
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
constexpr int kEqLoMax = 10;  // variables in the lower eq table of a trip
struct Eq3Plan {
  int nv = 0;
  std::vector<Trip> trips;
  std::vector<uint32_t> hi_off, lo_off;  // per trip, offsets into S_EQPARTS
  std::vector<int> h;                    // per trip, variables in the lower table
};
// Plan the trips of an eq-sumcheck over 2^nv entries for claim point z and
// launch the kernel that builds their eq tables (S_EQPARTS).
static int eq3_prepare(gkr_ctx* c, const qm31* z, int nv, Eq3Plan* pl) {
  pl->nv = nv;
  pl->trips = plan_trips(nv, kHostTailEq3, trip_k(1ull << nv));
  pl->hi_off.clear();
  pl->lo_off.clear();
  pl->h.clear();
  if (pl->trips.empty()) return GKR_OK;
  EqPartsArg arg;
  memset(&arg, 0, sizeof arg);
  arg.z = make_point(z, nv);
  uint32_t total = 0;
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
  HostTimer ht(c, K_HOST_LAUNCH);
  qm31* parts;
  TRY(ensureT(c, S_EQPARTS, total, &parts));
  {
    TimedLaunch tl(c, K_EQ_TABLE, 16ull * total);
    hipLaunchKernelGGL(k_eq_parts, dim3(grid_for(total)), dim3(kBlock), 0, c->stream, arg, total, parts);
  }
  return check_launch();
}
// Launch trip j of the plan over sources w, d (np pending challenges pend),
// folded vectors to dw, dd when given.
static int eq3_launch_trip(gkr_ctx* c, const Eq3Plan& pl, size_t j, const qm31* w, const qm31* d, int np,
                           const qm31* pend, qm31* dw, qm31* dd, int slot, RoundSink* sk) {
  qm31* parts = (qm31*)c->buf[S_EQPARTS];
  const Trip& tr = pl.trips[j];
  return launch_trip(c, 1, tr.K, w, d, tr.n, np, pend, dw, dd, parts + pl.hi_off[j], parts + pl.lo_off[j], pl.h[j],
                     slot, sk);
}
// The sumcheck for claim point z over w0, d0 (overwritten: the trips' folded
// vectors go to w1/d1 (n/2 entries) and w0/d0 alternately).  pre0: trip 0
// already launched (eq3_launch_trip, any slot).  Writes 4 * nv round
// coefficients, nv challenges and the final (eq, w, d) values.
static int eq3_sumcheck(gkr_ctx* c, PoseidonChannel& C, const qm31* z, const Eq3Plan& pl, qm31* w0, qm31* d0,
                        qm31* w1, qm31* d1, gkr_qm31* rp_out, qm31* chal, qm31 fin[3],
                        const RoundSink* pre0 = nullptr) {
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
  const qm31* sw = w0;
  const qm31* sd = d0;
  int np = 0;
  const qm31* pend = nullptr;
  qm31 cpre = qm31_one();  // prod of eqlin(z_l, r_l) over the rounds done
  for (size_t j = 0; j < pl.trips.size(); j++) {
    const Trip& tr = pl.trips[j];
    const bool last = j + 1 == pl.trips.size();
    qm31 g[kMaxSums];
    RoundSink sk;
    if (j == 0 && pre0) {
      sk = *pre0;
    } else {
      qm31* dw = j == 0 ? nullptr : bw[(j - 1) & 1];
      qm31* dd = j == 0 ? nullptr : bd[(j - 1) & 1];
      TRY(eq3_launch_trip(c, pl, j, sw, sd, np, pend, dw, dd, 0, &sk));
      if (j > 0) {
        sw = dw;
        sd = dd;
      }
    }
    if (last) TRY(ho.launch<2>(sw, sd, tr.n, tr.K));
    TRY(wait_trip(c, sk, trip_nq(1, tr.K), g));
    for (int i = 0; i < tr.K; i++) {
      qm31 sums[4];
      trip_round_gram(g, tr.K, i, chal + tr.t, 4, xs, sums, z + tr.t, cpre);
      absorb3(tr.t + i, sums);
    }
    for (int i = 0; i < tr.K; i++) cpre = qm31_mul(cpre, eqlin(z[tr.t + i], chal[tr.t + i]));
    np = tr.K;
    pend = chal + tr.t;
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
    qm31 sums[4] = {qm31_zero(), qm31_zero(), qm31_zero(), qm31_zero()};
    {
      HostTimer ht(c, K_HOST_FINISH);
      for (size_t i = 0; i < half; i++) {
        const qm31 e0 = E[i], e1 = E[i + half], w0v = W[i], w1v = W[i + half], d0v = D[i], d1v = D[i + half];
        sums[0] = qm31_add(sums[0], qm31_mul(qm31_mul(e0, w0v), d0v));
        sums[1] = qm31_add(sums[1], qm31_mul(qm31_mul(e1, w1v), d1v));
        const qm31 de = qm31_sub(e1, e0), dw = qm31_sub(w1v, w0v), dd = qm31_sub(d1v, d0v);
        const qm31 e2 = qm31_add(e1, de), w2 = qm31_add(w1v, dw), d2 = qm31_add(d1v, dd);
        sums[2] = qm31_add(sums[2], qm31_mul(qm31_mul(e2, w2), d2));
        sums[3] = qm31_add(sums[3], qm31_mul(qm31_mul(qm31_add(e2, de), qm31_add(w2, dw)), qm31_add(d2, dd)));
      }
    }
    absorb3(t, sums);
    HostTimer ht(c, K_HOST_FINISH);
    for (size_t i = 0; i < half; i++) {
      E[i] = qm31_fold(E[i], E[i + half], chal[t]);
      W[i] = qm31_fold(W[i], W[i + half], chal[t]);
      D[i] = qm31_fold(D[i], D[i + half], chal[t]);
    }
    E.resize(half);
    W.resize(half);
    D.resize(half);
  }
  fin[0] = E[0];
  fin[1] = W[0];
  fin[2] = D[0];
  return GKR_OK;
}

extern "C" int gkr_prove_activation_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                          const gkr_qm31* claim_value, const gkr_matrix* input, uint32_t tag,
                                          uint32_t table_log, gkr_channel* ch, gkr_proof* proof, gkr_logup_out* out) {
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
  if (!out->multiplicities || !out->mult_round_polys) return fail(GKR_ERR_INVALID, "null output arrays");
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  std::vector<qm31> cpt(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(claim_point[l])) return fail(GKR_ERR_INVALID, "claim point not canonical");
    cpt[l] = Q(claim_point[l]);
  }
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  PoseidonChannel& C = ch->ch;
  const uint64_t tsize = 1ull << table_log;
  const uint32_t mask = (uint32_t)(tsize - 1);
  const std::vector<uint32_t>& table = cached_table(c, tag, table_log);

  uint32_t *d_table, *d_mult, *d_min, *d_mout;
  qm31 *d_d0, *d_d1, *d_w0, *d_w1, *d_e0, *m0, *m1;
  TRY(ensureT(c, S_TABLE, tsize, &d_table));
  TRY(ensureT(c, S_MULT, tsize, &d_mult));
  TRY(ensureT(c, S_MIN, n, &d_min));
  TRY(ensureT(c, S_MOUT, n, &d_mout));
  TRY(ensureT(c, S_D0, n, &d_d0));
  TRY(ensureT(c, S_D1, n / 2 + 1, &d_d1));
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_W1, n / 2 + 1, &d_w1));
  TRY(ensureT(c, S_E0, n, &d_e0));
  TRY(ensureT(c, S_M0, tsize, &m0));
  TRY(ensureT(c, S_M1, tsize / 2 + 1, &m1));
  TRY(ensure_host_mult(c, tsize));
  const uint64_t table_key = ((uint64_t)tag << 32) | table_log;
  if (c->table_on_device != table_key) {
    c->table_on_device = 0;
    HIP_TRY(hipMemcpyAsync(d_table, table.data(), tsize * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    c->table_on_device = table_key;
  }
  HIP_TRY(hipMemsetAsync(d_mult, 0, tsize * sizeof(uint32_t), c->stream));
  // eq(claim point, x): the input MLE at the claim point (accumulated by the
  // prepare pass) and the eq vector of the eq-sumcheck
  TRY(eq_table(c, cpt.data(), nv, n, d_e0));

  // Fiat-Shamir: LOG tag, type tag, gamma, beta (prover.rs:6451-6454)
  C.mix_u64(0x4C4F47ull);
  C.mix_u64(tag);
  qm31 gb[2];
  C.draw_qm31s(gb, 2);
  const qm31 gamma = gb[0], beta = gb[1];
  out->gamma = G(gamma);
  out->beta = G(beta);

  // Launched back to back, read when needed (each result in its own slot):
  //   prepare -> (trace sum, input MLE at the claim point)      kSlotPrep
  //   table-side sum over the multiplicities                     kSlotTable
  //   multiplicities -> pinned host copy
  //   multiplicity sumcheck trip 0 (no challenge needed)         kSlotMult0
  //   eq tables of the eq-sumcheck trips, eq-sumcheck trip 0     kSlotEq0
  RoundSink sk_prep, sk_table, sk_mult0, sk_eq0;
  {
    HostTimer ht(c, K_HOST_LAUNCH);
    TRY(make_sink(c, &sk_prep, kSlotPrep));
    {
      TimedLaunch tl(c, K_LOGUP_PREP, 4 * input->rows * input->cols + 16 * n + 8 * n + 32 * n);
      hipLaunchKernelGGL(k_logup_prepare, dim3(partial_grid(n)), dim3(kBlock), 0, c->stream, input->dev,
                         input->rows, input->cols, log2_exact(pcol), n, d_table, mask, gamma, beta, d_e0, d_min,
                         d_mout, d_d0, d_w0, d_mult, sk_prep);
    }
    TRY(launch_finish<2>(c, sk_prep, partial_grid(n)));
    TRY(make_sink(c, &sk_table, kSlotTable));
    hipLaunchKernelGGL(k_logup_table_sum, dim3(partial_grid(tsize)), dim3(kBlock), 0, c->stream, d_table, d_mult,
                       tsize, gamma, beta, sk_table);
    TRY(launch_finish<1>(c, sk_table, partial_grid(tsize)));
    HIP_TRY(hipMemcpyAsync(c->h_mult, d_mult, tsize * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
    hipLaunchKernelGGL(k_u32_to_q, dim3(grid_for(tsize)), dim3(kBlock), 0, c->stream, d_mult, tsize, m0);
    TRY(check_launch());
  }
  const std::vector<Trip> mtrips = plan_trips((int)table_log, kHostTailSum, kTripMaxK);
  TRY(launch_trip(c, 2, mtrips[0].K, m0, nullptr, tsize, 0, nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                  kSlotMult0, &sk_mult0));
  Eq3Plan epl;
  TRY(eq3_prepare(c, cpt.data(), nv, &epl));
  const bool eq_pre = nv > 0;
  if (eq_pre) TRY(eq3_launch_trip(c, epl, 0, d_w0, d_d0, 0, nullptr, nullptr, nullptr, kSlotEq0, &sk_eq0));

  qm31 prep[2], tsum[1];
  TRY(wait_sink<1>(c, sk_table, tsum));  // implies the prepare results (earlier on the stream)
  for (int q = 0; q < 2; q++) prep[q] = c->h_out[kSlotPrep + q];
  const qm31 trace_sum = prep[0], input_eval = prep[1], table_sum = tsum[0];
  if (!qm31_eq(trace_sum, table_sum))
    return fail(GKR_ERR_LOGUP, "Activation LogUp sum mismatch: trace=(%u,%u,%u,%u) table=(%u,%u,%u,%u)", trace_sum.a,
                trace_sum.b, trace_sum.c, trace_sum.d, table_sum.a, table_sum.b, table_sum.c, table_sum.d);
  C.mix_secure_field(trace_sum);
  out->claimed_sum = G(trace_sum);

  // eq-sumcheck: sum eq(r, x) w(x) d(x) = 1 over the hypercube
  std::vector<qm31> chal(nv);
  qm31 fin[3];
  TRY(eq3_sumcheck(c, C, cpt.data(), epl, d_w0, d_d0, d_w1, d_d1, out->eq_round_polys, chal.data(), fin,
                   eq_pre ? &sk_eq0 : nullptr));
  const qm31 w_eval = fin[1];
  // MLE(masked_in), MLE(masked_out) at the eq-sumcheck challenges, one pass
  qm31 io[2];
  TRY(eq_table(c, chal.data(), nv, n, d_e0));
  {
    RoundSink sk;
    TRY(make_sink(c, &sk));
    hipLaunchKernelGGL(k_dot2_m31, dim3(partial_grid(n)), dim3(kBlock), 0, c->stream, d_min, d_mout, d_e0, n, sk);
    TRY(launch_finish<2>(c, sk, partial_grid(n)));
    TRY(wait_sink<2>(c, sk, io));
  }
  const qm31 in_eval = io[0], out_eval = io[1];
  out->w_eval = G(w_eval);
  out->in_eval = G(in_eval);
  out->out_eval = G(out_eval);

  // Multiplicity sumcheck (prover.rs:9449-9511): degree-1 rounds over
  // 2^table_log entries.  The multiplicities reached the pinned copy before
  // the kernels whose results were waited for above; they count every padded
  // input once, so their sum is n.
  memcpy(out->multiplicities, c->h_mult, tsize * sizeof(uint32_t));
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
    const qm31* src = m0;
    int np = 0;
    const qm31* pend = nullptr;
    std::vector<qm31> mchal(table_log);
    for (size_t j = 0; j < mtrips.size(); j++) {
      const Trip& tr = mtrips[j];
      const bool last = j + 1 == mtrips.size();
      RoundSink sk;
      if (j == 0) {
        sk = sk_mult0;
      } else {
        qm31* dst = bm[(j - 1) & 1];
        TRY(launch_trip(c, 2, tr.K, src, nullptr, tr.n, np, pend, dst, nullptr, nullptr, nullptr, 0, 0, &sk));
        src = dst;
      }
      if (last) TRY(ho.launch<1>(src, nullptr, tr.n, tr.K));
      qm31 g[kMaxSums];
      TRY(wait_trip(c, sk, trip_nq(2, tr.K), g));
      for (int i = 0; i < tr.K; i++) {
        qm31 sums[2];
        trip_round_sum(g, tr.K, i, mchal.data() + tr.t, sums);
        absorb1((uint32_t)(tr.t + i), sums);
        mchal[tr.t + i] = alpha;
      }
      np = tr.K;
      pend = mchal.data() + tr.t;
    }
    const int t_end = mtrips.back().t + mtrips.back().K;
    std::vector<qm31> v[1];
    TRY(ho.post(pend, np));
    TRY(ho.fetch(tsize >> t_end, 1, v));
    std::vector<qm31>& V = v[0];
    for (int t = t_end; t < (int)table_log; t++) {
      const size_t half = V.size() / 2;
      qm31 sums[2] = {qm31_zero(), qm31_zero()};
      {
        HostTimer ht(c, K_HOST_FINISH);
        for (size_t i = 0; i < half; i++) {
          sums[0] = qm31_add(sums[0], V[i]);
          sums[1] = qm31_add(sums[1], V[i + half]);
        }
      }
      absorb1((uint32_t)t, sums);
      HostTimer ht(c, K_HOST_FINISH);
      for (size_t i = 0; i < half; i++) V[i] = qm31_fold(V[i], V[i + half], alpha);
      V.resize(half);
    }
    mfin[0] = V[0];
  }
  out->mult_final_eval = G(mfin[0]);
  out->mult_claimed_sum = G(mult_sum);

  // Table commitment = poseidon_hash_many([type_tag, log_size]) (prover.rs:8365-8373)
  felt tc_in[2] = {felt_from_u64(tag), felt_from_u64(table_log)};
  const felt tc = poseidon_hash_many(tc_in, 2);
  out->table_commitment = felt_to_abi(tc);
  C.mix_secure_field(input_eval);
  C.mix_secure_field(Q(*claim_value));
  out->input_eval = G(input_eval);
  out->output_eval = *claim_value;

  if (proof) {
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
    L.mults.assign(out->multiplicities, out->multiplicities + tsize);
    for (uint32_t t = 0; t < 2 * table_log; t++) L.mult_rp.push_back(Q(out->mult_round_polys[t]));
    L.mult_final = mfin[0];
    L.mult_sum = mult_sum;
    proof->layers.push_back(L);
  }
  return GKR_OK;
}

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
  if (hipMemsetAsync(src, 1, n * 16, c->stream) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess) {
    rc = fail(GKR_ERR_DEVICE, "copy setup");
  } else {
    hipLaunchKernelGGL(k_copy16, dim3(g), dim3(kBlock), 0, c->stream, src, dst, n);  // warm-up
    (void)hipEventRecord(e0, c->stream);
    for (int i = 0; i < iters; i++) hipLaunchKernelGGL(k_copy16, dim3(g), dim3(kBlock), 0, c->stream, src, dst, n);
    (void)hipEventRecord(e1, c->stream);
    (void)hipEventSynchronize(e1);
    (void)hipEventElapsedTime(&ms, e0, e1);
    *copy_gbps = 2.0 * n * 16 * iters / (ms * 1e-3) / 1e9;
    (void)hipEventRecord(e0, c->stream);
    for (int i = 0; i < iters; i++)
      hipLaunchKernelGGL(k_read16, dim3(g), dim3(kBlock), 0, c->stream, src, n, (uint32_t*)dst);
    (void)hipEventRecord(e1, c->stream);
    (void)hipEventSynchronize(e1);
    (void)hipEventElapsedTime(&ms, e0, e1);
    *read_gbps = (double)n * 16 * iters / (ms * 1e-3) / 1e9;
    if (hipGetLastError() != hipSuccess) rc = fail(GKR_ERR_DEVICE, "copy kernels failed");
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(src);
  (void)hipFree(dst);
  return rc;
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
  hipLaunchKernelGGL(k_fill_synth_q, dim3(partial_grid(n) * 8), dim3(kBlock), 0, c->stream, d, n, seed);
  int rc = check_launch();
  if (rc == GKR_OK) rc = sync(c);
  if (rc != GKR_OK) {
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
  return rc;
}

/* ------------------------------------------------------------------ MLE commitments
 * Poseidon Merkle roots (merkle.h).  A batch runs level by level: launch L
 * moves every unfinished tree from level s to s + d, writing the real nodes
 * of level s + d into buffer L % 2 and reading level s from the other one.
 * d is the largest of 4..2 that still gives 2^18 output nodes over the
 * batch, else 1 (the upper levels are latency-bound: one hash per thread per
 * launch keeps them short). */
struct MerkleTreeSpec {
  uint32_t kind;  // 0 matrix, 1 QM31 vector
  const uint32_t* src;
  uint64_t rows, cols;
  uint32_t log_pk, height;
  uint64_t mle_len;
};

static uint32_t log2_ceil(uint64_t v) {
  uint32_t l = 0;
  while ((1ull << l) < v) l++;
  return l;
}

static int merkle_consts(gkr_ctx* c, const MerkleConsts** out) {
  if (!c->merkle_consts) {
    const f9::setup& S = f9::host_setup();
    std::unique_ptr<MerkleConsts> h(new MerkleConsts());
    h->hk = S.k;
    h->r2 = S.r2;
    h->one = S.one;
    const felt two124 = felt_to_mont(felt{{0, (uint64_t)1 << 60, 0, 0}});  // securefield_to_felt(0) = 2^124
    felt z = two124, zz = felt_zero();
    for (int s = 0; s < 64; s++) {
      h->z[s] = f9::from_host_mont(z);
      h->zz[s] = f9::from_host_mont(zz);
      z = poseidon_hash(z, z);
      zz = poseidon_hash(zz, zz);
    }
    MerkleConsts* d = nullptr;
    HIP_TRY(hipMalloc(&d, sizeof(MerkleConsts)));
    if (hipMemcpy(d, h.get(), sizeof(MerkleConsts), hipMemcpyHostToDevice) != hipSuccess) {
      (void)hipFree(d);
      return fail(GKR_ERR_DEVICE, "copy of the Merkle constants failed");
    }
    c->merkle_consts = d;
  }
  *out = c->merkle_consts;
  return GKR_OK;
}

// kept == nullptr: roots only (ping-pong level buffers).  Otherwise every level
// of every tree is kept in one arena (one level per launch) and described in
// (*kept)[i] for path extraction; the arena stays valid until the next call.
static int merkle_roots(gkr_ctx* c, const std::vector<MerkleTreeSpec>& trees, gkr_felt* roots,
                        std::vector<MerkleKept>* kept = nullptr) {
  const size_t nt = trees.size();
  if (nt == 0) return GKR_OK;
  const MerkleConsts* K;
  TRY(merkle_consts(c, &K));
  struct Launch {
    uint32_t s;
    size_t first_step, n_steps;
    uint64_t total;
  };
  std::vector<Launch> launches;
  std::vector<MerkleStep> steps;
  std::vector<uint64_t> step_off;  // node offset of each step's output in its buffer (arena when kept)
  std::vector<std::pair<size_t, size_t>> root_at(nt);  // (launch, step) producing each root
  uint64_t need[2] = {1, 1}, arena = 0;
  uint32_t smax = 0;
  for (const auto& t : trees) smax = std::max(smax, t.height);
  for (uint32_t s = 0; s < smax;) {
    auto outputs = [&](uint32_t D) {
      uint64_t n = 0;
      for (const auto& t : trees)
        if (t.height > s) n += merkle_real_count(t.kind, t.rows, t.cols, t.log_pk, s + std::min(D, t.height - s));
      return n;
    };
    uint32_t D = 1;
    if (!kept)
      for (uint32_t cand = kMerkleMaxD; cand >= 2; cand--)
        if (outputs(cand) >= (1ull << 18)) {
          D = cand;
          break;
        }
    Launch L{s, steps.size(), 0, 0};
    uint64_t off = 0;
    for (size_t i = 0; i < nt; i++) {
      const auto& t = trees[i];
      if (t.height <= s) continue;
      MerkleStep st{};
      st.src = t.src;
      st.rows = t.rows;
      st.cols = t.cols;
      st.mle_len = t.mle_len;
      st.kind = t.kind;
      st.log_pk = t.log_pk;
      st.d = std::min(D, t.height - s);
      st.n_out = merkle_real_count(t.kind, t.rows, t.cols, t.log_pk, s + st.d);
      st.thread_begin = L.total;
      L.total += st.n_out;
      step_off.push_back(kept ? arena : off);
      off += st.n_out;
      arena += st.n_out;
      if (s + st.d == t.height) root_at[i] = {launches.size(), steps.size()};
      steps.push_back(st);
    }
    L.n_steps = steps.size() - L.first_step;
    need[launches.size() & 1] = std::max(need[launches.size() & 1], off);
    launches.push_back(L);
    s += D;
  }
  f9::fe* buf[2] = {nullptr, nullptr};
  if (kept) {
    TRY(ensureT(c, S_MK0, arena, &buf[0]));
    kept->assign(nt, MerkleKept{});
    for (size_t i = 0; i < nt; i++) {
      MerkleKept& k = (*kept)[i];
      k.src = trees[i].src;
      k.rows = trees[i].rows;
      k.cols = trees[i].cols;
      k.mle_len = trees[i].mle_len;
      k.kind = trees[i].kind;
      k.log_pk = trees[i].log_pk;
      k.height = trees[i].height;
    }
  } else {
    TRY(ensureT(c, S_MK0, need[0], &buf[0]));
    TRY(ensureT(c, S_MK1, need[1], &buf[1]));
  }
  void* droot;
  TRY(ensure(c, S_MKROOT, nt * (sizeof(f9::fe) + sizeof(void*) + 32), &droot));
  f9::fe* root_nodes = (f9::fe*)droot;
  const f9::fe** dptr = (const f9::fe**)(root_nodes + nt);
  uint32_t* dwords = (uint32_t*)(dptr + nt);
  // wire the buffers: a tree's input is its previous output.  Roots only:
  // launch l writes buf[l & 1], and a tree's last launch writes its root to
  // root_nodes (later launches reuse the ping-pong buffers).  Kept: every
  // output has its own place in the arena.
  std::vector<const f9::fe*> prev(nt, nullptr);
  for (size_t l = 0; l < launches.size(); l++) {
    size_t k = launches[l].first_step;
    for (size_t i = 0; i < nt; i++) {
      if (trees[i].height <= launches[l].s) continue;
      steps[k].in = prev[i];
      if (kept) {
        steps[k].out = buf[0] + step_off[k];
        (*kept)[i].level[launches[l].s + steps[k].d] = steps[k].out;
      } else {
        steps[k].out = root_at[i].second == k ? root_nodes + i : buf[l & 1] + step_off[k];
      }
      prev[i] = steps[k].out;
      k++;
    }
  }
  MerkleStep* dsteps;
  TRY(ensureT(c, S_MKSTEP, steps.size(), &dsteps));
  HIP_TRY(hipMemcpyAsync(dsteps, steps.data(), steps.size() * sizeof(MerkleStep), hipMemcpyHostToDevice, c->stream));
  for (const auto& L : launches) {
    const uint64_t blocks = (L.total + kMerkleBlock - 1) / kMerkleBlock;
    uint64_t hashes = 0;  // the timer's byte counter holds the hash count of this kernel
    for (size_t k = L.first_step; k < L.first_step + L.n_steps; k++) hashes += steps[k].n_out * ((1ull << steps[k].d) - 1);
    TimedLaunch tl(c, K_MERKLE, hashes);
    k_merkle_level<<<dim3((uint32_t)blocks), dim3(kMerkleBlock), 0, c->stream>>>(dsteps + L.first_step, (int)L.n_steps,
                                                                              L.s, L.total, K);
    HIP_TRY(hipGetLastError());
  }
  std::vector<const f9::fe*> rp(nt);
  for (size_t i = 0; i < nt; i++) rp[i] = kept ? steps[root_at[i].second].out : root_nodes + i;
  HIP_TRY(hipMemcpyAsync(dptr, rp.data(), nt * sizeof(void*), hipMemcpyHostToDevice, c->stream));
  k_merkle_roots<<<dim3((uint32_t)((nt + 63) / 64)), dim3(64), 0, c->stream>>>(dptr, (int)nt, K, dwords);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipMemcpyAsync(roots, dwords, nt * 32, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return GKR_OK;
}

static int weight_tree(const gkr_matrix* m, MerkleTreeSpec* t) {
  if (!m || !m->dev || m->rows == 0 || m->cols == 0) return fail(GKR_ERR_INVALID, "weight commitment: empty matrix");
  t->kind = 0;
  t->src = m->dev;
  t->rows = m->rows;
  t->cols = m->cols;
  t->log_pk = log2_ceil(m->rows);
  const uint32_t log_pn = log2_ceil(m->cols);
  if (t->log_pk + log_pn > 48) return fail(GKR_ERR_INVALID, "weight commitment: padded MLE above 2^48 entries");
  t->mle_len = 1ull << (t->log_pk + log_pn);
  t->height = std::max(1u, t->log_pk + log_pn);
  return GKR_OK;
}

extern "C" int gkr_weight_commitment(gkr_ctx* c, const gkr_matrix* b, gkr_felt* root) {
  if (!c || !root) return fail(GKR_ERR_INVALID, "null argument");
  return gkr_weight_commitments(c, &b, 1, root);
}

extern "C" int gkr_weight_commitments(gkr_ctx* c, const gkr_matrix* const* mats, size_t count, gkr_felt* roots) {
  if (!c || (count && (!mats || !roots))) return fail(GKR_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(c->device));
  std::vector<MerkleTreeSpec> trees(count);
  for (size_t i = 0; i < count; i++) TRY(weight_tree(mats[i], &trees[i]));
  return merkle_roots(c, trees, roots);
}

extern "C" int gkr_mle_commitment(gkr_ctx* c, const gkr_qvec* evals, gkr_felt* root) {
  if (!c || !evals || !root) return fail(GKR_ERR_INVALID, "null argument");
  if (evals->n == 0) return fail(GKR_ERR_INVALID, "MLE commitment: empty vector");
  HIP_TRY(hipSetDevice(c->device));
  MerkleTreeSpec t{};
  t.kind = 1;
  t.src = (const uint32_t*)evals->dev;
  t.rows = evals->n;
  t.cols = 1;
  t.mle_len = evals->n;
  t.height = std::max(1u, log2_ceil(evals->n));
  if (t.height > 48) return fail(GKR_ERR_INVALID, "MLE commitment: above 2^48 entries");
  return merkle_roots(c, {t}, root);
}

/* ------------------------------------------------------------------ forward GEMM
 * C = A * B mod P for canonical M31 matrices (gemm.h).  B's digit planes (only
 * up to its highest non-zero plane) are built once per matrix and kept with
 * it; A's four planes are built per call into a context slot.  One wave per 32 x 32 tile
 * of C and K split; the splits (each at most 16384 deep, enough of them for
 * ~2048 workgroups) are added by k_gemm_reduce. */
static int digit_planes_needed(gkr_ctx* c, const uint32_t* X, uint64_t count, int* nplanes) {
  uint32_t* dmask;
  TRY(ensureT(c, S_GEMMP, 1, &dmask));
  HIP_TRY(hipMemsetAsync(dmask, 0, 4, c->stream));
  const uint64_t blocks = std::min<uint64_t>((count + 255) / 256, 256);
  k_digit_mask<<<dim3((uint32_t)std::max<uint64_t>(blocks, 1)), dim3(256), 0, c->stream>>>(X, count, dmask);
  HIP_TRY(hipGetLastError());
  uint32_t mask = 0;
  HIP_TRY(hipMemcpyAsync(&mask, dmask, 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  int np = 1;
  for (int p = 0; p < 4; p++)
    if (mask & (1u << p)) np = p + 1;
  *nplanes = np;
  return GKR_OK;
}

static int pack_planes(gkr_ctx* c, const uint32_t* X, uint64_t outer, uint64_t K, bool kmajor, int np, int8_t* out,
                       uint32_t* mask = nullptr) {
  const uint64_t ntiles = (outer + kGemmTile - 1) / kGemmTile, nsteps = (K + kGemmK - 1) / kGemmK;
  const uint64_t slots = ntiles * nsteps * 64;
  k_digit_pack<<<dim3((uint32_t)((slots + 255) / 256)), dim3(256), 0, c->stream>>>(X, outer, K, kmajor, np, ntiles,
                                                                                  nsteps, out, mask);
  HIP_TRY(hipGetLastError());
  return GKR_OK;
}

static int weight_planes(gkr_ctx* c, gkr_matrix* b) {
  if (b->bplanes) return GKR_OK;
  int np;
  TRY(digit_planes_needed(c, b->dev, b->rows * b->cols, &np));
  const uint64_t ntiles = (b->cols + kGemmTile - 1) / kGemmTile, nsteps = (b->rows + kGemmK - 1) / kGemmK;
  int8_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, (size_t)np * ntiles * nsteps * kGemmBlockBytes));
  const int rc = pack_planes(c, b->dev, b->cols, b->rows, true, np, d);
  if (rc != GKR_OK) {
    (void)hipFree(d);
    return rc;
  }
  b->bplanes = d;
  b->bnplanes = np;
  return GKR_OK;
}

template <int PA, int PB, int U>
static void launch_gemm(gkr_ctx* c, dim3 grid, const int8_t* ap, uint64_t apb, const uint32_t* amask,
                        const int8_t* bp, uint64_t bpb, uint64_t m, uint64_t n, uint64_t nsteps, uint64_t rt,
                        uint64_t ctl, uint64_t sps, uint32_t* out) {
  k_gemm_m31<PA, PB, U><<<grid, dim3(256), 0, c->stream>>>(ap, apb, amask, bp, bpb, m, n, nsteps, rt, ctl, sps, out);
}

static int matmul_forward(gkr_ctx* c, const gkr_matrix* a, gkr_matrix* b, uint32_t* C) {
  const uint64_t m = a->rows, k = a->cols, n = b->cols;
  TRY(weight_planes(c, b));
  const uint64_t nsteps = (k + kGemmK - 1) / kGemmK;
  const uint64_t rtiles = (m + kGemmTile - 1) / kGemmTile, ctiles = (n + kGemmTile - 1) / kGemmTile;
  const uint64_t a_plane = rtiles * nsteps * kGemmBlockBytes, b_plane = ctiles * nsteps * kGemmBlockBytes;
  // A: all four planes packed (A is small) with its non-zero mask on the device;
  // B: 1 plane (int8-range weights) or 4
  const int PB = b->bnplanes == 1 ? 1 : 4;
  void* abuf;
  TRY(ensure(c, S_GEMMA, 256 + (size_t)4 * a_plane, &abuf));
  uint32_t* amask = (uint32_t*)abuf;
  int8_t* ap = (int8_t*)abuf + 256;
  HIP_TRY(hipMemsetAsync(amask, 0, 4, c->stream));
  TRY(pack_planes(c, a->dev, m, k, false, 4, ap, amask));
  const int8_t* bp = b->bplanes;
  if (PB > b->bnplanes) {  // a 2- or 3-plane weight: extend with zero planes in scratch
    int8_t* ext;
    TRY(ensureT(c, S_GEMMB, (size_t)4 * b_plane, &ext));
    HIP_TRY(hipMemcpyAsync(ext, b->bplanes, (size_t)b->bnplanes * b_plane, hipMemcpyDeviceToDevice, c->stream));
    HIP_TRY(hipMemsetAsync(ext + (size_t)b->bnplanes * b_plane, 0, (size_t)(4 - b->bnplanes) * b_plane, c->stream));
    bp = ext;
  }
  const uint64_t waves = rtiles * ctiles, blocks_x = (waves + 3) / 4;
  uint64_t splits = (2048 + blocks_x - 1) / blocks_x;
  splits = std::min<uint64_t>(splits, std::max<uint64_t>(1, nsteps / 16));
  splits = std::max<uint64_t>(splits, (nsteps * kGemmK + kGemmMaxKPass - 1) / kGemmMaxKPass);
  const uint64_t sps = (nsteps + splits - 1) / splits;
  splits = (nsteps + sps - 1) / sps;
  if (blocks_x > 0x7fffffffull || splits > 65535) return fail(GKR_ERR_INVALID, "forward GEMM: grid too large");
  uint32_t* part = C;
  if (splits > 1) TRY(ensureT(c, S_GEMMP, splits * m * n, &part));
  const dim3 grid((uint32_t)blocks_x, (uint32_t)splits);
  // exactly one of each pair works (the other reads the mask and returns)
  if (PB == 1) {
    launch_gemm<1, 1, 16>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
    launch_gemm<4, 1, 4>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
  } else {
    launch_gemm<1, 4, 4>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
    launch_gemm<4, 4, 2>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
  }
  HIP_TRY(hipGetLastError());
  if (splits > 1) {
    const uint64_t count = m * n;
    k_gemm_reduce<<<dim3((uint32_t)((count + 255) / 256)), dim3(256), 0, c->stream>>>(part, count, (int)splits, C);
    HIP_TRY(hipGetLastError());
  }
  return GKR_OK;
}

extern "C" int gkr_matmul_forward_into(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, gkr_matrix* out) {
  if (!c || !a || !b || !out || !out->dev) return fail(GKR_ERR_INVALID, "null argument");
  if (a->cols != b->rows || out->rows != a->rows || out->cols != b->cols)
    return fail(GKR_ERR_INVALID, "forward GEMM: A %llux%llu . B %llux%llu into %llux%llu", (unsigned long long)a->rows,
                (unsigned long long)a->cols, (unsigned long long)b->rows, (unsigned long long)b->cols,
                (unsigned long long)out->rows, (unsigned long long)out->cols);
  if (out == a || out == b) return fail(GKR_ERR_INVALID, "forward GEMM: output aliases an input");
  HIP_TRY(hipSetDevice(c->device));
  if (out->bplanes || out->r8 || out->r8_state) {  // the contents change: drop the derived copies
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (out->bplanes) (void)hipFree(out->bplanes);
    if (out->r8) (void)hipFree(out->r8);
    out->bplanes = nullptr;
    out->bnplanes = 0;
    out->r8 = nullptr;
    out->r8_state = 0;
  }
  if (c->mm.a == out || c->mm.b == out) c->mm.valid = false;
  return matmul_forward(c, a, const_cast<gkr_matrix*>(b), out->dev);
}

extern "C" int gkr_matmul_forward(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, gkr_matrix** out) {
  if (!c || !a || !b || !out) return fail(GKR_ERR_INVALID, "null argument");
  if (a->cols != b->rows)
    return fail(GKR_ERR_INVALID, "forward GEMM: A is %llux%llu, B is %llux%llu", (unsigned long long)a->rows,
                (unsigned long long)a->cols, (unsigned long long)b->rows, (unsigned long long)b->cols);
  if (a->rows == 0 || a->cols == 0 || b->cols == 0) return fail(GKR_ERR_INVALID, "forward GEMM: empty matrix");
  HIP_TRY(hipSetDevice(c->device));
  uint32_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, a->rows * b->cols * sizeof(uint32_t)));
  int rc = matmul_forward(c, a, const_cast<gkr_matrix*>(b), d);
  if (rc == GKR_OK) rc = sync(c);
  if (rc != GKR_OK) {
    (void)hipFree(d);
    return rc;
  }
  *out = new_matrix(c, d, a->rows, b->cols, true);
  return GKR_OK;
}

/* ------------------------------------------------------------------ weight openings
 * prove_mle_opening_with_commitment (engine/src/crypto/mle_opening.rs:1654-1915)
 * over matrix_to_mle_col_major_padded(B):
 *   layer 0 = the padded MLE (read from B), layer t+1 = fold of layer t on its
 *   top variable with eval_point[t]; the Merkle tree of every layer longer
 *   than 1 is built once with all its levels kept (the reference rebuilds
 *   them for the query phase); roots are mixed in layer order; query pairs are
 *   drawn (low 64 bits of draw_felt252 mod len/2, then mod max(mid/2, 1) per
 *   round); values and auth paths are gathered on the device.
 * Layers 1..log2(pn) keep B's zero rows (a grid with `rows` real rows, kind 2
 * trees); later layers are plain QM31 vectors (kind 1).  The record holds the
 * serialized claim and MleOpeningProof (cairo_serde.rs:341-369, 1759-1767). */
constexpr size_t kMleQueries = 10;  // MLE_N_QUERIES, mle_opening.rs:47

static int weight_opening(gkr_ctx* c, const gkr_matrix* b, const gkr_qm31* point, uint32_t n_point,
                          const gkr_qm31* expected, PoseidonChannel& C, felt* commitment, std::vector<felt>& rec) {
  MerkleTreeSpec t0;
  TRY(weight_tree(b, &t0));
  const uint32_t log_pk = t0.log_pk, log_pn = log2_ceil(b->cols), nv = log_pk + log_pn;
  if (n_point != nv) return fail(GKR_ERR_INVALID, "weight opening: point has %u vars, the padded MLE has %u", n_point, nv);
  for (uint32_t t = 0; t < nv; t++)
    if (!canonical_q(point[t])) return fail(GKR_ERR_INVALID, "weight opening: point not canonical");
  const uint64_t N = 1ull << nv;
  // folded layers 1..nv, back to back (N - 1 values)
  qm31* lay = nullptr;
  TRY(ensureT(c, S_OPL, N, &lay));
  std::vector<qm31*> L(nv + 1, nullptr);
  for (uint64_t t = 1, off = 0; t <= nv; t++) {
    L[t] = lay + off;
    off += N >> t;
  }
  for (uint32_t t = 0; t < nv; t++) {
    const uint64_t mid = N >> (t + 1);
    const uint32_t blocks = (uint32_t)((mid + 255) / 256);
    if (t == 0)
      k_open_fold_matrix<<<dim3(blocks), dim3(256), 0, c->stream>>>(b->dev, b->rows, b->cols, log_pk, mid,
                                                                    Q(point[0]), L[1]);
    else
      k_open_fold<<<dim3(blocks), dim3(256), 0, c->stream>>>(L[t], mid, Q(point[t]), L[t + 1]);
    HIP_TRY(hipGetLastError());
  }
  // trees of layers 0..nv-1 (layer 0 also when nv == 0: one leaf padded to two)
  std::vector<MerkleTreeSpec> trees(1, t0);
  for (uint32_t t = 1; t < nv; t++) {
    MerkleTreeSpec s{};
    s.src = (const uint32_t*)L[t];
    s.mle_len = N >> t;
    s.height = nv - t;
    if (t <= log_pn) {
      s.kind = 2;
      s.rows = b->rows;
      s.cols = 1ull << (log_pn - t);
      s.log_pk = log_pk;
    } else {
      s.kind = 1;
      s.rows = N >> t;
      s.cols = 1;
    }
    trees.push_back(s);
  }
  std::vector<gkr_felt> roots(trees.size());
  std::vector<MerkleKept> kept;
  TRY(merkle_roots(c, trees, roots.data(), &kept));
  qm31 final_value;
  if (nv == 0) {
    uint32_t v;
    HIP_TRY(hipMemcpy(&v, b->dev, 4, hipMemcpyDeviceToHost));
    final_value = qm31_from_m31(v);
  } else {
    HIP_TRY(hipMemcpy(&final_value, L[nv], sizeof(qm31), hipMemcpyDeviceToHost));
  }
  if (expected && !qm31_eq(final_value, Q(*expected)))
    return fail(GKR_ERR_INVALID, "weight opening: the MLE at the point differs from the expected value");
  std::vector<felt> rf(trees.size());
  for (size_t t = 0; t < trees.size(); t++) rf[t] = felt_canon_from_words(roots[t].w);
  *commitment = rf[0];
  for (size_t t = 0; t < trees.size(); t++) C.mix_felt(felt_to_mont(rf[t]));
  // queries
  const uint64_t half = N / 2;
  const size_t nq = (size_t)std::min<uint64_t>(kMleQueries, half);
  std::vector<uint64_t> pairs(nq);
  for (size_t q = 0; q < nq; q++) {
    const felt f = felt_from_mont(C.draw_felt252());
    pairs[q] = f.l[0] % half;
  }
  std::vector<MerkleGather> items;
  for (size_t q = 0; q < nq; q++) {
    uint64_t idx = pairs[q];
    for (uint32_t t = 0; t < nv; t++) {
      const uint64_t mid = (N >> t) / 2, li = idx, ri = mid + idx;
      items.push_back(MerkleGather{t, 0, 1, 0, li});
      items.push_back(MerkleGather{t, 0, 1, 0, ri});
      for (uint64_t k0 : {li, ri}) {
        uint64_t k = k0;
        for (uint32_t lv = 0; lv < trees[t].height; lv++) {
          items.push_back(MerkleGather{t, lv, 0, 0, k ^ 1});
          k >>= 1;
        }
      }
      idx %= std::max<uint64_t>(mid / 2, 1);
    }
  }
  std::vector<uint32_t> got(8 * items.size());
  if (!items.empty()) {
    void* dio;
    const size_t kbytes = kept.size() * sizeof(MerkleKept), ibytes = items.size() * sizeof(MerkleGather);
    TRY(ensure(c, S_OPI, kbytes + ibytes + got.size() * 4, &dio));
    MerkleKept* dk = (MerkleKept*)dio;
    MerkleGather* di = (MerkleGather*)((char*)dio + kbytes);
    uint32_t* dout = (uint32_t*)((char*)dio + kbytes + ibytes);
    HIP_TRY(hipMemcpyAsync(dk, kept.data(), kbytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(di, items.data(), ibytes, hipMemcpyHostToDevice, c->stream));
    const MerkleConsts* K;
    TRY(merkle_consts(c, &K));
    k_merkle_gather<<<dim3((uint32_t)((items.size() + 63) / 64)), dim3(64), 0, c->stream>>>(dk, di, (int)items.size(),
                                                                                          K, dout);
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipMemcpyAsync(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
  }
  // record: claim point, expected value, MleOpeningProof
  auto fu = [&](uint64_t v) { rec.push_back(felt{{v, 0, 0, 0}}); };
  auto fq = [&](const qm31& x) { fu(x.a); fu(x.b); fu(x.c); fu(x.d); };
  fu(nv);
  for (uint32_t t = 0; t < nv; t++) fq(Q(point[t]));
  fq(expected ? Q(*expected) : final_value);
  fu(nv > 0 ? nv - 1 : 0);
  for (uint32_t t = 1; t < nv; t++) rec.push_back(rf[t]);
  fu(nq);
  size_t it = 0;
  for (size_t q = 0; q < nq; q++) {
    fu(pairs[q]);
    fu(nv);
    for (uint32_t t = 0; t < nv; t++) {
      for (int side = 0; side < 2; side++, it++) fq(qm31{got[8 * it], got[8 * it + 1], got[8 * it + 2], got[8 * it + 3]});
      for (int side = 0; side < 2; side++) {
        fu(trees[t].height);
        for (uint32_t lv = 0; lv < trees[t].height; lv++, it++) rec.push_back(felt_canon_from_words(&got[8 * it]));
      }
    }
  }
  fq(final_value);
  return GKR_OK;
}

extern "C" int gkr_prove_weight_opening(gkr_ctx* c, const gkr_matrix* b, const gkr_qm31* eval_point, uint32_t n_point,
                                        const gkr_qm31* expected_value, gkr_channel* ch, gkr_proof* proof,
                                        gkr_felt* commitment) {
  CH_CHECK(ch);
  if (!c || !b || !proof || (!eval_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (expected_value && !canonical_q(*expected_value)) return fail(GKR_ERR_INVALID, "expected value not canonical");
  HIP_TRY(hipSetDevice(c->device));
  felt cm;
  std::vector<felt> rec;
  TRY(weight_opening(c, b, eval_point, n_point, expected_value, ch->ch, &cm, rec));
  proof->weight_commitments.push_back(cm);
  proof->weight_openings.push_back(std::move(rec));
  if (commitment) felt_canon_to_words(cm, commitment->w);
  return GKR_OK;
}

extern "C" int gkr_prove_weight_openings(gkr_ctx* c, gkr_channel* ch, gkr_proof* proof) {
  return gkr_prove_weight_binding(c, ch, proof, GKR_WEIGHT_SEQUENTIAL);
}

// The weight phase of the GKR prover (prover.rs:2059-2200) over the claims the
// proof recorded, in recording order.
//   SEQUENTIAL: one opening per claim on the main channel (prover.rs:2160-2190).
//   AGGREGATED_RLC: the reference default, the aggregated oracle sumcheck without
//     the full binding proof (prover.rs:368-658): the commitment of every claimed
//     weight (one batch) goes into the proof, then rho = draw_qm31 and
//     mix_secure_field(sum rho^i v_i) (prover.rs:1335-1345); no openings.
//   RLC_DIRECT: apply_aggregated_rlc_binding (prover.rs:669-699): rho and the
//     combined value only, no commitments.
extern "C" int gkr_prove_weight_binding(gkr_ctx* c, gkr_channel* ch, gkr_proof* proof, int mode) {
  CH_CHECK(ch);
  if (!c || !proof) return fail(GKR_ERR_INVALID, "null argument");
  if (mode != GKR_WEIGHT_SEQUENTIAL && mode != GKR_WEIGHT_AGGREGATED_RLC && mode != GKR_WEIGHT_RLC_DIRECT)
    return fail(GKR_ERR_INVALID, "unknown weight binding mode %d", mode);
  auto& claims = proof->weight_claims;
  if (mode == GKR_WEIGHT_SEQUENTIAL) {
    for (const WeightClaimRec& w : claims) {
      const gkr_qm31* pt = reinterpret_cast<const gkr_qm31*>(w.point.data());
      const gkr_qm31 v = {{w.value.a, w.value.b, w.value.c, w.value.d}};
      TRY(gkr_prove_weight_opening(c, w.b, pt, (uint32_t)w.point.size(), &v, ch, proof, nullptr));
    }
    claims.clear();
    return GKR_OK;
  }
  if (claims.empty()) return GKR_OK;
  if (mode == GKR_WEIGHT_AGGREGATED_RLC) {
    // one root per distinct matrix, repeated per claim
    std::vector<const gkr_matrix*> uniq;
    std::map<const gkr_matrix*, size_t> at;
    for (const auto& w : claims)
      if (at.emplace(w.b, uniq.size()).second) uniq.push_back(w.b);
    std::vector<gkr_felt> roots(uniq.size());
    TRY(gkr_weight_commitments(c, uniq.data(), uniq.size(), roots.data()));
    for (const auto& w : claims) proof->weight_commitments.push_back(felt_canon_from_words(roots[at[w.b]].w));
  }
  PoseidonChannel& C = ch->ch;
  const qm31 rho = C.draw_qm31();
  qm31 pw = qm31_one(), combined = qm31_zero();
  for (const auto& w : claims) {
    combined = qm31_add(combined, qm31_mul(pw, w.value));
    pw = qm31_mul(pw, rho);
  }
  C.mix_secure_field(combined);
  claims.clear();
  return GKR_OK;
}

// ------------------------------------------------------------------ Mul layer
// reduce_mul_layer (gkr/prover.rs:6172-6271) over the padded QM31 MLEs held in
// S_W0 (lhs) and S_D0 (rhs), n = 2^nv entries each.
static int mul_layer_core(gkr_ctx* c, const std::vector<qm31>& cpt, const qm31& claim, int nv, gkr_channel* ch,
                          gkr_proof* proof, gkr_mul_out* out) {
  const uint64_t n = 1ull << nv;
  qm31 *d_w0, *d_w1, *d_d0, *d_d1;
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_W1, n / 2 + 1, &d_w1));
  TRY(ensureT(c, S_D0, n, &d_d0));
  TRY(ensureT(c, S_D1, n / 2 + 1, &d_d1));
  PoseidonChannel& C = ch->ch;
  Eq3Plan epl;  // eq over the first nv claim coordinates, kept factored
  TRY(eq3_prepare(c, cpt.data(), nv, &epl));
  C.mix_u64(0x4D554Cull);  // "MUL"
  C.mix_secure_field(claim);
  std::vector<qm31> chal(nv);
  qm31 fin[3];
  TRY(eq3_sumcheck(c, C, cpt.data(), epl, d_w0, d_d0, d_w1, d_d1, out->eq_round_polys, chal.data(), fin));
  const qm31 lhs = fin[1], rhs = fin[2];
  C.mix_secure_field(lhs);
  C.mix_secure_field(rhs);
  const qm31 alpha = C.draw_qm31();
  const qm31 comb = qm31_add(qm31_mul(alpha, lhs), qm31_mul(qm31_sub(qm31_one(), alpha), rhs));
  out->lhs_eval = G(lhs);
  out->rhs_eval = G(rhs);
  out->alpha = G(alpha);
  out->next_value = G(comb);
  out->n_vars = (uint32_t)nv;
  if (proof) {
    LayerRec L;
    L.tag = 2;
    L.claim_value = claim;
    L.rp.resize(4 * (size_t)nv);
    for (size_t i = 0; i < L.rp.size(); i++) L.rp[i] = Q(out->eq_round_polys[i]);
    L.final_a = lhs;
    L.final_b = rhs;
    proof->layers.push_back(std::move(L));
  }
  return GKR_OK;
}
static int mul_check_claim(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value, int nv,
                           gkr_mul_out* out, std::vector<qm31>* cpt) {
  if (!claim_value || !out || (!claim_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (nv > kMaxVars) return fail(GKR_ERR_INVALID, "mul layer too large");
  if ((int)n_point < nv) return fail(GKR_ERR_INVALID, "claim point too short for MLE size (%u < %d)", n_point, nv);
  if (!out->eq_round_polys && nv > 0) return fail(GKR_ERR_INVALID, "null eq_round_polys");
  if (!canonical_q(*claim_value)) return fail(GKR_ERR_INVALID, "claim value not canonical");
  cpt->resize(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(claim_point[l])) return fail(GKR_ERR_INVALID, "claim point not canonical");
    (*cpt)[l] = Q(claim_point[l]);
  }
  return GKR_OK;
}
// Padded QM31 MLEs of two resident matrices into S_W0 / S_D0; returns nv.
static int mul_stage_matrices(gkr_ctx* c, const gkr_matrix* lhs, const gkr_matrix* rhs, int* nv_out) {
  if (!lhs || !rhs) return fail(GKR_ERR_INVALID, "null matrix");
  if (lhs->ctx != c || rhs->ctx != c) return fail(GKR_ERR_INVALID, "matrix belongs to another context");
  const uint64_t nl = next_pow2(lhs->rows) * next_pow2(lhs->cols);
  const uint64_t nr = next_pow2(rhs->rows) * next_pow2(rhs->cols);
  if (nl != nr) return fail(GKR_ERR_INVALID, "lhs and rhs must have same length (%llu vs %llu)",
                            (unsigned long long)nl, (unsigned long long)nr);
  const int nv = log2_exact(nl);
  if (nv > kMaxVars) return fail(GKR_ERR_INVALID, "mul layer too large");
  qm31 *d_w0, *d_d0;
  TRY(ensureT(c, S_W0, nl, &d_w0));
  TRY(ensureT(c, S_D0, nl, &d_d0));
  hipLaunchKernelGGL(k_pad_q, dim3(grid_for(nl)), dim3(kBlock), 0, c->stream, lhs->dev, lhs->rows, lhs->cols,
                     log2_exact(next_pow2(lhs->cols)), nl, d_w0);
  TRY(check_launch());
  hipLaunchKernelGGL(k_pad_q, dim3(grid_for(nl)), dim3(kBlock), 0, c->stream, rhs->dev, rhs->rows, rhs->cols,
                     log2_exact(next_pow2(rhs->cols)), nl, d_d0);
  TRY(check_launch());
  *nv_out = nv;
  return GKR_OK;
}

extern "C" int gkr_prove_mul_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                   const gkr_qm31* claim_value, const gkr_matrix* lhs, const gkr_matrix* rhs,
                                   gkr_channel* ch, gkr_proof* proof, gkr_mul_out* out) {
  CH_CHECK(ch);
  if (!c) return fail(GKR_ERR_INVALID, "null context");
  HIP_TRY(hipSetDevice(c->device));
  int nv = 0;
  TRY(mul_stage_matrices(c, lhs, rhs, &nv));
  std::vector<qm31> cpt;
  TRY(mul_check_claim(claim_point, n_point, claim_value, nv, out, &cpt));
  c->mm.valid = false;
  return mul_layer_core(c, cpt, Q(*claim_value), nv, ch, proof, out);
}

extern "C" int gkr_reduce_mul_layer(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point,
                                    const gkr_qm31* claim_value, const gkr_qm31* lhs_vals, const gkr_qm31* rhs_vals,
                                    uint64_t n, gkr_channel* ch, gkr_proof* proof, gkr_mul_out* out) {
  CH_CHECK(ch);
  if (!c || !lhs_vals || !rhs_vals) return fail(GKR_ERR_INVALID, "null argument");
  if (n == 0 || (n & (n - 1))) return fail(GKR_ERR_INVALID, "MLE size must be power of 2 (got %llu)",
                                          (unsigned long long)n);
  const int nv = log2_exact(n);
  std::vector<qm31> cpt;
  TRY(mul_check_claim(claim_point, n_point, claim_value, nv, out, &cpt));
  for (uint64_t i = 0; i < n; i++)
    if (!canonical_q(lhs_vals[i]) || !canonical_q(rhs_vals[i]))
      return fail(GKR_ERR_INVALID, "MLE value %llu not canonical", (unsigned long long)i);
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  qm31 *d_w0, *d_d0;
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_D0, n, &d_d0));
  HIP_TRY(hipMemcpyAsync(d_w0, lhs_vals, n * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(d_d0, rhs_vals, n * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
  return mul_layer_core(c, cpt, Q(*claim_value), nv, ch, proof, out);
}

// MLE of lhs (.) rhs (padded) at `point`: sum_x eq(point, x) lhs(x) rhs(x),
// one eq-weighted pass (a trip of no rounds; eq as a product of two tables).
extern "C" int gkr_mul_output_claim(gkr_ctx* c, const gkr_matrix* lhs, const gkr_matrix* rhs,
                                    const gkr_qm31* point, uint32_t n_point, gkr_qm31* out) {
  if (!c || !out || (!point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(c->device));
  int nv = 0;
  TRY(mul_stage_matrices(c, lhs, rhs, &nv));
  if ((int)n_point != nv) return fail(GKR_ERR_INVALID, "point has %u vars, product MLE has %d", n_point, nv);
  std::vector<qm31> pt(n_point);
  for (uint32_t l = 0; l < n_point; l++) {
    if (!canonical_q(point[l])) return fail(GKR_ERR_INVALID, "point not canonical");
    pt[l] = Q(point[l]);
  }
  c->mm.valid = false;
  const uint64_t n = 1ull << nv;
  qm31 *d_w0, *d_d0;
  TRY(ensureT(c, S_W0, n, &d_w0));
  TRY(ensureT(c, S_D0, n, &d_d0));
  const int h = nv < kEqLoMax ? nv : kEqLoMax;
  EqPartsArg arg;
  memset(&arg, 0, sizeof arg);
  arg.z = make_point(pt.data(), nv);
  arg.count = 2;
  arg.s[0] = 0;
  arg.m[0] = nv - h;
  arg.off[0] = 0;
  arg.s[1] = nv - h;
  arg.m[1] = h;
  arg.off[1] = 1u << (nv - h);
  const uint32_t total = arg.off[1] + (1u << h);
  qm31* parts;
  TRY(ensureT(c, S_EQPARTS, total, &parts));
  hipLaunchKernelGGL(k_eq_parts, dim3(grid_for(total)), dim3(kBlock), 0, c->stream, arg, total, parts);
  TRY(check_launch());
  RoundSink sk;
  TRY(launch_trip(c, 1, 0, d_w0, d_d0, n, 0, nullptr, nullptr, nullptr, parts, parts + arg.off[1], h, 0, &sk));
  qm31 v[1];
  TRY(wait_trip(c, sk, 1, v));
  *out = G(v[0]);
  return GKR_OK;
}

// ------------------------------------------------------------------ GKR walk
extern "C" int gkr_prove_walk(gkr_ctx* c, gkr_channel* ch, const gkr_step* steps, size_t n_steps,
                              const gkr_qm31* init_point, uint32_t n_init, const gkr_qm31* init_value,
                              gkr_proof* proof, gkr_qm31* final_point, uint32_t* n_final, gkr_qm31* final_value) {
  CH_CHECK(ch);
  if (!c || (!steps && n_steps) || !final_point || !n_final || !final_value)
    return fail(GKR_ERR_INVALID, "null argument");
  std::vector<gkr_qm31> point(init_point ? init_point : nullptr, init_point ? init_point + n_init : nullptr);
  gkr_qm31 value = init_value ? *init_value : G(qm31_zero());
  bool have_claim = init_value != nullptr;
  std::vector<gkr_qm31> rp, npnt(64);
  std::vector<uint32_t> mults;
  for (size_t si = 0; si < n_steps; si++) {
    const gkr_step& st = steps[si];
    if (!st.a) return fail(GKR_ERR_INVALID, "step %zu: null matrix", si);
    if (st.kind == GKR_STEP_MATMUL) {
      if (!st.b) return fail(GKR_ERR_INVALID, "step %zu: null weight matrix", si);
      const uint32_t nv = (uint32_t)(log2_exact(next_pow2(st.a->rows)) + log2_exact(next_pow2(st.b->cols)));
      if (st.claim == GKR_CLAIM_FRESH) {
        point.resize(nv);
        {
          HostTimer ht(c, K_HOST_DRAW);
          TRY(gkr_channel_draw_qm31s(ch, nv, point.data()));
        }
        TRY(gkr_matmul_output_claim(c, st.a, st.b, point.data(), nv, &value));
        ch->ch.mix_secure_field(Q(value));
      } else if (!have_claim) {
        return fail(GKR_ERR_INVALID, "step %zu: chained claim but no previous claim", si);
      }
      const int T = log2_exact(next_pow2(st.a->cols));
      rp.resize(3 * (size_t)(T > 0 ? T : 1));
      gkr_qm31 fa, fb, nval;
      TRY(gkr_prove_matmul_layer(c, point.data(), (uint32_t)point.size(), &value, st.a, st.b, ch, proof, rp.data(),
                                 &fa, &fb, npnt.data(), &nval));
      const uint32_t nn = (uint32_t)(log2_exact(next_pow2(st.a->rows)) + T);
      point.assign(npnt.begin(), npnt.begin() + nn);
      value = nval;
    } else if (st.kind == GKR_STEP_MUL) {
      if (!st.b) return fail(GKR_ERR_INVALID, "step %zu: null rhs matrix", si);
      const uint32_t nv = (uint32_t)(log2_exact(next_pow2(st.a->rows)) + log2_exact(next_pow2(st.a->cols)));
      if (st.claim == GKR_CLAIM_FRESH) {
        point.resize(nv);
        {
          HostTimer ht(c, K_HOST_DRAW);
          TRY(gkr_channel_draw_qm31s(ch, nv, point.data()));
        }
        TRY(gkr_mul_output_claim(c, st.a, st.b, point.data(), nv, &value));
        ch->ch.mix_secure_field(Q(value));
      } else if (!have_claim) {
        return fail(GKR_ERR_INVALID, "step %zu: chained claim but no previous claim", si);
      }
      rp.resize(4 * (size_t)(nv ? nv : 1));
      gkr_mul_out mo;
      memset(&mo, 0, sizeof mo);
      mo.eq_round_polys = rp.data();
      TRY(gkr_prove_mul_layer(c, point.data(), (uint32_t)point.size(), &value, st.a, st.b, ch, proof, &mo));
      value = mo.next_value;  // the claim point is unchanged (prover.rs:6260-6263)
    } else if (st.kind == GKR_STEP_ACTIVATION) {
      const uint32_t nv = (uint32_t)(log2_exact(next_pow2(st.a->rows)) + log2_exact(next_pow2(st.a->cols)));
      if (st.claim == GKR_CLAIM_FRESH) {
        point.resize(nv);
        {
          HostTimer ht(c, K_HOST_DRAW);
          TRY(gkr_channel_draw_qm31s(ch, nv, point.data()));
        }
        value = G(ch->ch.draw_qm31());
      } else if (!have_claim) {
        return fail(GKR_ERR_INVALID, "step %zu: chained claim but no previous claim", si);
      }
      const uint32_t tl = st.table_log_size ? st.table_log_size : act_default_log_size(st.activation_type);
      if (tl == 0 || tl > 24) return fail(GKR_ERR_INVALID, "step %zu: bad table size", si);
      rp.resize(4 * (size_t)(nv ? nv : 1));
      mults.resize((size_t)1 << tl);
      std::vector<gkr_qm31> mrp(2 * tl);
      gkr_logup_out out;
      memset(&out, 0, sizeof out);
      out.eq_round_polys = rp.data();
      out.multiplicities = mults.data();
      out.mult_round_polys = mrp.data();
      TRY(gkr_prove_activation_layer(c, point.data(), (uint32_t)point.size(), &value, st.a, st.activation_type, tl,
                                     ch, proof, &out));
      value = out.input_eval;  // the claim point is unchanged (prover.rs:6581-6584)
    } else {
      return fail(GKR_ERR_INVALID, "step %zu: unknown kind %u", si, st.kind);
    }
    have_claim = true;
  }
  if (point.size() > 64) return fail(GKR_ERR_BUFFER, "final claim has %zu variables", point.size());
  for (size_t l = 0; l < point.size(); l++) final_point[l] = point[l];
  *n_final = (uint32_t)point.size();
  *final_value = value;
  return GKR_OK;
}

// ------------------------------------------------------------------ verifier replay
static bool read_point(const gkr_qm31* p, uint32_t n, std::vector<qm31>* out) {
  out->resize(n);
  for (uint32_t l = 0; l < n; l++) {
    if (!canonical_q(p[l])) return false;
    (*out)[l] = Q(p[l]);
  }
  return true;
}
static int verify_fail(const VerifyError& e) { return fail(GKR_ERR_VERIFY, "%s", e.why.c_str()); }

extern "C" int gkr_verify_matmul_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                                       uint64_t m, uint64_t k, uint64_t n, const gkr_qm31* round_polys,
                                       uint32_t n_rounds, const gkr_qm31* final_a, const gkr_qm31* final_b,
                                       gkr_channel* ch, gkr_qm31* next_point, uint32_t* n_next,
                                       gkr_qm31* next_value) {
  CH_CHECK(ch);
  if (!claim_value || !final_a || !final_b || !next_point || !n_next || !next_value ||
      (!claim_point && n_point) || (!round_polys && n_rounds))
    return fail(GKR_ERR_INVALID, "null argument");
  if (m == 0 || k == 0 || n == 0) return fail(GKR_ERR_INVALID, "empty dimension");
  std::vector<qm31> pt, polys(3 * (size_t)n_rounds);
  if (!read_point(claim_point, n_point, &pt)) return fail(GKR_ERR_INVALID, "claim point not canonical");
  for (size_t i = 0; i < polys.size(); i++) {
    if (!canonical_q(round_polys[i])) return fail(GKR_ERR_INVALID, "round polynomial not canonical");
    polys[i] = Q(round_polys[i]);
  }
  std::vector<qm31> np;
  qm31 nv;
  VerifyError e;
  if (!verify_matmul(pt, Q(*claim_value), m, k, n, polys, Q(*final_a), Q(*final_b), ch->ch, &np, &nv, &e))
    return verify_fail(e);
  for (size_t l = 0; l < np.size(); l++) next_point[l] = G(np[l]);
  *n_next = (uint32_t)np.size();
  *next_value = G(nv);
  return GKR_OK;
}

extern "C" int gkr_verify_mul_layer(const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                                    const gkr_qm31* eq_round_polys, uint32_t n_rounds, const gkr_qm31* lhs_eval,
                                    const gkr_qm31* rhs_eval, gkr_channel* ch, gkr_qm31* next_value) {
  CH_CHECK(ch);
  if (!claim_value || !lhs_eval || !rhs_eval || !next_value || (!claim_point && n_point) ||
      (!eq_round_polys && n_rounds))
    return fail(GKR_ERR_INVALID, "null argument");
  std::vector<qm31> pt, polys(4 * (size_t)n_rounds);
  if (!read_point(claim_point, n_point, &pt)) return fail(GKR_ERR_INVALID, "claim point not canonical");
  for (size_t i = 0; i < polys.size(); i++) polys[i] = Q(eq_round_polys[i]);
  qm31 nv;
  VerifyError e;
  if (!verify_mul(pt, Q(*claim_value), polys, Q(*lhs_eval), Q(*rhs_eval), ch->ch, &nv, &e)) return verify_fail(e);
  *next_value = G(nv);
  return GKR_OK;
}

static const std::vector<uint32_t>& verifier_table(uint32_t tag, uint32_t log) {
  static std::mutex mu;
  static std::map<uint64_t, std::vector<uint32_t>> tables;
  std::lock_guard<std::mutex> lock(mu);
  const uint64_t key = ((uint64_t)tag << 32) | log;
  auto it = tables.find(key);
  if (it == tables.end()) it = tables.emplace(key, act_table(tag, log)).first;
  return it->second;
}

extern "C" int gkr_verify_activation_layer(const gkr_qm31* claim_point, uint32_t n_point, uint32_t activation_type,
                                           uint32_t table_log_size, uint32_t n_eq_rounds, const gkr_logup_out* proof,
                                           gkr_channel* ch, gkr_qm31* next_value) {
  CH_CHECK(ch);
  if (!proof || !next_value || (!claim_point && n_point)) return fail(GKR_ERR_INVALID, "null argument");
  if (!act_valid(activation_type)) return fail(GKR_ERR_INVALID, "unknown activation type %u", activation_type);
  if (!act_logup_valid(activation_type))
    return fail(GKR_ERR_INVALID, "activation type %u (ReLU) is proved algebraically, not by LogUp", activation_type);
  if (table_log_size == 0) table_log_size = act_default_log_size(activation_type);
  if (table_log_size > 24) return fail(GKR_ERR_INVALID, "table_log_size %u too large", table_log_size);
  if ((n_eq_rounds && !proof->eq_round_polys) || !proof->multiplicities || !proof->mult_round_polys)
    return fail(GKR_ERR_INVALID, "null proof arrays");
  std::vector<qm31> pt;
  if (!read_point(claim_point, n_point, &pt)) return fail(GKR_ERR_INVALID, "claim point not canonical");
  LogUpProofIn p;
  p.claimed_sum = Q(proof->claimed_sum);
  for (uint32_t i = 0; i < 4 * n_eq_rounds; i++) p.eq_polys.push_back(Q(proof->eq_round_polys[i]));
  p.w_eval = Q(proof->w_eval);
  p.in_eval = Q(proof->in_eval);
  p.out_eval = Q(proof->out_eval);
  p.mults.assign(proof->multiplicities, proof->multiplicities + (1ull << table_log_size));
  for (uint32_t i = 0; i < 2 * table_log_size; i++) p.mult_polys.push_back(Q(proof->mult_round_polys[i]));
  p.mult_final = Q(proof->mult_final_eval);
  p.mult_sum = Q(proof->mult_claimed_sum);
  p.input_eval = Q(proof->input_eval);
  p.output_eval = Q(proof->output_eval);
  if (!felt_abi_canonical(proof->table_commitment)) return fail(GKR_ERR_INVALID, "table commitment not canonical");
  p.table_commitment = felt_canon_from_words(proof->table_commitment.w);
  qm31 nv;
  VerifyError e;
  if (!verify_activation(pt, activation_type, table_log_size, verifier_table(activation_type, table_log_size), p,
                         ch->ch, &nv, &e))
    return verify_fail(e);
  *next_value = G(nv);
  return GKR_OK;
}

// A chained walk from serialize_gkr_model_proof calldata: every layer's
// claim is the previous layer's input claim, starting from init_*.  Checks
// the layer proofs and the input-claim section; the weight commitments,
// openings and IO commitment that follow are not examined.
extern "C" int gkr_verify_walk(const gkr_felt* calldata, size_t n_felts, const gkr_layer_shape* layers,
                               size_t n_layers, const gkr_qm31* init_point, uint32_t n_init,
                               const gkr_qm31* init_value, const gkr_qm31* fresh_values, size_t n_fresh,
                               gkr_channel* ch, gkr_qm31* final_point, uint32_t* n_final, gkr_qm31* final_value,
                               size_t* n_consumed) {
  CH_CHECK(ch);
  if (!calldata || !layers || !final_point || !n_final || !final_value || (!init_point && n_init) ||
      (!fresh_values && n_fresh))
    return fail(GKR_ERR_INVALID, "null argument");
  if (n_layers && layers[0].claim != GKR_CLAIM_FRESH && !init_value)
    return fail(GKR_ERR_INVALID, "the first layer's claim is chained but no initial claim is given");
  std::vector<qm31> point;
  if (!read_point(init_point, n_init, &point)) return fail(GKR_ERR_INVALID, "initial point not canonical");
  qm31 value = init_value ? Q(*init_value) : qm31_zero();
  size_t fresh_used = 0;
  FeltReader R{reinterpret_cast<const uint32_t*>(calldata), n_felts};
  auto bad = [&](const std::string& why) { return fail(GKR_ERR_VERIFY, "%s", why.c_str()); };
  const uint64_t nl = R.u();
  if (!R.ok) return bad(R.why);
  if (nl != n_layers) return bad("proof has " + std::to_string(nl) + " layers, circuit " + std::to_string(n_layers));
  for (size_t li = 0; li < n_layers; li++) {
    const gkr_layer_shape& L = layers[li];
    const std::string at = "layer " + std::to_string(li) + ": ";
    const uint64_t tag = R.u();
    if (!R.ok) return bad(R.why);
    if (L.claim == GKR_CLAIM_FRESH) {  // the prover's fresh-claim rule (gkr_prove_walk)
      if (L.kind != GKR_STEP_MATMUL && L.kind != GKR_STEP_MUL && L.kind != GKR_STEP_ACTIVATION)
        return fail(GKR_ERR_INVALID, "layer %zu: unknown kind %u", li, L.kind);
      const uint64_t out_cols = L.kind == GKR_STEP_MATMUL ? L.cols_b : L.cols;
      const int nv = v_log2(v_next_pow2(L.rows)) + v_log2(v_next_pow2(out_cols));
      if (nv > 64) return fail(GKR_ERR_INVALID, "layer %zu: output claim of %d variables", li, nv);
      point.resize(nv);
      ch->ch.draw_qm31s(point.data(), (size_t)nv);
      if (L.kind == GKR_STEP_ACTIVATION) {
        value = ch->ch.draw_qm31();
      } else {
        if (fresh_used >= n_fresh) return fail(GKR_ERR_INVALID, "layer %zu: no fresh claim value left", li);
        if (!canonical_q(fresh_values[fresh_used])) return fail(GKR_ERR_INVALID, "fresh claim value not canonical");
        value = Q(fresh_values[fresh_used++]);
        ch->ch.mix_secure_field(value);
      }
    } else if (L.claim != GKR_CLAIM_CHAINED) {
      return fail(GKR_ERR_INVALID, "layer %zu: unknown claim rule %u", li, L.claim);
    }
    VerifyError e;
    if (L.kind == GKR_STEP_MATMUL) {
      if (tag != 0) return bad(at + "expected a MatMul proof (tag 0), found tag " + std::to_string(tag));
      const uint64_t nr = R.u(64);
      std::vector<qm31> polys;
      for (uint64_t t = 0; t < nr && R.ok; t++) {
        const qm31 c0 = R.q(), c2 = R.q();
        polys.push_back(c0);
        polys.push_back(qm31_zero());
        polys.push_back(c2);
      }
      const qm31 fa = R.q(), fb = R.q();
      if (!R.ok) return bad(at + R.why);
      std::vector<qm31> np;
      if (!verify_matmul(point, value, L.rows, L.cols, L.cols_b, polys, fa, fb, ch->ch, &np, &value, &e, true))
        return bad(at + e.why);
      point = np;
    } else if (L.kind == GKR_STEP_MUL) {
      if (tag != 2) return bad(at + "expected a Mul proof (tag 2), found tag " + std::to_string(tag));
      const uint64_t nr = R.u(64);
      std::vector<qm31> polys;
      for (uint64_t t = 0; t < nr && R.ok; t++) {
        const qm31 c0 = R.q(), c2 = R.q(), c3 = R.q();
        polys.push_back(c0);
        polys.push_back(qm31_zero());
        polys.push_back(c2);
        polys.push_back(c3);
      }
      const qm31 lhs = R.q(), rhs = R.q();
      if (!R.ok) return bad(at + R.why);
      if (nr != (uint64_t)v_log2(v_next_pow2(L.rows) * v_next_pow2(L.cols)))
        return bad(at + "Mul proof has " + std::to_string(nr) + " rounds for a " + std::to_string(L.rows) + " x " +
                   std::to_string(L.cols) + " operand");
      if (!verify_mul(point, value, polys, lhs, rhs, ch->ch, &value, &e, true)) return bad(at + e.why);
    } else if (L.kind == GKR_STEP_ACTIVATION) {
      if (tag != 3) return bad(at + "expected an Activation proof (tag 3), found tag " + std::to_string(tag));
      const uint32_t act = (uint32_t)R.u(0xFFFFFFFFull);
      if (R.ok && act != L.activation_type)
        return bad(at + "activation type " + std::to_string(act) + ", circuit " + std::to_string(L.activation_type));
      if (!act_valid(act)) return bad(at + "unknown activation type");
      if (!act_logup_valid(act)) return bad(at + "ReLU is proved algebraically, not by LogUp");
      const uint32_t tlog = L.table_log_size ? L.table_log_size : act_default_log_size(act);
      if (tlog > 24) return bad(at + "table size too large");
      LogUpProofIn p;
      p.input_eval = R.q();
      p.output_eval = R.q();
      p.table_commitment = R.f();
      if (R.u(1) != 1 || !R.ok) return bad(at + "activation proof without a LogUp proof");
      p.claimed_sum = R.q();
      const uint64_t nr = R.u(64);
      for (uint64_t t = 0; t < nr && R.ok; t++) {
        const qm31 c0 = R.q(), c2 = R.q(), c3 = R.q();
        p.eq_polys.push_back(c0);
        p.eq_polys.push_back(qm31_zero());
        p.eq_polys.push_back(c2);
        p.eq_polys.push_back(c3);
      }
      p.w_eval = R.q();
      p.in_eval = R.q();
      p.out_eval = R.q();
      const uint64_t nm = R.u(1ull << 24);
      for (uint64_t j = 0; j < nm && R.ok; j++) p.mults.push_back((uint32_t)R.u(0xFFFFFFFFull));
      if (R.u(1) != 1 || !R.ok) return bad(at + "activation proof without a multiplicity sumcheck");
      const uint64_t nmr = R.u(64);
      for (uint64_t t = 0; t < nmr && R.ok; t++) {
        p.mult_polys.push_back(R.q());
        p.mult_polys.push_back(R.q());
      }
      p.mult_final = R.q();
      p.mult_sum = R.q();
      const uint64_t has_prod = R.u(1), has_pw = R.u(1);
      if (!R.ok) return bad(at + R.why);
      if (has_prod || has_pw) return bad(at + "product / piecewise activation proofs are not supported");
      if (nr != (uint64_t)v_log2(v_next_pow2(L.rows) * v_next_pow2(L.cols)))
        return bad(at + "activation proof has " + std::to_string(nr) + " eq rounds for a " + std::to_string(L.rows) +
                   " x " + std::to_string(L.cols) + " input");
      if (nmr != tlog) return bad(at + "multiplicity sumcheck has " + std::to_string(nmr) + " rounds");
      if (!verify_activation(point, act, tlog, verifier_table(act, tlog), p, ch->ch, &value, &e, true))
        return bad(at + e.why);
    } else {
      return fail(GKR_ERR_INVALID, "layer %zu: unknown kind %u", li, L.kind);
    }
  }
  // the input claim the proof states must be the one the walk arrived at
  const uint64_t npt = R.u(64);
  std::vector<qm31> ipt;
  for (uint64_t l = 0; l < npt && R.ok; l++) ipt.push_back(R.q());
  const qm31 ival = R.q();
  if (!R.ok) return bad(R.why);
  bool same = ipt.size() == point.size() && qm31_eq(ival, value);
  for (size_t l = 0; same && l < ipt.size(); l++) same = qm31_eq(ipt[l], point[l]);
  if (!same) return bad("input claim in the proof differs from the claim the walk reached");
  if (fresh_used != n_fresh)
    return fail(GKR_ERR_INVALID, "%zu fresh claim values given, the circuit uses %zu", n_fresh, fresh_used);
  if (point.size() > 64) return fail(GKR_ERR_BUFFER, "final claim has %zu variables", point.size());
  for (size_t l = 0; l < point.size(); l++) final_point[l] = G(point[l]);
  *n_final = (uint32_t)point.size();
  *final_value = G(value);
  if (n_consumed) *n_consumed = R.pos;
  return GKR_OK;
}
