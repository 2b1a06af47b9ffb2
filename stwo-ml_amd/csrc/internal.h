// Shared internals of the host side of the MI355X GKR prover (not part of
// the C ABI): the error convention, the device context and its buffers, the
// result sinks and waits, the hand-over session, the multi-round trip
// planner and launcher, the channel and proof records, and the functions
// one translation unit provides to the others.  Each .hip file of this
// directory implements one part of include/gkr_mi355x.h on top of it.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <deque>

#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/gkr_mi355x.h"
#include "field.h"
#include <functional>

#include "kernels.h"
#include "launcher.h"
#include "poseidon.h"
#include "trace.h"
#include "hostfield.h"

namespace gkr {
struct MerkleConsts;  // merkle.h
}
using namespace gkr;

// The words of QM31 values, for the host-side AVX2 rounds (hostfield.h), which
// take the array-of-structs layout as plain u32 words.
static_assert(sizeof(qm31) == 16 && alignof(qm31) == 4, "qm31 is four packed u32 words");
inline uint32_t* qwords(qm31* q) { return reinterpret_cast<uint32_t*>(q); }
inline const uint32_t* qwords(const qm31* q) { return reinterpret_cast<const uint32_t*>(q); }

// ------------------------------------------------------------------ errors
// Records the message of a failure for gkr_last_error() and returns code.
int fail(int code, const char* fmt, ...);
// Every HIP call made through HIP_TRY first drains the launch ring of the
// context `c` in scope (launcher.h), so it never overtakes a launch queued
// before it on that context.  HIP_CHECK is for calls that touch no stream
// or device memory (device queries), made where no context exists yet.
#define HIP_CHECK(expr)                                                                     \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess) return fail(GKR_ERR_DEVICE, "%s: %s (%s:%d)", #expr,              \
                                      hipGetErrorString(e_), __FILE__, __LINE__);           \
  } while (0)
#define HIP_TRY(expr) \
  do {                \
    drain(c);         \
    HIP_CHECK(expr);  \
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
inline bool felt_abi_canonical(const gkr_felt& f) {
  felt c = felt_canon_from_words(f.w);
  return !felt_detail::geq_p(c.l);
}

// ------------------------------------------------------------------ context
enum Slot {
  S_LI, S_LJ, S_FA0, S_FA1, S_FB0, S_FB1, S_PART, S_RES, S_EQHI, S_EQLO, S_MLE, S_EQ, S_OUT,
  S_MULT, S_MIN, S_MOUT, S_D0, S_D1, S_W0, S_W1, S_E0, S_M0, S_M1, S_COLPART,
  S_MK0, S_MK1, S_MKSTEP, S_MKROOT, S_OPL, S_OPI, S_GEMMA, S_GEMMB, S_GEMMP, S_FA2, S_FB2, S_EQPARTS, S_TRIPCNT, S_TRIPMB, S_LKINV, S_LKHIST, S_LDIG, S_R8FLAG, S_PTWAIT, S_EXTA, S_EXTB, S_GRAM, S_NORMSUM, S_NORMROW,
  S_LKARENA, S_LKFOLD, S_LKDESC, S_LKPART, S_LKRES, S_LKTAB,
  S_BIND, S_BINDEQ, S_BINDDESC, S_BINDPART, S_BINDRES, S_BINDVIRT, S_NSLOTS
};
// Timer ids: device kernels (HIP events) and host-side phases (Fiat-Shamir
// hashing inside the reducers, waiting for trip results, waiting for the
// hand-over of the last vectors).
enum KernelId { K_RESTRICT_COLS = 0, K_RESTRICT_ROWS = 1, K_MM_ROUND = 2, K_EQ3_ROUND = 3, K_LOGUP_PREP = 4,
                K_EQ_TABLE = 5, K_HOST_FS = 6, K_HOST_WAIT = 7, K_HOST_WAIT_TAIL = 8, K_MERKLE = 9,
                K_HOST_DRAW = 10, K_HOST_LAUNCH = 11, K_HOST_FINISH = 12, K_NORM = 13, K_LOOKUP = 14,
                K_HOST_GRAM = 15, K_HOST_PROOF = 16, K_HOST_WALK_MM = 17, K_HOST_WALK_ACT = 18,
                K_WALK_RETRY = 19, K_ACT_AHEAD = 20, K_NKERNELS = 21 };
constexpr int kMaxPartialBlocks = 1024;
constexpr int kMaxSums = 64;  // values per partial row (a 3-round trip's 4^3 cross sums)
static_assert(kMaxPartialBlocks <= kCountedMaxRows && kCountedMaxRows % kBlock == 0,
              "partial_grid launches must fit the in-kernel finish");
// Result slots in the coherent host area (h_out): 0 .. 63 serve the result in
// flight; results launched ahead of time and read later have their own.
constexpr int kSlotEq0 = 64;     // eq-sumcheck trip 0 (up to 64 values)
constexpr int kSlotPrep = 128;   // LogUp prepare: trace sum, input MLE
constexpr int kSlotTable = 130;  // LogUp table-side sum
constexpr int kSlotMult0 = 136;  // multiplicity sumcheck trip 0 (up to 8 values)
constexpr int kSlotIO = 144;     // LogUp input / output MLEs at the eq-sumcheck challenges
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
  // (gemm.h), built on first use; kept until the contents change (written
  // by gkr_matmul_forward_into, or declared changed by gkr_matrix_invalidate)
  int8_t* bplanes = nullptr;
  int bnplanes = 0;
  // int8 copy for the weight-side restriction (1 KB tiles of 16 rows x 64
  // columns, the MFMA operand layout of k_restrict_cols8; r8_nst column
  // steps per row tile), built on first use when every entry is int8-range;
  // r8_state: 0 not yet checked, 1 copy present, -1 not int8-range
  int8_t* r8 = nullptr;
  uint64_t r8_nst = 0;
  int r8_state = 0;
  // the weight commitment (Poseidon Merkle root of the column-major padded
  // MLE, canonical words), once computed or supplied by the caller
  bool have_root = false;
  gkr_felt root;
};

// Drops the copies derived from m's contents (int8 copy, digit planes, the
// cached commitment root) and a matmul claim computed over m; they are
// rebuilt on the next use.
int drop_derived(gkr_ctx* c, gkr_matrix* m);

struct gkr_qvec {
  gkr_ctx* ctx;
  qm31* dev;
  uint64_t n;
};

// Pinned host staging buffers (grow-only, hipHostMalloc).
enum HostSlot { H_LKDESC, H_LKRES, H_LKTAB, H_NSLOTS };

// Coherent pinned buffers for the LogUp multiplicities, one per activation
// layer in flight: a layer's table pass writes its slot, and the layer's proof
// record copies the slot into the record (on the proof stream's thread when the
// proof is streamed, so the transcript thread does not) and then frees it.  A
// layer takes the next slot once its previous record has copied it.  Records
// share ownership of the ring, so a slot outlives a context destroyed first.
struct MultRing {
  static constexpr int kSlots = 4;
  uint32_t* buf[kSlots] = {};
  size_t cap = 0;
  std::atomic<int> busy[kSlots];  // 1 from the layer's table pass until its record copied the slot
  int next = 0;
  MultRing() {
    for (auto& b : busy) b.store(0, std::memory_order_relaxed);
  }
  ~MultRing() {
    for (uint32_t* b : buf)
      if (b) (void)hipHostFree(b);
  }
};

struct gkr_ctx {
  int device = 0;
  void* hbuf[H_NSLOTS] = {};
  size_t hcap[H_NSLOTS] = {};
  hipStream_t stream = nullptr;
  void* buf[S_NSLOTS] = {};
  size_t cap[S_NSLOTS] = {};
  qm31* h_res = nullptr;  // pinned result staging (64 QM31)
  std::shared_ptr<MultRing> mring;  // LogUp multiplicities, host side (ensure_host_mult)
  uint32_t* h_mult = nullptr;  // the current activation layer's slot of mring (written by its table pass)
  int h_mult_slot = -1;
  qm31* h_vec = nullptr;       // coherent pinned: vectors handed over by k_handover (2 x kHandMax)
  qm31* h_out = nullptr;      // coherent pinned: results delivered by kernels (RoundSink)
  uint32_t* h_flag = nullptr; // coherent pinned: sequence number of the last delivery
  Mailbox* mailbox = nullptr;  // coherent pinned: challenges posted to persistent tail kernels
  // coherent pinned: values posted after a claim point to kernels launched
  // ahead of both (an activation layer's gamma and beta, prelaunch_activation)
  Mailbox* vmailbox = nullptr;
  uint32_t seq = 0;            // last result sequence number handed out
  uint32_t mb_seq = 0;         // last mailbox sequence number handed out
  int timing = 0;  // 0 off; 1: sampled events on the critical-path kernels + host timers; 2: events on every timed kernel
  uint64_t event_seq[K_NKERNELS] = {};  // launches of each timer id since the last reset (level-1 sampling)
  KernelStat stats[K_NKERNELS];
  std::map<std::pair<int, uint64_t>, KernelStat> size_stats;  // per (timer id, bytes of one launch)
  std::vector<PendingTiming> pending;
  std::vector<hipEvent_t> free_events;
  MatMulCache mm;
  std::map<uint64_t, std::vector<uint32_t>> tables;  // (tag << 32 | log) -> table outputs
  std::set<gkr_matrix*> matrices;  // live matrices; detached when the context is destroyed
  std::set<gkr_qvec*> qvecs;       // live QM31 vectors; detached likewise
  uint64_t mult_zero_entries = 0;  // leading entries of S_MULT known to be zero once the queued work is done
  std::map<uint64_t, uint32_t*> dev_tables;  // (tag << 32 | log) -> resident device copy of the table outputs
  std::map<uint64_t, felt> table_commitments;  // (tag << 32 | log) -> poseidon_hash_many([tag, log])
  MerkleConsts* merkle_consts = nullptr;  // device copy, built on first use
  bool fb_pending = false;  // f_b of the last restriction still as column-chunk partials (S_COLPART)
  uint64_t fb_rows = 0, fb_pk = 0;
  int fb_chunks = 0;
  uint32_t trip_count = 0;         // value of the fused trips' arrival counter (S_TRIPCNT) after the queued launches
  bool trip_count_valid = false;   // false: zero the counter before the next fused trip
  bool tripmb_valid = false;       // false: zero the flags of the trips launched ahead (S_TRIPMB) before use
  bool int8_weights = true;        // int8 weight-side restriction for int8-range weights (GKR_INT8_WEIGHTS=0: off)
  // allocation-free mode (gkr_sumcheck_product_noalloc): ensure() hands out
  // the partial rows and the arrival counter from the device's static
  // scratch array (scratch_dev: its address on this context's device) and
  // refuses every other slot
  uint8_t* scratch_dev = nullptr;
  bool noalloc = false;
  // launches go through this thread's ring (null: GKR_ASYNC_LAUNCH=0, issued by the caller's thread)
  std::unique_ptr<Launcher> launcher;
  LaunchEvents armed;  // a TimedLaunch's events for the next launch (take_armed)
  // kernels launched ahead of their claim point, behind a k_point_wait for
  // mailbox sequence `want`: a matmul restriction (prelaunch_matmul; a, b the
  // operands) or an activation layer's first kernels (prelaunch_activation,
  // act; a the input, with its table and the sinks of its first results)
  struct {
    bool active = false;
    bool act = false;
    uint32_t want = 0;
    const gkr_matrix* a = nullptr;
    const gkr_matrix* b = nullptr;
    uint32_t tag = 0, table_log = 0;
    RoundSink sk_prep, sk_eq0;
    uint32_t want_vals = 0;  // act: vmailbox sequence of gamma and beta
    bool hold_vals = false;  // test hook: gamma, beta posted only after that wait expired
  } pre;
  // (variables, table_log) of the activation layers proved on this context:
  // their buffers exist, so such a layer's first kernels can be launched ahead
  std::set<std::pair<int, uint32_t>> act_shapes;
  uint32_t point_mb = 0;  // the posted point's sequence, until the first trip's results confirm it arrived
  uint32_t vals_mb = 0;   // likewise for values posted through vmailbox
  // set by the walk for one step: called at that step's last launch
  std::function<int()> prelaunch;
  // test hooks (gkr_ctx_debug), each consumed by the next hand-over (or trip launched ahead)
  bool debug_handover_cancel = false;  // the host leaves before posting the challenges
  uint32_t debug_handover_spins = 0;   // nonzero: the kernel's bounded wait, posted only after it expired
  uint32_t debug_trip_spins = 0;       // the same for the next trip launched ahead of its challenges
  // set when a call failed because a kernel's bounded wait for the host gave
  // up (the host fell more than the wait's length behind); the walk then
  // proves the step again
  bool wait_expired = false;
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

int ensure(gkr_ctx* c, Slot s, size_t bytes, void** out);
template <typename T>
inline int ensureT(gkr_ctx* c, Slot s, size_t count, T** out) {
  void* p;
  TRY(ensure(c, s, count * sizeof(T), &p));
  *out = (T*)p;
  return GKR_OK;
}

// A multiplicity ring of n-entry slots, then the next slot: c->h_mult,
// c->h_mult_slot, marked busy (waits until its previous record copied it).
int ensure_host_mult(gkr_ctx* c, uint64_t n);

// Kernel launch on the context's stream: GKR_LAUNCH(c, kernel, grid, block,
// shared bytes, kernel arguments...).  The arguments are evaluated and
// converted to the kernel's parameter types at this point; the launch itself
// is issued by the context's launcher thread when it has one.
#define GKR_LAUNCH(ctx, KERN_, GRID_, BLOCK_, SHMEM_, ...)                                     \
  (void)launch_kernel((ctx)->launcher.get(), take_armed(ctx), KERN_, dim3(GRID_), dim3(BLOCK_), \
                      (uint32_t)(SHMEM_), (ctx)->stream, __VA_ARGS__)
// The events a TimedLaunch armed for the next launch (consumed by it).
inline LaunchEvents take_armed(gkr_ctx* c) {
  const LaunchEvents ev = c->armed;
  c->armed = LaunchEvents{};
  return ev;
}
// Waits until every launch queued on the context has been issued.
inline void drain(const gkr_ctx* c) {
  if (c && c->launcher) c->launcher->drain();
}
hipEvent_t get_event(gkr_ctx* c);
// An event record in stream order (through the launcher when there is one).
inline void record_event(gkr_ctx* c, hipEvent_t e) {
  hipStream_t s = c->stream;
  if (c->launcher)
    c->launcher->submit([e, s]() -> hipError_t { return hipEventRecord(e, s); });
  else
    (void)hipEventRecord(e, s);
}
// Times the launches of its scope for timer `kid`.  Timing a dispatch costs
// the queue about 4 us next to each neighbouring kernel (kernel trace of the
// 48-layer walk: 3.9-4.0 us gaps on both sides of every timed dispatch,
// whether its events are records or carried in the dispatch), so level 1
// times every kEventSample-th launch of the kernels on the walk's critical
// path (ids 0 and 4) and every launch of ids 1, 9, 13 and 14.
// single: the scope makes exactly one launch, which carries the events in
// its own dispatch (hipExtLaunchKernel); otherwise a pair of event records
// brackets the scope.
constexpr uint64_t kEventSample = 8;
struct TimedLaunch {
  gkr_ctx* c;
  int kid;
  uint64_t bytes;
  bool single;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  TimedLaunch(gkr_ctx* c_, int kid_, uint64_t bytes_, bool single_ = false)
      : c(c_), kid(kid_), bytes(bytes_), single(single_) {
    bool on = c->timing >= 2;
    if (c->timing == 1) {
      if (kid == K_RESTRICT_COLS || kid == K_LOGUP_PREP)
        on = c->event_seq[kid]++ % kEventSample == 0;
      else if (kid == K_RESTRICT_ROWS || kid == K_MERKLE || kid == K_NORM || kid == K_LOOKUP)
        on = true;
    }
    if (on) {
      e0 = get_event(c);
      e1 = get_event(c);
      if (!e0 || !e1) {
        e0 = e1 = nullptr;
      } else if (single) {
        c->armed = LaunchEvents{e0, e1};
      } else {
        record_event(c, e0);
      }
    }
  }
  ~TimedLaunch() {
    if (!e0 || !e1) return;
    if (single && c->armed.start == e0) {  // no launch took them (an error path)
      c->armed = LaunchEvents{};
      c->free_events.push_back(e0);
      c->free_events.push_back(e1);
      return;
    }
    if (!single) record_event(c, e1);
    c->pending.push_back({kid, e0, e1, bytes});
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
void collect_timing(gkr_ctx* c);
int sync(gkr_ctx* c);
// Launch errors of the calling thread and of c's launcher thread (the first
// error its ring's launches returned), never another context's.
inline int check_launch(gkr_ctx* c) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && c && c->launcher) e = c->launcher->take_error();
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

PointArg make_point(const qm31* r, int n);
int eq_split(gkr_ctx* c, const qm31* r, int n, qm31** hi, qm31** lo, int* h);
int arrival_counter(gkr_ctx* c, unsigned grid, uint32_t** counter, uint32_t* base);
int deliver_args(gkr_ctx* c, unsigned grid, uint32_t** counter, uint32_t* base);
int dot2_evals(gkr_ctx* c, const qm31* z, int nv, const uint32_t* v0, const uint32_t* v1, qm31 out[2]);
// The same pass, launched only: its two values arrive in host slot `slot` (wait_sink<2>).
int dot2_launch(gkr_ctx* c, const qm31* z, int nv, const uint32_t* v0, const uint32_t* v1, int slot, RoundSink* sk);

// eq(r, x) for x < count (r[0] on the most significant bit of x).
int eq_table(gkr_ctx* c, const qm31* r, int n, uint64_t count, qm31* out);

// Result and mailbox sequence numbers come in consecutive ranges and restart
// at 1 before they reach the cancel code reserved at the top of the u32 range
// (kWaitCancel); waits compare them modulo 2^32.
constexpr uint32_t kSeqLimit = 0xFFFFFF00u;
inline uint32_t alloc_seq(uint32_t* counter, uint32_t n) {
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
int make_sink(gkr_ctx* c, RoundSink* sk, int slot = 0);
// Launch the one-workgroup finisher that adds `nblocks` partial rows and
// delivers the NQ results (after a multi-workgroup reducing kernel).
template <int NQ>
static int launch_finish(gkr_ctx* c, const RoundSink& sk, unsigned nblocks) {
  TRY(check_launch(c));
  GKR_LAUNCH(c, k_finish<NQ>, dim3(1), dim3(kBlock), 0, sk, (uint32_t)nblocks);
  return check_launch(c);
}
// The finisher of a launch made with deliver_args (none when it delivers itself).
template <int NQ>
static int deliver_finish(gkr_ctx* c, const RoundSink& sk, unsigned nblocks, const uint32_t* counter) {
  if (counter) return check_launch(c);
  return launch_finish<NQ>(c, sk, nblocks);
}
// Wait until result `seq` has been published and copy NQ values.  The wait
// spins on the coherent flag and never blocks on the stream (a hand-over
// kernel queued behind the result may be waiting for the host): once it has
// waited kWaitQuerySeconds it queries the stream, and again every
// kWaitQuerySeconds, so a device error, or a drained stream without the
// result, is reported; after kWaitWallSeconds it gives up.  hand_mb != 0:
// the result comes from the hand-over waiting for mailbox sequence hand_mb,
// whose expiry is reported at once.
//
// The query is kept off ordinary waits: a stream query puts a marker packet
// behind the kernels already queued, and the command processor takes about
// 5 us over it before the next kernel starts.  While the host waits for a
// trip's sums, the queue already holds the next trip launched ahead, so a
// query then delayed the following mailbox wait, and with it the trip after
// (kernel trace: about 5 us before most eq-sumcheck mailbox waits, 1.4 ms per
// 48-layer proof, when the stream was queried every 65536 spins).
constexpr double kWaitWallSeconds = 60.0;
constexpr double kWaitQuerySeconds = 0.002;
template <int NQ>
static int wait_result(gkr_ctx* c, uint32_t seq, qm31* host_out, int timer = K_HOST_WAIT_TAIL, int slot = 0,
                       uint32_t hand_mb = 0) {
  TRY(check_launch(c));
  HostTimer ht(c, timer);
  volatile uint32_t* flag = c->h_flag;
  volatile uint32_t* expired = &c->mailbox->expired;
  std::chrono::steady_clock::time_point t0, next_query;
  // the flag only moves forward (mod 2^32): a later delivery implies this one
  for (uint64_t spins = 0; (int32_t)(*flag - seq) < 0; spins++) {
    if (hand_mb && *expired == hand_mb) {
      c->wait_expired = true;
      return fail(GKR_ERR_DEVICE, "kernel launched ahead stopped waiting for its challenges (mailbox %u)", hand_mb);
    }
    if ((spins & 0xFFF) != 0xFFF) continue;
    const auto now = std::chrono::steady_clock::now();
    if (spins == 0xFFF) {
      t0 = now;
      next_query = now + std::chrono::duration_cast<std::chrono::steady_clock::duration>(
                             std::chrono::duration<double>(kWaitQuerySeconds));
      continue;
    }
    if (now < next_query) continue;
    next_query = now + std::chrono::duration_cast<std::chrono::steady_clock::duration>(
                           std::chrono::duration<double>(kWaitQuerySeconds));
    TRY(check_launch(c));
    // while launches are still being issued the stream has not drained
    const hipError_t e = c->launcher && !c->launcher->idle() ? hipErrorNotReady : hipStreamQuery(c->stream);
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
// Post k challenges into the mailbox under sequence `want`.
inline void post_mailbox(gkr_ctx* c, uint32_t want, const qm31* chal, int k) {
  for (int r = 0; r < k; r++) c->mailbox->alpha[r] = chal[r];
  __atomic_store_n(&c->mailbox->seq, want, __ATOMIC_RELEASE);
}
// Host side of a k_handover launch over the last trip's vectors, folded by
// that trip's k challenges: the kernel folds the first kd = k - 1 levels as
// the host posts their challenges (post_one, one at a time as they are drawn,
// so each fold runs while the host draws the next; or post, the rest at once)
// and hands the vectors over while the host draws the last challenge, which
// the host folds itself (fetch).  The session holds kd consecutive mailbox
// sequence numbers from mb_seq: challenge i < kd is posted under mb_seq + i.
// If the host leaves before posting (an error), the guard posts the cancel
// code so the kernel stops waiting at once, drains the stream, and clears the
// mailbox so that the next hand-over does not read the cancel code.
struct HandoverSession {
  gkr_ctx* c;
  uint32_t res_seq = 0, mb_seq = 0;
  int k = 0, kd = 0, posted = 0;
  qm31 last = {0, 0, 0, 0};  // challenge k - 1, folded by the host
  bool launched = false, done = false;
  bool cancel_before_post = false;  // test hook (gkr_ctx_debug): leave without posting
  bool hold_post = false;           // test hook (gkr_ctx_debug): post only after the kernel's wait expired
  explicit HandoverSession(gkr_ctx* c_) : c(c_) {}
  // Launch k_handover<NV> over the vectors a (, b) of length len, to be folded by k challenges.
  template <int NV>
  int launch(const qm31* a, const qm31* b, uint64_t len, int k_, const CarriedFinish* fin = nullptr) {
    HostTimer ht(c, K_HOST_LAUNCH);
    if (len > (uint64_t)kHandMax || k_ < 0 || k_ > kTripMaxK || (len >> k_) == 0)
      return fail(GKR_ERR_DEVICE, "hand-over of %llu entries folded %d times", (unsigned long long)len, k_);
    k = k_;
    kd = k > 0 ? k - 1 : 0;
    posted = 0;
    res_seq = alloc_seq(&c->seq, 1);
    mb_seq = alloc_seq(&c->mb_seq, kd > 0 ? kd : 1);
    uint32_t spin_limit = kWaitSpinLimit;
    if (c->debug_handover_spins) {  // test hook: a short bounded wait that expires before the post
      spin_limit = c->debug_handover_spins;
      c->debug_handover_spins = 0;
      hold_post = kd > 0;  // only a kernel that waits can expire
    }
    if (c->debug_handover_cancel) {
      cancel_before_post = true;
      c->debug_handover_cancel = false;
    }
    CarriedFinish none;
    memset(&none, 0, sizeof none);
    GKR_LAUNCH(c, k_handover<NV>, dim3(1), dim3(kBlock), 0, a, b, (uint32_t)len, kd, c->mailbox,
                       mb_seq, spin_limit, c->h_vec, c->h_flag, res_seq, fin ? *fin : none);
    launched = true;
    return check_launch(c);
  }
  // Checks before a post: the test hooks leave without posting, or post only
  // once the kernel's wait has expired.
  int before_post() {
    if (!launched) return fail(GKR_ERR_DEVICE, "hand-over challenges posted before its launch");
    if (cancel_before_post) return fail(GKR_ERR_DEVICE, "hand-over cancelled before the challenges were posted");
    if (hold_post && posted == 0) {
      const auto t0 = std::chrono::steady_clock::now();
      volatile uint32_t* expired = &c->mailbox->expired;
      while (*expired != mb_seq && std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < 10.0) {
      }
    }
    return GKR_OK;
  }
  // Post challenge i (i == the number posted so far) as soon as it is drawn.
  int post_one(int i, const qm31& r) {
    if (i != posted || i >= k) return fail(GKR_ERR_DEVICE, "hand-over challenge %d posted out of order", i);
    TRY(before_post());
    posted = i + 1;
    if (i == k - 1) {  // the host's own fold
      last = r;
      return GKR_OK;
    }
    c->mailbox->alpha[i] = r;
    __atomic_store_n(&c->mailbox->seq, mb_seq + (uint32_t)i, __ATOMIC_RELEASE);
    return GKR_OK;
  }
  // Post the challenges not yet posted: chal holds all k.
  int post(const qm31* chal, int k_) {
    if (k_ != k) return fail(GKR_ERR_DEVICE, "hand-over folded %d times, %d challenges posted", k, k_);
    if (posted == k) return GKR_OK;
    TRY(before_post());
    const int from = posted;
    for (int r = from; r < kd; r++) c->mailbox->alpha[r] = chal[r];
    if (from < kd) __atomic_store_n(&c->mailbox->seq, mb_seq + (uint32_t)(kd - 1), __ATOMIC_RELEASE);
    last = chal[k - 1];
    posted = k;
    return GKR_OK;
  }
  // The folded vectors: count vectors of len entries each (the kernel's
  // vectors, twice as long, folded here by the last challenge).
  int fetch(uint64_t len, int count, std::vector<qm31>* out) {
    if (posted != k) return fail(GKR_ERR_DEVICE, "hand-over fetched before its %d challenges were posted", k);
    TRY(wait_result<0>(c, res_seq, nullptr, K_HOST_WAIT_TAIL, 0, kd > 0 ? mb_seq : 0));
    const uint64_t dl = k > 0 ? 2 * len : len;
    for (int v = 0; v < count; v++) out[v].assign(c->h_vec + v * dl, c->h_vec + (v + 1) * dl);
    done = true;
    if (k > 0) {
      HostTimer ht(c, K_HOST_FINISH);
      for (int v = 0; v < count; v++) {
        hostfield::fold(qwords(out[v].data()), len, qwords(&last));
        out[v].resize(len);
      }
    }
    return GKR_OK;
  }
  ~HandoverSession() {
    if (launched && !done) {
      __atomic_store_n(&c->mailbox->seq, kWaitCancel, __ATOMIC_RELEASE);
      drain(c);  // kernels still queued see the cancel code when they run
      (void)hipStreamSynchronize(c->stream);
      __atomic_store_n(&c->mailbox->seq, 0u, __ATOMIC_RELEASE);  // 0 is never a wanted sequence
    }
  }
};

// ------------------------------------------------------------------ multi-round trips (host side)
// A sumcheck over 2^T entries runs as a few device trips of K <= 3 rounds
// each (k_trip: one launch plus the finisher per trip), then k_handover
// folds the last trip's vectors by all of that trip's challenges but the last
// (the host folds the last one) and the host finishes the rounds on vectors
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
// Result delivery of the reducing kernels: k_finish / k_finish_wide launched
// behind them.  With GKR_TRIP_FUSED=1, trips whose one-entry-per-thread grid
// is at most kTripFusedGrid workgroups run on at most kTripFusedMax
// workgroups and finish in the kernel itself (an arrival counter, the last
// workgroup adds the rows); measured on MI355X this is slower than the
// finisher kernel (the Qwen layer's trips: 450 us with fused trips of up to
// 256 workgroups, 402 us plus one kernel boundary per trip without), so it
// is off.  Vectors of at most kTripSplitLanes / 2 entries use the
// two-lanes-per-entry layout.
#ifndef GKR_TRIP_FUSED
#define GKR_TRIP_FUSED 0
#endif
#ifndef GKR_TRIP_FUSED_GRID
#define GKR_TRIP_FUSED_GRID 64
#endif
constexpr unsigned kTripFusedGrid = GKR_TRIP_FUSED_GRID;
constexpr uint64_t kTripSplitLanes = 256ull * kBlock;
std::vector<Trip> plan_trips(int T, uint64_t host_len, int k0);
static inline int trip_nq(int kind, int K) { return kind == 2 ? (1 << K) : (1 << (2 * K)); }
// eqlin(z, X) = (1 - z)(1 - X) + z X, the multilinear eq factor of one coordinate.
static inline qm31 eqlin(const qm31& z, const qm31& x) {
  const qm31 one = qm31_one();
  return qm31_add(qm31_mul(qm31_sub(one, z), qm31_sub(one, x)), qm31_mul(z, x));
}
// Lagrange weights E[u] (u < 2^j, first challenge on the MSB) of r[0..j).
void lagrange_weights(const qm31* r, int j, qm31* E);
// The K rounds of a product-type trip from its cross sums G (4^K, row-major
// over sub-vectors c, c'), one after another.  Round j's polynomial is
//   p(X) = sum_v sum_{u,u',b,b'} E[u] E[u'] eqlin(X,b) eqlin(X,b') G[(u,b,v)][(u',b',v)]
// with E the Lagrange weights of the trip's challenges r_0 .. r_{j-1} (the
// first on the most significant bit) and v over the trip's later variables.
// Applying E on both sides is folding the rows and the columns of G on their
// top bit by each challenge as it is drawn, so round j reads a 2^(K-j) x
// 2^(K-j) matrix F:
//   p(X) = sum_v eqv(v) sum_{b,b'} eqlin(X,b) eqlin(X,b') F[(b,v)][(b',v)].
// For the eq-sumcheck (zt: the claim coordinates of the trip's variables;
// cpre: prod of eqlin(z_l, r_l) over the earlier rounds) v is weighted by
// eq(zt_{>j}, v) and p(X) multiplied by cpre * prod_{i<j} eqlin(zt_i, r_i) *
// eqlin(zt_j, X).
struct TripGram {
  int K, j = 0, dim;
  qm31 F[kMaxSums];
  const qm31* zt;
  qm31 pre;
  TripGram(const qm31* G, int K_, const qm31* zt_, const qm31& cpre) : K(K_), dim(1 << K_), zt(zt_), pre(cpre) {
    for (int q = 0; q < dim * dim; q++) F[q] = G[q];
  }
  // p(xs[k]) for the current round
  void values(int nx, const qm31* xs, qm31* out) const {
    const int h = dim / 2;
    qm31 H00 = qm31_zero(), H01 = qm31_zero(), H10 = qm31_zero(), H11 = qm31_zero();
    for (int v = 0; v < h; v++) {
      qm31 f00 = F[v * dim + v], f01 = F[v * dim + h + v], f10 = F[(h + v) * dim + v], f11 = F[(h + v) * dim + h + v];
      if (zt) {
        qm31 ez = qm31_one();
        for (int i = 0; i < K - j - 1; i++)
          ez = qm31_mul(ez, ((v >> (K - j - 2 - i)) & 1) ? zt[j + 1 + i] : qm31_sub(qm31_one(), zt[j + 1 + i]));
        f00 = qm31_mul(ez, f00);
        f01 = qm31_mul(ez, f01);
        f10 = qm31_mul(ez, f10);
        f11 = qm31_mul(ez, f11);
      }
      H00 = qm31_add(H00, f00);
      H01 = qm31_add(H01, f01);
      H10 = qm31_add(H10, f10);
      H11 = qm31_add(H11, f11);
    }
    const qm31 Hx = qm31_add(H01, H10);
    for (int k = 0; k < nx; k++) {
      const qm31 e1 = xs[k], e0 = qm31_sub(qm31_one(), e1);
      qm31 p = qm31_add(qm31_mul(qm31_mul(e0, e0), H00),
                        qm31_add(qm31_mul(qm31_mul(e0, e1), Hx), qm31_mul(qm31_mul(e1, e1), H11)));
      if (zt) p = qm31_mul(p, qm31_mul(pre, eqlin(zt[j], e1)));
      out[k] = p;
    }
  }
  // the current round's challenge r: fold to the next round's matrix
  void fold(const qm31& r) {
    const int h = dim / 2;
    const qm31 omr = qm31_sub(qm31_one(), r);
    const qm31 w00 = qm31_mul(omr, omr), w01 = qm31_mul(omr, r), w11 = qm31_mul(r, r);
    qm31 N[kMaxSums];
    for (int a = 0; a < h; a++)
      for (int b = 0; b < h; b++) {
        const qm31 cross = qm31_add(F[a * dim + b + h], F[(a + h) * dim + b]);
        N[a * h + b] = qm31_add(qm31_add(qm31_mul(w00, F[a * dim + b]), qm31_mul(w01, cross)),
                                qm31_mul(w11, F[(a + h) * dim + b + h]));
      }
    for (int q = 0; q < h * h; q++) F[q] = N[q];
    if (zt) pre = qm31_mul(pre, eqlin(zt[j], r));
    j++;
    dim = h;
  }
};
// Round j of a degree-1 trip from its 2^K sums S: p(0), p(1).
void trip_round_sum(const qm31* S, int K, int j, const qm31* r, qm31* out);
// tw given: the trip is launched ahead of its np pending challenges, which
// it takes from the mailbox (pend unused).
// carry_out given: no finisher is launched; the rows' finishing is described
// there for the next kernel of the chain (carry_in of the next trip launched
// ahead, or the hand-over), which adds them before it waits.
int launch_trip(gkr_ctx* c, int kind, int K, const qm31* sa, const qm31* sb, uint64_t n, int np,
                       const qm31* pend, qm31* da, qm31* db, const qm31* hi, const qm31* lo, int h, int slot,
                       RoundSink* sk, uint64_t b_rows = 0, int b_chunks = 0, const TripWait* tw = nullptr,
                       CarriedFinish* carry_out = nullptr, const CarriedFinish* carry_in = nullptr);
// Wait for a trip's nq sums (want: the mailbox sequence of a trip launched
// ahead, whose expired wait is then reported at once).
int wait_trip(gkr_ctx* c, const RoundSink& sk, int nq, qm31* out, uint32_t want = 0);

// The trips of one sumcheck launched ahead of their challenges, all at once
// behind the first: make() gives the next launch its mailbox wait, post()
// delivers its challenges (in launch order: one mailbox serves them all,
// since a trip has read its challenges before the host, having received its
// sums, posts the next).  Leaving with posts outstanding (an error) cancels
// the waiting kernels, drains the stream and forgets the arrival counter's
// value (cancelled trips do not arrive).  Off in the allocation-free mode,
// whose device memory is shared by every context.
struct AheadTrips {
  gkr_ctx* c;
  int outstanding = 0;
  uint32_t hold_want = 0;  // test hook (gkr_ctx_debug): this wait is posted only after it expired
  explicit AheadTrips(gkr_ctx* c_) : c(c_) {}
  bool enabled() const { return !c->noalloc; }
  int make(TripWait* tw) {
    uint32_t* words;
    TRY(ensureT(c, S_TRIPMB, 16, &words));  // status word, then kTripMaxK challenges at 16-byte offset
    if (!c->tripmb_valid) {  // fresh memory: the status may not hold a future sequence number
      GKR_LAUNCH(c, k_zero_u32, dim3(1), dim3(64), 0, words, 16u);
      TRY(check_launch(c));
      c->tripmb_valid = true;
    }
    tw->mb = c->mailbox;
    tw->want = alloc_seq(&c->mb_seq, 1);
    tw->spin_limit = kWaitSpinLimit;
    if (c->debug_trip_spins) {  // test hook: a short bounded wait that expires before the post
      tw->spin_limit = c->debug_trip_spins;
      c->debug_trip_spins = 0;
      hold_want = tw->want;
    }
    tw->status = words;
    tw->chal = reinterpret_cast<qm31*>(words + 4);
    outstanding++;
    return GKR_OK;
  }
  int post(const TripWait& tw, const qm31* chal, int np) {
    if (tw.want == hold_want) {
      const auto t0 = std::chrono::steady_clock::now();
      volatile uint32_t* expired = &c->mailbox->expired;
      while (*expired != tw.want &&
             std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < 10.0) {
      }
    }
    post_mailbox(c, tw.want, chal, np);
    outstanding--;
    return GKR_OK;
  }
  ~AheadTrips() {
    if (outstanding > 0) {
      __atomic_store_n(&c->mailbox->seq, kWaitCancel, __ATOMIC_RELEASE);
      drain(c);  // kernels still queued see the cancel code when they run
      (void)hipStreamSynchronize(c->stream);
      __atomic_store_n(&c->mailbox->seq, 0u, __ATOMIC_RELEASE);
      c->trip_count_valid = false;
    }
  }
};

int fetch_q(gkr_ctx* c, const qm31* dev, int count, qm31* host_out);

// ------------------------------------------------------------------ launches ahead of a walk step
int prelaunch_matmul(gkr_ctx* c, const gkr_matrix* A, const gkr_matrix* B, bool* launched);
int prelaunch_activation(gkr_ctx* c, const gkr_matrix* input, uint32_t tag, uint32_t table_log, bool* launched);
// gkr_prove_activation_layer without its copy of the multiplicities when
// out->multiplicities is null (the walk: the proof record holds them)
int prove_activation(gkr_ctx* c, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
                     const gkr_matrix* input, uint32_t tag, uint32_t table_log, gkr_channel* ch, gkr_proof* proof,
                     gkr_logup_out* out);
// S_PTWAIT: k_point_wait's status word at 0, the values' wait status at 64
// (prelaunch_activation), the copied point at 256, posted values (gamma,
// beta) at kPtWaitVals
constexpr size_t kPtWaitVals = 256 + ((sizeof(PointArg) + 15) & ~(size_t)15);
constexpr size_t kPtWaitBytes = kPtWaitVals + 4 * sizeof(qm31);
// The current step's last launch is done: launch what the walk queued for the next step.
inline int run_prelaunch(gkr_ctx* c) {
  if (!c->prelaunch) return GKR_OK;
  std::function<int()> f = std::move(c->prelaunch);
  c->prelaunch = nullptr;
  return f();
}
// After the first results of a restriction launched ahead: its point wait saw the post.
inline int check_point_wait(gkr_ctx* c) {
  const uint32_t w = c->point_mb, v = c->vals_mb;
  c->point_mb = 0;
  c->vals_mb = 0;
  if (w && __atomic_load_n(&c->mailbox->expired, __ATOMIC_ACQUIRE) == w) {
    c->wait_expired = true;
    return fail(GKR_ERR_DEVICE, "kernels launched ahead stopped waiting for their claim point (mailbox %u)", w);
  }
  if (v && __atomic_load_n(&c->vmailbox->expired, __ATOMIC_ACQUIRE) == v) {
    c->wait_expired = true;
    return fail(GKR_ERR_DEVICE, "kernels launched ahead stopped waiting for their posted values (mailbox %u)", v);
  }
  return GKR_OK;
}
// Drops kernels launched ahead that will not be used: the cancel code ends
// their waits, the stream drains, the mailboxes are cleared.
inline void cancel_prelaunch(gkr_ctx* c) {
  c->prelaunch = nullptr;
  if (!c->pre.active) return;
  __atomic_store_n(&c->mailbox->seq, kWaitCancel, __ATOMIC_RELEASE);
  __atomic_store_n(&c->vmailbox->seq, kWaitCancel, __ATOMIC_RELEASE);
  drain(c);
  (void)hipStreamSynchronize(c->stream);
  __atomic_store_n(&c->mailbox->seq, 0u, __ATOMIC_RELEASE);
  __atomic_store_n(&c->vmailbox->seq, 0u, __ATOMIC_RELEASE);
  c->pre.active = false;
  c->pre.act = false;
  c->pre.hold_vals = false;
  c->point_mb = 0;
  c->vals_mb = 0;
  c->fb_pending = false;
  c->mm.valid = false;
}

// sum_i v[i] * eq[i] (v M31-valued, length n).
int dot_m31(gkr_ctx* c, const uint32_t* v, const qm31* eq, uint64_t n, qm31* out);


// ------------------------------------------------------------------ channel and proof records
struct gkr_channel {
  PoseidonChannel ch;
};
#define CH_CHECK(ch) \
  if (!(ch)) return fail(GKR_ERR_INVALID, "null channel")

// A LayerNorm (tag 4) or RMSNorm (tag 8) layer's proof fields (types.rs
// LayerProof::LayerNorm / RMSNorm): RMSNorm keeps rms^2 in mean_eval, the
// square sum in sum0, its final input in p0_final0, (input, scale) finals in
// lin_final0/1, the per-row rms^2 in rows0.
struct NormRec {
  qm31 input_eval, output_eval, mean_eval, rsqrt_eval, var_eval;
  uint32_t n_active = 0;
  qm31 sum0, sum1;
  std::vector<qm31> p0, lin, logup;  // c0..c3 per round
  qm31 p0_final0, p0_final1, lin_final0, lin_final1, cb_input, cb_mean;
  qm31 claimed_sum, w_eval, in_eval, out_eval;
  std::vector<uint32_t> mults;
  std::vector<qm31> mult_rp;  // c0, c1 per round
  qm31 mult_final, mult_sum;
  felt table_commitment;
  std::vector<uint32_t> rows0, rows1;  // per padded row
};
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
  // Activation: mults still in slot mult_slot of mult_ring (mult_count
  // entries) until layer_take_mults copies them; -1: in mults
  std::shared_ptr<MultRing> mult_ring;
  int mult_slot = -1;
  size_t mult_count = 0;
  std::vector<qm31> mult_rp;  // c0,c1 per round
  qm31 mult_final, mult_sum;
  NormRec norm;  // tags 4 (LayerNorm) and 8 (RMSNorm)
};
// A MatMul layer's claim on its weight: MLE(B)(r_j || sumcheck challenges) =
// final_b (push_matmul_weight_data, prover.rs:1465-1483).
struct WeightClaimRec {
  const gkr_matrix* b;
  std::vector<qm31> point;
  qm31 value;
};
// Serialization of a proof's layers while the proof is built
// (gkr_proof_stream_to); defined with the serializer.
struct ProofStream;
struct gkr_proof {
  gkr_proof();
  ~gkr_proof();
  // a deque: appending keeps earlier records in place (the stream's thread reads them)
  std::deque<LayerRec> layers;
  std::vector<qm31> in_point;
  qm31 in_value = {0, 0, 0, 0};
  std::vector<felt> weight_commitments;
  std::vector<WeightClaimRec> weight_claims;      // recorded by the MatMul layers, in proving order
  std::vector<std::vector<felt>> weight_openings;  // serialized opening records (claim + MleOpeningProof)
  std::vector<std::vector<gkr_felt>> binding_groups;  // serialized aggregated binding proofs
  felt io_commitment = {{0, 0, 0, 0}};
  std::unique_ptr<ProofStream> stream;
};
// Appends a layer record (and hands it to the proof's stream, if any).
void proof_add_layer(gkr_proof* p, LayerRec&& L);
// Copies an activation record's multiplicities out of its ring slot and frees the slot.
void layer_take_mults(LayerRec& L);
// Drops the records after the first n (a walk step proved again).
void proof_truncate(gkr_proof* p, size_t n);

// ------------------------------------------------------------------ provided by one unit to the others
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

constexpr int kEqLoMax = 10;  // variables in the lower eq table of a trip
struct Eq3Plan {
  int nv = 0;
  std::vector<Trip> trips;
  std::vector<uint32_t> hi_off, lo_off;  // per trip, offsets into S_EQPARTS
  std::vector<int> h;                    // per trip, variables in the lower table
  // with_split: eq(z, .) as the product of a table over z[0, nv - split_h)
  // and one over z[nv - split_h, nv) (split_h = nv / 2, as eq_split), offsets
  // into S_EQPARTS
  int split_h = 0;
  uint32_t split_hi_off = 0, split_lo_off = 0;
};

// A new matrix handle (owned: freed with the handle).
gkr_matrix* new_matrix(gkr_ctx* c, uint32_t* dev, uint64_t rows, uint64_t cols, bool owned);
// Trip 0 of a product sumcheck as product_sumcheck launches it: the
// weight-side column-chunk partials it adds into in_b on the way
// (b_chunks > 0), and a hook called with its sums before the first round
// (the walk's fresh matmul claim, whose value is the trace of those sums).
struct FirstTrip {
  const qm31* b_partials = nullptr;
  uint64_t b_rows = 0;
  int b_chunks = 0;
  std::function<int(const qm31* g, int K)> on_sums;
};
// The walk's matmul step with a fresh claim (matmul.hip): the claim value
// and the layer proof in one pass, k > 1.
int walk_matmul_fresh(gkr_ctx* c, const gkr_qm31* point, uint32_t n_point, gkr_qm31* value, const gkr_matrix* a,
                      const gkr_matrix* b, gkr_channel* ch, gkr_proof* proof, gkr_qm31* round_polys,
                      gkr_qm31* final_a, gkr_qm31* final_b, gkr_qm31* next_point, gkr_qm31* next_value);
// Degree-2 product sumcheck over 2^T entries (matmul.hip).
int product_sumcheck(gkr_ctx* c, PoseidonChannel& ch, int T, const qm31* in_a, const qm31* in_b,
                            qm31* const bufs_a[2], qm31* const bufs_b[2], const qm31* g0, int k0,
                            gkr_qm31* round_polys, gkr_qm31* challenges, gkr_qm31* final_a, gkr_qm31* final_b,
                            const qm31* scale3 = nullptr, const FirstTrip* ft = nullptr);
// Eq-weighted degree-3 sumcheck sum_x eq(z, x) w(x) d(x) (logup.hip): plan and eq tables,
int eq3_prepare(gkr_ctx* c, const qm31* z, int nv, Eq3Plan* pl, bool with_split = false);
// one trip,
int eq3_launch_trip(gkr_ctx* c, const Eq3Plan& pl, size_t j, const qm31* w, const qm31* d, int np,
                           const qm31* pend, qm31* dw, qm31* dd, int slot, RoundSink* sk,
                           const TripWait* tw = nullptr, CarriedFinish* carry_out = nullptr,
                           const CarriedFinish* carry_in = nullptr);
// the whole sumcheck; after_last, when given, is called right after its last
// launch (the hand-over), to queue work that must not sit between its trips
// and may not allocate.
int eq3_sumcheck(gkr_ctx* c, PoseidonChannel& C, const qm31* z, const Eq3Plan& pl, qm31* w0, qm31* d0,
                        qm31* w1, qm31* d1, gkr_qm31* rp_out, qm31* chal, qm31 fin[3],
                        const RoundSink* pre0 = nullptr, const std::function<int()>* after_last = nullptr);
// LayerNorm (ln) or RMSNorm layer reducer (norm.hip); commit_gamma: fill
// gamma_commitment (one Poseidon mix per scale entry; the walk, which neither
// mixes nor serializes it, skips it).
int prove_norm(gkr_ctx* c, bool ln, const gkr_qm31* claim_point, uint32_t n_point, const gkr_qm31* claim_value,
               const gkr_matrix* X, uint64_t dim, const uint32_t* gamma, uint64_t ng, gkr_channel* ch,
               gkr_proof* proof, gkr_norm_out* out, bool commit_gamma);
// prove_mle_opening_with_commitment (crypto/mle_opening.rs:1654-1915) over
// a weight's column-major padded MLE (b) or a resident QM31 vector (q, qn
// entries, a power of two) (commit.hip); the record gets the claim first when
// with_claim is set, then the MleOpeningProof.
struct OpenSrc {
  const gkr_matrix* b;
  const qm31* q;
  uint64_t qn;
};
int mle_opening(gkr_ctx* c, const OpenSrc& src, const gkr_qm31* point, uint32_t n_point, const gkr_qm31* expected,
                PoseidonChannel& C, felt* commitment, std::vector<felt>& rec, bool with_claim);
// Activation table outputs (host copy, cached per context).
const std::vector<uint32_t>& cached_table(gkr_ctx* c, uint32_t tag, uint32_t log_size);
