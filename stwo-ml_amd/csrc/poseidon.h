// Starknet Poseidon (Hades over felt252) and the Fiat-Shamir channel of the
// GKR prover, on the host.
//
// Hades: 91 rounds over a 3-element state; rounds 0-3 and 87-90 are full
// (x^3 on every lane), rounds 4-86 are partial (x^3 on lane 2 only).  Each
// round adds its three round constants to the three lanes, applies the
// S-box, then the MDS matrix [[3,1,1],[1,-1,1],[1,1,-2]] (evaluated below in
// the equivalent compressed-constant form)
// (reference: engine/src/recursive/hades_air.rs:1892-2012 for the round
// structure and MDS; constants per engine/src/crypto/poseidon_constants.rs).
//
// Channel semantics follow engine/src/crypto/poseidon_channel.rs:83-308:
//   mix_felt(v):  digest = hades([digest, v, 2])[0], n_draws = 0
//   draw_felt252: hades([digest, n_draws, 3])[0],   n_draws += 1
//   draw_qm31:    four 31-bit limbs of one draw, LSB first, each mod P
//   mix_poly_coeffs(c0,c1,c2): digest = hash_many([digest, pack(c0,c1), pack(c2)])
//   mix_poly_coeffs_deg3(c0..c3): hash_many([digest, pack(c0,c1), pack(c2,c3)])
//   mix_felts(qs): hash_many([digest, pack(pairs)..., pack(last single)])
// where pack(v...) = fold(1, acc * 2^31 + v) over the M31 words.
#pragma once
#include <stdint.h>
#include <stdlib.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#include "felt252.h"
#include "field.h"

namespace gkr {

#include "hades_constants.inc"

// Round constants in the compressed form: rounds 0-3 and 88-90 keep their
// three raw constants; the constants that partial rounds 4-86 add to lanes 0
// and 1 (which skip the S-box) are pushed through the linear layer and
// folded into round 87, so a partial round adds a single constant to lane 2.
// The permutation is unchanged (hades_air.rs:1137-1180 states the same
// compression).
struct hades_rc {
  felt full_first[4][3];
  felt partial[83];
  felt full_last[4][3];
  static void mds(felt s[3]) {
    felt t = felt_add(felt_add(s[0], s[1]), s[2]);
    felt n0 = felt_add(t, felt_add(s[0], s[0]));
    felt n1 = felt_sub(t, felt_add(s[1], s[1]));
    felt n2 = felt_sub(t, felt_add(felt_add(s[2], s[2]), s[2]));
    s[0] = n0;
    s[1] = n1;
    s[2] = n2;
  }
  hades_rc() {
    felt raw[91][3];
    for (int r = 0; r < 91; r++)
      for (int j = 0; j < 3; j++) {
        const uint64_t* c = kHadesRoundConstants[3 * r + j];
        raw[r][j] = felt_to_mont(felt{{c[0], c[1], c[2], c[3]}});
      }
    for (int r = 0; r < 4; r++)
      for (int j = 0; j < 3; j++) full_first[r][j] = raw[r][j];
    felt acc[3] = {felt_zero(), felt_zero(), felt_zero()};
    for (int r = 0; r < 83; r++) {
      for (int j = 0; j < 3; j++) acc[j] = felt_add(acc[j], raw[4 + r][j]);
      partial[r] = acc[2];
      acc[2] = felt_zero();
      mds(acc);
    }
    for (int j = 0; j < 3; j++) full_last[0][j] = felt_add(acc[j], raw[87][j]);
    for (int r = 1; r < 4; r++)
      for (int j = 0; j < 3; j++) full_last[r][j] = raw[87 + r][j];
  }
};
inline const hades_rc& hades_constants() {
  static const hades_rc k;
  return k;
}

// The permutation with values kept in [0, 2p) inside (felt_*_lazy) and
// reduced once at the end.  A partial round x = s2 + c, y = x^3 followed by
// the MDS layer (t = s0 + s1 + y; s0 = t + 2 s0, s1 = t - 2 s1, s2 = t - 3y)
// is evaluated as s0' = (3 s0 + s1) + y, s1' = (s0 - s1) + y and
// s2' = (s0 + s1) - 2y with the next round's constant folded into (s0 + s1):
// one square, one product and seven additions per partial round.
inline void hades_permute(felt s[3]) {
  const hades_rc& k = hades_constants();
  felt a = s[0], b = s[1], c = s[2];
  auto full = [&](const felt* rc) {
    const felt x0 = felt_add_lazy(a, rc[0]), x1 = felt_add_lazy(b, rc[1]), x2 = felt_add_lazy(c, rc[2]);
    const felt y0 = felt_mul_lazy(felt_sqr_lazy(x0), x0);
    const felt y1 = felt_mul_lazy(felt_sqr_lazy(x1), x1);
    const felt y2 = felt_mul_lazy(felt_sqr_lazy(x2), x2);
    const felt t = felt_add_lazy(felt_add_lazy(y0, y1), y2);
    a = felt_add_lazy(t, felt_add_lazy(y0, y0));
    b = felt_sub_lazy(t, felt_add_lazy(y1, y1));
    c = felt_sub_lazy(t, felt_add_lazy(felt_add_lazy(y2, y2), y2));
  };
  for (int r = 0; r < 4; r++) full(k.full_first[r]);
  felt x = felt_add_lazy(c, k.partial[0]);
  for (int r = 0; r < 83; r++) {
    const felt u = felt_add_lazy(a, b);
    const felt A = felt_add_lazy(felt_add_lazy(a, a), u);  // 3 s0 + s1
    const felt B = felt_sub_lazy(a, b);                    // s0 - s1
    const felt un = r + 1 < 83 ? felt_add_lazy(u, k.partial[r + 1]) : u;
    const felt y = felt_mul_lazy(felt_sqr_lazy(x), x);
    a = felt_add_lazy(A, y);
    b = felt_add_lazy(B, y);
    x = felt_sub_lazy(un, felt_add_lazy(y, y));
  }
  c = x;
  for (int r = 0; r < 4; r++) full(k.full_last[r]);
  s[0] = felt_reduce_once(a);
  s[1] = felt_reduce_once(b);
  s[2] = felt_reduce_once(c);
}

// hash(a, b) = hades([a, b, 2])[0]
inline felt poseidon_hash(const felt& a, const felt& b) {
  felt s[3] = {a, b, felt_from_u64(2)};
  hades_permute(s);
  return s[0];
}

// Rate-2 sponge from the zero state.  A trailing single input x absorbs
// [x, 1]; an even count finishes by absorbing [1, 0].  Output lane 0.
inline felt poseidon_hash_many(const felt* in, int n) {
  felt s[3] = {felt_zero(), felt_zero(), felt_zero()};
  const felt one = felt_one();
  int i = 0;
  for (; i + 1 < n; i += 2) {
    s[0] = felt_add(s[0], in[i]);
    s[1] = felt_add(s[1], in[i + 1]);
    hades_permute(s);
  }
  if (i < n) {
    s[0] = felt_add(s[0], in[i]);
    s[1] = felt_add(s[1], one);
  } else {
    s[0] = felt_add(s[0], one);
  }
  hades_permute(s);
  return s[0];
}

// 1 || v0 || v1 || ... with 31 bits per word (n <= 8 keeps it below 2^249,
// hence canonical without reduction).  Returns Montgomery form.
inline felt pack_m31s(const uint32_t* v, int n) {
  uint64_t l[4] = {1, 0, 0, 0};
  for (int k = 0; k < n; k++) {
    // l = l << 31 | v[k]
    l[3] = (l[3] << 31) | (l[2] >> 33);
    l[2] = (l[2] << 31) | (l[1] >> 33);
    l[1] = (l[1] << 31) | (l[0] >> 33);
    l[0] = (l[0] << 31) | (uint64_t)v[k];
  }
  return felt_to_mont(felt{{l[0], l[1], l[2], l[3]}});
}
inline felt securefield_to_felt(const qm31& q) {
  uint32_t w[4] = {q.a, q.b, q.c, q.d};
  return pack_m31s(w, 4);
}

// A batch of draws from one channel state, draw i = hades([digest, base + i, 3])[0],
// has no dependency between draws: DrawPool spreads them over worker threads
// (the caller works too).  Items are claimed through one atomic word holding
// (batch id << 32 | batch size << 16 | next index): every decision of a
// worker reads only that word, a worker only ever takes items of the batch it
// has seen, and the batch's fields (read after a successful claim) cannot
// change before all its items are done.  Workers spin for GKR_DRAW_SPIN_US
// (default 2000) after a batch, then sleep on a condition variable.  One batch
// at a time; a second caller (another thread) computes its batch alone.
// Threads: GKR_DRAW_THREADS, default min(8, hardware threads - 1); 0 disables
// the pool.
class DrawPool {
 public:
  static DrawPool& instance() {
    static DrawPool* p = new DrawPool();  // never destroyed: detached workers may still wait at exit
    return *p;
  }
  template <typename F>
  bool run(const felt& digest, uint64_t base, size_t n, F&& conv, qm31* out) {
    if (workers_ == 0 || n >= (1u << 16)) return false;
    std::unique_lock<std::mutex> busy(busy_, std::try_to_lock);
    if (!busy.owns_lock()) return false;
    const uint64_t job = ++job_ & 0xffffffffull;
    digest_ = digest;
    base_ = base;
    n_ = n;
    out_ = out;
    done_.store(0, std::memory_order_relaxed);
    claim_.store((job << 32) | ((uint64_t)n << 16), std::memory_order_release);
    {
      std::lock_guard<std::mutex> g(sleep_mu_);
      gen_.store(job, std::memory_order_release);
    }
    if (sleepers_.load(std::memory_order_acquire) > 0) sleep_cv_.notify_all();
    work(job, conv);
    while (done_.load(std::memory_order_acquire) < n) {
    }
    return true;
  }

 private:
  DrawPool() {
    int t = (int)std::thread::hardware_concurrency() - 1;
    if (t > 8) t = 8;
    if (const char* e = getenv("GKR_DRAW_THREADS")) t = atoi(e);
    if (t < 0) t = 0;
    workers_ = t;
    if (const char* e = getenv("GKR_DRAW_SPIN_US")) spin_us_ = atoi(e);
    for (int i = 0; i < t; i++) std::thread([this] { loop(); }).detach();
  }
  template <typename F>
  void work(uint64_t job, F&& conv) {
    uint64_t c = claim_.load(std::memory_order_acquire);
    for (;;) {
      if ((c >> 32) != (job & 0xffffffffull) || (c & 0xffffull) >= ((c >> 16) & 0xffffull)) return;
      if (!claim_.compare_exchange_weak(c, c + 1, std::memory_order_acq_rel, std::memory_order_acquire)) continue;
      const size_t i = (size_t)(c & 0xffffull);
      out_[i] = conv(digest_, base_ + i);
      done_.fetch_add(1, std::memory_order_release);
      c = claim_.load(std::memory_order_acquire);
    }
  }
  void loop();
  int workers_ = 0;
  int spin_us_ = 2000;  // a prover posts batches a few hundred microseconds apart
  std::mutex busy_;
  uint64_t job_ = 0;  // written by the poster only, under busy_
  felt digest_{};
  uint64_t base_ = 0;
  size_t n_ = 0;
  qm31* out_ = nullptr;
  std::atomic<uint64_t> claim_{0};
  std::atomic<size_t> done_{0};
  std::atomic<uint64_t> gen_{0};
  std::atomic<int> sleepers_{0};
  std::mutex sleep_mu_;
  std::condition_variable sleep_cv_;
};

class PoseidonChannel {
 public:
  felt digest;  // Montgomery form
  uint32_t n_draws = 0;
  uint64_t hash_count = 0;

  PoseidonChannel() : digest(felt_zero()) {}

  void mix_felt(const felt& v) {
    felt s[3] = {digest, v, felt_from_u64(2)};
    hades_permute(s);
    digest = s[0];
    n_draws = 0;
    hash_count++;
  }
  void mix_u64(uint64_t v) { mix_felt(felt_from_u64(v)); }
  void mix_secure_field(const qm31& v) { mix_felt(securefield_to_felt(v)); }

  felt draw_felt252() {  // returns Montgomery form
    felt s[3] = {digest, felt_from_u64(n_draws), felt_from_u64(3)};
    hades_permute(s);
    n_draws++;
    hash_count++;
    return s[0];
  }
  // draw_qm31: four 31-bit limbs of the drawn felt, LSB first, each mod P
  // (poseidon_channel.rs:176-200).
  static qm31 felt_to_qm31(const felt& mont) {
    const felt x = felt_from_mont(mont);
    uint32_t m[4];
    for (int k = 0; k < 4; k++) {
      const int bit = 31 * k, limb = bit >> 6, off = bit & 63;
      uint64_t v = x.l[limb] >> off;
      if (off > 33 && limb < 3) v |= x.l[limb + 1] << (64 - off);
      m[k] = m31_from_u32((uint32_t)(v & 0x7fffffffull));
    }
    return qm31{m[0], m[1], m[2], m[3]};
  }
  qm31 draw_qm31() { return felt_to_qm31(draw_felt252()); }
  // One draw without advancing the channel: hades([digest, index, 3])[0].
  static qm31 draw_at(const felt& digest, uint64_t index) {
    felt s[3] = {digest, felt_from_u64(index), felt_from_u64(3)};
    hades_permute(s);
    return felt_to_qm31(s[0]);
  }
  void draw_qm31s(qm31* out, size_t n) {
    if (n >= 2 && DrawPool::instance().run(digest, n_draws, n, draw_at, out)) {
      n_draws += (uint32_t)n;
      hash_count += n;
      return;
    }
    for (size_t i = 0; i < n; i++) out[i] = draw_qm31();
  }
  void mix_poly_coeffs(const qm31& c0, const qm31& c1, const qm31& c2) {
    const uint32_t w[12] = {c0.a, c0.b, c0.c, c0.d, c1.a, c1.b, c1.c, c1.d, c2.a, c2.b, c2.c, c2.d};
    felt in[3] = {digest, pack_m31s(w, 8), pack_m31s(w + 8, 4)};
    digest = poseidon_hash_many(in, 3);
    n_draws = 0;
    hash_count++;
  }
  void mix_poly_coeffs_deg3(const qm31& c0, const qm31& c1, const qm31& c2, const qm31& c3) {
    const uint32_t w[16] = {c0.a, c0.b, c0.c, c0.d, c1.a, c1.b, c1.c, c1.d,
                            c2.a, c2.b, c2.c, c2.d, c3.a, c3.b, c3.c, c3.d};
    felt in[3] = {digest, pack_m31s(w, 8), pack_m31s(w + 8, 8)};
    digest = poseidon_hash_many(in, 3);
    n_draws = 0;
    hash_count++;
  }
  // Poseidon252Channel::mix_felts (stwo core/channel/poseidon252.rs:70-84),
  // the channel of STWO's LogUp-GKR batch: the same packing as mix_felts, but
  // an empty slice still hashes [digest] and resets n_draws.
  void mix_felts_stwo(const qm31* q, int n) {
    if (n > 0) return mix_felts(q, n);
    digest = poseidon_hash_many(&digest, 1);
    n_draws = 0;
    hash_count++;
  }
  // PoseidonChannel::mix_felts (poseidon_channel.rs:261-297): an empty slice
  // leaves the channel unchanged.
  void mix_felts(const qm31* q, int n) {
    if (n <= 0) return;
    felt* in = new felt[1 + (n + 1) / 2];
    int m = 0;
    in[m++] = digest;
    for (int i = 0; i < n; i += 2) {
      if (i + 1 < n) {
        const uint32_t w[8] = {q[i].a, q[i].b, q[i].c, q[i].d, q[i + 1].a, q[i + 1].b, q[i + 1].c, q[i + 1].d};
        in[m++] = pack_m31s(w, 8);
      } else {
        in[m++] = securefield_to_felt(q[i]);
      }
    }
    digest = poseidon_hash_many(in, m);
    delete[] in;
    n_draws = 0;
    hash_count++;
  }

  // State in the reference's to_gpu_state layout (poseidon_channel.rs:109-135):
  // 8 little-endian u32 digest words, n_draws, hash_count lo, hash_count hi.
  void export_state(uint32_t st[11]) const {
    felt_canon_to_words(felt_from_mont(digest), st);
    st[8] = n_draws;
    st[9] = (uint32_t)hash_count;
    st[10] = (uint32_t)(hash_count >> 32);
  }
  void import_state(const uint32_t st[11]) {
    digest = felt_to_mont(felt_canon_from_words(st));
    n_draws = st[8];
    hash_count = (uint64_t)st[9] | ((uint64_t)st[10] << 32);
  }
};

inline void DrawPool::loop() {
  uint64_t seen = gen_.load(std::memory_order_acquire);
  for (;;) {
    // spin for spin_us_ waiting for a batch, then sleep until one is posted
    const auto t0 = std::chrono::steady_clock::now();
    uint64_t g;
    while ((g = gen_.load(std::memory_order_acquire)) == seen) {
      if (std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(spin_us_)) {
        std::unique_lock<std::mutex> lk(sleep_mu_);
        sleepers_.fetch_add(1, std::memory_order_acq_rel);
        sleep_cv_.wait(lk, [&] { return gen_.load(std::memory_order_acquire) != seen; });
        sleepers_.fetch_sub(1, std::memory_order_acq_rel);
      }
    }
    seen = g;
    work(g, PoseidonChannel::draw_at);
  }
}

}  // namespace gkr
