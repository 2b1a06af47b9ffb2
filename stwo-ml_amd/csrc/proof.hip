// Proof container and serialize_gkr_model_proof (engine/src/cairo_serde.rs).
#include "internal.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <mutex>
#include <thread>
// ------------------------------------------------------------------ proof container
gkr_proof::gkr_proof() = default;
gkr_proof::~gkr_proof() = default;  // a stream's thread is stopped and joined first (~ProofStream)
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
// A counting pass (constant time per layer: runs of u32 values are counted,
// not visited) gives every layer's offset; the layers are then written
// straight into the caller's buffer by several threads.
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
  void us(const uint32_t* v, size_t count) {  // count felts of u32 values
    if (out)
      for (size_t i = 0; i < count; i++) {
        gkr_felt& f = out[n + i];
        f.w[0] = v[i];
        for (int k = 1; k < 8; k++) f.w[k] = 0;
      }
    n += count;
  }
  void q(const qm31& x) { u(x.a); u(x.b); u(x.c); u(x.d); }
  void f(const felt& canon) {
    if (out) felt_canon_to_words(canon, out[n].w);
    n++;
  }
};
// (c0, c2, c3) per round, c1 omitted
static void ser_deg3(const std::vector<qm31>& rp, Ser& s) {
  const size_t nr = rp.size() / 4;
  s.u(nr);
  for (size_t r = 0; r < nr; r++) {
    s.q(rp[4 * r]);
    s.q(rp[4 * r + 2]);
    s.q(rp[4 * r + 3]);
  }
}
// LayerProof::LayerNorm (cairo_serde.rs:1388-1484) and LayerProof::RMSNorm
// (1648-1720; no multiplicity sumcheck in this format), non-SIMD, with their
// Part 0 proofs; per-row statistics only for more than one padded row.
static void serialize_norm(const LayerRec& L, Ser& s) {
  const NormRec& N = L.norm;
  const bool ln = L.tag == 4;
  s.u(L.tag);
  s.q(N.input_eval);
  s.q(N.output_eval);
  s.q(N.mean_eval);
  s.q(N.rsqrt_eval);
  s.f(N.table_commitment);
  s.u(0);  // simd_combined
  s.u(1);  // Part 0 present
  s.u(N.n_active);
  s.q(N.sum0);
  if (ln) s.q(N.sum1);
  ser_deg3(N.p0, s);
  s.q(N.p0_final0);
  if (ln) s.q(N.p0_final1);
  ser_deg3(N.lin, s);
  s.q(N.lin_final0);
  s.q(N.lin_final1);
  if (ln) {
    s.q(N.cb_input);
    s.q(N.cb_mean);
  }
  s.u(1);  // LogUp proof (serialize_logup_proof, with multiplicities: cairo_serde.rs:1071-1105)
  s.q(N.claimed_sum);
  ser_deg3(N.logup, s);
  s.q(N.w_eval);
  s.q(N.in_eval);
  s.q(N.out_eval);
  s.u(N.mults.size());
  s.us(N.mults.data(), N.mults.size());
  const bool multi_row = N.rows0.size() > 1;
  if (ln) {
    s.u(1);  // serialize_multiplicity_sumcheck (cairo_serde.rs:1138-1156)
    s.u(N.mult_rp.size() / 2);
    for (const qm31& c : N.mult_rp) s.q(c);
    s.q(N.mult_final);
    s.q(N.mult_sum);
    s.q(N.var_eval);
    for (const std::vector<uint32_t>* rv : {&N.rows0, &N.rows1}) {
      s.u(multi_row ? 1 : 0);
      if (multi_row) {
        s.u(rv->size());
        s.us(rv->data(), rv->size());
      }
    }
  } else {
    s.u(multi_row ? 1 : 0);
    if (multi_row) {
      s.u(N.rows0.size());
      s.us(N.rows0.data(), N.rows0.size());
    }
  }
}
static void serialize_layer(const LayerRec& L, Ser& s) {
  {
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
    } else if (L.tag == 4 || L.tag == 8) {
      serialize_norm(L, s);
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
      s.us(L.mults.data(), L.mults.size());
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
}
static void serialize_tail(const gkr_proof* p, Ser& s) {
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
// ------------------------------------------------------------------ serialization while proving
// A thread of the proof writes each layer record, as the reducers append it,
// into the caller's buffer at the offset the records before it leave (layer
// 0 at felt 1, after the layer count), so that serializing the finished
// proof only writes the count and the tail.  A layer that does not fit ends
// the streaming (gkr_proof_serialize then writes every layer itself).
//
// The thread spins on the queue length for a while before it sleeps, and the
// reducer's thread notifies it only when it sleeps: a condition-variable wake
// per record (a futex call) would land on the transcript's critical path.
struct ProofStream {
  static constexpr double kSpinSeconds = 0.005;
  gkr_felt* out;
  size_t cap;
  std::mutex m;
  std::condition_variable work, idle;
  std::vector<const LayerRec*> queue;  // records handed over, in proof order
  size_t written = 0;                  // queue entries written (or counted, after an overflow)
  std::vector<size_t> off{1};          // off[i]: first felt of layer i, for i <= written
  bool overflow = false, stop = false;
  std::atomic<size_t> queued{0};       // queue.size(), read without the lock while spinning
  std::atomic<bool> sleeping{false}, stopping{false};
  std::thread th;
  ProofStream(gkr_felt* o, size_t c) : out(o), cap(c) { th = std::thread([this] { run(); }); }
  ~ProofStream() {
    {
      std::lock_guard<std::mutex> lk(m);
      stop = true;
      stopping.store(true, std::memory_order_release);
    }
    work.notify_all();
    th.join();
    for (size_t i = written; i < queue.size(); i++) layer_take_mults(*const_cast<LayerRec*>(queue[i]));
  }
  void run() {
    std::unique_lock<std::mutex> lk(m);
    for (;;) {
      if (!stop && written == queue.size()) {  // spin, then sleep until add() or the destructor wakes it
        const size_t w = written;
        lk.unlock();
        const auto t0 = std::chrono::steady_clock::now();
        for (uint32_t i = 1;; i++) {
          _mm_pause();
          if (queued.load(std::memory_order_acquire) != w || stopping.load(std::memory_order_acquire)) break;
          if ((i & 1023) == 0 &&
              std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kSpinSeconds)
            break;
        }
        lk.lock();
        sleeping.store(true, std::memory_order_seq_cst);
        work.wait(lk, [&] { return stop || written < queue.size(); });
        sleeping.store(false, std::memory_order_seq_cst);
      }
      if (stop) return;
      const LayerRec* L = queue[written];
      const size_t at = off[written];
      bool fits = !overflow;
      lk.unlock();
      // the record is this thread's until it is counted as written
      layer_take_mults(*const_cast<LayerRec*>(L));
      Ser count{nullptr};
      serialize_layer(*L, count);
      fits = fits && at + count.n <= cap;
      if (fits) {
        Ser w{out};
        w.n = at;
        serialize_layer(*L, w);
      }
      lk.lock();
      if (!fits) overflow = true;
      off.push_back(at + count.n);
      written++;
      idle.notify_all();
    }
  }
  void add(const LayerRec* L) {
    {
      std::lock_guard<std::mutex> lk(m);
      queue.push_back(L);
      queued.store(queue.size(), std::memory_order_release);
    }
    // the thread sets `sleeping` under the lock before its last look at the
    // queue, so either it sees this record or this load sees it sleeping
    if (sleeping.load(std::memory_order_seq_cst)) work.notify_one();
  }
  // Returns once every record handed over is written.
  void sync() {
    std::unique_lock<std::mutex> lk(m);
    idle.wait(lk, [&] { return written == queue.size(); });
  }
  void truncate(size_t n) {
    sync();
    std::lock_guard<std::mutex> lk(m);
    if (n < queue.size()) {
      queue.resize(n);
      written = n;
      off.resize(n + 1);
      queued.store(n, std::memory_order_release);
    }
  }
};
void layer_take_mults(LayerRec& L) {
  if (L.mult_slot < 0) return;
  const uint32_t* src = L.mult_ring->buf[L.mult_slot];
  L.mults.assign(src, src + L.mult_count);
  L.mult_ring->busy[L.mult_slot].store(0, std::memory_order_release);
  L.mult_slot = -1;
  L.mult_ring.reset();
}
void proof_add_layer(gkr_proof* p, LayerRec&& L) {
  p->layers.push_back(std::move(L));
  if (p->stream)
    p->stream->add(&p->layers.back());  // its thread copies the multiplicities before writing the record
  else
    layer_take_mults(p->layers.back());
}
void proof_truncate(gkr_proof* p, size_t n) {
  if (p->stream) p->stream->truncate(n);
  if (n < p->layers.size()) p->layers.resize(n);
}
extern "C" int gkr_proof_stream_to(gkr_proof* p, gkr_felt* out, size_t cap) {
  if (!p || (!out && cap)) return fail(GKR_ERR_INVALID, "null argument");
  p->stream.reset();
  if (!out) return GKR_OK;
  p->stream.reset(new ProofStream(out, cap));
  for (const LayerRec& L : p->layers) p->stream->add(&L);
  return GKR_OK;
}

extern "C" int gkr_proof_serialize(const gkr_proof* p, gkr_felt* out, size_t cap, size_t* n_out) {
  if (!p || !n_out || (!out && cap)) return fail(GKR_ERR_INVALID, "null argument");
  const size_t nl = p->layers.size();
  if (p->stream) {
    ProofStream& st = *p->stream;
    st.sync();  // nothing is appended while serializing: the stream is idle from here on
    if (st.out == out && st.cap == cap && !st.overflow && st.written == nl) {
      Ser tail_count{nullptr};
      serialize_tail(p, tail_count);
      *n_out = st.off[nl] + tail_count.n;
      if (cap < *n_out) return fail(GKR_ERR_BUFFER, "need %zu felts, have %zu", *n_out, cap);
      Ser head{out};
      head.u(nl);
      Ser tail{out};
      tail.n = st.off[nl];
      serialize_tail(p, tail);
      return GKR_OK;
    }
  }
  std::vector<size_t> off(nl + 1);
  off[0] = 1;  // the layer count
  for (size_t l = 0; l < nl; l++) {
    Ser count{nullptr};
    serialize_layer(p->layers[l], count);
    off[l + 1] = off[l] + count.n;
  }
  Ser tail_count{nullptr};
  serialize_tail(p, tail_count);
  *n_out = off[nl] + tail_count.n;
  if (cap < *n_out) return fail(GKR_ERR_BUFFER, "need %zu felts, have %zu", *n_out, cap);
  Ser head{out};
  head.u(nl);
  // layers in contiguous chunks of about equal felt counts, one per thread
  const size_t total = off[nl] - off[0];
  const unsigned hw = std::thread::hardware_concurrency();
  const size_t nt = std::min<size_t>({(size_t)(hw ? hw : 1), (size_t)8, nl ? nl : 1, total / (1u << 16) + 1});
  auto write_range = [&](size_t l0, size_t l1) {
    for (size_t l = l0; l < l1; l++) {
      Ser w{out};
      w.n = off[l];
      serialize_layer(p->layers[l], w);
    }
  };
  if (nt <= 1) {
    write_range(0, nl);
  } else {
    std::vector<std::thread> th;
    size_t l0 = 0;
    for (size_t t = 0; t < nt && l0 < nl; t++) {
      const size_t target = off[0] + total * (t + 1) / nt;
      size_t l1 = l0;
      while (l1 < nl && (off[l1 + 1] <= target || l1 == l0)) l1++;
      if (t + 1 == nt) l1 = nl;
      th.emplace_back(write_range, l0, l1);
      l0 = l1;
    }
    for (auto& x : th) x.join();
  }
  Ser tail{out};
  tail.n = off[nl];
  serialize_tail(p, tail);
  return GKR_OK;
}

