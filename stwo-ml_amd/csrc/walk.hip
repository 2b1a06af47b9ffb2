// The GKR walk: a list of layer steps proved on one channel.
#include "internal.h"
#include "activations.h"
// ------------------------------------------------------------------ GKR walk
extern "C" int gkr_prove_walk(gkr_ctx* c, gkr_channel* ch, const gkr_step* steps, size_t n_steps,
                              const gkr_qm31* init_point, uint32_t n_init, const gkr_qm31* init_value,
                              gkr_proof* proof, gkr_qm31* final_point, uint32_t* n_final, gkr_qm31* final_value) {
  CH_CHECK(ch);
  if (!c || (!steps && n_steps) || !final_point || !n_final || !final_value)
    return fail(GKR_ERR_INVALID, "null argument");
  TraceScope trace;
  std::vector<gkr_qm31> point(init_point ? init_point : nullptr, init_point ? init_point + n_init : nullptr);
  gkr_qm31 value = init_value ? *init_value : G(qm31_zero());
  bool have_claim = init_value != nullptr;
  std::vector<gkr_qm31> rp, npnt(64);
  // A fresh matmul step whose predecessor is a matmul or activation step has
  // its restriction launched ahead, at the predecessor's last launch, waiting
  // on the device for its claim point (prelaunch_matmul): the host then only
  // posts the point.  A LogUp activation step after such a step has its first
  // kernels launched the same way (prelaunch_activation), waiting for its
  // claim point and gamma, beta.  Whatever is left of it on any exit is
  // cancelled.
  struct PreGuard {
    gkr_ctx* c;
    ~PreGuard() { cancel_prelaunch(c); }
  } pre_guard{c};
  auto fused_matmul = [](const gkr_step& s) {
    return s.kind == GKR_STEP_MATMUL && s.claim == GKR_CLAIM_FRESH && s.a && s.b && s.a->cols > 1;
  };
  auto table_log_of = [](const gkr_step& s) {
    return s.table_log_size ? s.table_log_size : act_default_log_size(s.activation_type);
  };
  auto logup_act = [](const gkr_step& s) {
    return s.kind == GKR_STEP_ACTIVATION && s.a && act_valid(s.activation_type) && act_logup_valid(s.activation_type);
  };
  // the kernels launched ahead are the ones step s needs
  auto pre_matches = [&](const gkr_step& s) {
    if (c->pre.act)
      return logup_act(s) && c->pre.a == s.a && c->pre.tag == s.activation_type && c->pre.table_log == table_log_of(s);
    return fused_matmul(s) && c->pre.a == s.a && c->pre.b == s.b;
  };
  if (n_steps > 1) {
    uint8_t* pw;
    TRY(ensureT(c, S_PTWAIT, kPtWaitBytes, &pw));
  }
  for (size_t si = 0; si < n_steps; si++) {
    const gkr_step& st = steps[si];
    if (!st.a) return fail(GKR_ERR_INVALID, "step %zu: null matrix", si);
    if (c->pre.active && !pre_matches(st)) cancel_prelaunch(c);
    auto prove_step = [&]() -> int {
      c->prelaunch = nullptr;
      if (si + 1 < n_steps && (fused_matmul(st) || st.kind == GKR_STEP_ACTIVATION)) {
        const gkr_step& ns = steps[si + 1];
        if (fused_matmul(ns)) {
          const gkr_matrix* na = ns.a;
          const gkr_matrix* nb = ns.b;
          c->prelaunch = [c, na, nb]() -> int {
            bool launched;
            return prelaunch_matmul(c, na, nb, &launched);
          };
        } else if (logup_act(ns)) {
          const gkr_matrix* na = ns.a;
          const uint32_t tag = ns.activation_type, tl = table_log_of(ns);
          c->prelaunch = [c, na, tag, tl]() -> int {
            bool launched;
            return prelaunch_activation(c, na, tag, tl, &launched);
          };
        }
      }
      if (st.kind == GKR_STEP_MATMUL) {
        HostTimer hw(c, K_HOST_WALK_MM);
        if (!st.b) return fail(GKR_ERR_INVALID, "step %zu: null weight matrix", si);
        const uint32_t nv = (uint32_t)(log2_exact(next_pow2(st.a->rows)) + log2_exact(next_pow2(st.b->cols)));
        const int T = log2_exact(next_pow2(st.a->cols));
        // a fresh claim with k > 1: its value comes out of the layer proof's first trip
        const bool fused = st.claim == GKR_CLAIM_FRESH && T > 0;
        if (st.claim == GKR_CLAIM_FRESH) {
          point.resize(nv);
          {
            HostTimer ht(c, K_HOST_DRAW);
            TRY(gkr_channel_draw_qm31s(ch, nv, point.data()));
          }
          if (!fused) {
            TRY(gkr_matmul_output_claim(c, st.a, st.b, point.data(), nv, &value));
            ch->ch.mix_secure_field(Q(value));
          }
        } else if (!have_claim) {
          return fail(GKR_ERR_INVALID, "step %zu: chained claim but no previous claim", si);
        }
        rp.resize(3 * (size_t)(T > 0 ? T : 1));
        gkr_qm31 fa, fb, nval;
        if (fused)
          TRY(walk_matmul_fresh(c, point.data(), (uint32_t)point.size(), &value, st.a, st.b, ch, proof, rp.data(), &fa,
                                &fb, npnt.data(), &nval));
        else
          TRY(gkr_prove_matmul_layer(c, point.data(), (uint32_t)point.size(), &value, st.a, st.b, ch, proof,
                                     rp.data(), &fa, &fb, npnt.data(), &nval));
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
        HostTimer hw(c, K_HOST_WALK_ACT);
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
        std::vector<gkr_qm31> mrp(2 * tl);
        gkr_logup_out out;
        memset(&out, 0, sizeof out);
        out.eq_round_polys = rp.data();
        out.multiplicities = nullptr;  // the proof record holds them
        out.mult_round_polys = mrp.data();
        TRY(prove_activation(c, point.data(), (uint32_t)point.size(), &value, st.a, st.activation_type, tl, ch,
                             proof, &out));
        value = out.input_eval;  // the claim point is unchanged (prover.rs:6581-6584)
      } else if (st.kind == GKR_STEP_LAYERNORM || st.kind == GKR_STEP_RMSNORM) {
        const uint32_t nv = (uint32_t)(log2_exact(next_pow2(st.a->rows)) + log2_exact(next_pow2(st.a->cols)));
        const uint64_t dim = st.dim ? st.dim : st.a->cols;
        std::vector<uint32_t> gamma;
        if (st.kind == GKR_STEP_RMSNORM && st.b) {  // the learned scale, one row
          if (st.b->rows != 1) return fail(GKR_ERR_INVALID, "step %zu: gamma must be a 1 x n matrix", si);
          gamma.resize(st.b->cols);
          TRY(gkr_matrix_download(c, st.b, gamma.data()));
        }
        if (st.claim == GKR_CLAIM_FRESH) {
          point.resize(nv);
          {
            HostTimer ht(c, K_HOST_DRAW);
            TRY(gkr_channel_draw_qm31s(ch, nv, point.data()));
          }
          TRY(gkr_norm_output_claim(c, st.kind, st.a, dim, gamma.data(), gamma.size(), point.data(), nv, &value));
          ch->ch.mix_secure_field(Q(value));
        } else if (!have_claim) {
          return fail(GKR_ERR_INVALID, "step %zu: chained claim but no previous claim", si);
        }
        std::vector<gkr_qm31> p0(4 * nv), lin(4 * nv), lg(4 * nv), mrp(32);
        std::vector<uint32_t> nm(1u << 16), r0(next_pow2(st.a->rows)), r1(next_pow2(st.a->rows));
        gkr_norm_out out;
        memset(&out, 0, sizeof out);
        out.p0_round_polys = p0.data();
        out.lin_round_polys = lin.data();
        out.logup_round_polys = lg.data();
        out.multiplicities = nm.data();
        out.mult_round_polys = mrp.data();
        out.row_stats0 = r0.data();
        out.row_stats1 = r1.data();
        TRY(prove_norm(c, st.kind == GKR_STEP_LAYERNORM, point.data(), (uint32_t)point.size(), &value, st.a, dim,
                       gamma.empty() ? nullptr : gamma.data(), gamma.size(), ch, proof, &out, false));
        value = out.input_eval;  // the claim point is unchanged (prover.rs:8351-8354)
      } else {
        return fail(GKR_ERR_INVALID, "step %zu: unknown kind %u", si, st.kind);
      }
      return GKR_OK;
    };
    // A kernel's bounded wait for the host gives up after about 5.5 s (2^22
    // polls of the mailbox, 1.3 us each on MI355X): a host thread held up that
    // long fails the step with every kernel exited.  The step is then proved
    // again, once, from the channel, claim and proof as they were before it
    // (the transcript is deterministic, so the proof is the same), without the
    // launches made ahead for it.
    const PoseidonChannel ch_before = ch->ch;
    const std::vector<gkr_qm31> point_before = point;
    const gkr_qm31 value_before = value;
    const size_t layers_before = proof ? proof->layers.size() : 0;
    const size_t claims_before = proof ? proof->weight_claims.size() : 0;
    c->wait_expired = false;
    int rc = prove_step();
    if (rc != GKR_OK && c->wait_expired) {
      cancel_prelaunch(c);
      ch->ch = ch_before;
      point = point_before;
      value = value_before;
      if (proof) {
        proof_truncate(proof, layers_before);
        proof->weight_claims.resize(claims_before);
      }
      c->wait_expired = false;
      c->stats[K_WALK_RETRY].launches++;
      rc = prove_step();
    }
    TRY(rc);
    c->prelaunch = nullptr;
    have_claim = true;
    trace_point(ch->ch, "walk.step", (long)si);
  }
  if (point.size() > 64) return fail(GKR_ERR_BUFFER, "final claim has %zu variables", point.size());
  for (size_t l = 0; l < point.size(); l++) final_point[l] = point[l];
  *n_final = (uint32_t)point.size();
  *final_value = value;
  return GKR_OK;
}

