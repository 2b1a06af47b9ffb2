// Poseidon permutation, hash and channel ABI (engine/src/crypto/
// poseidon_channel.rs) and the GKR driver seeding (gkr/prover.rs:1527-1537).
#include "internal.h"
// ------------------------------------------------------------------ error / version

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

// ------------------------------------------------------------------ transcript trace
namespace {
thread_local int tl_trace_depth = 0;
thread_local bool tl_trace_on = false;
thread_local std::string tl_trace_path;  // empty: stderr
std::mutex g_trace_mu;
}  // namespace
gkr::TraceScope::TraceScope() {
  if (tl_trace_depth++ != 0) return;
  const char* p = getenv("GKR_CHANNEL_TRACE");
  tl_trace_on = false;
  tl_trace_path.clear();
  if (p && *p) {
    tl_trace_on = true;
    if (strcmp(p, "-") != 0 && strcmp(p, "stderr") != 0) tl_trace_path = p;
  } else if (getenv("STWO_CHANNEL_TRACE")) {
    tl_trace_on = true;
  }
}
gkr::TraceScope::~TraceScope() { tl_trace_depth--; }
bool gkr::trace_enabled() { return tl_trace_on && tl_trace_depth > 0; }
void gkr::trace_point_impl(const PoseidonChannel& ch, const char* label, long index) {
  const gkr_felt d = felt_to_abi(ch.digest);
  char line[160];
  int n = index >= 0 ? snprintf(line, sizeof line, "%s %ld 0x", label, index) : snprintf(line, sizeof line, "%s 0x", label);
  for (int w = 7; w >= 0; w--) n += snprintf(line + n, sizeof line - n, "%08x", d.w[w]);
  snprintf(line + n, sizeof line - n, " %u\n", ch.n_draws);
  std::lock_guard<std::mutex> lk(g_trace_mu);
  if (tl_trace_path.empty()) {
    fputs(line, stderr);
    return;
  }
  if (FILE* f = fopen(tl_trace_path.c_str(), "a")) {
    fputs(line, f);
    fclose(f);
  }
}

// ------------------------------------------------------------------ channel ABI
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
// ------------------------------------------------------------------ proof-generation policy
extern "C" int gkr_policy_preset(const char* name, gkr_policy* out) {
  if (!name || !out) return fail(GKR_ERR_INVALID, "null argument");
  std::string n(name);
  for (char& ch : n) ch = (char)tolower((unsigned char)ch);
  // field order: norm, logup, segment | rms_sq, piecewise, batch, stark | mode | full, rlc | io, packed, double | chain
  if (n == "strict")  // policy.rs:131-155
    *out = gkr_policy{0, 0, 0, 0, 1, 0, 0, 1, 1, 0, 1, 1, 1, 1};
  else if (n == "standard")  // policy.rs:160-184
    *out = gkr_policy{1, 1, 0, 1, 0, 1, 1, 1, 1, 0, 1, 1, 1, 1};
  else if (n == "relaxed")  // policy.rs:189-203
    *out = gkr_policy{1, 1, 1, 1, 1, 1, 1, 1, 0, 0, 1, 1, 1, 0};
  else
    return fail(GKR_ERR_INVALID, "unknown policy preset '%s'", name);
  return GKR_OK;
}
extern "C" int gkr_policy_commitment(const gkr_policy* p, gkr_felt* out) {
  if (!p || !out) return fail(GKR_ERR_INVALID, "null argument");
  const uint8_t v[14] = {p->allow_missing_norm_proof, p->allow_logup_activation, p->allow_missing_segment_binding,
                         p->skip_rms_sq_proof,        p->piecewise_activation,   p->skip_batch_tokens,
                         p->skip_unified_stark,       p->weight_binding_mode,    p->aggregated_full_binding,
                         p->aggregated_rlc_only,      p->io_packing,             p->packed_proof,
                         p->double_packed_proof,      p->validate_decode_chain};
  felt in[15];
  in[0] = felt_from_u64(0x504F4C01ull);  // "POL" + version 1 (policy.rs:28)
  for (int i = 0; i < 14; i++) {
    if (v[i] > (i == 7 ? 3 : 1)) return fail(GKR_ERR_INVALID, "policy field %d out of range (%u)", i, v[i]);
    in[1 + i] = felt_from_u64(v[i]);
  }
  *out = felt_to_abi(poseidon_hash_many(in, 15));
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

