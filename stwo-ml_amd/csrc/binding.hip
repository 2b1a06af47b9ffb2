// Aggregated weight binding: prove_aggregated_binding_streaming
// (engine/src/crypto/aggregated_opening.rs:1647-1720) over resident weights,
// its verifier replay (verify_aggregated_binding, :1774-1905) and
// serialize_aggregated_binding_proof (engine/src/cairo_serde.rs:3885-3920).
//
// The unified oracle W(s, x) = sum_k sel_k(s) W_k(x[n_max - n_k ..]) over
// selector bits s and n_max local variables; the mismatch sumcheck's round
// polynomial at round j is
//   S_j(X) = sum_i beta_i eqp_i eq(g_i[j], X) (W(r_<j, X, g_i[>j]) - v_i)
// (the identity sum_x eq(a, x) f(x) = f(a) for multilinear f, :412-620).  In
// a selector round every W_k is evaluated at claim i's own local point:
// E[k][i], computed once.  In local round j' matrix k (offset
// off_k = n_max - n_k) contributes E[k][i] while j' < off_k, then
//   D_{k,i}(X) = sum_x F_k[X, x] eq(x, g_i_loc[j' + 1 ..])
// with F_k its column-major MLE folded by the local challenges so far: the
// device keeps F_k resident, folds it by the previous challenge on the fly
// and forms all claims' two half sums in one pass (eq weights factored into
// per-claim hi and lo tables).  The host combines the sums into the degree-2
// round polynomial, runs the transcript, and at the end opens the virtual
// MLE (m_padded slots of 2^n_max entries) with the resident opening code.
#include "internal.h"

#include <array>

namespace {

constexpr int kBindMaxClaims = 8;
constexpr int kBindIter = 4;  // entries per thread and workgroup pass

struct BindDesc {
  const qm31* src;  // F (2^m entries), or with a pending fold the previous table (2^(m+1))
  qm31* dst;        // the folded table (pending fold)
  qm31 x;           // the pending fold's challenge
  uint32_t pend, m, wg0, slot;
};

static __global__ void k_bind_colmajor(const uint32_t* __restrict__ B, uint64_t rows, uint64_t cols, int log_pk,
                                       uint64_t n, qm31* __restrict__ F) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const uint64_t c = idx >> log_pk, r = idx & ((1ull << log_pk) - 1);
  st_q(F, idx, qm31_from_m31((r < rows && c < cols) ? m31_from_u32(B[r * cols + c]) : 0u));
}

// hi_i[u] = eq(bits(u), coords_i[0 .. L - h)), lo_i[v] = eq(bits(v), coords_i[L - h .. L)),
// first coordinate on the most significant bit; hi_i at hi + i 2^(L-h), lo_i at lo + i 2^h.
static __global__ void k_bind_eq(const qm31* __restrict__ coords, int P, int L, int h, qm31* __restrict__ hi,
                                 qm31* __restrict__ lo) {
  const uint64_t nhi = 1ull << (L - h), nlo = 1ull << h, per = nhi + nlo;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= per * (uint64_t)P) return;
  const int i = (int)(t / per);
  const uint64_t e = t - (uint64_t)i * per;
  const qm31* cd = coords + (uint64_t)i * L;
  qm31 acc = qm31_one();
  if (e < nhi) {
    const int nb = L - h;
    for (int c = 0; c < nb; c++)
      acc = qm31_mul(acc, ((e >> (nb - 1 - c)) & 1ull) ? cd[c] : qm31_sub(qm31_one(), cd[c]));
    st_q(hi, (uint64_t)i * nhi + e, acc);
  } else {
    const uint64_t v = e - nhi;
    for (int c = 0; c < h; c++)
      acc = qm31_mul(acc, ((v >> (h - 1 - c)) & 1ull) ? cd[L - h + c] : qm31_sub(qm31_one(), cd[L - h + c]));
    st_q(lo, (uint64_t)i * nlo + v, acc);
  }
}

template <typename T>
__device__ __forceinline__ uint32_t bind_find(const T* d, uint32_t n) {
  __shared__ uint32_t s_idx;
  if (threadIdx.x == 0) {
    uint32_t a = 0, b = n - 1;
    while (a < b) {
      const uint32_t mid = (a + b + 1) >> 1;
      if (d[mid].wg0 <= blockIdx.x)
        a = mid;
      else
        b = mid - 1;
    }
    s_idx = a;
  }
  __syncthreads();
  return s_idx;
}

// Per table: the pending fold (written to dst) and, for every claim i < P,
// sum_x F[X 2^(m-1) + x] hi_i[x >> h] lo_i[x & (2^h - 1)] for X = 0, 1.
template <int NP>
static __global__ void __launch_bounds__(kBlock) k_bind_dots(const BindDesc* __restrict__ desc, uint32_t n_desc, int P,
                                                              int h, const qm31* __restrict__ hi, uint64_t nhi,
                                                              const qm31* __restrict__ lo,
                                                              qm31* __restrict__ partials) {
  const BindDesc D = desc[bind_find(desc, n_desc)];
  const uint64_t half = 1ull << (D.m - 1), full = 1ull << D.m;
  const uint64_t base = (uint64_t)(blockIdx.x - D.wg0) * kBlock * kBindIter;
  const uint64_t nlo = 1ull << h;
  qm31 v[2 * NP];
#pragma unroll
  for (int q = 0; q < 2 * NP; q++) v[q] = qm31_zero();
  for (int it = 0; it < kBindIter; it++) {
    const uint64_t x = base + (uint64_t)it * kBlock + threadIdx.x;
    if (x >= half) break;
    qm31 f0, f1;
    if (D.pend) {
      f0 = qm31_fold(ld_q(D.src, x), ld_q(D.src, x + full), D.x);
      f1 = qm31_fold(ld_q(D.src, x + half), ld_q(D.src, x + half + full), D.x);
      st_q(D.dst, x, f0);
      st_q(D.dst, x + half, f1);
    } else {
      f0 = ld_q(D.src, x);
      f1 = ld_q(D.src, x + half);
    }
#pragma unroll
    for (int i = 0; i < NP; i++) {
      if (i >= P) break;
      const qm31 w = qm31_mul(ld_q(hi, (uint64_t)i * nhi + (x >> h)), ld_q(lo, (uint64_t)i * nlo + (x & (nlo - 1))));
      v[2 * i] = qm31_add(v[2 * i], qm31_mul(f0, w));
      v[2 * i + 1] = qm31_add(v[2 * i + 1], qm31_mul(f1, w));
    }
  }
  block_sum_store<2 * NP>(v, partials + (uint64_t)(2 * NP) * blockIdx.x);
}

template <int NP>
static __global__ void __launch_bounds__(kBlock) k_bind_finish(const BindDesc* __restrict__ desc,
                                                                const qm31* __restrict__ partials,
                                                                qm31* __restrict__ res) {
  const BindDesc D = desc[blockIdx.x];
  const uint64_t half = 1ull << (D.m - 1);
  const uint32_t nwg = (uint32_t)((half + (uint64_t)kBlock * kBindIter - 1) / ((uint64_t)kBlock * kBindIter));
  qacc acc[2 * NP];
#pragma unroll
  for (int q = 0; q < 2 * NP; q++) acc[q].zero();
  for (uint32_t b = threadIdx.x; b < nwg; b += blockDim.x)
#pragma unroll
    for (int q = 0; q < 2 * NP; q++) acc[q].add(ld_q(partials, (uint64_t)(2 * NP) * (D.wg0 + b) + q));
  qm31 tot[2 * NP];
#pragma unroll
  for (int q = 0; q < 2 * NP; q++) tot[q] = acc[q].reduce();
  block_sum_store<2 * NP>(tot, res + (uint64_t)(2 * NP) * D.slot);
}

struct VirtualSlots {
  const qm31* f[kBindMaxClaims];
  uint64_t len[kBindMaxClaims];
};
// The virtual MLE: slot k of 2^n_max entries holds F_k (2^n_k entries) then zeros.
static __global__ void k_bind_virtual(VirtualSlots vs, int n_claims, int n_max, uint64_t total,
                                      qm31* __restrict__ V) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint64_t slot = idx >> n_max, local = idx & ((1ull << n_max) - 1);
  qm31 v = qm31_zero();
  if (slot < (uint64_t)n_claims && local < vs.len[slot]) v = ld_q(vs.f[slot], local);
  st_q(V, idx, v);
}

// ------------------------------------------------------------------ host side
qm31 eq1(const qm31& a, const qm31& b) {
  return qm31_add(qm31_mul(a, b), qm31_mul(qm31_sub(qm31_one(), a), qm31_sub(qm31_one(), b)));
}

struct Cfg {
  int sel = 0, n_max = 0, m_padded = 1, n_global = 0, n_claims = 0;
};
Cfg bind_config(const std::vector<int>& nvars) {
  Cfg c;
  c.n_claims = (int)nvars.size();
  for (int n : nvars) c.n_max = std::max(c.n_max, n);
  while (c.m_padded < c.n_claims) c.m_padded *= 2;
  while ((1 << c.sel) < c.m_padded) c.sel++;
  c.n_global = c.sel + c.n_max;
  return c;
}

felt zero_leaf() { return felt_to_mont(felt_raw(0, 1ull << 60, 0, 0)); }  // securefield_to_felt(0) = 2^124

// build_super_root (aggregated_opening.rs:181-227); felts in Montgomery form.
void super_root(const Cfg& cfg, const std::vector<int>& nvars, const std::vector<felt>& commit, felt* root,
                std::vector<felt>* subs) {
  std::vector<felt> zeros(cfg.n_max + 1);
  zeros[0] = zero_leaf();
  for (int k = 1; k <= cfg.n_max; k++) zeros[k] = poseidon_hash(zeros[k - 1], zeros[k - 1]);
  subs->clear();
  for (size_t i = 0; i < nvars.size(); i++) {
    felt r = commit[i];
    for (int k = 0; k < cfg.n_max - nvars[i]; k++) r = poseidon_hash(r, zeros[nvars[i] + k]);
    subs->push_back(r);
  }
  while ((int)subs->size() < cfg.m_padded) subs->push_back(zeros[cfg.n_max]);
  std::vector<felt> cur(*subs);
  while (cur.size() > 1) {
    std::vector<felt> nx(cur.size() / 2);
    for (size_t i = 0; i < nx.size(); i++) nx[i] = poseidon_hash(cur[2 * i], cur[2 * i + 1]);
    cur.swap(nx);
  }
  *root = cur[0];
}

// global_point (aggregated_opening.rs:328-356): selector bits of the claim's
// slot (most significant first), zeros for a smaller matrix, its point.
std::vector<qm31> global_point(const Cfg& cfg, int index, int nv, const qm31* point) {
  std::vector<qm31> g;
  for (int b = cfg.sel - 1; b >= 0; b--) g.push_back(qm31_from_m31((index >> b) & 1));
  for (int k = 0; k < cfg.n_max - nv; k++) g.push_back(qm31_zero());
  for (int k = 0; k < nv; k++) g.push_back(point[k]);
  return g;
}

qm31 selector_weight(int k, const qm31* sel, int nb) {  // compute_selector_weight (:289-309)
  qm31 w = qm31_one();
  for (int j = 0; j < nb; j++) w = qm31_mul(w, eq1(sel[j], qm31_from_m31((k >> (nb - 1 - j)) & 1)));
  return w;
}

// serialized felts of the proof (serialize_aggregated_binding_proof) given the opening's length
size_t bind_felts(const Cfg& cfg, size_t opening) { return 5 + 1 + 12 * (size_t)cfg.n_global + 4 + 1 + 1 + cfg.m_padded + opening; }
size_t opening_felts(uint32_t nv) {  // MleOpeningProof: roots, queries, final value
  if (nv == 0) return 1 + 1 + 4;
  const uint64_t half = 1ull << (nv - 1);
  const size_t nq = (size_t)std::min<uint64_t>(10, half);
  size_t per = 2;
  for (uint32_t t = 0; t < nv; t++) per += 8 + 2 + 2 * (size_t)(nv - t);
  return 1 + (nv - 1) + 1 + nq * per + 4;
}

struct BindClaim {
  const gkr_matrix* b;
  int nv, log_pk;
  std::vector<qm31> point;
  qm31 value;
  felt commitment;  // Montgomery
};

int bind_prepare(const gkr_binding_claim* claims, size_t n, gkr_ctx* c, std::vector<BindClaim>* out) {
  if (!claims || n == 0) return fail(GKR_ERR_INVALID, "aggregated binding: no claims");
  if (n > (size_t)kBindMaxClaims)
    return fail(GKR_ERR_INVALID, "aggregated binding: %zu claims (at most %d per proof; the walk uses groups of 4)", n,
                kBindMaxClaims);
  for (size_t i = 0; i < n; i++) {
    const gkr_binding_claim& x = claims[i];
    if (!x.weight || !x.weight->dev || (c && x.weight->ctx != c)) return fail(GKR_ERR_INVALID, "claim %zu: no weight", i);
    BindClaim b;
    b.b = x.weight;
    b.log_pk = log2_exact(next_pow2(x.weight->rows));
    b.nv = b.log_pk + log2_exact(next_pow2(x.weight->cols));
    if ((int)x.n_point != b.nv) return fail(GKR_ERR_INVALID, "claim %zu: point of %u vars, weight MLE of %d", i, x.n_point, b.nv);
    if (!x.eval_point && x.n_point) return fail(GKR_ERR_INVALID, "claim %zu: null point", i);
    for (uint32_t k = 0; k < x.n_point; k++) {
      if (!canonical_q(x.eval_point[k])) return fail(GKR_ERR_INVALID, "claim %zu: point not canonical", i);
      b.point.push_back(Q(x.eval_point[k]));
    }
    if (!canonical_q(x.expected_value) || !felt_abi_canonical(x.commitment))
      return fail(GKR_ERR_INVALID, "claim %zu: value or commitment not canonical", i);
    b.value = Q(x.expected_value);
    b.commitment = felt_to_mont(felt_canon_from_words(x.commitment.w));
    out->push_back(std::move(b));
  }
  return GKR_OK;
}

}  // namespace

extern "C" int gkr_prove_aggregated_binding(gkr_ctx* c, gkr_channel* ch, const gkr_binding_claim* claims,
                                            size_t n_claims, gkr_felt* out, size_t cap, size_t* n_felts) {
  if (!c || !n_felts || (!out && cap)) return fail(GKR_ERR_INVALID, "null argument");
  CH_CHECK(ch);
  std::vector<BindClaim> B;
  TRY(bind_prepare(claims, n_claims, c, &B));
  std::vector<int> nvars;
  for (const auto& b : B) nvars.push_back(b.nv);
  const Cfg cfg = bind_config(nvars);
  const size_t need = bind_felts(cfg, opening_felts((uint32_t)cfg.n_global));
  *n_felts = need;
  if (cap < need) return fail(GKR_ERR_BUFFER, "need %zu felts, have %zu", need, cap);
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  PoseidonChannel& C = ch->ch;
  const int P = (int)B.size();
  // 1. super root, 2. beta weights
  std::vector<felt> commits, subs;
  for (const auto& b : B) commits.push_back(b.commitment);
  felt root;
  super_root(cfg, nvars, commits, &root, &subs);
  C.mix_felt(root);
  const qm31 rho = C.draw_qm31();
  std::vector<qm31> beta(P);
  beta[0] = qm31_one();
  for (int i = 1; i < P; i++) beta[i] = qm31_mul(beta[i - 1], rho);
  std::vector<std::vector<qm31>> g(P);
  for (int i = 0; i < P; i++) g[i] = global_point(cfg, i, B[i].nv, B[i].point.data());

  // resident column-major MLEs and their fold buffers
  std::vector<qm31*> F0(P), fb[2];
  fb[0].resize(P);
  fb[1].resize(P);
  size_t arena = 0;
  for (const auto& b : B) arena += 2 * (1ull << b.nv) + 2;
  qm31* a;
  TRY(ensureT(c, S_BIND, arena, &a));
  for (int k = 0; k < P; k++) {
    const uint64_t len = 1ull << B[k].nv;
    F0[k] = a;
    a += len;
    fb[0][k] = a;
    a += len / 2 + 1;
    fb[1][k] = a;
    a += len / 2 + 1;
    GKR_LAUNCH(c, k_bind_colmajor, dim3(grid_for(len)), dim3(kBlock), 0, B[k].b->dev, B[k].b->rows,
                       B[k].b->cols, B[k].log_pk, len, F0[k]);
    TRY(check_launch(c));
  }
  int NP = 1;
  while (NP < P) NP *= 2;
  const int local0 = cfg.sel;  // first local round
  const int nloc = cfg.n_max;

  // One device pass: for each listed matrix, the half sums of all claims
  // against the suffix g_i_loc[jl + 1 ..] (L = n_max - jl - 1 coordinates),
  // folding by `x` first when pend is set.  res[k][i] = (D(0), D(1)).
  std::vector<std::array<qm31, 2 * kBindMaxClaims>> dres(P);
  auto run_dots = [&](int jl, const std::vector<int>& ks, const std::vector<const qm31*>& src,
                      const std::vector<qm31*>& dst, const std::vector<int>& m, bool pend, const qm31& x) -> int {
    const int L = nloc - jl - 1;
    const int h = L / 2;
    std::vector<qm31> coords((size_t)P * std::max(L, 1));
    for (int i = 0; i < P; i++)
      for (int t = 0; t < L; t++) coords[(size_t)i * L + t] = g[i][local0 + jl + 1 + t];
    const uint64_t nhi = 1ull << (L - h), nlo = 1ull << h;
    qm31 *dco, *dhi, *dlo, *part, *res;
    TRY(ensureT(c, S_BINDEQ, coords.size() + (size_t)P * (nhi + nlo), &dco));
    dhi = dco + coords.size();
    dlo = dhi + (size_t)P * nhi;
    HIP_TRY(hipMemcpyAsync(dco, coords.data(), coords.size() * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
    GKR_LAUNCH(c, k_bind_eq, dim3(grid_for((uint64_t)P * (nhi + nlo))), dim3(kBlock), 0, dco, P, L, h,
                       dhi, dlo);
    TRY(check_launch(c));
    std::vector<BindDesc> d;
    uint32_t wg = 0;
    for (size_t q = 0; q < ks.size(); q++) {
      BindDesc e;
      memset(&e, 0, sizeof e);
      e.src = src[q];
      e.dst = dst[q];
      e.x = x;
      e.pend = pend ? 1u : 0u;
      e.m = (uint32_t)m[q];
      e.wg0 = wg;
      e.slot = (uint32_t)q;
      const uint64_t half = 1ull << (m[q] - 1);
      wg += (uint32_t)((half + (uint64_t)kBlock * kBindIter - 1) / ((uint64_t)kBlock * kBindIter));
      d.push_back(e);
    }
    void* dv;
    TRY(ensure(c, S_BINDDESC, d.size() * sizeof(BindDesc), &dv));
    TRY(ensureT(c, S_BINDPART, (size_t)2 * NP * wg, &part));
    TRY(ensureT(c, S_BINDRES, (size_t)2 * NP * d.size(), &res));
    HIP_TRY(hipMemcpyAsync(dv, d.data(), d.size() * sizeof(BindDesc), hipMemcpyHostToDevice, c->stream));
    const BindDesc* dd = static_cast<const BindDesc*>(dv);
    switch (NP) {
      case 1:
        GKR_LAUNCH(c, k_bind_dots<1>, dim3(wg), dim3(kBlock), 0, dd, (uint32_t)d.size(), P, h, dhi, nhi, dlo, part);
        GKR_LAUNCH(c, k_bind_finish<1>, dim3((unsigned)d.size()), dim3(kBlock), 0, dd, part, res);
        break;
      case 2:
        GKR_LAUNCH(c, k_bind_dots<2>, dim3(wg), dim3(kBlock), 0, dd, (uint32_t)d.size(), P, h, dhi, nhi, dlo, part);
        GKR_LAUNCH(c, k_bind_finish<2>, dim3((unsigned)d.size()), dim3(kBlock), 0, dd, part, res);
        break;
      case 4:
        GKR_LAUNCH(c, k_bind_dots<4>, dim3(wg), dim3(kBlock), 0, dd, (uint32_t)d.size(), P, h, dhi, nhi, dlo, part);
        GKR_LAUNCH(c, k_bind_finish<4>, dim3((unsigned)d.size()), dim3(kBlock), 0, dd, part, res);
        break;
      default:
        GKR_LAUNCH(c, k_bind_dots<8>, dim3(wg), dim3(kBlock), 0, dd, (uint32_t)d.size(), P, h, dhi, nhi, dlo, part);
        GKR_LAUNCH(c, k_bind_finish<8>, dim3((unsigned)d.size()), dim3(kBlock), 0, dd, part, res);
        break;
    }
    TRY(check_launch(c));
    std::vector<qm31> hres((size_t)2 * NP * d.size());
    HIP_TRY(hipMemcpyAsync(hres.data(), res, hres.size() * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
    TRY(sync(c));
    for (size_t q = 0; q < ks.size(); q++)
      for (int i = 0; i < 2 * P; i++) dres[ks[q]][i] = hres[(size_t)2 * NP * q + i];
    return GKR_OK;
  };

  // E[k][i] = W_k(g_i_loc[off_k ..]) from the first pass of each matrix (its
  // local round off_k, no fold yet); those sums also serve that round
  std::vector<std::vector<qm31>> E(P, std::vector<qm31>(P));
  std::vector<std::array<qm31, 2 * kBindMaxClaims>> d0(P);
  std::vector<qm31> single(P, qm31_zero());  // a 1 x 1 weight (no variables): its value
  for (int k = 0; k < P; k++)
    if (B[k].nv == 0) {
      uint32_t v;
      HIP_TRY(hipMemcpy(&v, B[k].b->dev, 4, hipMemcpyDeviceToHost));
      single[k] = qm31_from_m31(m31_from_u32(v));
      for (int i = 0; i < P; i++) E[k][i] = single[k];
    }
  for (int off = 0; off < nloc; off++) {
    std::vector<int> ks, m;
    std::vector<const qm31*> src;
    std::vector<qm31*> dst;
    for (int k = 0; k < P; k++)
      if (B[k].nv > 0 && nloc - B[k].nv == off) {
        ks.push_back(k);
        src.push_back(F0[k]);
        dst.push_back(nullptr);
        m.push_back(B[k].nv);
      }
    if (ks.empty()) continue;
    TRY(run_dots(off, ks, src, dst, m, false, qm31_zero()));
    for (int k : ks) {
      d0[k] = dres[k];
      for (int i = 0; i < P; i++) E[k][i] = qm31_fold(dres[k][2 * i], dres[k][2 * i + 1], g[i][local0 + off]);
    }
  }

  // the mismatch sumcheck (aggregated_opening.rs:412-515)
  std::vector<qm31> eqp(P, qm31_one()), chal;
  std::vector<qm31> polys;
  const qm31 inv2 = qm31_from_m31(1u << 30), two = qm31_from_m31(2);
  std::vector<qm31> sigma(P);
  for (int j = 0; j < cfg.n_global; j++) {
    qm31 S[3] = {qm31_zero(), qm31_zero(), qm31_zero()};
    const qm31 xs[3] = {qm31_zero(), qm31_one(), two};
    if (j < cfg.sel) {
      for (int i = 0; i < P; i++)
        for (int xi = 0; xi < 3; xi++) {
          std::vector<qm31> sel(chal);
          sel.push_back(xs[xi]);
          for (int l = j + 1; l < cfg.sel; l++) sel.push_back(g[i][l]);
          qm31 w = qm31_zero();
          for (int k = 0; k < P; k++) w = qm31_add(w, qm31_mul(selector_weight(k, sel.data(), cfg.sel), E[k][i]));
          const qm31 t = qm31_mul(qm31_mul(beta[i], eqp[i]), qm31_mul(eq1(g[i][j], xs[xi]), qm31_sub(w, B[i].value)));
          S[xi] = qm31_add(S[xi], t);
        }
    } else {
      const int jl = j - cfg.sel;
      if (jl == 0)
        for (int k = 0; k < P; k++) sigma[k] = selector_weight(k, chal.data(), cfg.sel);
      // device sums for the matrices past their first local round
      std::vector<int> ks, m;
      std::vector<const qm31*> src;
      std::vector<qm31*> dst;
      for (int k = 0; k < P; k++) {
        const int off = nloc - B[k].nv;
        if (B[k].nv == 0 || jl <= off) continue;
        const int p = jl - off;  // folds so far after this round's pending one
        ks.push_back(k);
        src.push_back(p == 1 ? F0[k] : fb[p & 1][k]);
        dst.push_back(fb[(p - 1) & 1][k]);
        m.push_back(B[k].nv - p);
      }
      if (!ks.empty()) TRY(run_dots(jl, ks, src, dst, m, true, chal.back()));
      for (int k = 0; k < P; k++)
        if (B[k].nv > 0 && jl == nloc - B[k].nv) dres[k] = d0[k];
      for (int i = 0; i < P; i++) {
        qm31 w[3] = {qm31_zero(), qm31_zero(), qm31_zero()};
        for (int k = 0; k < P; k++) {
          qm31 v0, v1;
          if (B[k].nv == 0 || jl < nloc - B[k].nv) {
            v0 = v1 = E[k][i];
          } else {
            v0 = dres[k][2 * i];
            v1 = dres[k][2 * i + 1];
          }
          const qm31 v2 = qm31_sub(qm31_add(v1, v1), v0);
          w[0] = qm31_add(w[0], qm31_mul(sigma[k], v0));
          w[1] = qm31_add(w[1], qm31_mul(sigma[k], v1));
          w[2] = qm31_add(w[2], qm31_mul(sigma[k], v2));
        }
        for (int xi = 0; xi < 3; xi++) {
          const qm31 t = qm31_mul(qm31_mul(beta[i], eqp[i]), qm31_mul(eq1(g[i][j], xs[xi]), qm31_sub(w[xi], B[i].value)));
          S[xi] = qm31_add(S[xi], t);
        }
      }
    }
    const qm31 c0 = S[0];
    const qm31 c2 = qm31_mul(qm31_add(qm31_sub(S[0], qm31_add(S[1], S[1])), S[2]), inv2);
    const qm31 c1 = qm31_sub(qm31_sub(S[1], S[0]), c2);
    qm31 r;
    {
      HostTimer ht(c, K_HOST_FS);
      C.mix_poly_coeffs(c0, c1, c2);
      r = C.draw_qm31();
    }
    polys.insert(polys.end(), {c0, c1, c2});
    chal.push_back(r);
    for (int i = 0; i < P; i++) eqp[i] = qm31_mul(eqp[i], eq1(r, g[i][j]));
  }
  // oracle value at the challenge point: the last round's two values per matrix, folded
  if (cfg.sel > 0 && cfg.n_max == 0)
    for (int k = 0; k < P; k++) sigma[k] = selector_weight(k, chal.data(), cfg.sel);
  if (cfg.sel == 0)
    for (int k = 0; k < P; k++) sigma[k] = qm31_one();
  qm31 oracle_eval = qm31_zero();
  for (int k = 0; k < P; k++) {
    const qm31 wk = B[k].nv == 0 ? single[k] : qm31_fold(dres[k][0], dres[k][1], chal.back());
    oracle_eval = qm31_add(oracle_eval, qm31_mul(sigma[k], wk));
  }
  C.mix_felts(&oracle_eval, 1);
  // the virtual MLE and its opening at the challenge point
  const uint64_t vtotal = (uint64_t)cfg.m_padded << cfg.n_max;
  qm31* V;
  TRY(ensureT(c, S_BINDVIRT, vtotal, &V));
  VirtualSlots vs;
  memset(&vs, 0, sizeof vs);
  for (int k = 0; k < P; k++) {
    vs.f[k] = F0[k];
    vs.len[k] = 1ull << B[k].nv;
  }
  GKR_LAUNCH(c, k_bind_virtual, dim3(grid_for(vtotal)), dim3(kBlock), 0, vs, P, cfg.n_max, vtotal, V);
  TRY(check_launch(c));
  std::vector<gkr_qm31> pt(chal.size());
  for (size_t k = 0; k < chal.size(); k++) pt[k] = G(chal[k]);
  felt cm;
  std::vector<felt> rec;
  TRY(mle_opening(c, OpenSrc{nullptr, V, vtotal}, pt.data(), (uint32_t)pt.size(), nullptr, C, &cm, rec, false));
  // serialize_aggregated_binding_proof (cairo_serde.rs:3885-3920)
  size_t n = 0;
  auto fu = [&](uint64_t v) {
    gkr_felt& f = out[n++];
    f.w[0] = (uint32_t)v;
    f.w[1] = (uint32_t)(v >> 32);
    for (int k = 2; k < 8; k++) f.w[k] = 0;
  };
  auto fq = [&](const qm31& q) { fu(q.a); fu(q.b); fu(q.c); fu(q.d); };
  auto ff = [&](const felt& canon) { felt_canon_to_words(canon, out[n++].w); };
  fu(cfg.sel);
  fu(cfg.n_max);
  fu(cfg.m_padded);
  fu(cfg.n_global);
  fu(cfg.n_claims);
  fu(cfg.n_global);
  for (const qm31& q : polys) fq(q);
  fq(oracle_eval);
  ff(felt_from_mont(root));
  fu(subs.size());
  for (const felt& s : subs) ff(felt_from_mont(s));
  if (n + rec.size() != need) return fail(GKR_ERR_INVALID, "aggregated binding: proof of %zu felts, expected %zu", n + rec.size(), need);
  for (const felt& f : rec) ff(f);
  return GKR_OK;
}
