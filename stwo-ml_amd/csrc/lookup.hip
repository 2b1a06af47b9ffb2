// STWO's LogUp-GKR and grand-product batch prover: prove_batch
// (stwo-gpu/crates/stwo/src/prover/lookups/gkr_prover.rs:396-500) over device
// columns, the verifier replay partially_verify_batch (gkr_verifier.rs:17-157)
// and serialize_stwo_gkr_batch_proof (engine/src/cairo_serde.rs:3330-3420).
//
// Device:
//  - k_lk_tree builds the circuit of every instance, nine levels per launch
//    (a workgroup reduces 512 entries of a level to one entry eight levels up
//    through LDS, writing each level on the way): pairs (2i, 2i + 1) combine
//    as fractions (LogUp) or products (grand product);
//  - k_lk_round runs one sumcheck round for every instance that takes part in
//    it: it folds the previous challenge into the vectors on the fly (writing
//    the folded vectors) and sums, for t = 0 and t = 2, the weighted fraction
//    sums of the pairs with eq weights over the suffix of the layer point;
//    k_lk_finish adds the workgroup rows per instance.
// Host: the transcript, the round polynomials from the sums (r(0), r(2) from
// the device, r(1) = claim - r(0), r(b) = 0 at the root of the eq factor:
// the unique cubic through them, gkr_prover.rs:518-566), the instance
// combination, the masks and the layer points.
#include "internal.h"

namespace {

constexpr int kLkLevels = 9;   // circuit levels per tree launch
constexpr int kLkTab = 10;     // suffix eq tables up to 2^10 entries come from the host
constexpr int kLkMaxVars = 28;
constexpr int kLkRes = 12;     // result QM31 per instance and round: 4 sums, then 4 num + 4 den values

enum : uint32_t { NF_NONE = 0, NF_Q = 1, NF_M31 = 2, NF_ONE = 3 };  // numerator formats

struct LkTree {
  const void* num;
  const qm31* den;
  qm31* out_num;  // level k at offset 2^k - 1
  qm31* out_den;
  uint32_t fmt, gp, src_log, levels, wg0, pad;
};

struct LkRound {
  const void* src_num;
  const qm31* src_den;
  qm31* dst_num;
  qm31* dst_den;
  qm31 x;         // pending fold challenge
  uint32_t fmt;   // numerator format of the source
  uint32_t gp;    // grand product: den holds the column
  uint32_t pend;  // fold the source (2^(m+1) entries) with x first
  uint32_t m;     // variables of the vector summed
  uint32_t wg0;   // first workgroup
  uint32_t slot;  // result slot
};

struct LkTop {
  const void* num1;  // level 1 (2 entries): the input when it has one variable
  const qm31* den1;
  const qm31* num0;  // level 0 (1 entry)
  const qm31* den0;
  uint32_t fmt1, gp, pad[2];
};

__device__ __forceinline__ qm31 lk_num(const void* p, uint32_t fmt, uint64_t i) {
  if (fmt == NF_Q) return ld_q(reinterpret_cast<const qm31*>(p), i);
  if (fmt == NF_M31) return qm31_from_m31(reinterpret_cast<const uint32_t*>(p)[i]);
  return qm31_one();
}

template <typename T>
__device__ __forceinline__ uint32_t find_desc(const T* d, uint32_t n) {
  __shared__ uint32_t s_idx;
  if (threadIdx.x == 0) {
    uint32_t lo = 0, hi = n - 1;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (d[mid].wg0 <= blockIdx.x)
        lo = mid;
      else
        hi = mid - 1;
    }
    s_idx = lo;
  }
  __syncthreads();
  return s_idx;
}

// One launch: per instance, `levels` circuit levels below level src_log.
// Workgroup w of an instance covers entries [512 w, 512 w + 512) of the
// source level (all of it when smaller).
static __global__ void __launch_bounds__(kBlock) k_lk_tree(const LkTree* __restrict__ desc, uint32_t n_desc) {
  const LkTree D = desc[find_desc(desc, n_desc)];
  const uint32_t wl = blockIdx.x - D.wg0;
  const uint64_t half = 1ull << (D.src_log - 1);
  const uint32_t per = half < (uint64_t)kBlock ? (uint32_t)half : (uint32_t)kBlock;
  __shared__ qm31 sn[kBlock], sd[kBlock];
  const uint32_t t = threadIdx.x;
  if (t < per) {
    const uint64_t i = (uint64_t)wl * kBlock + t;
    const qm31 d0 = ld_q(D.den, 2 * i), d1 = ld_q(D.den, 2 * i + 1);
    qm31 n = qm31_zero(), d;
    if (D.gp) {
      d = qm31_mul(d0, d1);
    } else {
      const qm31 n0 = lk_num(D.num, D.fmt, 2 * i), n1 = lk_num(D.num, D.fmt, 2 * i + 1);
      n = qm31_add(qm31_mul(n0, d1), qm31_mul(n1, d0));
      d = qm31_mul(d0, d1);
    }
    const uint64_t off = half - 1;
    st_q(D.out_den, off + i, d);
    if (!D.gp) st_q(D.out_num, off + i, n);
    sn[t] = n;
    sd[t] = d;
  }
  for (uint32_t e = 1; e < D.levels; e++) {
    const uint32_t cnt = per >> e;
    __syncthreads();
    qm31 n = qm31_zero(), d = qm31_zero();
    if (t < cnt) {
      const qm31 d0 = sd[2 * t], d1 = sd[2 * t + 1];
      d = qm31_mul(d0, d1);
      if (!D.gp) n = qm31_add(qm31_mul(sn[2 * t], d1), qm31_mul(sn[2 * t + 1], d0));
      const uint64_t lvl_n = half >> e;  // entries of this level
      const uint64_t i = (uint64_t)wl * cnt + t;
      st_q(D.out_den, lvl_n - 1 + i, d);
      if (!D.gp) st_q(D.out_num, lvl_n - 1 + i, n);
    }
    __syncthreads();
    if (t < cnt) {
      sn[t] = n;
      sd[t] = d;
    }
  }
}

// The two top levels of every instance: out[6 i ..] = num0, den0, num1[0],
// num1[1], den1[0], den1[1] (grand product: the column in den).
static __global__ void k_lk_top(const LkTop* __restrict__ desc, uint32_t n, qm31* __restrict__ out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const LkTop D = desc[i];
  qm31* o = out + 6ull * i;
  o[0] = D.gp ? qm31_zero() : ld_q(D.num0, 0);
  o[1] = ld_q(D.den0, 0);
  o[2] = D.gp ? qm31_zero() : lk_num(D.num1, D.fmt1, 0);
  o[3] = D.gp ? qm31_zero() : lk_num(D.num1, D.fmt1, 1);
  o[4] = ld_q(D.den1, 0);
  o[5] = ld_q(D.den1, 1);
}

// eq weight of term j over the suffix of length s of the layer point y (n_y
// coordinates): tab holds eq(bits(j), y[n_y - s ..]) for s <= kLkTab at
// offset 2^s - 1; longer suffixes split as hi(j >> kLkTab) * tab_kLkTab.
__device__ __forceinline__ qm31 lk_hi(const qm31* __restrict__ y, int n_y, int s, uint64_t u) {
  const int nh = s - kLkTab;
  qm31 e = qm31_one();
  for (int c = 0; c < nh; c++) {
    const qm31 yc = y[n_y - s + c];
    e = qm31_mul(e, ((u >> (nh - 1 - c)) & 1ull) ? yc : qm31_sub(qm31_one(), yc));
  }
  return e;
}

__device__ __forceinline__ qm31 fold_ld(const qm31* p, uint64_t i, uint64_t h, bool pend, qm31 x) {
  const qm31 a = ld_q(p, i);
  return pend ? qm31_fold(a, ld_q(p, i + h), x) : a;
}
__device__ __forceinline__ qm31 fold_num(const void* p, uint32_t fmt, uint64_t i, uint64_t h, bool pend, qm31 x) {
  const qm31 a = lk_num(p, fmt, i);
  if (!pend || fmt == NF_ONE) return a;
  return qm31_fold(a, lk_num(p, fmt, i + h), x);
}

static __global__ void __launch_bounds__(kBlock) k_lk_round(const LkRound* __restrict__ desc, uint32_t n_desc,
                                                             const qm31* __restrict__ tab, const qm31* __restrict__ y,
                                                             int n_y, qm31* __restrict__ partials,
                                                             qm31* __restrict__ res) {
  const LkRound D = desc[find_desc(desc, n_desc)];
  const int s = (int)D.m - 2;
  const uint64_t nt = 1ull << s;
  const uint64_t j = (uint64_t)(blockIdx.x - D.wg0) * kBlock + threadIdx.x;
  __shared__ qm31 s_hi;
  if (s > kLkTab && threadIdx.x == 0) s_hi = lk_hi(y, n_y, s, j >> kLkTab);
  __syncthreads();
  qm31 v[4] = {qm31_zero(), qm31_zero(), qm31_zero(), qm31_zero()};
  if (j < nt) {
    const uint64_t h = 1ull << D.m;  // fold distance in the source
    const bool pend = D.pend != 0;
    const uint64_t pos[4] = {2 * j, 2 * j + 1, 2 * (nt + j), 2 * (nt + j) + 1};
    qm31 dv[4], nv[4];
#pragma unroll
    for (int q = 0; q < 4; q++) dv[q] = fold_ld(D.src_den, pos[q], h, pend, D.x);
    if (!D.gp) {
#pragma unroll
      for (int q = 0; q < 4; q++) nv[q] = fold_num(D.src_num, D.fmt, pos[q], h, pend, D.x);
    }
    if (pend) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        st_q(D.dst_den, pos[q], dv[q]);
        if (!D.gp && D.fmt != NF_ONE) st_q(D.dst_num, pos[q], nv[q]);
      }
    }
    const qm31 w = s <= kLkTab ? ld_q(tab, (1ull << s) - 1 + j)
                               : qm31_mul(s_hi, ld_q(tab, (1ull << kLkTab) - 1 + (j & ((1ull << kLkTab) - 1))));
    // t = 2 by extrapolation: f(2) = 2 f(1) - f(0) along the first variable
    const qm31 d20 = qm31_sub(qm31_add(dv[2], dv[2]), dv[0]), d21 = qm31_sub(qm31_add(dv[3], dv[3]), dv[1]);
    if (D.gp) {
      v[0] = qm31_mul(w, qm31_mul(dv[0], dv[1]));
      v[2] = qm31_mul(w, qm31_mul(d20, d21));
    } else {
      qm31 num0, num2;
      if (D.fmt == NF_ONE) {
        num0 = qm31_add(dv[0], dv[1]);
        num2 = qm31_add(d20, d21);
      } else {
        const qm31 n20 = qm31_sub(qm31_add(nv[2], nv[2]), nv[0]), n21 = qm31_sub(qm31_add(nv[3], nv[3]), nv[1]);
        num0 = qm31_add(qm31_mul(nv[0], dv[1]), qm31_mul(nv[1], dv[0]));
        num2 = qm31_add(qm31_mul(n20, d21), qm31_mul(n21, d20));
      }
      v[0] = qm31_mul(w, num0);
      v[1] = qm31_mul(w, qm31_mul(dv[0], dv[1]));
      v[2] = qm31_mul(w, num2);
      v[3] = qm31_mul(w, qm31_mul(d20, d21));
    }
    if (nt == 1) {  // the last round of this instance: its four values per column
      qm31* o = res + (uint64_t)kLkRes * D.slot + 4;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        o[q] = D.gp ? qm31_zero() : nv[q];
        o[4 + q] = dv[q];
      }
    }
  }
  block_sum_store<4>(v, partials + 4ull * blockIdx.x);
}

// Per instance (one workgroup each): the sum of its workgroup rows.
static __global__ void __launch_bounds__(kBlock) k_lk_finish(const LkRound* __restrict__ desc,
                                                              const qm31* __restrict__ partials,
                                                              qm31* __restrict__ res) {
  const LkRound D = desc[blockIdx.x];
  const uint64_t nt = 1ull << (D.m - 2);
  const uint32_t nwg = (uint32_t)((nt + kBlock - 1) / kBlock);
  qacc acc[4];
#pragma unroll
  for (int q = 0; q < 4; q++) acc[q].zero();
  for (uint32_t b = threadIdx.x; b < nwg; b += blockDim.x)
#pragma unroll
    for (int q = 0; q < 4; q++) acc[q].add(ld_q(partials, 4ull * (D.wg0 + b) + q));
  qm31 tot[4];
#pragma unroll
  for (int q = 0; q < 4; q++) tot[q] = acc[q].reduce();
  block_sum_store<4>(tot, res + (uint64_t)kLkRes * D.slot);
}

// ------------------------------------------------------------------ host side
qm31 eq1(const qm31& x, const qm31& y) {
  return qm31_add(qm31_mul(x, y), qm31_mul(qm31_sub(qm31_one(), x), qm31_sub(qm31_one(), y)));
}

// Polynomial of at most 4 coefficients, leading zeros dropped (UnivariatePoly, utils.rs:14-69).
struct Poly {
  qm31 c[4];
  int len = 0;
  void trunc() {
    while (len > 0 && qm31_eq(c[len - 1], qm31_zero())) len--;
  }
  qm31 eval(const qm31& x) const {
    qm31 acc = qm31_zero();
    for (int i = len - 1; i >= 0; i--) acc = qm31_add(qm31_mul(acc, x), c[i]);
    return acc;
  }
};

// The round polynomial of correct_sum_as_poly_in_first_variable
// (gkr_prover.rs:518-566) is the unique cubic r with r(0), r(1), r(2) given and
// r(b) = 0, b = (1 - y) / (1 - 2 y) the root of eq(t, y).  Written as
// r(t) = (t - b) q(t) with q the quadratic through q(k) = r(k) / (k - b),
// k = 0, 1, 2; the reciprocals depend only on y, so instances of one size
// share them within a round.
struct RootInv {
  qm31 y, b, i0, i1, i2;  // i_k = 1 / (k - b)
  bool valid = false;
};
RootInv root_inv(const qm31& y) {
  RootInv r;
  r.y = y;
  r.b = qm31_mul(qm31_sub(qm31_one(), y), qm31_inv(qm31_sub(qm31_one(), qm31_add(y, y))));
  const qm31 d0 = qm31_neg(r.b), d1 = qm31_sub(qm31_one(), r.b), d2 = qm31_sub(qm31_from_m31(2), r.b);
  const qm31 p01 = qm31_mul(d0, d1), inv = qm31_inv(qm31_mul(p01, d2)), t = qm31_mul(inv, d2);
  r.i2 = qm31_mul(inv, p01);
  r.i1 = qm31_mul(t, d0);
  r.i0 = qm31_mul(t, d1);
  r.valid = true;
  return r;
}
Poly cubic_with_root(const qm31& r0, const qm31& r1, const qm31& r2, const RootInv& ri) {
  const qm31 inv2 = qm31_from_m31(1u << 30);
  const qm31 q0 = qm31_mul(r0, ri.i0), q1 = qm31_mul(r1, ri.i1), q2 = qm31_mul(r2, ri.i2);
  const qm31 a2 = qm31_mul(qm31_add(qm31_sub(q2, qm31_add(q1, q1)), q0), inv2);  // q = a0 + a1 t + a2 t^2
  const qm31 a1 = qm31_sub(qm31_sub(q1, q0), a2), a0 = q0;
  Poly p;
  p.c[0] = qm31_neg(qm31_mul(ri.b, a0));
  p.c[1] = qm31_sub(a0, qm31_mul(ri.b, a1));
  p.c[2] = qm31_sub(a1, qm31_mul(ri.b, a2));
  p.c[3] = a2;
  p.len = 4;
  p.trunc();
  return p;
}

qm31 horner(const qm31* v, int n, const qm31& a) {  // random_linear_combination: v0 + a v1 + ...
  qm31 acc = qm31_zero();
  for (int i = n - 1; i >= 0; i--) acc = qm31_add(qm31_mul(acc, a), v[i]);
  return acc;
}

struct Inst {
  uint32_t kind, nv;
  const void* num;
  const qm31* den;
  qm31* arena_num = nullptr;  // levels 0 .. nv-1
  qm31* arena_den = nullptr;
  qm31* fold_num[2] = {nullptr, nullptr};
  qm31* fold_den[2] = {nullptr, nullptr};
  qm31 top[6];
  // GKR state
  bool active = false;
  int nclaims = 0;
  qm31 claims[2];
  bool gp() const { return kind == GKR_LOOKUP_GRAND_PRODUCT; }
  uint32_t in_fmt() const {
    return kind == GKR_LOOKUP_LOGUP_GENERIC ? NF_Q : kind == GKR_LOOKUP_LOGUP_MULTIPLICITIES ? NF_M31
                                                   : kind == GKR_LOOKUP_LOGUP_SINGLES          ? NF_ONE
                                                                                               : NF_NONE;
  }
  // the layer with lv variables: source pointers and numerator format
  void layer(int lv, const void** n, const qm31** d, uint32_t* fmt) const {
    if (lv == (int)nv) {
      *n = num;
      *d = den;
      *fmt = in_fmt();
    } else {
      const uint64_t off = (1ull << lv) - 1;
      *n = gp() ? nullptr : arena_num + off;
      *d = arena_den + off;
      *fmt = gp() ? NF_NONE : NF_Q;
    }
  }
};

int ensure_host(gkr_ctx* c, int hs, size_t bytes, void** out) {
  if (c->hcap[hs] < bytes) {
    if (c->hbuf[hs]) {
      HIP_TRY(hipStreamSynchronize(c->stream));
      (void)hipHostFree(c->hbuf[hs]);
    }
    c->hbuf[hs] = nullptr;
    c->hcap[hs] = 0;
    const size_t want = bytes < 4096 ? 4096 : bytes;
    HIP_TRY(hipHostMalloc(&c->hbuf[hs], want, hipHostMallocDefault));
    c->hcap[hs] = want;
  }
  *out = c->hbuf[hs];
  return GKR_OK;
}

int lk_check(const gkr_lookup_instance* in, size_t n) {
  if (!in || n == 0) return fail(GKR_ERR_INVALID, "empty lookup batch");
  for (size_t i = 0; i < n; i++) {
    const gkr_lookup_instance& x = in[i];
    if (x.kind > GKR_LOOKUP_LOGUP_SINGLES) return fail(GKR_ERR_INVALID, "instance %zu: kind %u", i, x.kind);
    if (x.n_vars < 1 || x.n_vars > (uint32_t)kLkMaxVars)
      return fail(GKR_ERR_INVALID, "instance %zu: %u variables (1 .. %d)", i, x.n_vars, kLkMaxVars);
    if (!x.denominators) return fail(GKR_ERR_INVALID, "instance %zu: no denominators", i);
    if ((x.kind == GKR_LOOKUP_LOGUP_GENERIC || x.kind == GKR_LOOKUP_LOGUP_MULTIPLICITIES) && !x.numerators)
      return fail(GKR_ERR_INVALID, "instance %zu: no numerators", i);
    // try_into_mask is unimplemented for a multiplicities layer that is never folded (gkr_prover.rs:359)
    if (x.kind == GKR_LOOKUP_LOGUP_MULTIPLICITIES && x.n_vars == 1)
      return fail(GKR_ERR_INVALID, "instance %zu: a multiplicities layer needs 2 or more variables", i);
  }
  return GKR_OK;
}

// gen_layers (gkr_prover.rs:503-508) for every instance, then levels 0 and 1 to the host.
int lk_build(gkr_ctx* c, std::vector<Inst>& I) {
  size_t arena = 0, folds = 0;
  for (const Inst& x : I) {
    const size_t cols = x.gp() ? 1 : 2;
    arena += cols * (((size_t)1 << x.nv) - 1);
    folds += cols * 2 * ((size_t)1 << (x.nv - 1));
  }
  qm31 *a, *f, *top;
  TRY(ensureT(c, S_LKARENA, arena, &a));
  TRY(ensureT(c, S_LKFOLD, folds, &f));
  for (Inst& x : I) {
    const size_t len = ((size_t)1 << x.nv) - 1, half = (size_t)1 << (x.nv - 1);
    x.arena_den = a;
    a += len;
    if (!x.gp()) {
      x.arena_num = a;
      a += len;
    }
    for (int k = 0; k < 2; k++) {
      x.fold_den[k] = f;
      f += half;
      if (!x.gp()) {
        x.fold_num[k] = f;
        f += half;
      }
    }
  }
  // stages of up to kLkLevels levels each
  std::vector<int> lvl(I.size());
  for (size_t i = 0; i < I.size(); i++) lvl[i] = (int)I[i].nv;
  for (;;) {
    std::vector<LkTree> d;
    uint32_t wg = 0;
    uint64_t bytes = 0;
    for (size_t i = 0; i < I.size(); i++) {
      if (lvl[i] == 0) continue;
      const Inst& x = I[i];
      LkTree t;
      memset(&t, 0, sizeof t);
      const void* n;
      const qm31* dd;
      uint32_t fmt;
      x.layer(lvl[i], &n, &dd, &fmt);
      t.num = n;
      t.den = dd;
      t.fmt = fmt;
      t.gp = x.gp();
      t.out_num = x.arena_num;
      t.out_den = x.arena_den;
      t.src_log = (uint32_t)lvl[i];
      t.levels = (uint32_t)std::min(kLkLevels, lvl[i]);
      t.wg0 = wg;
      const uint64_t half = 1ull << (lvl[i] - 1);
      wg += (uint32_t)((half + kBlock - 1) / kBlock);
      bytes += (16 + (fmt == NF_Q ? 16 : fmt == NF_M31 ? 4 : 0)) * (2 * half) + (x.gp() ? 16 : 32) * 2 * half;
      d.push_back(t);
      lvl[i] -= (int)t.levels;
    }
    if (d.empty()) break;
    void *dv, *h;
    TRY(ensure(c, S_LKDESC, d.size() * sizeof(LkTree), &dv));
    LkTree* dd = static_cast<LkTree*>(dv);
    TRY(ensure_host(c, H_LKDESC, d.size() * sizeof(LkTree), &h));
    memcpy(h, d.data(), d.size() * sizeof(LkTree));
    HIP_TRY(hipMemcpyAsync(dd, h, d.size() * sizeof(LkTree), hipMemcpyHostToDevice, c->stream));
    {
      TimedLaunch tl(c, K_LOOKUP, bytes);
      GKR_LAUNCH(c, k_lk_tree, dim3(wg), dim3(kBlock), 0, dd, (uint32_t)d.size());
    }
    TRY(check_launch(c));
    TRY(sync(c));  // the staging buffer is reused by the next stage
  }
  std::vector<LkTop> td(I.size());
  for (size_t i = 0; i < I.size(); i++) {
    const Inst& x = I[i];
    LkTop& t = td[i];
    memset(&t, 0, sizeof t);
    const void* n;
    const qm31* dd;
    uint32_t fmt;
    x.layer(1, &n, &dd, &fmt);
    t.num1 = n;
    t.den1 = dd;
    t.fmt1 = fmt;
    t.num0 = x.arena_num;
    t.den0 = x.arena_den;
    t.gp = x.gp();
  }
  void *dv, *h;
  TRY(ensure(c, S_LKDESC, td.size() * sizeof(LkTop), &dv));
  LkTop* dt = static_cast<LkTop*>(dv);
  TRY(ensureT(c, S_LKRES, 6 * I.size(), &top));
  TRY(ensure_host(c, H_LKDESC, td.size() * sizeof(LkTop), &h));
  memcpy(h, td.data(), td.size() * sizeof(LkTop));
  HIP_TRY(hipMemcpyAsync(dt, h, td.size() * sizeof(LkTop), hipMemcpyHostToDevice, c->stream));
  GKR_LAUNCH(c, k_lk_top, dim3(grid_for(I.size())), dim3(kBlock), 0, dt, (uint32_t)I.size(), top);
  TRY(check_launch(c));
  void* hr;
  TRY(ensure_host(c, H_LKRES, 6 * I.size() * sizeof(qm31), &hr));
  HIP_TRY(hipMemcpyAsync(hr, top, 6 * I.size() * sizeof(qm31), hipMemcpyDeviceToHost, c->stream));
  TRY(sync(c));
  const qm31* r = static_cast<const qm31*>(hr);
  for (size_t i = 0; i < I.size(); i++)
    for (int k = 0; k < 6; k++) I[i].top[k] = r[6 * i + k];
  return GKR_OK;
}

// Suffix eq tables of the layer point y (n_y coordinates) for suffix lengths
// 0 .. min(kLkTab, n_y), then y itself, to the device.
int lk_tables(gkr_ctx* c, const std::vector<qm31>& y, qm31** d_tab, qm31** d_y) {
  const int smax = std::min(kLkTab, (int)y.size());
  const size_t ntab = ((size_t)1 << (smax + 1)) - 1;
  std::vector<qm31> t(ntab + y.size() + 1);
  t[0] = qm31_one();
  for (int s = 1; s <= smax; s++) {  // T_s = eq over y[n_y - s] (new top bit) times T_{s-1}
    const qm31 ys = y[y.size() - s], om = qm31_sub(qm31_one(), ys);
    const size_t prev = ((size_t)1 << (s - 1)) - 1, cur = ((size_t)1 << s) - 1, h = (size_t)1 << (s - 1);
    for (size_t j = 0; j < h; j++) {
      t[cur + j] = qm31_mul(om, t[prev + j]);
      t[cur + h + j] = qm31_mul(ys, t[prev + j]);
    }
  }
  for (size_t k = 0; k < y.size(); k++) t[ntab + k] = y[k];
  qm31* d;
  void* h;
  TRY(ensureT(c, S_LKTAB, t.size(), &d));
  TRY(ensure_host(c, H_LKTAB, t.size() * sizeof(qm31), &h));
  memcpy(h, t.data(), t.size() * sizeof(qm31));
  HIP_TRY(hipMemcpyAsync(d, h, t.size() * sizeof(qm31), hipMemcpyHostToDevice, c->stream));
  *d_tab = d;
  *d_y = d + ntab;
  return GKR_OK;
}

}  // namespace

extern "C" int gkr_prove_lookup_batch(gkr_ctx* c, gkr_channel* ch, const gkr_lookup_instance* instances,
                                      size_t n_instances, gkr_lookup_batch* out) {
  if (!c || !out) return fail(GKR_ERR_INVALID, "null argument");
  CH_CHECK(ch);
  TRY(lk_check(instances, n_instances));
  if (!out->output_claims || !out->round_polys || !out->round_poly_lens || !out->masks || !out->ood_point ||
      !out->claims_to_verify)
    return fail(GKR_ERR_INVALID, "null output arrays");
  HIP_TRY(hipSetDevice(c->device));
  c->mm.valid = false;
  PoseidonChannel& C = ch->ch;
  const size_t ni = n_instances;
  std::vector<Inst> I(ni);
  int n_layers = 0;
  for (size_t i = 0; i < ni; i++) {
    I[i].kind = instances[i].kind;
    I[i].nv = instances[i].n_vars;
    I[i].num = instances[i].numerators;
    I[i].den = reinterpret_cast<const qm31*>(instances[i].denominators);
    n_layers = std::max(n_layers, (int)I[i].nv);
  }
  TRY(lk_build(c, I));
  memset(out->masks, 0, (size_t)n_layers * ni * 4 * sizeof(gkr_qm31));
  std::vector<qm31> ood;
  size_t round = 0;
  const qm31 inv2 = qm31_from_m31(1u << 30), two = qm31_from_m31(2);
  for (int layer = 0; layer < n_layers; layer++) {
    const int n_rem = n_layers - layer;
    for (size_t i = 0; i < ni; i++)
      if ((int)I[i].nv == n_rem) {  // output layer values
        Inst& x = I[i];
        x.active = true;
        if (x.gp()) {
          x.nclaims = 1;
          x.claims[0] = x.top[1];
        } else {
          x.nclaims = 2;
          x.claims[0] = x.top[0];
          x.claims[1] = x.top[1];
        }
        for (int k = 0; k < 2; k++) out->output_claims[2 * i + k] = G(k < x.nclaims ? x.claims[k] : qm31_zero());
      }
    {
      HostTimer ht(c, K_HOST_FS);
      for (size_t i = 0; i < ni; i++)
        if (I[i].active) C.mix_felts_stwo(I[i].claims, I[i].nclaims);
    }
    const qm31 alpha = C.draw_qm31(), lambda = C.draw_qm31();
    // per active instance: layer variables lv, oracle variables k = lv - 1
    std::vector<size_t> act;
    std::vector<int> lv(ni, 0);
    std::vector<qm31> sc(ni), corr(ni, qm31_one()), pend_x(ni);
    std::vector<Poly> polys(ni);
    for (size_t i = 0; i < ni; i++)
      if (I[i].active) {
        act.push_back(i);
        lv[i] = layer - (n_layers - (int)I[i].nv) + 1;
        sc[i] = horner(I[i].claims, I[i].nclaims, lambda);
        sc[i] = qm31_mul_m31(sc[i], 1u << (layer - (lv[i] - 1)));  // claim doubling for unused variables
      }
    qm31 *d_tab = nullptr, *d_y = nullptr;
    if (layer > 0) TRY(lk_tables(c, ood, &d_tab, &d_y));
    std::vector<qm31> assign(layer);
    std::vector<qm31> snap(ni * 8);
    for (int r = 0; r < layer; r++) {
      // the instances in their own rounds, and their launch descriptors
      std::vector<LkRound> d;
      std::vector<size_t> real;
      uint32_t wg = 0;
      uint64_t bytes = 0;
      for (size_t i : act) {
        const int k = lv[i] - 1;
        if (layer - r > k) continue;
        const int rho = r - (layer - k);
        const Inst& x = I[i];
        LkRound e;
        memset(&e, 0, sizeof e);
        const void* n0;
        const qm31* d0;
        uint32_t fmt0;
        x.layer(lv[i], &n0, &d0, &fmt0);
        const uint32_t fmt_folded = fmt0 == NF_ONE ? NF_ONE : x.gp() ? NF_NONE : NF_Q;
        // own round rho reads the layer (rho <= 1) or the buffer round rho - 1
        // wrote, and (rho >= 1) folds into buffer (rho - 1) & 1
        if (rho <= 1) {
          e.src_num = n0;
          e.src_den = d0;
          e.fmt = fmt0;
        } else {
          e.src_num = x.fold_num[rho & 1];
          e.src_den = x.fold_den[rho & 1];
          e.fmt = fmt_folded;
        }
        if (rho >= 1) {
          const int b = (rho - 1) & 1;
          e.dst_num = x.fold_num[b];
          e.dst_den = x.fold_den[b];
          e.pend = 1;
          e.x = pend_x[i];
        }
        e.gp = x.gp();
        e.m = (uint32_t)(lv[i] - rho);
        e.wg0 = wg;
        e.slot = (uint32_t)real.size();
        const uint64_t nt = 1ull << (e.m - 2);
        wg += (uint32_t)((nt + kBlock - 1) / kBlock);
        const uint64_t ent = 4 * nt, per_num = e.fmt == NF_Q ? 16 : e.fmt == NF_M31 ? 4 : 0;
        bytes += (e.pend ? 2 : 1) * ent * (16 + per_num) + (e.pend ? ent * (16 + (fmt_folded == NF_Q ? 16 : 0)) : 0);
        d.push_back(e);
        real.push_back(i);
      }
      if (!d.empty()) {
        qm31 *part, *res;
        void *dv, *h, *hr;
        TRY(ensure(c, S_LKDESC, d.size() * sizeof(LkRound), &dv));
        LkRound* dd = static_cast<LkRound*>(dv);
        TRY(ensureT(c, S_LKPART, 4ull * wg, &part));
        TRY(ensureT(c, S_LKRES, (size_t)kLkRes * d.size(), &res));
        TRY(ensure_host(c, H_LKDESC, d.size() * sizeof(LkRound), &h));
        TRY(ensure_host(c, H_LKRES, (size_t)kLkRes * d.size() * sizeof(qm31), &hr));
        memcpy(h, d.data(), d.size() * sizeof(LkRound));
        {
          HostTimer ht(c, K_HOST_LAUNCH);
          HIP_TRY(hipMemcpyAsync(dd, h, d.size() * sizeof(LkRound), hipMemcpyHostToDevice, c->stream));
          {
            TimedLaunch tl(c, K_LOOKUP, bytes);
            GKR_LAUNCH(c, k_lk_round, dim3(wg), dim3(kBlock), 0, dd, (uint32_t)d.size(), d_tab, d_y,
                               layer, part, res);
          }
          TRY(check_launch(c));
          GKR_LAUNCH(c, k_lk_finish, dim3((unsigned)d.size()), dim3(kBlock), 0, dd, part, res);
          TRY(check_launch(c));
          HIP_TRY(hipMemcpyAsync(hr, res, (size_t)kLkRes * d.size() * sizeof(qm31), hipMemcpyDeviceToHost,
                                 c->stream));
        }
        {
          HostTimer ht(c, K_HOST_WAIT);
          TRY(sync(c));
        }
        const qm31* rv = static_cast<const qm31*>(hr);
        RootInv roots[kLkMaxVars + 2];
        for (size_t a = 0; a < real.size(); a++) {
          const size_t i = real[a];
          const qm31* s = rv + (size_t)kLkRes * a;
          const qm31 S0 = I[i].gp() ? s[0] : qm31_add(s[0], qm31_mul(lambda, s[1]));
          const qm31 S2 = I[i].gp() ? s[2] : qm31_add(s[2], qm31_mul(lambda, s[3]));
          const int m = (int)d[a].m;
          const qm31 yc = ood[layer - m + 1];
          const qm31 r0 = qm31_mul(qm31_mul(S0, corr[i]), eq1(qm31_zero(), yc));
          const qm31 r2 = qm31_mul(qm31_mul(S2, corr[i]), eq1(two, yc));
          if (!roots[m].valid) roots[m] = root_inv(yc);
          polys[i] = cubic_with_root(r0, qm31_sub(sc[i], r0), r2, roots[m]);
          if (m == 2)
            for (int q = 0; q < 8; q++) snap[8 * i + q] = s[4 + q];
        }
      }
      Poly comb;
      for (size_t a = act.size(); a-- > 0;) {
        const size_t i = act[a];
        const int k = lv[i] - 1;
        if (layer - r > k) {  // a constant round of a smaller instance
          polys[i].c[0] = qm31_mul(sc[i], inv2);
          polys[i].len = 1;
          polys[i].trunc();
        }
        if (!qm31_eq(qm31_add(polys[i].eval(qm31_zero()), polys[i].eval(qm31_one())), sc[i]))
          return fail(GKR_ERR_INVALID, "lookup batch: round %d of layer %d does not sum to the claim (degenerate input)",
                      r, layer);
        for (int q = 0; q < comb.len; q++) comb.c[q] = qm31_mul(comb.c[q], alpha);
        const int len = std::max(comb.len, polys[i].len);
        for (int q = 0; q < len; q++)
          comb.c[q] = qm31_add(q < comb.len ? comb.c[q] : qm31_zero(), q < polys[i].len ? polys[i].c[q] : qm31_zero());
        comb.len = len;
      }
      qm31 xr;
      {
        HostTimer ht(c, K_HOST_FS);
        C.mix_felts_stwo(comb.c, comb.len);
        xr = C.draw_qm31();
      }
      for (int q = 0; q < 4; q++) out->round_polys[4 * round + q] = G(q < comb.len ? comb.c[q] : qm31_zero());
      out->round_poly_lens[round] = (uint32_t)comb.len;
      round++;
      assign[r] = xr;
      for (size_t i : act) sc[i] = polys[i].eval(xr);
      for (size_t a = 0; a < real.size(); a++) {
        const size_t i = real[a];
        corr[i] = qm31_mul(corr[i], eq1(xr, ood[layer - (int)d[a].m + 1]));
        pend_x[i] = xr;
      }
    }
    // masks: an instance with rounds folds its last four values with the last
    // challenge; a newly joined one gives its level-1 values
    std::vector<qm31> mk(4 * ni);
    {
      HostTimer ht(c, K_HOST_FS);
      for (size_t i : act) {
        const Inst& x = I[i];
        qm31* m = &mk[4 * i];
        if (lv[i] == 1) {
          m[0] = x.gp() ? x.top[4] : x.top[2];
          m[1] = x.gp() ? x.top[5] : x.top[3];
          m[2] = x.top[4];
          m[3] = x.top[5];
        } else {
          const qm31* s = &snap[8 * i];
          const qm31 xl = assign[layer - 1];
          const qm31 n0 = qm31_fold(s[0], s[2], xl), n1 = qm31_fold(s[1], s[3], xl);
          const qm31 d0 = qm31_fold(s[4], s[6], xl), d1 = qm31_fold(s[5], s[7], xl);
          m[0] = x.gp() ? d0 : n0;
          m[1] = x.gp() ? d1 : n1;
          m[2] = d0;
          m[3] = d1;
        }
        const int nq = x.gp() ? 2 : 4;
        C.mix_felts_stwo(m, nq);
        for (int q = 0; q < 4; q++)
          out->masks[4 * ((size_t)layer * ni + i) + q] = G(q < nq ? m[q] : qm31_zero());
      }
    }
    const qm31 cz = C.draw_qm31();
    ood = assign;
    ood.push_back(cz);
    for (size_t i : act) {
      const qm31* m = &mk[4 * i];
      I[i].claims[0] = qm31_fold(m[0], m[1], cz);
      if (!I[i].gp()) I[i].claims[1] = qm31_fold(m[2], m[3], cz);
    }
  }
  out->n_layers = (uint32_t)n_layers;
  for (size_t k = 0; k < ood.size(); k++) out->ood_point[k] = G(ood[k]);
  for (size_t i = 0; i < ni; i++)
    for (int k = 0; k < 2; k++) out->claims_to_verify[2 * i + k] = G(k < I[i].nclaims ? I[i].claims[k] : qm31_zero());
  return GKR_OK;
}

extern "C" const uint32_t* gkr_matrix_device_ptr(const gkr_matrix* m) { return m ? m->dev : nullptr; }

namespace {

bool lk_canon(const gkr_qm31& q) { return q.v[0] < P && q.v[1] < P && q.v[2] < P && q.v[3] < P; }

int lk_shape(const uint32_t* gates, const uint32_t* n_vars, size_t n, int* n_layers) {
  if (!gates || !n_vars || n == 0) return fail(GKR_ERR_INVALID, "empty lookup batch");
  *n_layers = 0;
  for (size_t i = 0; i < n; i++) {
    if (gates[i] > 1) return fail(GKR_ERR_INVALID, "instance %zu: gate %u", i, gates[i]);
    if (n_vars[i] < 1 || n_vars[i] > (uint32_t)kLkMaxVars)
      return fail(GKR_ERR_INVALID, "instance %zu: %u variables", i, n_vars[i]);
    *n_layers = std::max(*n_layers, (int)n_vars[i]);
  }
  return GKR_OK;
}

}  // namespace

// partially_verify_batch (gkr_verifier.rs:17-157) with sumcheck::partially_verify
// (sumcheck.rs:151-180) and Gate::eval (gkr_verifier.rs:198-232).
extern "C" int gkr_verify_lookup_batch(const uint32_t* gates, const uint32_t* n_vars, size_t n_instances,
                                       const gkr_lookup_batch* p, gkr_channel* ch, gkr_qm31* ood_out,
                                       gkr_qm31* claims_out) {
  int n_layers = 0;
  TRY(lk_shape(gates, n_vars, n_instances, &n_layers));
  if (!p || !ood_out || !claims_out || !p->output_claims || !p->round_polys || !p->round_poly_lens || !p->masks)
    return fail(GKR_ERR_INVALID, "null argument");
  CH_CHECK(ch);
  if ((int)p->n_layers != n_layers)
    return fail(GKR_ERR_VERIFY, "proof has %u layers, the instances %d", p->n_layers, n_layers);
  PoseidonChannel& C = ch->ch;
  const size_t ni = n_instances;
  std::vector<qm31> claims(2 * ni);
  std::vector<int> ncl(ni, 0);
  std::vector<qm31> ood;
  size_t round = 0;
  for (int layer = 0; layer < n_layers; layer++) {
    for (size_t i = 0; i < ni; i++)
      if ((int)n_vars[i] == n_layers - layer) {
        ncl[i] = gates[i] == 0 ? 1 : 2;
        for (int k = 0; k < ncl[i]; k++) {
          if (!lk_canon(p->output_claims[2 * i + k])) return fail(GKR_ERR_VERIFY, "output claim not canonical");
          claims[2 * i + k] = Q(p->output_claims[2 * i + k]);
        }
      }
    for (size_t i = 0; i < ni; i++)
      if (ncl[i]) C.mix_felts_stwo(&claims[2 * i], ncl[i]);
    const qm31 alpha = C.draw_qm31(), lambda = C.draw_qm31();
    std::vector<qm31> cl;
    for (size_t i = 0; i < ni; i++)
      if (ncl[i]) {
        const int unused = n_layers - (int)n_vars[i];
        cl.push_back(qm31_mul_m31(horner(&claims[2 * i], ncl[i], lambda), 1u << unused));
      }
    qm31 sum = horner(cl.data(), (int)cl.size(), alpha);
    std::vector<qm31> pt(layer);
    for (int r = 0; r < layer; r++, round++) {
      Poly q;
      q.len = (int)p->round_poly_lens[round];
      if (q.len < 0 || q.len > 4)
        return fail(GKR_ERR_VERIFY, "layer %d round %d: degree above 3", layer, r);
      for (int k = 0; k < q.len; k++) {
        if (!lk_canon(p->round_polys[4 * round + k])) return fail(GKR_ERR_VERIFY, "round polynomial not canonical");
        q.c[k] = Q(p->round_polys[4 * round + k]);
      }
      if (!qm31_eq(qm31_add(q.eval(qm31_zero()), q.eval(qm31_one())), sum))
        return fail(GKR_ERR_VERIFY, "layer %d round %d: p(0) + p(1) differs from the claim", layer, r);
      C.mix_felts_stwo(q.c, q.len);
      pt[r] = C.draw_qm31();
      sum = q.eval(pt[r]);
    }
    std::vector<qm31> ev;
    for (size_t i = 0; i < ni; i++)
      if (ncl[i]) {
        const int unused = n_layers - (int)n_vars[i];
        const gkr_qm31* m = p->masks + 4 * ((size_t)layer * ni + i);
        for (int k = 0; k < (gates[i] ? 4 : 2); k++)
          if (!lk_canon(m[k])) return fail(GKR_ERR_VERIFY, "mask not canonical");
        qm31 g[2];
        int ng;
        if (gates[i] == 0) {
          g[0] = qm31_mul(Q(m[0]), Q(m[1]));
          ng = 1;
        } else {
          g[0] = qm31_add(qm31_mul(Q(m[0]), Q(m[3])), qm31_mul(Q(m[1]), Q(m[2])));
          g[1] = qm31_mul(Q(m[2]), Q(m[3]));
          ng = 2;
        }
        qm31 e = qm31_one();
        for (int k = unused; k < layer; k++) e = qm31_mul(e, eq1(ood[k], pt[k]));
        ev.push_back(qm31_mul(e, horner(g, ng, lambda)));
      }
    if (!qm31_eq(horner(ev.data(), (int)ev.size(), alpha), sum))
      return fail(GKR_ERR_VERIFY, "layer %d: the circuit at the sumcheck point differs from the sumcheck", layer);
    for (size_t i = 0; i < ni; i++)
      if (ncl[i]) {
        const gkr_qm31* m = p->masks + 4 * ((size_t)layer * ni + i);
        qm31 v[4];
        const int nv = gates[i] ? 4 : 2;
        for (int k = 0; k < nv; k++) v[k] = Q(m[k]);
        C.mix_felts_stwo(v, nv);
      }
    const qm31 c = C.draw_qm31();
    ood = pt;
    ood.push_back(c);
    for (size_t i = 0; i < ni; i++)
      if (ncl[i]) {
        const gkr_qm31* m = p->masks + 4 * ((size_t)layer * ni + i);
        for (int k = 0; k < ncl[i]; k++) claims[2 * i + k] = qm31_fold(Q(m[2 * k]), Q(m[2 * k + 1]), c);
      }
  }
  for (size_t k = 0; k < ood.size(); k++) ood_out[k] = G(ood[k]);
  for (size_t i = 0; i < ni; i++)
    for (int k = 0; k < 2; k++) claims_out[2 * i + k] = G(k < ncl[i] ? claims[2 * i + k] : qm31_zero());
  return GKR_OK;
}

extern "C" int gkr_serialize_lookup_batch(const uint32_t* gates, const uint32_t* n_vars, size_t n_instances,
                                          const gkr_lookup_batch* p, gkr_felt* out, size_t cap, size_t* n_felts) {
  int n_layers = 0;
  TRY(lk_shape(gates, n_vars, n_instances, &n_layers));
  if (!p || !n_felts || (!out && cap)) return fail(GKR_ERR_INVALID, "null argument");
  for (size_t i = 0; i < n_instances; i++)
    if ((int)n_vars[i] != n_layers)
      return fail(GKR_ERR_INVALID, "serialize_stwo_gkr_batch_proof indexes masks by layer: instance %zu has %u of %d "
                                   "variables", i, n_vars[i], n_layers);
  size_t n = 0;
  auto u = [&](uint64_t v) {
    if (out && n < cap) {
      out[n].w[0] = (uint32_t)v;
      out[n].w[1] = (uint32_t)(v >> 32);
      for (int k = 2; k < 8; k++) out[n].w[k] = 0;
    }
    n++;
  };
  auto q = [&](const gkr_qm31& x) {
    for (int k = 0; k < 4; k++) u(x.v[k]);
  };
  const size_t ni = n_instances;
  u(ni);
  for (size_t i = 0; i < ni; i++) {
    u(gates[i]);
    u(n_vars[i]);
    const int nc = gates[i] ? 2 : 1;
    u((uint64_t)nc);
    for (int k = 0; k < nc; k++) q(p->output_claims[2 * i + k]);
  }
  u((uint64_t)n_layers);
  size_t round = 0;
  const gkr_qm31 zero = {{0, 0, 0, 0}};
  for (int layer = 0; layer < n_layers; layer++) {
    u((uint64_t)layer);
    for (int r = 0; r < layer; r++, round++) {
      const uint32_t len = p->round_poly_lens[round];
      for (uint32_t k = 0; k < 4; k++) q(k < len ? p->round_polys[4 * round + k] : zero);
      u(len);
    }
    u(ni);
    for (size_t i = 0; i < ni; i++) {
      const int nv = gates[i] ? 4 : 2;
      u((uint64_t)nv);
      for (int k = 0; k < nv; k++) q(p->masks[4 * ((size_t)layer * ni + i) + k]);
      u((uint64_t)(nv / 2));
    }
  }
  *n_felts = n;
  if (cap < n) return fail(GKR_ERR_BUFFER, "need %zu felts, have %zu", n, cap);
  return GKR_OK;
}
