/* STWO's LogUp-GKR / grand-product batch prover and verifier, restated for
 * the CPU backend.  TEST INFRASTRUCTURE ONLY: the checker of the product's
 * gkr_prove_lookup_batch; nothing in the product links it.
 *
 * Follows stwo-gpu/crates/stwo/src/prover/lookups/:
 *   gkr_prover.rs:396-500   prove_batch (layer loop, claims, alpha / lambda, masks)
 *   gkr_prover.rs:503-508   gen_layers
 *   gkr_prover.rs:518-566   correct_sum_as_poly_in_first_variable
 *   gkr_prover.rs:304-319   GkrMultivariatePolyOracle::fix_first_variable
 *   gkr_prover.rs:343-368   try_into_mask
 *   sumcheck.rs:61-131      sumcheck::prove_batch (claim doubling, random linear
 *                           combination of the round polynomials)
 *   sumcheck.rs:151-180     partially_verify
 *   gkr_verifier.rs:17-157  partially_verify_batch; :198-232 Gate::eval
 *   utils.rs:14-69          UnivariatePoly (leading zeros dropped), interpolate_lagrange
 *   backend/cpu/lookups/gkr.rs:17-288  gen_eq_evals, next_layer, the eval sums
 * The channel is the Poseidon252 channel (stwo core/channel/poseidon252.rs):
 * mix_felts packs pairs of QM31 and hashes [digest, packs...], also for an
 * empty slice (a zero round polynomial has no coefficients left), and
 * draw_secure_felt takes the low four 31-bit limbs of a draw: the operations
 * of orc_mix_felts_stwo / orc_draw_qm31. */
#include "oracle_internal.h"

enum { L_GP = 0, L_GEN = 1, L_MULT = 2, L_SINGLE = 3 };

typedef struct {
  int kind, nv;
  qm* num;       /* L_GEN */
  uint32_t* nm;  /* L_MULT: M31 numerators */
  qm* den;       /* every LogUp kind; L_GP: the column */
} layer_t;

static qm q_m(uint32_t v) { return q_from_m31(v); }
static qm q_dbl(qm x) { return q_add(x, x); }

static void layer_free(layer_t* l) {
  free(l->num);
  free(l->nm);
  free(l->den);
  memset(l, 0, sizeof *l);
}
static qm lnum(const layer_t* l, size_t i) {
  return l->kind == L_GEN ? l->num[i] : l->kind == L_MULT ? q_m(l->nm[i]) : q_one();
}

/* next_layer (backend/cpu/lookups/gkr.rs:250-288): pairs (2i, 2i + 1) */
static layer_t next_layer(const layer_t* l) {
  layer_t o;
  memset(&o, 0, sizeof o);
  o.nv = l->nv - 1;
  const size_t h = (size_t)1 << o.nv;
  if (l->kind == L_GP) {
    o.kind = L_GP;
    o.den = (qm*)malloc(h * sizeof(qm));
    for (size_t i = 0; i < h; i++) o.den[i] = q_mul(l->den[2 * i], l->den[2 * i + 1]);
    return o;
  }
  o.kind = L_GEN;
  o.num = (qm*)malloc(h * sizeof(qm));
  o.den = (qm*)malloc(h * sizeof(qm));
  for (size_t i = 0; i < h; i++) {
    const qm n0 = lnum(l, 2 * i), n1 = lnum(l, 2 * i + 1), d0 = l->den[2 * i], d1 = l->den[2 * i + 1];
    o.num[i] = q_add(q_mul(n0, d1), q_mul(n1, d0)); /* Fraction add, utils.rs / core/fraction */
    o.den[i] = q_mul(d0, d1);
  }
  return o;
}

/* Mle::fix_first_variable: v[i] + x (v[i + h] - v[i]) on the most significant variable */
static layer_t fix_first(layer_t* l, qm x) {
  layer_t o;
  memset(&o, 0, sizeof o);
  if (l->nv == 0) return *l;
  o.nv = l->nv - 1;
  const size_t h = (size_t)1 << o.nv;
  o.den = (qm*)malloc(h * sizeof(qm));
  for (size_t i = 0; i < h; i++) o.den[i] = q_add(l->den[i], q_mul(x, q_sub(l->den[i + h], l->den[i])));
  if (l->kind == L_GP || l->kind == L_SINGLE) {
    o.kind = l->kind;
  } else {  /* multiplicities become generic (gkr_prover.rs:186-192) */
    o.kind = L_GEN;
    o.num = (qm*)malloc(h * sizeof(qm));
    for (size_t i = 0; i < h; i++) {
      const qm a = lnum(l, i), b = lnum(l, i + h);
      o.num[i] = q_add(a, q_mul(x, q_sub(b, a)));
    }
  }
  layer_free(l);
  return o;
}

/* eq(x, y) for single coordinates */
static qm eq1(qm x, qm y) { return q_add(q_mul(x, y), q_mul(q_sub(q_one(), x), q_sub(q_one(), y))); }

/* gen_eq_evals (backend/cpu/lookups/gkr.rs:229-246): eq(x, y) v, x over
 * {0,1}^|y| with the last coordinate on the least significant bit. */
static void gen_eq_evals(const qm* y, int n, qm v, qm* out) {
  size_t len = 1;
  out[0] = v;
  for (int k = n - 1; k >= 0; k--) {
    for (size_t j = 0; j < len; j++) {
      const qm t = q_mul(out[j], y[k]);
      out[len + j] = t;
      out[j] = q_sub(out[j], t);
    }
    len *= 2;
  }
}

/* UnivariatePoly of at most 4 coefficients; len drops leading zeros */
typedef struct {
  qm c[4];
  int len;
} upoly;
static void up_trunc(upoly* p) {
  while (p->len > 0 && q_eq(p->c[p->len - 1], q_zero())) p->len--;
}
static qm up_eval(const upoly* p, qm x) {
  qm acc = q_zero();
  for (int i = p->len - 1; i >= 0; i--) acc = q_add(q_mul(acc, x), p->c[i]);
  return acc;
}
/* interpolate_lagrange (utils.rs:23-48) on 4 points */
static upoly interp4(const qm* xs, const qm* ys) {
  upoly r;
  memset(&r, 0, sizeof r);
  r.len = 4;
  for (int i = 0; i < 4; i++) r.c[i] = q_zero();
  for (int i = 0; i < 4; i++) {
    qm prod = ys[i];
    for (int j = 0; j < 4; j++)
      if (j != i) prod = q_mul(prod, q_inv(q_sub(xs[i], xs[j])));
    qm t[4] = {prod, q_zero(), q_zero(), q_zero()};
    int deg = 0;
    for (int j = 0; j < 4; j++) {
      if (j == i) continue;
      /* t *= (X - xs[j]) */
      for (int k = deg + 1; k >= 1; k--) t[k] = q_sub(t[k - 1], q_mul(xs[j], t[k]));
      t[0] = q_neg(q_mul(xs[j], t[0]));
      deg++;
    }
    for (int k = 0; k < 4; k++) r.c[k] = q_add(r.c[k], t[k]);
  }
  up_trunc(&r);
  return r;
}

/* the oracle of one instance in one GKR layer (GkrMultivariatePolyOracle) */
typedef struct {
  layer_t L;        /* input layer of the oracle: n_variables = L.nv - 1 */
  qm corr;          /* eq_fixed_var_correction */
  qm lambda;
} oracle_t;

/* sum_as_poly_in_first_variable (backend/cpu/lookups/gkr.rs:39-68) with the
 * extended eq_evals of the layer, then correct_sum_as_poly_in_first_variable */
static int sum_as_poly(const oracle_t* h, const qm* eq_evals, const qm* y, int ny, qm claim, upoly* out) {
  const int nv = h->L.nv - 1;
  if (nv <= 0) return 1;
  const size_t n_terms = (size_t)1 << (nv - 1);
  const layer_t* L = &h->L;
  qm e0 = q_zero(), e2 = q_zero();
  for (size_t i = 0; i < n_terms; i++) {
    const qm w = eq_evals[i];
    if (L->kind == L_GP) {
      const qm a0 = L->den[2 * i], a1 = L->den[2 * i + 1];
      const qm b0 = L->den[2 * (n_terms + i)], b1 = L->den[2 * (n_terms + i) + 1];
      const qm c0 = q_sub(q_dbl(b0), a0), c1 = q_sub(q_dbl(b1), a1);
      e0 = q_add(e0, q_mul(w, q_mul(a0, a1)));
      e2 = q_add(e2, q_mul(w, q_mul(c0, c1)));
    } else {
      const qm n00 = lnum(L, 2 * i), n01 = lnum(L, 2 * i + 1);
      const qm n10 = lnum(L, 2 * (n_terms + i)), n11 = lnum(L, 2 * (n_terms + i) + 1);
      const qm d00 = L->den[2 * i], d01 = L->den[2 * i + 1];
      const qm d10 = L->den[2 * (n_terms + i)], d11 = L->den[2 * (n_terms + i) + 1];
      const qm n20 = q_sub(q_dbl(n10), n00), n21 = q_sub(q_dbl(n11), n01);
      const qm d20 = q_sub(q_dbl(d10), d00), d21 = q_sub(q_dbl(d11), d01);
      qm num0, den0, num2, den2;
      if (L->kind == L_SINGLE) { /* Reciprocal add: (a + b) / (a b) */
        num0 = q_add(d00, d01);
        num2 = q_add(d20, d21);
      } else {
        num0 = q_add(q_mul(n00, d01), q_mul(n01, d00));
        num2 = q_add(q_mul(n20, d21), q_mul(n21, d20));
      }
      den0 = q_mul(d00, d01);
      den2 = q_mul(d20, d21);
      e0 = q_add(e0, q_mul(w, q_add(num0, q_mul(h->lambda, den0))));
      e2 = q_add(e2, q_mul(w, q_add(num2, q_mul(h->lambda, den2))));
    }
  }
  e0 = q_mul(e0, h->corr);
  e2 = q_mul(e2, h->corr);
  /* correct_sum_as_poly_in_first_variable (gkr_prover.rs:518-566), k = nv */
  const int k = nv, n = ny;
  if (k > n) return 2;
  qm a = q_one();
  for (int j = 0; j < n - k + 1; j++) a = q_mul(a, eq1(q_zero(), y[j]));
  a = q_inv(a);
  const qm yk = y[n - k];
  const qm b = q_mul(q_sub(q_one(), yk), q_inv(q_sub(q_one(), q_dbl(yk))));
  const qm r0 = q_mul(q_mul(e0, eq1(q_zero(), yk)), a);
  const qm r1 = q_sub(claim, r0);
  const qm r2 = q_mul(q_mul(e2, eq1(q_m(2), yk)), a);
  const qm xs[4] = {q_zero(), q_one(), q_m(2), b}, ys[4] = {r0, r1, r2, q_zero()};
  *out = interp4(xs, ys);
  return 0;
}

static void oracle_fix(oracle_t* h, const qm* y, int ny, qm x) {
  const int nv = h->L.nv - 1;
  if (nv == 0) return;
  const qm z0 = y[ny - nv];
  h->corr = q_mul(h->corr, eq1(x, z0));
  h->L = fix_first(&h->L, x);
}

/* columns of the constant oracle (try_into_mask): 2 values each */
static int oracle_mask(const oracle_t* h, qm cols[4], int* ncols) {
  const layer_t* L = &h->L;
  if (L->nv != 1) return 1;
  if (L->kind == L_GP) {
    cols[0] = L->den[0];
    cols[1] = L->den[1];
    *ncols = 1;
  } else if (L->kind == L_MULT) {
    return 2; /* unimplemented!() in the reference */
  } else {
    cols[0] = lnum(L, 0);
    cols[1] = lnum(L, 1);
    cols[2] = L->den[0];
    cols[3] = L->den[1];
    *ncols = 2;
  }
  return 0;
}

static qm draw(orc_channel* ch) {
  uint32_t w[4];
  orc_draw_qm31(ch, w);
  return q_load(w);
}
static void mix_q(orc_channel* ch, const qm* v, size_t n) {
  uint32_t* w = (uint32_t*)malloc((n ? n : 1) * 16);
  for (size_t i = 0; i < n; i++) q_store(w + 4 * i, v[i]);
  orc_mix_felts_stwo(ch, w, n);
  free(w);
}
/* random_linear_combination: v0 + a v1 + ... (Horner) */
static qm rlc(const qm* v, int n, qm a) {
  qm acc = q_zero();
  for (int i = n - 1; i >= 0; i--) acc = q_add(q_mul(acc, a), v[i]);
  return acc;
}

int orc_prove_lookup_batch(orc_channel* ch, const orc_lookup_layer* inst, size_t n_inst, orc_lookup_out* out) {
  if (n_inst == 0) return 1;
  int n_layers = 0;
  for (size_t i = 0; i < n_inst; i++) {
    if (inst[i].n_vars < 1 || inst[i].n_vars > 26 || inst[i].kind > 3) return 1;
    if (inst[i].kind == L_MULT && inst[i].n_vars == 1) return 1;
    if ((int)inst[i].n_vars > n_layers) n_layers = (int)inst[i].n_vars;
  }
  /* gen_layers: layers[i][k] holds the layer with k variables */
  layer_t** layers = (layer_t**)calloc(n_inst, sizeof(layer_t*));
  for (size_t i = 0; i < n_inst; i++) {
    const int nv = (int)inst[i].n_vars;
    const size_t n = (size_t)1 << nv;
    layers[i] = (layer_t*)calloc((size_t)nv + 1, sizeof(layer_t));
    layer_t* top = &layers[i][nv];
    top->kind = (int)inst[i].kind;
    top->nv = nv;
    top->den = (qm*)malloc(n * sizeof(qm));
    for (size_t j = 0; j < n; j++) top->den[j] = q_load(inst[i].den + 4 * j);
    if (top->kind == L_GEN) {
      top->num = (qm*)malloc(n * sizeof(qm));
      for (size_t j = 0; j < n; j++) top->num[j] = q_load(inst[i].num + 4 * j);
    } else if (top->kind == L_MULT) {
      top->nm = (uint32_t*)malloc(n * sizeof(uint32_t));
      for (size_t j = 0; j < n; j++) top->nm[j] = m31_from(inst[i].num[j]);
    }
    for (int k = nv - 1; k >= 0; k--) layers[i][k] = next_layer(&layers[i][k + 1]);
  }
  qm* claims = (qm*)calloc(2 * n_inst, sizeof(qm));
  int* n_claims = (int*)calloc(n_inst, sizeof(int));
  qm* ood = (qm*)calloc((size_t)n_layers + 1, sizeof(qm));
  int n_ood = 0;
  size_t round = 0;
  int rc = 0;
  memset(out->masks, 0, (size_t)n_layers * n_inst * 16 * sizeof(uint32_t));
  for (int layer = 0; layer < n_layers && !rc; layer++) {
    const int n_rem = n_layers - layer;
    for (size_t i = 0; i < n_inst; i++)
      if ((int)inst[i].n_vars == n_rem) {
        const layer_t* o = &layers[i][0];
        if (o->kind == L_GP) {
          claims[2 * i] = o->den[0];
          n_claims[i] = 1;
        } else {
          claims[2 * i] = lnum(o, 0);
          claims[2 * i + 1] = o->den[0];
          n_claims[i] = 2;
        }
        for (int c = 0; c < 2; c++) q_store(out->output_claims + 8 * i + 4 * c, c < n_claims[i] ? claims[2 * i + c] : q_zero());
      }
    for (size_t i = 0; i < n_inst; i++)
      if (n_claims[i]) mix_q(ch, claims + 2 * i, (size_t)n_claims[i]);
    /* EqEvals::generate(ood): eq((0, x), y) over x in {0,1}^(|y| - 1) */
    const size_t n_eq = n_ood ? (size_t)1 << (n_ood - 1) : 1;
    qm* eq_evals = (qm*)malloc(n_eq * sizeof(qm));
    if (n_ood == 0)
      eq_evals[0] = q_one();
    else
      gen_eq_evals(ood + 1, n_ood - 1, eq1(q_zero(), ood[0]), eq_evals);
    const qm alpha = draw(ch), lambda = draw(ch);
    /* the oracles of the active instances, in instance order */
    oracle_t* orc = (oracle_t*)calloc(n_inst, sizeof(oracle_t));
    size_t* who = (size_t*)calloc(n_inst, sizeof(size_t));
    qm* sc = (qm*)calloc(n_inst, sizeof(qm));
    size_t na = 0;
    for (size_t i = 0; i < n_inst; i++)
      if (n_claims[i]) {
        const int lv = layer - (n_layers - (int)inst[i].n_vars) + 1; /* variables of the layer consumed now */
        orc[na].L = layers[i][lv];
        memset(&layers[i][lv], 0, sizeof(layer_t)); /* the oracle owns it now */
        orc[na].corr = q_one();
        orc[na].lambda = lambda;
        sc[na] = rlc(claims + 2 * i, n_claims[i], lambda);
        who[na++] = i;
      }
    /* sumcheck::prove_batch */
    int nvars = 0;
    for (size_t a = 0; a < na; a++)
      if (orc[a].L.nv - 1 > nvars) nvars = orc[a].L.nv - 1;
    for (size_t a = 0; a < na; a++) {
      const int unused = nvars - (orc[a].L.nv - 1);
      sc[a] = q_mul(sc[a], q_m(1u << unused));
    }
    qm* assign = (qm*)calloc((size_t)nvars + 1, sizeof(qm));
    upoly* polys = (upoly*)calloc(na, sizeof(upoly));
    const qm inv2 = q_inv(q_m(2));
    for (int r = 0; r < nvars && !rc; r++) {
      const int n_rr = nvars - r;
      for (size_t a = 0; a < na && !rc; a++) {
        if (n_rr == orc[a].L.nv - 1) {
          if (sum_as_poly(&orc[a], eq_evals, ood, n_ood, sc[a], &polys[a])) rc = 3;
        } else {
          memset(&polys[a], 0, sizeof(upoly));
          polys[a].c[0] = q_mul(sc[a], inv2);
          polys[a].len = 1;
          up_trunc(&polys[a]);
        }
        if (!rc && !q_eq(q_add(up_eval(&polys[a], q_zero()), up_eval(&polys[a], q_one())), sc[a])) rc = 4;
      }
      if (rc) break;
      /* random_linear_combination of the polynomials (sumcheck.rs:134-141): rfold, lengths kept */
      upoly comb;
      memset(&comb, 0, sizeof comb);
      for (size_t a = na; a-- > 0;) {
        for (int k = 0; k < comb.len; k++) comb.c[k] = q_mul(comb.c[k], alpha);
        const int len = polys[a].len > comb.len ? polys[a].len : comb.len;
        for (int k = 0; k < len; k++) {
          const qm x = k < comb.len ? comb.c[k] : q_zero();
          const qm yv = k < polys[a].len ? polys[a].c[k] : q_zero();
          comb.c[k] = q_add(x, yv);
        }
        comb.len = len;
      }
      mix_q(ch, comb.c, (size_t)comb.len);
      const qm x = draw(ch);
      for (int k = 0; k < 4; k++) q_store(out->round_polys + 16 * round + 4 * k, k < comb.len ? comb.c[k] : q_zero());
      out->round_poly_lens[round] = (uint32_t)comb.len;
      round++;
      for (size_t a = 0; a < na; a++) sc[a] = up_eval(&polys[a], x);
      for (size_t a = 0; a < na; a++)
        if (n_rr == orc[a].L.nv - 1) oracle_fix(&orc[a], ood, n_ood, x);
      assign[r] = x;
    }
    /* masks, mixed in instance order */
    for (size_t a = 0; a < na && !rc; a++) {
      qm cols[4];
      int ncol = 0;
      if (oracle_mask(&orc[a], cols, &ncol)) {
        rc = 5;
        break;
      }
      mix_q(ch, cols, (size_t)(2 * ncol));
      for (int c = 0; c < 2 * ncol; c++) q_store(out->masks + 16 * ((size_t)layer * n_inst + who[a]) + 4 * c, cols[c]);
      /* claims for the layer above: reduce_at_point, after the challenge */
    }
    if (!rc) {
      const qm c = draw(ch);
      for (int r = 0; r < nvars; r++) ood[r] = assign[r];
      ood[nvars] = c;
      n_ood = nvars + 1;
      for (size_t a = 0; a < na; a++) {
        qm cols[4];
        int ncol = 0;
        oracle_mask(&orc[a], cols, &ncol);
        const size_t i = who[a];
        for (int k = 0; k < ncol; k++) claims[2 * i + k] = q_add(cols[2 * k], q_mul(c, q_sub(cols[2 * k + 1], cols[2 * k])));
      }
    }
    for (size_t a = 0; a < na; a++) layer_free(&orc[a].L);
    free(orc);
    free(who);
    free(sc);
    free(assign);
    free(polys);
    free(eq_evals);
  }
  if (!rc) {
    out->n_layers = (uint32_t)n_layers;
    for (int k = 0; k < n_ood; k++) q_store(out->ood_point + 4 * k, ood[k]);
    for (size_t i = 0; i < n_inst; i++)
      for (int c = 0; c < 2; c++)
        q_store(out->claims_to_verify + 8 * i + 4 * c, c < n_claims[i] ? claims[2 * i + c] : q_zero());
  }
  for (size_t i = 0; i < n_inst; i++) {
    for (int k = 0; k <= (int)inst[i].n_vars; k++) layer_free(&layers[i][k]);
    free(layers[i]);
  }
  free(layers);
  free(claims);
  free(n_claims);
  free(ood);
  return rc;
}

/* partially_verify_batch (gkr_verifier.rs:17-157).  gates: 0 grand product,
 * 1 LogUp.  Returns 0 and the artifact, or a nonzero code naming the check. */
int orc_verify_lookup_batch(const uint32_t* gates, const uint32_t* n_vars, size_t n_inst, const orc_lookup_out* p,
                            orc_channel* ch, uint32_t* ood_out, uint32_t* claims_out) {
  int n_layers = 0;
  for (size_t i = 0; i < n_inst; i++)
    if ((int)n_vars[i] > n_layers) n_layers = (int)n_vars[i];
  if (n_inst == 0 || (uint32_t)n_layers != p->n_layers) return 1;
  qm* claims = (qm*)calloc(2 * n_inst, sizeof(qm));
  int* n_claims = (int*)calloc(n_inst, sizeof(int));
  qm* ood = (qm*)calloc((size_t)n_layers + 1, sizeof(qm));
  int n_ood = 0, rc = 0;
  size_t round = 0;
  for (int layer = 0; layer < n_layers && !rc; layer++) {
    const int n_rem = n_layers - layer;
    for (size_t i = 0; i < n_inst; i++)
      if ((int)n_vars[i] == n_rem) {
        n_claims[i] = gates[i] == 0 ? 1 : 2;
        for (int c = 0; c < n_claims[i]; c++) claims[2 * i + c] = q_load(p->output_claims + 8 * i + 4 * c);
      }
    for (size_t i = 0; i < n_inst; i++)
      if (n_claims[i]) mix_q(ch, claims + 2 * i, (size_t)n_claims[i]);
    const qm alpha = draw(ch), lambda = draw(ch);
    qm sum = q_zero();
    {
      qm* cl = (qm*)calloc(n_inst, sizeof(qm));
      int nc = 0;
      for (size_t i = 0; i < n_inst; i++)
        if (n_claims[i]) {
          const int unused = n_layers - (int)n_vars[i];
          cl[nc++] = q_mul(rlc(claims + 2 * i, n_claims[i], lambda), q_m(1u << unused));
        }
      sum = rlc(cl, nc, alpha);
      free(cl);
    }
    /* sumcheck::partially_verify over `layer` rounds */
    qm* pt = (qm*)calloc((size_t)layer + 1, sizeof(qm));
    for (int r = 0; r < layer; r++, round++) {
      upoly q;
      memset(&q, 0, sizeof q);
      q.len = (int)p->round_poly_lens[round];
      if (q.len > 4) {
        rc = 2;
        break;
      }
      for (int k = 0; k < q.len; k++) q.c[k] = q_load(p->round_polys + 16 * round + 4 * k);
      if (!q_eq(q_add(up_eval(&q, q_zero()), up_eval(&q, q_one())), sum)) {
        rc = 3;
        break;
      }
      mix_q(ch, q.c, (size_t)q.len);
      pt[r] = draw(ch);
      sum = up_eval(&q, pt[r]);
    }
    if (rc) {
      free(pt);
      break;
    }
    /* the circuit at the sumcheck point */
    qm* evals = (qm*)calloc(n_inst, sizeof(qm));
    int ne = 0;
    for (size_t i = 0; i < n_inst; i++)
      if (n_claims[i]) {
        const int unused = n_layers - (int)n_vars[i];
        const uint32_t* m = p->masks + 16 * ((size_t)layer * n_inst + i);
        qm out2[2];
        int no;
        if (gates[i] == 0) {
          out2[0] = q_mul(q_load(m), q_load(m + 4));
          no = 1;
        } else {
          const qm na = q_load(m), nb = q_load(m + 4), da = q_load(m + 8), db = q_load(m + 12);
          out2[0] = q_add(q_mul(na, db), q_mul(nb, da));
          out2[1] = q_mul(da, db);
          no = 2;
        }
        qm e = q_one();
        for (int k = unused; k < layer; k++) e = q_mul(e, eq1(ood[k], pt[k]));
        evals[ne++] = q_mul(e, rlc(out2, no, lambda));
      }
    const qm layer_eval = rlc(evals, ne, alpha);
    free(evals);
    if (!q_eq(layer_eval, sum)) {
      free(pt);
      rc = 4;
      break;
    }
    for (size_t i = 0; i < n_inst; i++)
      if (n_claims[i]) {
        const uint32_t* m = p->masks + 16 * ((size_t)layer * n_inst + i);
        qm v[4];
        const int nv = gates[i] == 0 ? 2 : 4;
        for (int k = 0; k < nv; k++) v[k] = q_load(m + 4 * k);
        mix_q(ch, v, (size_t)nv);
      }
    const qm c = draw(ch);
    for (int r = 0; r < layer; r++) ood[r] = pt[r];
    ood[layer] = c;
    n_ood = layer + 1;
    free(pt);
    for (size_t i = 0; i < n_inst; i++)
      if (n_claims[i]) {
        const uint32_t* m = p->masks + 16 * ((size_t)layer * n_inst + i);
        for (int k = 0; k < n_claims[i]; k++) {
          const qm v0 = q_load(m + 8 * k), v1 = q_load(m + 8 * k + 4);
          claims[2 * i + k] = q_add(v0, q_mul(c, q_sub(v1, v0)));
        }
      }
  }
  if (!rc) {
    for (int k = 0; k < n_ood; k++) q_store(ood_out + 4 * k, ood[k]);
    for (size_t i = 0; i < n_inst; i++)
      for (int c = 0; c < 2; c++) q_store(claims_out + 8 * i + 4 * c, c < n_claims[i] ? claims[2 * i + c] : q_zero());
  }
  free(claims);
  free(n_claims);
  free(ood);
  return rc;
}
