/* Starknet Poseidon and the GKR Poseidon channel, restated for the oracle.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 *  - round constants: sha256("Hades<idx>") mod p, the published derivation of
 *    StarkWare's poseidon3.txt that engine/src/crypto/poseidon_constants.rs
 *    embeds (computed here at first use with a FIPS 180-4 SHA-256)
 *  - permutation: the compressed form of engine/src/recursive/hades_air.rs:
 *    1137-1180 (constant compression) and 1892-2012 (4 full, 83 partial,
 *    4 full rounds, x^3, MDS t+2s0 / t-2s1 / t-3s2)
 *  - sponge: poseidon_hash_many, stwo-gpu/.../backend/gpu/fft.rs:2543-2572
 *  - channel: engine/src/crypto/poseidon_channel.rs:83-308
 * felt252 products use separated-operand-scanning Montgomery reduction with
 * the generic limbs of p = 2^251 + 17*2^192 + 1.
 */
#include <pthread.h>
#include <stdio.h>

#include "oracle_internal.h"

typedef unsigned __int128 u128;
static const uint64_t FP[4] = {1ull, 0ull, 0ull, 0x0800000000000011ull};

static int fe_geq_p(const uint64_t* t) {
  for (int i = 3; i >= 0; i--) {
    if (t[i] != FP[i]) return t[i] > FP[i];
  }
  return 1;
}
static void fe_sub_p(uint64_t* t) {
  uint64_t br = 0;
  for (int i = 0; i < 4; i++) {
    u128 d = (u128)t[i] - FP[i] - br;
    t[i] = (uint64_t)d;
    br = (uint64_t)(d >> 127);
  }
}
static fe fe_add(fe a, fe b) {
  fe r;
  uint64_t c = 0;
  for (int i = 0; i < 4; i++) {
    u128 s = (u128)a.v[i] + b.v[i] + c;
    r.v[i] = (uint64_t)s;
    c = (uint64_t)(s >> 64);
  }
  if (fe_geq_p(r.v)) fe_sub_p(r.v);
  return r;
}
static fe fe_sub(fe a, fe b) {
  fe r;
  uint64_t br = 0;
  for (int i = 0; i < 4; i++) {
    u128 d = (u128)a.v[i] - b.v[i] - br;
    r.v[i] = (uint64_t)d;
    br = (uint64_t)(d >> 127);
  }
  if (br) {
    uint64_t c = 0;
    for (int i = 0; i < 4; i++) {
      u128 s = (u128)r.v[i] + FP[i] + c;
      r.v[i] = (uint64_t)s;
      c = (uint64_t)(s >> 64);
    }
  }
  return r;
}
/* SOS: full 512-bit product, then four word-by-word Montgomery steps. */
static fe fe_mul(fe a, fe b) {
  uint64_t t[9] = {0};
  for (int i = 0; i < 4; i++) {
    uint64_t c = 0;
    for (int j = 0; j < 4; j++) {
      u128 x = (u128)a.v[i] * b.v[j] + t[i + j] + c;
      t[i + j] = (uint64_t)x;
      c = (uint64_t)(x >> 64);
    }
    t[i + 4] = c;
  }
  const uint64_t ninv = 0xffffffffffffffffull; /* -p^-1 mod 2^64 (p = 1 mod 2^64) */
  for (int i = 0; i < 4; i++) {
    uint64_t m = t[i] * ninv;
    uint64_t c = 0;
    for (int j = 0; j < 4; j++) {
      u128 x = (u128)m * FP[j] + t[i + j] + c;
      t[i + j] = (uint64_t)x;
      c = (uint64_t)(x >> 64);
    }
    for (int j = i + 4; j < 9 && c; j++) {
      u128 x = (u128)t[j] + c;
      t[j] = (uint64_t)x;
      c = (uint64_t)(x >> 64);
    }
  }
  fe r = {{t[4], t[5], t[6], t[7]}};
  if (t[8] || fe_geq_p(r.v)) fe_sub_p(r.v);
  return r;
}

static fe R2;      /* 2^512 mod p */
static fe ONE_M;   /* Montgomery 1 */
static fe COMP[107];
static pthread_once_t once = PTHREAD_ONCE_INIT;

static fe fe_canon_to_mont(const uint64_t c[4]) {
  fe x = {{c[0], c[1], c[2], c[3]}};
  return fe_mul(x, R2);
}
static void fe_mont_to_canon(fe x, uint64_t c[4]) {
  fe one = {{1, 0, 0, 0}};
  fe r = fe_mul(x, one);
  memcpy(c, r.v, 32);
}

/* ---------------------------------------------------------------- SHA-256 */
static const uint32_t K256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
#define ROTR(x, n) (((x) >> (n)) | ((x) << (32 - (n))))
static void sha256_block(uint32_t h[8], const uint8_t* b) {
  uint32_t w[64];
  for (int i = 0; i < 16; i++)
    w[i] = ((uint32_t)b[4 * i] << 24) | ((uint32_t)b[4 * i + 1] << 16) | ((uint32_t)b[4 * i + 2] << 8) | b[4 * i + 3];
  for (int i = 16; i < 64; i++) {
    uint32_t s0 = ROTR(w[i - 15], 7) ^ ROTR(w[i - 15], 18) ^ (w[i - 15] >> 3);
    uint32_t s1 = ROTR(w[i - 2], 17) ^ ROTR(w[i - 2], 19) ^ (w[i - 2] >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t a = h[0], bb = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
  for (int i = 0; i < 64; i++) {
    uint32_t S1 = ROTR(e, 6) ^ ROTR(e, 11) ^ ROTR(e, 25);
    uint32_t ch = (e & f) ^ (~e & g);
    uint32_t t1 = hh + S1 + ch + K256[i] + w[i];
    uint32_t S0 = ROTR(a, 2) ^ ROTR(a, 13) ^ ROTR(a, 22);
    uint32_t mj = (a & bb) ^ (a & c) ^ (bb & c);
    uint32_t t2 = S0 + mj;
    hh = g; g = f; f = e; e = d + t1; d = c; c = bb; bb = a; a = t1 + t2;
  }
  h[0] += a; h[1] += bb; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}
void orc_sha256(const uint8_t* msg, size_t len, uint8_t out[32]) {
  uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
  size_t i = 0;
  for (; i + 64 <= len; i += 64) sha256_block(h, msg + i);
  uint8_t tail[128] = {0};
  size_t rem = len - i;
  memcpy(tail, msg + i, rem);
  tail[rem] = 0x80;
  size_t tl = (rem + 9 <= 64) ? 64 : 128;
  uint64_t bits = (uint64_t)len * 8;
  for (int k = 0; k < 8; k++) tail[tl - 1 - k] = (uint8_t)(bits >> (8 * k));
  sha256_block(h, tail);
  if (tl == 128) sha256_block(h, tail + 64);
  for (int k = 0; k < 8; k++) {
    out[4 * k] = (uint8_t)(h[k] >> 24);
    out[4 * k + 1] = (uint8_t)(h[k] >> 16);
    out[4 * k + 2] = (uint8_t)(h[k] >> 8);
    out[4 * k + 3] = (uint8_t)h[k];
  }
}

/* raw constant idx = int(sha256("Hades<idx>"), big endian) mod p, canonical limbs */
static void raw_constant(int idx, uint64_t c[4]) {
  char msg[32];
  int len = snprintf(msg, sizeof msg, "Hades%d", idx);
  uint8_t d[32];
  orc_sha256((const uint8_t*)msg, (size_t)len, d);
  for (int l = 0; l < 4; l++) {
    uint64_t v = 0;
    for (int k = 0; k < 8; k++) v = (v << 8) | d[(3 - l) * 8 + k];
    c[l] = v;
  }
  while (fe_geq_p(c)) fe_sub_p(c); /* value < 2^256 < 32 p */
}
void orc_hades_constant(int idx, uint32_t out[8]) {
  uint64_t c[4];
  raw_constant(idx, c);
  for (int l = 0; l < 4; l++) {
    out[2 * l] = (uint32_t)c[l];
    out[2 * l + 1] = (uint32_t)(c[l] >> 32);
  }
}

static void mds(fe s[3]) {
  fe t = fe_add(fe_add(s[0], s[1]), s[2]);
  fe n0 = fe_add(t, fe_add(s[0], s[0]));
  fe n1 = fe_sub(t, fe_add(s[1], s[1]));
  fe n2 = fe_sub(t, fe_add(fe_add(s[2], s[2]), s[2]));
  s[0] = n0; s[1] = n1; s[2] = n2;
}

static void init_once(void) {
  fe x = {{1, 0, 0, 0}};
  for (int i = 0; i < 512; i++) x = fe_add(x, x); /* canonical doubling: 2^512 mod p */
  R2 = x;
  uint64_t one[4] = {1, 0, 0, 0};
  ONE_M = fe_canon_to_mont(one);
  /* constant compression (hades_air.rs:1137-1180) */
  fe raw[91][3];
  for (int r = 0; r < 91; r++)
    for (int j = 0; j < 3; j++) {
      uint64_t c[4];
      raw_constant(3 * r + j, c);
      raw[r][j] = fe_canon_to_mont(c);
    }
  int k = 0;
  for (int r = 0; r < 4; r++)
    for (int j = 0; j < 3; j++) COMP[k++] = raw[r][j];
  fe st[3] = {{{0}}, {{0}}, {{0}}};
  int idx = 4;
  for (int r = 0; r < 83; r++, idx++) {
    for (int j = 0; j < 3; j++) st[j] = fe_add(st[j], raw[idx][j]);
    COMP[k++] = st[2];
    memset(&st[2], 0, sizeof(fe));
    mds(st);
  }
  for (int j = 0; j < 3; j++) st[j] = fe_add(st[j], raw[idx][j]);
  COMP[k++] = st[0];
  COMP[k++] = st[1];
  COMP[k++] = st[2];
  idx++;
  for (; idx < 91; idx++)
    for (int j = 0; j < 3; j++) COMP[k++] = raw[idx][j];
}
static void ensure_init(void) { pthread_once(&once, init_once); }

static fe cube(fe x) { return fe_mul(fe_mul(x, x), x); }
static void hades(fe s[3]) {
  int idx = 0;
  for (int r = 0; r < 4; r++, idx += 3) {
    for (int j = 0; j < 3; j++) s[j] = cube(fe_add(s[j], COMP[idx + j]));
    mds(s);
  }
  for (int r = 0; r < 83; r++, idx++) {
    s[2] = cube(fe_add(s[2], COMP[idx]));
    mds(s);
  }
  for (int r = 0; r < 4; r++, idx += 3) {
    for (int j = 0; j < 3; j++) s[j] = cube(fe_add(s[j], COMP[idx + j]));
    mds(s);
  }
}

/* poseidon_hash(a, b) = hades([a, b, 2])[0] */
fe fe_hash2(fe a, fe b) {
  ensure_init();
  fe s[3] = {a, b, fe_from_u64(2)};
  hades(s);
  return s[0];
}
fe fe_from_u64(uint64_t x) {
  ensure_init();
  uint64_t c[4] = {x, 0, 0, 0};
  return fe_canon_to_mont(c);
}
fe fe_from_words(const uint32_t w[8]) {
  ensure_init();
  uint64_t c[4];
  for (int l = 0; l < 4; l++) c[l] = (uint64_t)w[2 * l] | ((uint64_t)w[2 * l + 1] << 32);
  return fe_canon_to_mont(c);
}
void fe_to_words(fe x, uint32_t w[8]) {
  uint64_t c[4];
  fe_mont_to_canon(x, c);
  for (int l = 0; l < 4; l++) {
    w[2 * l] = (uint32_t)c[l];
    w[2 * l + 1] = (uint32_t)(c[l] >> 32);
  }
}

void orc_hades(uint32_t state[24]) {
  ensure_init();
  fe s[3];
  for (int i = 0; i < 3; i++) s[i] = fe_from_words(state + 8 * i);
  hades(s);
  for (int i = 0; i < 3; i++) fe_to_words(s[i], state + 8 * i);
}

fe fe_hash_many(const fe* in, size_t n) {
  ensure_init();
  fe s[3];
  memset(s, 0, sizeof s);
  size_t i = 0;
  while (i < n) {
    s[0] = fe_add(s[0], in[i]);
    i++;
    if (i < n) {
      s[1] = fe_add(s[1], in[i]);
      i++;
    } else {
      s[1] = fe_add(s[1], ONE_M);
      hades(s);
      return s[0];
    }
    hades(s);
  }
  s[0] = fe_add(s[0], ONE_M);
  hades(s);
  return s[0];
}
void orc_hash_many(const uint32_t* felts, size_t n, uint32_t out[8]) {
  fe* v = (fe*)malloc((n ? n : 1) * sizeof(fe));
  for (size_t i = 0; i < n; i++) v[i] = fe_from_words(felts + 8 * i);
  fe_to_words(fe_hash_many(v, n), out);
  free(v);
}

/* pack_m31s (poseidon_channel.rs:22-29): acc = 1; acc = acc * 2^31 + v, in the field */
fe fe_pack_m31s(const uint32_t* v, int n) {
  fe acc = fe_from_u64(1);
  const fe shift = fe_from_u64(1ull << 31);
  for (int i = 0; i < n; i++) acc = fe_add(fe_mul(acc, shift), fe_from_u64(v[i]));
  return acc;
}

/* ---------------------------------------------------------------- channel */
size_t orc_channel_size(void) { return sizeof(orc_channel); }
static fe ch_digest(const orc_channel* ch) { fe d; memcpy(d.v, ch->digest, 32); return d; }
static void ch_set(orc_channel* ch, fe d) {
  memcpy(ch->digest, d.v, 32);
  ch->n_draws = 0;
  ch->hash_count++;
}
void orc_channel_init(orc_channel* ch) {
  ensure_init();
  memset(ch, 0, sizeof *ch); /* digest 0 is 0 in Montgomery form too */
}
/* mix_felt: state = [digest, v, 2]; hades; digest = state[0] (poseidon_channel.rs:145-151) */
static void mix_fe(orc_channel* ch, fe v) {
  fe s[3] = {ch_digest(ch), v, fe_from_u64(2)};
  hades(s);
  ch_set(ch, s[0]);
}
void orc_mix_u64(orc_channel* ch, uint64_t v) { mix_fe(ch, fe_from_u64(v)); }
void orc_mix_felt(orc_channel* ch, const uint32_t w[8]) { mix_fe(ch, fe_from_words(w)); }
void orc_mix_secure_field(orc_channel* ch, const uint32_t q[4]) { mix_fe(ch, fe_pack_m31s(q, 4)); }
/* mix_poly_coeffs (poseidon_channel.rs:213-226) */
void orc_mix_poly_coeffs(orc_channel* ch, const uint32_t c[12]) {
  fe in[3] = {ch_digest(ch), fe_pack_m31s(c, 8), fe_pack_m31s(c + 8, 4)};
  ch_set(ch, fe_hash_many(in, 3));
}
void orc_mix_poly_coeffs_deg3(orc_channel* ch, const uint32_t c[16]) {
  fe in[3] = {ch_digest(ch), fe_pack_m31s(c, 8), fe_pack_m31s(c + 8, 8)};
  ch_set(ch, fe_hash_many(in, 3));
}
/* mix_felts (poseidon_channel.rs:261-297) */
void orc_mix_felts(orc_channel* ch, const uint32_t* q, size_t n) {
  if (n == 0) return;
  fe* in = (fe*)malloc((2 + n / 2 + 1) * sizeof(fe));
  size_t m = 0;
  in[m++] = ch_digest(ch);
  for (size_t i = 0; i < n;) {
    if (n - i >= 2) {
      in[m++] = fe_pack_m31s(q + 4 * i, 8);
      i += 2;
    } else {
      in[m++] = fe_pack_m31s(q + 4 * i, 4);
      i += 1;
    }
  }
  ch_set(ch, fe_hash_many(in, m));
  free(in);
}
/* Poseidon252Channel::mix_felts (stwo core/channel/poseidon252.rs:70-84), the
 * channel of STWO's LogUp-GKR batch: as orc_mix_felts, except that an empty
 * slice still hashes [digest] (poseidon_hash_many of one felt) and resets n_draws. */
void orc_mix_felts_stwo(orc_channel* ch, const uint32_t* q, size_t n) {
  if (n) {
    orc_mix_felts(ch, q, n);
    return;
  }
  fe in[1] = {ch_digest(ch)};
  ch_set(ch, fe_hash_many(in, 1));
}
/* Transcript trace (test infrastructure): with ORACLE_CHANNEL_TRACE set to a
 * path (or "-" for stderr), appends "<label>[ <index>] 0x<digest> <n_draws>"
 * at the points where the product traces under GKR_CHANNEL_TRACE, so the two
 * traces can be compared line by line.  The reference prints its channel at
 * such points under STWO_CHANNEL_TRACE (gkr/prover.rs:1523-1541, 6002-6012). */
void orc_trace(const orc_channel* ch, const char* label, long index) {
  const char* path = getenv("ORACLE_CHANNEL_TRACE");
  if (!path || !*path) return;
  uint32_t d[8];
  orc_digest(ch, d);
  FILE* f = strcmp(path, "-") == 0 ? stderr : fopen(path, "a");
  if (!f) return;
  if (index >= 0)
    fprintf(f, "%s %ld 0x", label, index);
  else
    fprintf(f, "%s 0x", label);
  for (int w = 7; w >= 0; w--) fprintf(f, "%08x", d[w]);
  fprintf(f, " %u\n", ch->n_draws);
  if (f != stderr) fclose(f);
}
/* draw_felt252: [digest, n_draws, 3] (poseidon_channel.rs:156-166) */
static fe draw_fe(orc_channel* ch) {
  fe s[3] = {ch_digest(ch), fe_from_u64(ch->n_draws), fe_from_u64(3)};
  hades(s);
  ch->n_draws++;
  ch->hash_count++;
  return s[0];
}
void orc_draw_felt252(orc_channel* ch, uint32_t out[8]) { fe_to_words(draw_fe(ch), out); }
/* draw_qm31: successive floor_div by 2^31, remainder mod P (poseidon_channel.rs:176-200) */
void orc_draw_qm31(orc_channel* ch, uint32_t out[4]) {
  uint64_t c[4];
  fe_mont_to_canon(draw_fe(ch), c);
  for (int k = 0; k < 4; k++) {
    uint64_t rem = c[0] & 0x7fffffffull;
    /* cur = cur >> 31 */
    c[0] = (c[0] >> 31) | (c[1] << 33);
    c[1] = (c[1] >> 31) | (c[2] << 33);
    c[2] = (c[2] >> 31) | (c[3] << 33);
    c[3] = c[3] >> 31;
    out[k] = (uint32_t)(rem % ORC_P);
  }
}
void orc_draw_qm31s(orc_channel* ch, size_t n, uint32_t* out) {
  for (size_t i = 0; i < n; i++) orc_draw_qm31(ch, out + 4 * i);
}
void orc_digest(const orc_channel* ch, uint32_t out[8]) { fe_to_words(ch_digest(ch), out); }
/* Channel state in the to_gpu_state layout (poseidon_channel.rs:109-135): 8 LE words of the
 * canonical digest, n_draws, hash_count lo, hash_count hi. */
void orc_channel_set_state(orc_channel* ch, const uint32_t st[11]) {
  ensure_init();
  const fe d = fe_from_words(st);
  memcpy(ch->digest, d.v, 32);
  ch->n_draws = st[8];
  ch->hash_count = (uint64_t)st[9] | ((uint64_t)st[10] << 32);
}
