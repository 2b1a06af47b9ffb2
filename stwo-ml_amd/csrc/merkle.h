// Poseidon Merkle roots of MLE commitments on the GPU.
//
// Tree (engine/src/crypto/poseidon_merkle.rs:255-280, root_only_parallel):
// leaves padded with FieldElement::ZERO to a power of two (at least 2),
// node = poseidon_hash(left, right).  Leaves are securefield_to_felt(v) =
// 1 || a || b || c || d in 31-bit fields (poseidon_channel.rs:59-69).
//
// Three leaf sources:
//   kind 0, a weight matrix B (rows x cols, row-major M31): the leaves are
//     matrix_to_mle_col_major_padded(B) (prover.rs:1021-1023), i.e. B[i][j]
//     at index j * pk + i of a pk x pn grid (next powers of two); grid cells
//     outside B hold SecureField ZERO, whose leaf is 2^124;
//   kind 1, n QM31 values (commit_mle_root_only, mle_opening.rs:630-641);
//   kind 2, a QM31 grid stored column-major with pk rows per column, of which
//     the first `rows` can be non-zero, `cols` columns (the folded layers of a
//     weight opening): kind 0's tree with QM31 leaves read from the grid.
//
// Only nodes whose subtree touches a real leaf are hashed and stored.  A
// subtree made only of grid padding (kind 0) has the value z[s] =
// H(z[s-1], z[s-1]) with z[0] = 2^124, one made only of tree padding has
// zz[s] with zz[0] = 0; both come from a table built on the host.  The root
// is the same as hashing every node.
//
// Storage of the real nodes of level s (at most the real leaf count / 2^s):
//   kind 0 with 2^s <= pk: node (column j, row block b), b < rb_s =
//     ceil(rows / 2^s), at j * rb_s + b; its index in the level is
//     (j << (log_pk - s)) + b;
//   kind 0 with 2^s > pk, and kind 1: the level index itself.
// One launch advances every tree of a batch from level s to s + d (d <= 4):
// a thread owns one output node and reduces its 2^d children depth-first,
// keeping pending left nodes in LDS.
#pragma once
#include <stdint.h>

#include "field.h"
#include "poseidon9.h"

namespace gkr {

struct MerkleConsts {
  f9::hades_consts hk;
  f9::fe r2;      // 2^522 mod p: canonical -> Montgomery
  f9::fe one;     // plain 1: Montgomery -> representative of the value
  f9::fe z[64];   // grid padding subtrees, Montgomery
  f9::fe zz[64];  // tree padding subtrees, Montgomery
};

// One tree's part of one level launch.
struct MerkleStep {
  const uint32_t* src;  // s == 0: the matrix (kind 0) or the QM31 words (kinds 1, 2)
  const f9::fe* in;     // s > 0: the real nodes of level s
  f9::fe* out;          // the real nodes of level s + d
  uint64_t rows, cols;  // kinds 0, 2: grid shape (real rows, columns); kind 1: rows = number of values
  uint64_t mle_len;     // leaves at index >= mle_len are tree padding
  uint64_t thread_begin;  // first thread of this tree in the launch
  uint64_t n_out;         // real nodes of level s + d
  uint32_t kind, log_pk, d, pad_;
};

// A tree whose levels are all kept (weight openings): real nodes of level s
// at level[s] (s >= 1); level 0 is read from src.
constexpr int kMerkleMaxHeight = 48;
struct MerkleKept {
  const uint32_t* src;
  uint64_t rows, cols, mle_len;
  uint32_t kind, log_pk, height, pad_;
  const f9::fe* level[kMerkleMaxHeight + 1];
};

__host__ __device__ inline uint64_t ceil_shr(uint64_t x, uint32_t s) { return s >= 64 ? (x != 0) : (x + (1ull << s) - 1) >> s; }

// Real nodes at level s.
__host__ __device__ inline uint64_t merkle_real_count(uint32_t kind, uint64_t rows, uint64_t cols, uint32_t log_pk,
                                                      uint32_t s) {
  if (kind == 1) return ceil_shr(rows, s);  // kinds 0 and 2 share the grid layout
  if (s <= log_pk) return cols * ceil_shr(rows, s);
  return ceil_shr(cols, s - log_pk);
}

// securefield_to_felt(a, b, c, d) as limbs (not Montgomery).
__device__ __forceinline__ void merkle_leaf_limbs(uint32_t a, uint32_t b, uint32_t c, uint32_t d, f9::fe& r) {
  uint32_t w[8];
  w[0] = d | (c << 31);
  w[1] = (c >> 1) | (b << 30);
  w[2] = (b >> 2) | (a << 29);
  w[3] = (a >> 3) | (1u << 28);
  w[4] = w[5] = w[6] = w[7] = 0;
  f9::from_words(w, r);
}

__device__ __forceinline__ void merkle_child(const MerkleStep& T, uint32_t s, uint64_t c, const MerkleConsts& C,
                                             f9::fe& v) {
  if ((c << s) >= T.mle_len) {
    v = C.zz[s];
    return;
  }
  if (T.kind == 1) {
    if (s == 0) {
      const uint4 q = *(const uint4*)(T.src + 4 * c);
      f9::fe x;
      merkle_leaf_limbs(q.x, q.y, q.z, q.w, x);
      f9::mul(x, C.r2, v);
    } else {
      v = T.in[c];
    }
    return;
  }
  if (s <= T.log_pk) {
    const uint32_t sh = T.log_pk - s;
    const uint64_t j = c >> sh, b = c & ((1ull << sh) - 1);
    const uint64_t rb = ceil_shr(T.rows, s);
    if (j >= T.cols || b >= rb) {
      v = C.z[s];
    } else if (s == 0) {
      f9::fe x;
      if (T.kind == 0) {
        merkle_leaf_limbs(T.src[b * T.cols + j], 0, 0, 0, x);
      } else {
        const uint4 q = *(const uint4*)(T.src + 4 * ((j << T.log_pk) + b));
        merkle_leaf_limbs(q.x, q.y, q.z, q.w, x);
      }
      f9::mul(x, C.r2, v);
    } else {
      v = T.in[j * rb + b];
    }
  } else {
    if (c >= ceil_shr(T.cols, s - T.log_pk))
      v = C.z[s];
    else
      v = T.in[c];
  }
}

constexpr int kMerkleBlock = 256;
constexpr int kMerkleMaxD = 4;

static __global__ void __launch_bounds__(kMerkleBlock) k_merkle_level(const MerkleStep* __restrict__ steps, int n_steps,
                                                               uint32_t s, uint64_t total,
                                                               const MerkleConsts* __restrict__ Cp) {
  __shared__ f9::fe stack[kMerkleMaxD][kMerkleBlock];
  const uint64_t g = (uint64_t)blockIdx.x * kMerkleBlock + threadIdx.x;
  if (g >= total) return;
  int lo = 0, hi = n_steps - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (steps[mid].thread_begin <= g)
      lo = mid;
    else
      hi = mid - 1;
  }
  const MerkleStep T = steps[lo];
  const MerkleConsts& C = *Cp;
  const uint64_t t = g - T.thread_begin;
  const uint32_t d = T.d, S = s + d;
  uint64_t slot, c0;
  if (T.kind != 1 && S <= T.log_pk) {  // grid trees (kinds 0 and 2)
    // consecutive threads take consecutive columns (coalesced leaf reads)
    const uint64_t b = t / T.cols, j = t - b * T.cols;
    slot = j * ceil_shr(T.rows, S) + b;
    c0 = (j << (T.log_pk - s)) + (b << d);
  } else {
    slot = t;
    c0 = t << d;
  }
  f9::fe v;
  for (uint32_t r = 0; r < (1u << d); r++) {
    merkle_child(T, s, c0 + r, C, v);
    uint32_t lvl = 0, rr = r;
    while (rr & 1) {
      const f9::fe left = stack[lvl][threadIdx.x];
      f9::hash2(left, v, C.hk, v);
      rr >>= 1;
      lvl++;
    }
    if (lvl < d) stack[lvl][threadIdx.x] = v;
  }
  T.out[slot] = v;
}

// Gather for opening proofs.  Item kinds: 0, the canonical felt of node c of
// level s of tree t (8 words); 1, value c of the layer behind tree t as QM31
// (4 words; kind 0 layers read the matrix, zero outside it).
struct MerkleGather {
  uint32_t tree, level, what, pad_;
  uint64_t index;
};

static __global__ void k_merkle_gather(const MerkleKept* __restrict__ trees, const MerkleGather* __restrict__ items, int n,
                                const MerkleConsts* __restrict__ Cp, uint32_t* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const MerkleGather it = items[i];
  const MerkleKept& K = trees[it.tree];
  uint32_t* o = out + 8 * (uint64_t)i;
  if (it.what == 1) {
    uint32_t q[4] = {0, 0, 0, 0};
    const uint64_t c = it.index;
    if (K.kind == 1) {
      for (int w = 0; w < 4; w++) q[w] = K.src[4 * c + w];
    } else {
      const uint64_t j = c >> K.log_pk, b = c & ((1ull << K.log_pk) - 1);
      if (j < K.cols && b < K.rows) {
        if (K.kind == 0)
          q[0] = K.src[b * K.cols + j];
        else
          for (int w = 0; w < 4; w++) q[w] = K.src[4 * c + w];
      }
    }
    for (int w = 0; w < 8; w++) o[w] = w < 4 ? q[w] : 0;
    return;
  }
  MerkleStep T{};
  T.src = K.src;
  T.in = K.level[it.level];
  T.rows = K.rows;
  T.cols = K.cols;
  T.mle_len = K.mle_len;
  T.kind = K.kind;
  T.log_pk = K.log_pk;
  f9::fe v, x;
  merkle_child(T, it.level, it.index, *Cp, v);
  f9::mul(v, Cp->one, x);
  f9::canonicalize(x);
  f9::to_words(x, o);
}

// Folds of a weight opening, f'[x] = f[x] + r (f[x + mid] - f[x]) on the top
// variable.  The first fold reads the column-major padded MLE of B (B[i][j] at
// j * pk + i, zero outside B) straight from the row-major matrix.
static __global__ void k_open_fold_matrix(const uint32_t* __restrict__ B, uint64_t rows, uint64_t cols, uint32_t log_pk,
                                   uint64_t mid, qm31 r, qm31* __restrict__ out) {
  const uint64_t x = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= mid) return;
  auto at = [&](uint64_t idx) -> uint32_t {
    const uint64_t j = idx >> log_pk, i = idx & ((1ull << log_pk) - 1);
    return (j < cols && i < rows) ? B[i * cols + j] : 0u;
  };
  out[x] = qm31_fold(qm31_from_m31(at(x)), qm31_from_m31(at(x + mid)), r);
}
static __global__ void k_open_fold(const qm31* __restrict__ in, uint64_t mid, qm31 r, qm31* __restrict__ out) {
  const uint64_t x = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= mid) return;
  out[x] = qm31_fold(in[x], in[x + mid], r);
}

// Montgomery roots -> canonical 8-word felts.
static __global__ void k_merkle_roots(const f9::fe* const* __restrict__ roots, int n, const MerkleConsts* __restrict__ Cp,
                               uint32_t* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  f9::fe x;
  f9::mul(*roots[i], Cp->one, x);
  f9::canonicalize(x);
  f9::to_words(x, out + 8 * i);
}

}  // namespace gkr
