// Forward-pass M31 matrix product C = A * B mod P on the matrix cores
// (the witness GEMM before the GKR walk; reference: m31_gemm_kernel /
// m31_gemv_kernel, engine/src/gpu_sumcheck.rs:418-460, gpu_matmul_m31_full
// :3104).  Exact for any canonical M31 inputs.
//
// Digit planes.  A value x in [0, P) is centered to v in (-P/2, P/2] and
// written as four balanced signed digits, v = sum_p d_p 256^p, d_p in
// [-128, 127].  Then
//   (A B)_ij = sum_s 256^s sum_{p+q=s} sum_k a_p[i][k] b_q[k][j]   (mod P),
// each inner sum an int8 GEMM on the matrix cores.  A group s holds at most 4
// pairs of products of magnitude <= 2^14, so K <= 16384 per pass stays inside
// int32.  Finally C_ij = sum_s 2^(8s mod 31) * group_s mod P (2^31 = 1 mod P).
// Planes that are zero everywhere are neither stored nor multiplied: int8-range
// data (|v| <= 127: the configs' weights and activations) has plane 0 only,
// so a weight streams 1 byte per entry and a K step costs one MFMA.
//
// Operand blocks.  v_mfma_i32_32x32x32_i8 takes, in lane l, row (A) or column
// (B) l % 32 and the 16 K values 16 (l / 32) .. + 15 of a 32-wide K step (any
// K order shared by A and B gives the same sum).  A plane is stored as 1 KB
// blocks, one per (32-row or 32-column tile, 32-wide K step), with lane l's
// 16 bytes at offset 16 l: one coalesced 16-byte load per lane.  Block (t, c)
// of a plane is at ((t * nsteps) + c) * 1024.  The accumulator holds rows
// 8 (v / 4) + 4 (l / 32) + v % 4 of column l % 32 in register v.
#pragma once
#include <stdint.h>

#include "field.h"

namespace gkr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kGemmK = 32;     // K per MFMA step
constexpr int kGemmTile = 32;  // rows / columns per wave tile
constexpr int kGemmBlockBytes = 1024;
constexpr uint64_t kGemmMaxKPass = 16384;  // K per accumulation pass (int32 bound)

__device__ __forceinline__ int32_t center_m31(uint32_t x) {
  return x > (P >> 1) ? (int32_t)x - (int32_t)P : (int32_t)x;
}
// Balanced digit p of v (p = 0..3); digits above 0 vanish for |v| <= 127.
__device__ __forceinline__ void balanced_digits(int32_t v, int32_t (&d)[4]) {
#pragma unroll
  for (int p = 0; p < 4; p++) {
    d[p] = (int32_t)(int8_t)(v & 0xff);
    v = (v - d[p]) >> 8;  // exact; after three digits |v| <= 64
  }
}

// Which planes of X (count canonical M31 values) are non-zero: bit p of
// *mask.  Grid-stride, an OR across the workgroup in LDS, then one vector
// atomic per workgroup (launch at most a few hundred workgroups).
static __global__ void __launch_bounds__(256) k_digit_mask(const uint32_t* __restrict__ X, uint64_t count,
                                                    uint32_t* __restrict__ mask) {
  __shared__ uint32_t wave_bits[4];
  uint32_t bits = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x) {
    int32_t d[4];
    balanced_digits(center_m31(X[i]), d);
#pragma unroll
    for (int p = 0; p < 4; p++) bits |= (d[p] != 0 ? 1u : 0u) << p;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) bits |= __shfl_xor(bits, off);
  if ((threadIdx.x & 63) == 0) wave_bits[threadIdx.x >> 6] = bits;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t all = wave_bits[0] | wave_bits[1] | wave_bits[2] | wave_bits[3];
    if (all) atomicOr(mask, all);
  }
}

// Pack planes 0..nplanes-1 of X into operand blocks.  kmajor = false: X is
// outer x K row-major (A: outer = row); kmajor = true: X is K x outer
// row-major (B: outer = column).  One thread fills one lane slot (16 bytes
// per plane) of one block; K and outer beyond the matrix are zero.  When mask
// is given (zeroed by the caller), bit p is set if plane p is non-zero.
static __global__ void __launch_bounds__(256) k_digit_pack(const uint32_t* __restrict__ X, uint64_t outer, uint64_t K,
                                                    bool kmajor, int nplanes, uint64_t ntiles, uint64_t nsteps,
                                                    int8_t* __restrict__ planes, uint32_t* __restrict__ mask) {
  __shared__ uint32_t wave_bits[4];
  const uint64_t slot = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (tile, step, lane)
  uint32_t bits = 0;
  if (slot < ntiles * nsteps * 64) {
    const int lane = (int)(slot & 63);
    const uint64_t blk = slot >> 6, tile = blk / nsteps, step = blk - tile * nsteps;
    const uint64_t o = tile * kGemmTile + (lane & 31);
    const uint64_t k0 = step * kGemmK + 16 * (lane >> 5);
    uint32_t w[4][4];
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
      for (int g = 0; g < 4; g++) w[p][g] = 0;
#pragma unroll
    for (int t = 0; t < 16; t++) {
      const uint64_t kk = k0 + t;
      uint32_t x = 0;
      if (o < outer && kk < K) x = kmajor ? X[kk * outer + o] : X[o * K + kk];
      int32_t d[4];
      balanced_digits(center_m31(x), d);
#pragma unroll
      for (int p = 0; p < 4; p++) w[p][t >> 2] |= ((uint32_t)d[p] & 0xffu) << (8 * (t & 3));
    }
    const uint64_t plane_bytes = ntiles * nsteps * kGemmBlockBytes;
    for (int p = 0; p < nplanes; p++) {
      uint4 v;
      v.x = w[p][0];
      v.y = w[p][1];
      v.z = w[p][2];
      v.w = w[p][3];
      *(uint4*)(planes + p * plane_bytes + blk * kGemmBlockBytes + 16 * lane) = v;
    }
#pragma unroll
    for (int p = 0; p < 4; p++) bits |= ((w[p][0] | w[p][1] | w[p][2] | w[p][3]) != 0 ? 1u : 0u) << p;
  }
  if (!mask) return;  // uniform: a kernel argument
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) bits |= __shfl_xor(bits, off);
  if ((threadIdx.x & 63) == 0) wave_bits[threadIdx.x >> 6] = bits;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t all = wave_bits[0] | wave_bits[1] | wave_bits[2] | wave_bits[3];
    if (all) atomicOr(mask, all);
  }
}

__device__ __forceinline__ uint32_t gemm_mod_p(int64_t x) {
  int64_t r = x % (int64_t)P;
  if (r < 0) r += P;
  return (uint32_t)r;
}

// One wave: C tile (row tile rt, column tile ct) over K steps [s0, s1);
// PA / PB planes of A / B (the planes above are zero).  Canonical partial
// sums go to out[split][row][col].  The host launches the PA = 1 and PA = 4
// variants back to back; *amask (A's non-zero planes, written by the A
// packing) makes exactly one of them work, so no host round trip decides.
template <int PA, int PB, int U>
static __global__ void __launch_bounds__(256) k_gemm_m31(const int8_t* __restrict__ Ap, uint64_t a_plane_bytes,
                                                  const uint32_t* __restrict__ amask,
                                                  const int8_t* __restrict__ Bp, uint64_t b_plane_bytes,
                                                  uint64_t m, uint64_t n, uint64_t nsteps, uint64_t rtiles,
                                                  uint64_t ctiles, uint64_t steps_per_split,
                                                  uint32_t* __restrict__ out) {
  constexpr int NG = PA + PB - 1;
  const bool high = (*amask & 0xeu) != 0;  // uniform
  if (PA == 1 ? high : !high) return;
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= rtiles * ctiles) return;
  const uint64_t rt = wave % rtiles, ct = wave / rtiles;  // the row tiles of a column tile are neighbours
  const uint64_t split = blockIdx.y;
  const uint64_t s0 = split * steps_per_split;
  const uint64_t s1 = s0 + steps_per_split < nsteps ? s0 + steps_per_split : nsteps;
  v16i acc[NG];
#pragma unroll
  for (int g = 0; g < NG; g++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[g][v] = 0;
  const int8_t* abase = Ap + (rt * nsteps) * kGemmBlockBytes + 16 * lane;
  const int8_t* bbase = Bp + (ct * nsteps) * kGemmBlockBytes + 16 * lane;
  uint64_t s = s0;  // U K steps' loads are issued together
  for (; s + U <= s1; s += U) {
    v4i a[U][PA], b[U][PB];
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
      for (int p = 0; p < PA; p++) a[u][p] = *(const v4i*)(abase + p * a_plane_bytes + (s + u) * kGemmBlockBytes);
#pragma unroll
      for (int q = 0; q < PB; q++)
        b[u][q] = __builtin_nontemporal_load((const v4i*)(bbase + q * b_plane_bytes + (s + u) * kGemmBlockBytes));
    }
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int p = 0; p < PA; p++)
#pragma unroll
        for (int q = 0; q < PB; q++)
          acc[p + q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u][p], b[u][q], acc[p + q], 0, 0, 0);
  }
  for (; s < s1; s++) {
    v4i a[PA], b[PB];
#pragma unroll
    for (int p = 0; p < PA; p++) a[p] = *(const v4i*)(abase + p * a_plane_bytes + s * kGemmBlockBytes);
#pragma unroll
    for (int q = 0; q < PB; q++) b[q] = *(const v4i*)(bbase + q * b_plane_bytes + s * kGemmBlockBytes);
#pragma unroll
    for (int p = 0; p < PA; p++)
#pragma unroll
      for (int q = 0; q < PB; q++) acc[p + q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[p], b[q], acc[p + q], 0, 0, 0);
  }
  const uint64_t col = ct * kGemmTile + (lane & 31);
  if (col >= n) return;
#pragma unroll
  for (int v = 0; v < 16; v++) {
    const uint64_t row = rt * kGemmTile + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
    if (row >= m) continue;
    uint64_t total = 0;
#pragma unroll
    for (int g = 0; g < NG; g++)
      total += (uint64_t)m31_reduce64((uint64_t)gemm_mod_p(acc[g][v]) << ((8 * g) % 31));
    out[(split * m + row) * n + col] = m31_reduce64(total);
  }
}

// C = sum over splits of the partials, mod P.
static __global__ void k_gemm_reduce(const uint32_t* __restrict__ part, uint64_t count, int splits, uint32_t* __restrict__ C) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  uint64_t s = 0;
  for (int t = 0; t < splits; t++) s += part[(uint64_t)t * count + i];
  C[i] = m31_reduce64(s);
}

}  // namespace gkr
