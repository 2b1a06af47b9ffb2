// Forward-pass M31 matrix product on the matrix cores (the witness).
#include "internal.h"
#include "gemm.h"
/* ------------------------------------------------------------------ forward GEMM
 * C = A * B mod P for canonical M31 matrices (gemm.h).  B's digit planes (only
 * up to its highest non-zero plane) are built once per matrix and kept with
 * it; A's four planes are built per call into a context slot.  One wave per 32 x 32 tile
 * of C and K split; the splits (each at most 16384 deep, enough of them for
 * ~2048 workgroups) are added by k_gemm_reduce. */
static int digit_planes_needed(gkr_ctx* c, const uint32_t* X, uint64_t count, int* nplanes) {
  uint32_t* dmask;
  TRY(ensureT(c, S_GEMMP, 1, &dmask));
  HIP_TRY(hipMemsetAsync(dmask, 0, 4, c->stream));
  const uint64_t blocks = std::min<uint64_t>((count + 255) / 256, 256);
  GKR_LAUNCH(c, k_digit_mask, dim3((uint32_t)std::max<uint64_t>(blocks, 1)), dim3(256), 0, X, count, dmask);
  HIP_TRY(hipGetLastError());
  uint32_t mask = 0;
  HIP_TRY(hipMemcpyAsync(&mask, dmask, 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  int np = 1;
  for (int p = 0; p < 4; p++)
    if (mask & (1u << p)) np = p + 1;
  *nplanes = np;
  return GKR_OK;
}

static int pack_planes(gkr_ctx* c, const uint32_t* X, uint64_t outer, uint64_t K, bool kmajor, int np, int8_t* out,
                       uint32_t* mask = nullptr) {
  const uint64_t ntiles = (outer + kGemmTile - 1) / kGemmTile, nsteps = (K + kGemmK - 1) / kGemmK;
  const uint64_t slots = ntiles * nsteps * 64;
  GKR_LAUNCH(c, k_digit_pack, dim3((uint32_t)((slots + 255) / 256)), dim3(256), 0, X, outer, K, kmajor, np, ntiles,
                                                                                  nsteps, out, mask);
  HIP_TRY(hipGetLastError());
  return GKR_OK;
}

static int weight_planes(gkr_ctx* c, gkr_matrix* b) {
  if (b->bplanes) return GKR_OK;
  int np;
  TRY(digit_planes_needed(c, b->dev, b->rows * b->cols, &np));
  const uint64_t ntiles = (b->cols + kGemmTile - 1) / kGemmTile, nsteps = (b->rows + kGemmK - 1) / kGemmK;
  int8_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, (size_t)np * ntiles * nsteps * kGemmBlockBytes));
  const int rc = pack_planes(c, b->dev, b->cols, b->rows, true, np, d);
  if (rc != GKR_OK) {
    drain(c);
    (void)hipFree(d);
    return rc;
  }
  b->bplanes = d;
  b->bnplanes = np;
  return GKR_OK;
}

template <int PA, int PB, int U>
static void launch_gemm(gkr_ctx* c, dim3 grid, const int8_t* ap, uint64_t apb, const uint32_t* amask,
                        const int8_t* bp, uint64_t bpb, uint64_t m, uint64_t n, uint64_t nsteps, uint64_t rt,
                        uint64_t ctl, uint64_t sps, uint32_t* out) {
  GKR_LAUNCH(c, (k_gemm_m31<PA, PB, U>), grid, dim3(256), 0, ap, apb, amask, bp, bpb, m, n, nsteps, rt, ctl, sps, out);
}

static int matmul_forward(gkr_ctx* c, const gkr_matrix* a, gkr_matrix* b, uint32_t* C) {
  const uint64_t m = a->rows, k = a->cols, n = b->cols;
  TRY(weight_planes(c, b));
  const uint64_t nsteps = (k + kGemmK - 1) / kGemmK;
  const uint64_t rtiles = (m + kGemmTile - 1) / kGemmTile, ctiles = (n + kGemmTile - 1) / kGemmTile;
  const uint64_t a_plane = rtiles * nsteps * kGemmBlockBytes, b_plane = ctiles * nsteps * kGemmBlockBytes;
  // A: all four planes packed (A is small) with its non-zero mask on the device;
  // B: 1 plane (int8-range weights) or 4
  const int PB = b->bnplanes == 1 ? 1 : 4;
  void* abuf;
  TRY(ensure(c, S_GEMMA, 256 + (size_t)4 * a_plane, &abuf));
  uint32_t* amask = (uint32_t*)abuf;
  int8_t* ap = (int8_t*)abuf + 256;
  HIP_TRY(hipMemsetAsync(amask, 0, 4, c->stream));
  TRY(pack_planes(c, a->dev, m, k, false, 4, ap, amask));
  const int8_t* bp = b->bplanes;
  if (PB > b->bnplanes) {  // a 2- or 3-plane weight: extend with zero planes in scratch
    int8_t* ext;
    TRY(ensureT(c, S_GEMMB, (size_t)4 * b_plane, &ext));
    HIP_TRY(hipMemcpyAsync(ext, b->bplanes, (size_t)b->bnplanes * b_plane, hipMemcpyDeviceToDevice, c->stream));
    HIP_TRY(hipMemsetAsync(ext + (size_t)b->bnplanes * b_plane, 0, (size_t)(4 - b->bnplanes) * b_plane, c->stream));
    bp = ext;
  }
  const uint64_t waves = rtiles * ctiles, blocks_x = (waves + 3) / 4;
  uint64_t splits = (2048 + blocks_x - 1) / blocks_x;
  splits = std::min<uint64_t>(splits, std::max<uint64_t>(1, nsteps / 16));
  splits = std::max<uint64_t>(splits, (nsteps * kGemmK + kGemmMaxKPass - 1) / kGemmMaxKPass);
  const uint64_t sps = (nsteps + splits - 1) / splits;
  splits = (nsteps + sps - 1) / sps;
  if (blocks_x > 0x7fffffffull || splits > 65535) return fail(GKR_ERR_INVALID, "forward GEMM: grid too large");
  uint32_t* part = C;
  if (splits > 1) TRY(ensureT(c, S_GEMMP, splits * m * n, &part));
  const dim3 grid((uint32_t)blocks_x, (uint32_t)splits);
  // exactly one of each pair works (the other reads the mask and returns)
  if (PB == 1) {
    launch_gemm<1, 1, 16>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
    launch_gemm<4, 1, 4>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
  } else {
    launch_gemm<1, 4, 4>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
    launch_gemm<4, 4, 2>(c, grid, ap, a_plane, amask, bp, b_plane, m, n, nsteps, rtiles, ctiles, sps, part);
  }
  HIP_TRY(hipGetLastError());
  if (splits > 1) {
    const uint64_t count = m * n;
    GKR_LAUNCH(c, k_gemm_reduce, dim3((uint32_t)((count + 255) / 256)), dim3(256), 0, part, count, (int)splits, C);
    HIP_TRY(hipGetLastError());
  }
  return GKR_OK;
}

extern "C" int gkr_matmul_forward_into(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, gkr_matrix* out) {
  if (!c || !a || !b || !out || !out->dev) return fail(GKR_ERR_INVALID, "null argument");
  if (a->cols != b->rows || out->rows != a->rows || out->cols != b->cols)
    return fail(GKR_ERR_INVALID, "forward GEMM: A %llux%llu . B %llux%llu into %llux%llu", (unsigned long long)a->rows,
                (unsigned long long)a->cols, (unsigned long long)b->rows, (unsigned long long)b->cols,
                (unsigned long long)out->rows, (unsigned long long)out->cols);
  if (out == a || out == b) return fail(GKR_ERR_INVALID, "forward GEMM: output aliases an input");
  HIP_TRY(hipSetDevice(c->device));
  TRY(drop_derived(c, out));  // the contents change
  return matmul_forward(c, a, const_cast<gkr_matrix*>(b), out->dev);
}

extern "C" int gkr_matmul_forward(gkr_ctx* c, const gkr_matrix* a, const gkr_matrix* b, gkr_matrix** out) {
  if (!c || !a || !b || !out) return fail(GKR_ERR_INVALID, "null argument");
  if (a->cols != b->rows)
    return fail(GKR_ERR_INVALID, "forward GEMM: A is %llux%llu, B is %llux%llu", (unsigned long long)a->rows,
                (unsigned long long)a->cols, (unsigned long long)b->rows, (unsigned long long)b->cols);
  if (a->rows == 0 || a->cols == 0 || b->cols == 0) return fail(GKR_ERR_INVALID, "forward GEMM: empty matrix");
  HIP_TRY(hipSetDevice(c->device));
  uint32_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, a->rows * b->cols * sizeof(uint32_t)));
  int rc = matmul_forward(c, a, const_cast<gkr_matrix*>(b), d);
  if (rc == GKR_OK) rc = sync(c);
  if (rc != GKR_OK) {
    drain(c);
    (void)hipFree(d);
    return rc;
  }
  *out = new_matrix(c, d, a->rows, b->cols, true);
  return GKR_OK;
}

