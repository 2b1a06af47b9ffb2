// The rsqrt lookup table of the LayerNorm and RMSNorm layers (host side).
//
// build_rsqrt_table (engine/src/components/layernorm.rs:116-151, shared by
// rmsnorm.rs:125): entry x maps to 2^16 / isqrt(x) (integer Newton square
// root), x = 0 to 2^16 - 1; 2^16 entries (LayerNormConfig / RMSNormConfig,
// layernorm.rs:41-47).  Row statistics are reduced to the table range by
// masking (prover.rs:7987-7990, 8459-8462).
#pragma once
#include <stdint.h>

namespace gkr {

constexpr uint32_t kNormTableLog = 16;
constexpr uint32_t kNormMask = (1u << kNormTableLog) - 1;
constexpr uint64_t kNormTagLN = 0x4C4E;  // "LN": LayerNorm linear part
constexpr uint64_t kNormTagMV = 0x4D56;  // "MV": LayerNorm mean-variance part
constexpr uint64_t kNormTagRS = 0x5253;  // "RS": LayerNorm rsqrt LogUp type tag, table commitment tag
constexpr uint64_t kNormTagRN = 0x524E;  // "RN": RMSNorm linear part and LogUp type tag
constexpr uint64_t kNormTagRQ = 0x5251;  // "RQ": RMSNorm square-sum part
constexpr uint64_t kNormTagGamma = 0x47414D4D41ull;  // "GAMMA": RMSNorm scale commitment

// floor(sqrt(n)) by Newton's iteration from 2^ceil(bits / 2) (layernorm.rs:139-151)
inline uint64_t norm_isqrt(uint64_t n) {
  if (n < 2) return n;
  const int bits = 64 - __builtin_clzll(n);
  uint64_t x = 1ull << ((bits + 1) / 2);
  for (;;) {
    const uint64_t x1 = (x + n / x) / 2;
    if (x1 >= x) return x;
    x = x1;
  }
}
inline uint32_t norm_rsqrt(uint32_t v) {
  if (v == 0) return (1u << 16) - 1;
  const uint64_t s = norm_isqrt(v);
  if (s == 0) return (1u << 16) - 1;
  const uint64_t r = (1ull << 16) / s;
  return (uint32_t)(r < (1ull << 31) - 2 ? r : (1ull << 31) - 2);
}

}  // namespace gkr
