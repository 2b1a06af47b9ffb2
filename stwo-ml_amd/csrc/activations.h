// Activation lookup tables of the LogUp layer (host side).
//
// Functions follow engine/src/gadgets/lookup_table.rs:192-342 (fixed-point
// scale 2^16, values above P/2 read as negative) and the type tags of
// engine/src/components/activation.rs:63-71.  Table j maps input j to f(j)
// for j < 2^log_size (PrecomputedTable::build, lookup_table.rs:30-75).
// SiLU and GELU evaluate exp/tanh in f64 through the C library, as the
// reference does through Rust's f64 methods on the same platform.
#pragma once
#include <math.h>
#include <stdint.h>

#include <vector>

namespace gkr {

enum ActivationType : uint32_t {
  ACT_RELU = 1,
  ACT_GELU = 2,
  ACT_SIGMOID = 3,
  ACT_SOFTMAX = 4,
  ACT_SILU = 5,
};

inline uint32_t act_default_log_size(uint32_t tag) {
  // ActivationType::recommended_table_log_size (activation.rs:38-46)
  return tag == ACT_SOFTMAX ? 20u : 16u;
}

namespace act_detail {
constexpr uint64_t kP = (1ull << 31) - 1;
constexpr uint32_t kHalfP = (1u << 30) - 1;
constexpr double kScale = 65536.0;

inline double to_real(uint32_t val) {
  return val <= kHalfP ? (double)val / kScale : -((double)(kP - (uint64_t)val)) / kScale;
}
inline uint32_t from_real(double y) {
  if (y >= 0.0) {
    double r = round(y * kScale);
    uint64_t u = (uint64_t)r;
    if (u > kP - 1) u = kP - 1;
    return (uint32_t)u;
  }
  uint64_t neg = (uint64_t)round(-y * kScale);
  if (neg > kP - 1) neg = kP - 1;
  return (uint32_t)(kP - neg);
}
}  // namespace act_detail

inline uint32_t act_relu(uint32_t v) { return v <= act_detail::kHalfP ? v : 0u; }

inline uint32_t act_gelu(uint32_t v) {
  if (v == 0) return 0;
  const double x = act_detail::to_real(v);
  const double k = sqrt(2.0 / M_PI);
  const double inner = k * (x + 0.044715 * x * x * x);
  return act_detail::from_real(0.5 * x * (1.0 + tanh(inner)));
}

inline uint32_t act_sigmoid(uint32_t v) {
  if (v > act_detail::kHalfP) return 0;
  if (v == 0) return 1u << 15;
  return 1u << 16;
}

inline uint32_t act_softmax_exp(uint32_t v) {
  const uint32_t scale = 1u << 16;
  if (v > act_detail::kHalfP) {
    const uint32_t neg = ((1u << 31) - 2) - v;
    uint32_t decay = neg / scale;
    if (decay > 20) decay = 20;
    const uint32_t r = scale >> decay;
    return r > 1 ? r : 1;
  }
  if (v == 0) return scale;
  uint32_t growth = v / scale;
  if (growth > 10) growth = 10;
  const uint64_t r = (uint64_t)scale << growth;
  const uint64_t cap = (1ull << 31) - 2;
  return (uint32_t)(r < cap ? r : cap);
}

inline uint32_t act_silu(uint32_t v) {
  if (v == 0) return 0;
  const double x = act_detail::to_real(v);
  return act_detail::from_real(x / (1.0 + exp(-x)));
}

inline bool act_valid(uint32_t tag) { return tag >= ACT_RELU && tag <= ACT_SILU; }
// Activations the reference proves with the LogUp reducer.  ReLU never goes
// through it: every dispatch sends ReLU to the algebraic proof
// (engine/src/gkr/prover.rs:1770-1776), so a LogUp proof of ReLU could not be
// byte-identical to the reference's and is refused.
inline bool act_logup_valid(uint32_t tag) { return act_valid(tag) && tag != ACT_RELU; }

inline uint32_t act_apply(uint32_t tag, uint32_t v) {
  switch (tag) {
    case ACT_RELU: return act_relu(v);
    case ACT_GELU: return act_gelu(v);
    case ACT_SIGMOID: return act_sigmoid(v);
    case ACT_SOFTMAX: return act_softmax_exp(v);
    default: return act_silu(v);
  }
}

// Output column of the table for inputs 0 .. 2^log_size - 1 (M31 values).
inline std::vector<uint32_t> act_table(uint32_t tag, uint32_t log_size) {
  std::vector<uint32_t> out((size_t)1 << log_size);
  for (size_t j = 0; j < out.size(); j++) {
    uint32_t r = act_apply(tag, (uint32_t)j);
    out[j] = r == (uint32_t)act_detail::kP ? 0u : r;
  }
  return out;
}

}  // namespace gkr
