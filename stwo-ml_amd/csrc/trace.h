// Transcript trace: the channel state at fixed points of the provers, the
// verifiers and the walk, one line per point, for finding where two
// transcripts part (the reference prints its channel under
// STWO_CHANNEL_TRACE, engine/src/gpu_sumcheck.rs:2708-2740,
// gkr/prover.rs:1523-1541, 6002-6012).
//
// GKR_CHANNEL_TRACE=<path> appends the lines to that file, GKR_CHANNEL_TRACE=-
// (or "stderr") writes them to stderr; STWO_CHANNEL_TRACE set to anything
// writes them to stderr.  The environment is read once per library call
// that runs a transcript (the outermost TraceScope), so a disabled trace
// costs one branch per point.  Line format:
//   <label>[ <index>] 0x<digest, 64 hex digits> <n_draws>
// Labels: matmul.rounds / matmul (a MatMul reduction after its rounds and
// after its final mixes), logup.gamma_beta / logup.eq / logup.mult / logup
// (an activation layer after gamma and beta, its eq-sumcheck, its
// multiplicity sumcheck and its final mixes), mul.eq / mul, layernorm /
// rmsnorm, and walk.step <i> after step i of a walk.
#pragma once
#include "poseidon.h"

namespace gkr {

struct TraceScope {
  TraceScope();
  ~TraceScope();
};
// The calling thread's trace setting, as read by its outermost TraceScope.
bool trace_enabled();
void trace_point_impl(const PoseidonChannel& ch, const char* label, long index);
inline void trace_point(const PoseidonChannel& ch, const char* label, long index = -1) {
  if (trace_enabled()) trace_point_impl(ch, label, index);
}

}  // namespace gkr
