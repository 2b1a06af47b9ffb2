"""ctypes binding of the MI355X GKR prover C ABI (include/gkr_mi355x.h).

The library is lib/libgkr_mi355x.so next to this file (built by the
package Makefile).  Loading fails loudly when it is missing: there is no
CPU fallback.  Class and method names follow the reference's Rust API
(PoseidonChannel in engine/src/crypto/poseidon_channel.rs, ZkmlOps in
engine/src/backend.rs, the GKR layer reducers in engine/src/gkr/prover.rs).
QM31 values are 4-tuples (a, b, c, d) = (a + b i) + (c + d i) u; felt252
values are Python ints.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import List, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# GKR_MI355X_LIB selects another build of the library (e.g. a tuning variant).
LIB_PATH = os.environ.get("GKR_MI355X_LIB") or os.path.join(HERE, "lib", "libgkr_mi355x.so")
P = (1 << 31) - 1
FELT_P = 2**251 + 17 * 2**192 + 1

QM31 = Tuple[int, int, int, int]


class GkrQM31(C.Structure):
    _fields_ = [("v", C.c_uint32 * 4)]


class GkrFelt(C.Structure):
    _fields_ = [("w", C.c_uint32 * 8)]


POLICY_FIELDS = ("allow_missing_norm_proof", "allow_logup_activation", "allow_missing_segment_binding",
                 "skip_rms_sq_proof", "piecewise_activation", "skip_batch_tokens", "skip_unified_stark",
                 "weight_binding_mode", "aggregated_full_binding", "aggregated_rlc_only", "io_packing", "packed_proof",
                 "double_packed_proof", "validate_decode_chain")


class GkrPolicy(C.Structure):
    _fields_ = [(f, C.c_uint8) for f in POLICY_FIELDS]


class GkrMulOut(C.Structure):
    _fields_ = [("eq_round_polys", C.POINTER(GkrQM31)), ("lhs_eval", GkrQM31), ("rhs_eval", GkrQM31),
                ("alpha", GkrQM31), ("next_value", GkrQM31), ("n_vars", C.c_uint32)]


class GkrLogupOut(C.Structure):
    _fields_ = [
        ("claimed_sum", GkrQM31),
        ("eq_round_polys", C.POINTER(GkrQM31)),
        ("w_eval", GkrQM31),
        ("in_eval", GkrQM31),
        ("out_eval", GkrQM31),
        ("multiplicities", C.POINTER(C.c_uint32)),
        ("mult_round_polys", C.POINTER(GkrQM31)),
        ("mult_final_eval", GkrQM31),
        ("mult_claimed_sum", GkrQM31),
        ("input_eval", GkrQM31),
        ("output_eval", GkrQM31),
        ("table_commitment", GkrFelt),
        ("gamma", GkrQM31),
        ("beta", GkrQM31),
    ]


class GkrStep(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("claim", C.c_uint32), ("a", C.c_void_p), ("b", C.c_void_p),
                ("activation_type", C.c_uint32), ("table_log_size", C.c_uint32), ("dim", C.c_uint64)]


class GkrNormOut(C.Structure):
    _fields_ = [("input_eval", GkrQM31), ("output_eval", GkrQM31), ("mean_eval", GkrQM31),
                ("rsqrt_eval", GkrQM31), ("var_eval", GkrQM31), ("n_active", C.c_uint32), ("sum0", GkrQM31),
                ("sum1", GkrQM31), ("p0_round_polys", C.POINTER(GkrQM31)), ("p0_final0", GkrQM31),
                ("p0_final1", GkrQM31), ("lin_round_polys", C.POINTER(GkrQM31)), ("lin_final0", GkrQM31),
                ("lin_final1", GkrQM31), ("cb_input", GkrQM31), ("cb_mean", GkrQM31), ("claimed_sum", GkrQM31),
                ("logup_round_polys", C.POINTER(GkrQM31)), ("w_eval", GkrQM31), ("in_eval", GkrQM31),
                ("out_eval", GkrQM31), ("multiplicities", C.POINTER(C.c_uint32)),
                ("mult_round_polys", C.POINTER(GkrQM31)), ("mult_final_eval", GkrQM31),
                ("mult_claimed_sum", GkrQM31), ("table_commitment", GkrFelt), ("n_rows", C.c_uint32),
                ("row_stats0", C.POINTER(C.c_uint32)), ("row_stats1", C.POINTER(C.c_uint32)),
                ("gamma_commitment", GkrFelt), ("gamma_eval", GkrQM31)]


STEP_MATMUL, STEP_MUL, STEP_ACTIVATION, STEP_LAYERNORM, STEP_RMSNORM = 0, 2, 3, 4, 8
NORM_TABLE_LOG = 16
# norm proof dict keys holding one QM31 (the oracle's norm proof dicts use the same names)
NORM_Q_KEYS = (("input_eval", "input_eval"), ("output_eval", "output_eval"), ("mean_eval", "mean_eval"),
               ("rsqrt_eval", "rsqrt_eval"), ("var_eval", "var_eval"), ("sum0", "sum0"), ("sum1", "sum1"),
               ("p0_final0", "p0_final0"), ("p0_final1", "p0_final1"), ("lin_final0", "lin_final0"),
               ("lin_final1", "lin_final1"), ("cb_input", "cb_input"), ("cb_mean", "cb_mean"),
               ("claimed_sum", "claimed_sum"), ("w_eval", "w_eval"), ("in_eval", "in_eval"), ("out_eval", "out_eval"),
               ("mult_final_eval", "mult_final"), ("mult_claimed_sum", "mult_sum"), ("gamma_eval", "gamma_eval"))
CLAIM_CHAINED, CLAIM_FRESH = 0, 1


def _next_pow2(v: int) -> int:
    return 1 << max(0, (v - 1).bit_length())


class GkrLayerShape(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("rows", C.c_uint64), ("cols", C.c_uint64), ("cols_b", C.c_uint64),
                ("activation_type", C.c_uint32), ("table_log_size", C.c_uint32), ("claim", C.c_uint32),
                ("dim", C.c_uint64)]


class GkrError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"gkr error {code}: {msg}")
        self.code = code


_lib: Optional[C.CDLL] = None

# (name, restype, argtypes) for every symbol of include/gkr_mi355x.h
_P = C.c_void_p
_PQ = C.POINTER(GkrQM31)
_PF = C.POINTER(GkrFelt)
_U32P = C.POINTER(C.c_uint32)
SIGNATURES = [
    ("gkr_last_error", C.c_char_p, []),
    ("gkr_version", C.c_char_p, []),
    ("gkr_hades_permute", C.c_int, [_PF]),
    ("gkr_poseidon_hash", C.c_int, [_PF, _PF, _PF]),
    ("gkr_poseidon_hash_many", C.c_int, [_PF, C.c_size_t, _PF]),
    ("gkr_channel_new", C.c_int, [C.POINTER(_P)]),
    ("gkr_channel_free", None, [_P]),
    ("gkr_channel_clone", C.c_int, [_P, C.POINTER(_P)]),
    ("gkr_channel_mix_u64", C.c_int, [_P, C.c_uint64]),
    ("gkr_channel_mix_felt", C.c_int, [_P, _PF]),
    ("gkr_channel_mix_secure_field", C.c_int, [_P, _PQ]),
    ("gkr_channel_mix_felts", C.c_int, [_P, _PQ, C.c_size_t]),
    ("gkr_channel_mix_poly_coeffs", C.c_int, [_P, _PQ]),
    ("gkr_channel_mix_poly_coeffs_deg3", C.c_int, [_P, _PQ]),
    ("gkr_channel_draw_felt252", C.c_int, [_P, _PF]),
    ("gkr_channel_draw_qm31", C.c_int, [_P, _PQ]),
    ("gkr_channel_draw_qm31s", C.c_int, [_P, C.c_size_t, _PQ]),
    ("gkr_channel_digest", C.c_int, [_P, _PF]),
    ("gkr_channel_hash_count", C.c_uint64, [_P]),
    ("gkr_channel_export", C.c_int, [_P, _U32P]),
    ("gkr_channel_import", C.c_int, [_P, _U32P]),
    ("gkr_ctx_create", C.c_int, [C.c_int, C.POINTER(_P)]),
    ("gkr_ctx_destroy", None, [_P]),
    ("gkr_ctx_synchronize", C.c_int, [_P]),
    ("gkr_ctx_set_timing", C.c_int, [_P, C.c_int]),
    ("gkr_ctx_kernel_time", C.c_int, [_P, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_uint64),
                                      C.POINTER(C.c_uint64)]),
    ("gkr_ctx_kernel_time_by_size", C.c_int, [_P, C.c_int, C.POINTER(C.c_uint64), C.POINTER(C.c_double),
                                              C.POINTER(C.c_uint64), C.c_size_t, C.POINTER(C.c_size_t)]),
    ("gkr_ctx_reset_timing", C.c_int, [_P]),
    ("gkr_ctx_debug", C.c_int, [_P, C.c_int, C.c_uint64]),
    ("gkr_matrix_upload", C.c_int, [_P, _U32P, C.c_uint64, C.c_uint64, C.POINTER(_P)]),
    ("gkr_matrix_wrap_device", C.c_int, [_P, _P, C.c_uint64, C.c_uint64, C.POINTER(_P)]),
    ("gkr_matrix_synthetic", C.c_int, [_P, C.c_uint64, C.c_uint64, C.c_int, C.c_uint64, C.POINTER(_P)]),
    ("gkr_matrix_download", C.c_int, [_P, _P, _U32P]),
    ("gkr_matrix_free", None, [_P]),
    ("gkr_synthetic_value", C.c_uint32, [C.c_int, C.c_uint64, C.c_uint64]),
    ("gkr_reduce_matmul_layer", C.c_int, [_P, _P, _P, _PQ, C.c_uint32, _PQ, C.c_uint32, C.c_uint64, _P, _PQ, _PQ,
                                          _PQ, _PQ]),
    ("gkr_evaluate_mle_at_point", C.c_int, [_P, _PQ, C.c_uint64, _PQ, C.c_uint32, _PQ]),
    ("gkr_restrict_mle", C.c_int, [_P, _PQ, C.c_uint64, _PQ, C.c_uint32, _PQ]),
    ("gkr_proof_new", C.c_int, [C.POINTER(_P)]),
    ("gkr_proof_free", None, [_P]),
    ("gkr_proof_num_layers", C.c_size_t, [_P]),
    ("gkr_proof_set_input_claim", C.c_int, [_P, _PQ, C.c_uint32, _PQ]),
    ("gkr_proof_layer_claim_value", C.c_int, [_P, C.c_size_t, _PQ]),
    ("gkr_proof_add_weight_commitment", C.c_int, [_P, _PF]),
    ("gkr_proof_set_io_commitment", C.c_int, [_P, _PF]),
    ("gkr_proof_serialize", C.c_int, [_P, _PF, C.c_size_t, C.POINTER(C.c_size_t)]),
    ("gkr_proof_stream_to", C.c_int, [_P, _PF, C.c_size_t]),
    ("gkr_seed_channel", C.c_int, [_P, C.c_uint64, C.c_uint64, C.c_uint64, _PF]),
    ("gkr_policy_preset", C.c_int, [C.c_char_p, C.POINTER(GkrPolicy)]),
    ("gkr_policy_commitment", C.c_int, [C.POINTER(GkrPolicy), _PF]),
    ("gkr_matmul_output_claim", C.c_int, [_P, _P, _P, _PQ, C.c_uint32, _PQ]),
    ("gkr_prove_matmul_layer", C.c_int, [_P, _PQ, C.c_uint32, _PQ, _P, _P, _P, _P, _PQ, _PQ, _PQ, _PQ, _PQ]),
    ("gkr_prove_matmul_layer_dual_simd", C.c_int,
     [_P, _PQ, C.c_uint32, _PQ, C.POINTER(_P), C.POINTER(_P), _PQ, C.c_uint32, _P, _P, _PQ, _PQ, _PQ]),
    ("gkr_prove_matmul_layer_simd", C.c_int,
     [_P, _PQ, C.c_uint32, _PQ, C.POINTER(_P), _PQ, C.c_uint32, _P, _P, _P, _PQ, _PQ, _PQ, _PQ, _PQ]),
    ("gkr_prove_activation_layer", C.c_int, [_P, _PQ, C.c_uint32, _PQ, _P, C.c_uint32, C.c_uint32, _P, _P,
                                             C.POINTER(GkrLogupOut)]),
    ("gkr_activation_table", C.c_int, [C.c_uint32, C.c_uint32, _U32P]),
    ("gkr_bench_copy", C.c_int, [_P, C.c_uint64, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    ("gkr_qvec_upload", C.c_int, [_P, _PQ, C.c_uint64, C.POINTER(_P)]),
    ("gkr_qvec_synthetic", C.c_int, [_P, C.c_uint64, C.c_uint64, C.POINTER(_P)]),
    ("gkr_qvec_download", C.c_int, [_P, _P, _PQ]),
    ("gkr_qvec_free", None, [_P]),
    ("gkr_qvec_device_ptr", _P, [_P]),
    ("gkr_matrix_device_ptr", _P, [_P]),
    ("gkr_matrix_invalidate", C.c_int, [_P, _P]),
    ("gkr_matrix_commitment_cached", C.c_int, [_P, _P, C.POINTER(C.c_int)]),
    ("gkr_matrix_set_commitment", C.c_int, [_P, _P, _P]),
    ("gkr_prove_aggregated_binding", C.c_int, [_P, _P, _P, C.c_size_t, _PF, C.c_size_t, C.POINTER(C.c_size_t)]),
    ("gkr_proof_num_binding_groups", C.c_size_t, [_P]),
    ("gkr_proof_binding_group", C.c_int, [_P, C.c_size_t, _PF, C.c_size_t, C.POINTER(C.c_size_t)]),
    ("gkr_prove_lookup_batch", C.c_int, [_P, _P, _P, C.c_size_t, _P]),
    ("gkr_verify_lookup_batch", C.c_int, [_U32P, _U32P, C.c_size_t, _P, _P, _PQ, _PQ]),
    ("gkr_serialize_lookup_batch", C.c_int, [_U32P, _U32P, C.c_size_t, _P, _PF, C.c_size_t,
                                             C.POINTER(C.c_size_t)]),
    ("gkr_sumcheck_product", C.c_int, [_P, _P, _P, _P, _PQ, _PQ, _PQ, _PQ]),
    ("gkr_sumcheck_product_noalloc", C.c_int, [_P, _PQ, _PQ, C.c_uint64, _P, _PQ, _PQ, _PQ, _PQ]),
    ("gkr_prove_mul_layer", C.c_int, [_P, _PQ, C.c_uint32, _PQ, _P, _P, _P, _P, C.POINTER(GkrMulOut)]),
    ("gkr_reduce_mul_layer", C.c_int, [_P, _PQ, C.c_uint32, _PQ, _PQ, _PQ, C.c_uint64, _P, _P,
                                       C.POINTER(GkrMulOut)]),
    ("gkr_mul_output_claim", C.c_int, [_P, _P, _P, _PQ, C.c_uint32, _PQ]),
    ("gkr_verify_matmul_layer", C.c_int, [_PQ, C.c_uint32, _PQ, C.c_uint64, C.c_uint64, C.c_uint64, _PQ,
                                          C.c_uint32, _PQ, _PQ, _P, _PQ, C.POINTER(C.c_uint32), _PQ]),
    ("gkr_verify_mul_layer", C.c_int, [_PQ, C.c_uint32, _PQ, _PQ, C.c_uint32, _PQ, _PQ, _P, _PQ]),
    ("gkr_verify_activation_layer", C.c_int, [_PQ, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                              C.POINTER(GkrLogupOut), _P, _PQ]),
    ("gkr_prove_layernorm_layer", C.c_int, [_P, _PQ, C.c_uint32, _PQ, _P, C.c_uint64, _P, _P, C.POINTER(GkrNormOut)]),
    ("gkr_prove_rmsnorm_layer", C.c_int, [_P, _PQ, C.c_uint32, _PQ, _P, C.c_uint64, _U32P, C.c_uint64, _P, _P,
                                          C.POINTER(GkrNormOut)]),
    ("gkr_norm_output_claim", C.c_int, [_P, C.c_uint32, _P, C.c_uint64, _U32P, C.c_uint64, _PQ, C.c_uint32, _PQ]),
    ("gkr_verify_layernorm_layer", C.c_int, [_PQ, C.c_uint32, _PQ, C.c_uint64, C.POINTER(GkrNormOut), _P, _PQ]),
    ("gkr_verify_rmsnorm_layer", C.c_int, [_PQ, C.c_uint32, _PQ, C.c_uint64, C.POINTER(GkrNormOut), _P, _PQ]),
    ("gkr_verify_walk", C.c_int, [C.POINTER(GkrFelt), C.c_size_t, C.POINTER(GkrLayerShape), C.c_size_t, _PQ,
                                  C.c_uint32, _PQ, _PQ, C.c_size_t, _P, _PQ, C.POINTER(C.c_uint32), _PQ,
                                  C.POINTER(C.c_size_t)]),
    ("gkr_prove_walk", C.c_int, [_P, _P, C.POINTER(GkrStep), C.c_size_t, _PQ, C.c_uint32, _PQ, _P, _PQ,
                                 C.POINTER(C.c_uint32), _PQ]),
    ("gkr_matmul_forward", C.c_int, [_P, _P, _P, C.POINTER(_P)]),
    ("gkr_matmul_forward_into", C.c_int, [_P, _P, _P, _P]),
    ("gkr_weight_commitment", C.c_int, [_P, _P, _PF]),
    ("gkr_weight_commitments", C.c_int, [_P, C.POINTER(_P), C.c_size_t, _PF]),
    ("gkr_mle_commitment", C.c_int, [_P, _P, _PF]),
    ("gkr_prove_weight_opening", C.c_int, [_P, _P, _PQ, C.c_uint32, _PQ, _P, _P, _PF]),
    ("gkr_prove_weight_openings", C.c_int, [_P, _P, _P]),
    ("gkr_prove_weight_binding", C.c_int, [_P, _P, _P, C.c_int]),
]
WEIGHT_SEQUENTIAL, WEIGHT_AGGREGATED_RLC, WEIGHT_RLC_DIRECT, WEIGHT_AGGREGATED_FULL = 0, 1, 2, 3
DEBUG_HANDOVER_CANCEL, DEBUG_HANDOVER_EXPIRE, DEBUG_TRIP_EXPIRE = 1, 2, 3


def lib() -> C.CDLL:
    """Load the HIP library (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C stwo-ml_amd` "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise GkrError(rc, lib().gkr_last_error().decode())


# ------------------------------------------------------------------ conversions
def q_to_c(q: Sequence[int]) -> GkrQM31:
    x = GkrQM31()
    for i in range(4):
        x.v[i] = int(q[i])
    return x


def q_from_c(x: GkrQM31) -> QM31:
    return (x.v[0], x.v[1], x.v[2], x.v[3])


def q_array(qs: Sequence[Sequence[int]]):
    arr = (GkrQM31 * max(1, len(qs)))()
    for i, q in enumerate(qs):
        for j in range(4):
            arr[i].v[j] = int(q[j])
    return arr


def felt_to_c(v: int) -> GkrFelt:
    f = GkrFelt()
    for i in range(8):
        f.w[i] = (v >> (32 * i)) & 0xFFFFFFFF
    return f


def felt_from_c(f: GkrFelt) -> int:
    return sum(int(f.w[i]) << (32 * i) for i in range(8))


# ------------------------------------------------------------------ Poseidon
def hades_permute(state: Sequence[int]) -> List[int]:
    arr = (GkrFelt * 3)(*[felt_to_c(v) for v in state])
    _check(lib().gkr_hades_permute(arr))
    return [felt_from_c(arr[i]) for i in range(3)]


def poseidon_hash(a: int, b: int) -> int:
    out = GkrFelt()
    _check(lib().gkr_poseidon_hash(C.byref(felt_to_c(a)), C.byref(felt_to_c(b)), C.byref(out)))
    return felt_from_c(out)


def poseidon_hash_many(xs: Sequence[int]) -> int:
    arr = (GkrFelt * max(1, len(xs)))(*[felt_to_c(v) for v in xs])
    out = GkrFelt()
    _check(lib().gkr_poseidon_hash_many(arr, len(xs), C.byref(out)))
    return felt_from_c(out)


def policy_preset(name: str) -> dict:
    """PolicyConfig::strict / standard / relaxed (engine/src/policy.rs:131-203) as a field dict."""
    p = GkrPolicy()
    _check(lib().gkr_policy_preset(name.encode(), C.byref(p)))
    return {f: int(getattr(p, f)) for f in POLICY_FIELDS}


def policy_commitment(policy: dict) -> int:
    """PolicyConfig::policy_commitment (engine/src/policy.rs:236-254)."""
    p = GkrPolicy(*[int(policy[f]) for f in POLICY_FIELDS])
    out = GkrFelt()
    _check(lib().gkr_policy_commitment(C.byref(p), C.byref(out)))
    return felt_from_c(out)


class PoseidonChannel:
    """engine/src/crypto/poseidon_channel.rs:83 -- host Fiat-Shamir channel."""

    def __init__(self, _handle: Optional[int] = None):
        if _handle is None:
            h = C.c_void_p()
            _check(lib().gkr_channel_new(C.byref(h)))
            _handle = h.value
        self._h = _handle

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.gkr_channel_free(self._h)
            self._h = None

    @property
    def handle(self) -> int:
        return self._h

    def clone(self) -> "PoseidonChannel":
        h = C.c_void_p()
        _check(lib().gkr_channel_clone(self._h, C.byref(h)))
        return PoseidonChannel(h.value)

    def mix_u64(self, v: int) -> None:
        _check(lib().gkr_channel_mix_u64(self._h, v))

    def mix_felt(self, v: int) -> None:
        _check(lib().gkr_channel_mix_felt(self._h, C.byref(felt_to_c(v))))

    def mix_secure_field(self, q: Sequence[int]) -> None:
        _check(lib().gkr_channel_mix_secure_field(self._h, C.byref(q_to_c(q))))

    def mix_felts(self, qs: Sequence[Sequence[int]]) -> None:
        _check(lib().gkr_channel_mix_felts(self._h, q_array(qs), len(qs)))

    def mix_poly_coeffs(self, c0, c1, c2) -> None:
        _check(lib().gkr_channel_mix_poly_coeffs(self._h, q_array([c0, c1, c2])))

    def mix_poly_coeffs_deg3(self, c0, c1, c2, c3) -> None:
        _check(lib().gkr_channel_mix_poly_coeffs_deg3(self._h, q_array([c0, c1, c2, c3])))

    def draw_felt252(self) -> int:
        out = GkrFelt()
        _check(lib().gkr_channel_draw_felt252(self._h, C.byref(out)))
        return felt_from_c(out)

    def draw_qm31(self) -> QM31:
        out = GkrQM31()
        _check(lib().gkr_channel_draw_qm31(self._h, C.byref(out)))
        return q_from_c(out)

    def draw_qm31s(self, n: int) -> List[QM31]:
        arr = (GkrQM31 * max(1, n))()
        _check(lib().gkr_channel_draw_qm31s(self._h, n, arr))
        return [q_from_c(arr[i]) for i in range(n)]

    def digest(self) -> int:
        out = GkrFelt()
        _check(lib().gkr_channel_digest(self._h, C.byref(out)))
        return felt_from_c(out)

    def hash_count(self) -> int:
        return int(lib().gkr_channel_hash_count(self._h))

    def export_state(self) -> List[int]:
        st = (C.c_uint32 * 11)()
        _check(lib().gkr_channel_export(self._h, st))
        return list(st)

    def import_state(self, st: Sequence[int]) -> None:
        arr = (C.c_uint32 * 11)(*st)
        _check(lib().gkr_channel_import(self._h, arr))

    def seed_gkr(self, num_layers: int, in_rows: int, in_cols: int, policy_commitment: Optional[int] = None):
        pc = C.byref(felt_to_c(policy_commitment)) if policy_commitment is not None else None
        _check(lib().gkr_seed_channel(self._h, num_layers, in_rows, in_cols, pc))


# ------------------------------------------------------------------ device
class Context:
    """A device context: one HIP stream plus its device buffers."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().gkr_ctx_create(device, C.byref(h)))
        self._h = h.value

    def close(self):
        if getattr(self, "_h", None):
            lib().gkr_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        if _lib is not None:
            self.close()

    @property
    def handle(self) -> int:
        return self._h

    def synchronize(self):
        _check(lib().gkr_ctx_synchronize(self._h))

    def set_timing(self, level):
        """0 off; 1 (or True): k_restrict_cols events + host timers; 2: events on every timed kernel."""
        _check(lib().gkr_ctx_set_timing(self._h, int(level)))

    def reset_timing(self):
        _check(lib().gkr_ctx_reset_timing(self._h))

    def debug(self, op: int, arg: int = 0) -> None:
        """Test hook for the failure paths of the device waits (DEBUG_HANDOVER_CANCEL / DEBUG_HANDOVER_EXPIRE /
        DEBUG_TRIP_EXPIRE)."""
        _check(lib().gkr_ctx_debug(self._h, op, arg))

    def kernel_time(self, kid: int) -> Tuple[float, int, int]:
        ms, n, b = C.c_double(), C.c_uint64(), C.c_uint64()
        _check(lib().gkr_ctx_kernel_time(self._h, kid, C.byref(ms), C.byref(n), C.byref(b)))
        return ms.value, n.value, b.value

    def kernel_time_by_size(self, kid: int) -> List[Tuple[int, float, int]]:
        """[(bytes of one launch, total ms, launches)] per distinct launch size, smallest first."""
        n = C.c_size_t()
        _check(lib().gkr_ctx_kernel_time_by_size(self._h, kid, None, None, None, 0, C.byref(n)))
        k = n.value
        b, ms, nl = (C.c_uint64 * max(k, 1))(), (C.c_double * max(k, 1))(), (C.c_uint64 * max(k, 1))()
        _check(lib().gkr_ctx_kernel_time_by_size(self._h, kid, b, ms, nl, k, C.byref(n)))
        return [(b[i], ms[i], nl[i]) for i in range(min(k, n.value))]

    def bench_copy(self, nbytes: int = 1 << 32, iters: int = 5) -> Tuple[float, float]:
        """(copy GB/s counting read + write, read-only GB/s) of plain 128-bit streaming kernels."""
        cp, rd = C.c_double(), C.c_double()
        _check(lib().gkr_bench_copy(self._h, nbytes, iters, C.byref(cp), C.byref(rd)))
        return cp.value, rd.value

    # matrices
    def upload(self, m: np.ndarray) -> "Matrix":
        m = np.ascontiguousarray(m, dtype=np.uint32)
        assert m.ndim == 2
        h = C.c_void_p()
        _check(lib().gkr_matrix_upload(self._h, m.ctypes.data_as(_U32P), m.shape[0], m.shape[1], C.byref(h)))
        return Matrix(self, h.value, m.shape[0], m.shape[1])

    def wrap_device(self, ptr: int, rows: int, cols: int) -> "Matrix":
        h = C.c_void_p()
        _check(lib().gkr_matrix_wrap_device(self._h, C.c_void_p(ptr), rows, cols, C.byref(h)))
        return Matrix(self, h.value, rows, cols)

    def synthetic(self, rows: int, cols: int, kind: int, seed: int) -> "Matrix":
        h = C.c_void_p()
        _check(lib().gkr_matrix_synthetic(self._h, rows, cols, kind, seed, C.byref(h)))
        return Matrix(self, h.value, rows, cols)

    # ZkmlOps
    def reduce_matmul_layer(self, a: "Matrix", b: "Matrix", r_i, r_j, pk: int, ch: PoseidonChannel):
        T = pk.bit_length() - 1
        rp = (GkrQM31 * max(1, 3 * T))()
        chal = (GkrQM31 * max(1, T))()
        fa, fb = GkrQM31(), GkrQM31()
        _check(lib().gkr_reduce_matmul_layer(self._h, a.handle, b.handle, q_array(r_i), len(r_i), q_array(r_j),
                                             len(r_j), pk, ch.handle, rp, chal, C.byref(fa), C.byref(fb)))
        polys = [(q_from_c(rp[3 * t]), q_from_c(rp[3 * t + 1]), q_from_c(rp[3 * t + 2])) for t in range(T)]
        return {"round_polys": polys, "challenges": [q_from_c(chal[t]) for t in range(T)],
                "final_a_eval": q_from_c(fa), "final_b_eval": q_from_c(fb)}

    def evaluate_mle_at_point(self, mle, point) -> QM31:
        out = GkrQM31()
        _check(lib().gkr_evaluate_mle_at_point(self._h, q_array(mle), len(mle), q_array(point), len(point),
                                               C.byref(out)))
        return q_from_c(out)

    def restrict_mle(self, mle, assignments) -> List[QM31]:
        rest = len(mle) >> len(assignments)
        out = (GkrQM31 * max(1, rest))()
        _check(lib().gkr_restrict_mle(self._h, q_array(mle), len(mle), q_array(assignments), len(assignments), out))
        return [q_from_c(out[i]) for i in range(rest)]

    # GKR layer reducers
    def matmul_output_claim(self, a: "Matrix", b: "Matrix", r_out) -> QM31:
        out = GkrQM31()
        _check(lib().gkr_matmul_output_claim(self._h, a.handle, b.handle, q_array(r_out), len(r_out), C.byref(out)))
        return q_from_c(out)

    def prove_matmul_layer(self, claim_point, claim_value, a: "Matrix", b: "Matrix", ch: PoseidonChannel,
                           proof: Optional["Proof"] = None):
        pm = 1 << (a.rows - 1).bit_length()
        pk = 1 << (a.cols - 1).bit_length()
        T = pk.bit_length() - 1
        lm = pm.bit_length() - 1
        rp = (GkrQM31 * max(1, 3 * T))()
        fa, fb, nv = GkrQM31(), GkrQM31(), GkrQM31()
        npnt = (GkrQM31 * max(1, lm + T))()
        _check(lib().gkr_prove_matmul_layer(self._h, q_array(claim_point), len(claim_point),
                                            C.byref(q_to_c(claim_value)), a.handle, b.handle, ch.handle,
                                            proof.handle if proof else None, rp, C.byref(fa), C.byref(fb), npnt,
                                            C.byref(nv)))
        polys = [(q_from_c(rp[3 * t]), q_from_c(rp[3 * t + 1]), q_from_c(rp[3 * t + 2])) for t in range(T)]
        return {"round_polys": polys, "final_a_eval": q_from_c(fa), "final_b_eval": q_from_c(fb),
                "next_point": [q_from_c(npnt[i]) for i in range(lm + T)], "next_value": q_from_c(nv)}

    def prove_matmul_layer_simd(self, claim_point, claim_value, a_blocks, block_weights, b: "Matrix",
                                ch: PoseidonChannel, proof: Optional["Proof"] = None):
        """gkr_prove_matmul_layer_simd: reduce_matmul_layer_simd_gpu (gkr/prover.rs:5422-5600) over
        activation blocks a_blocks (Matrix list, same shape) with QM31 block_weights and one weight b."""
        a0 = a_blocks[0]
        pm = 1 << (a0.rows - 1).bit_length()
        pk = 1 << (a0.cols - 1).bit_length()
        T = pk.bit_length() - 1
        lm = pm.bit_length() - 1
        rp = (GkrQM31 * max(1, 3 * T))()
        fa, fb, nv = GkrQM31(), GkrQM31(), GkrQM31()
        npnt = (GkrQM31 * max(1, lm + T))()
        handles = (_P * len(a_blocks))(*[m.handle for m in a_blocks])
        _check(lib().gkr_prove_matmul_layer_simd(self._h, q_array(claim_point), len(claim_point),
                                                 C.byref(q_to_c(claim_value)), handles, q_array(block_weights),
                                                 len(a_blocks), b.handle, ch.handle,
                                                 proof.handle if proof else None, rp, C.byref(fa), C.byref(fb),
                                                 npnt, C.byref(nv)))
        polys = [(q_from_c(rp[3 * t]), q_from_c(rp[3 * t + 1]), q_from_c(rp[3 * t + 2])) for t in range(T)]
        return {"round_polys": polys, "final_a_eval": q_from_c(fa), "final_b_eval": q_from_c(fb),
                "next_point": [q_from_c(npnt[i]) for i in range(lm + T)], "next_value": q_from_c(nv)}

    def prove_matmul_layer_dual_simd(self, claim_point, claim_value, a_blocks, b_blocks, block_weights,
                                     ch: PoseidonChannel, proof: Optional["Proof"] = None):
        """gkr_prove_matmul_layer_dual_simd: reduce_matmul_layer_dual_simd_gpu (gkr/prover.rs:5615-5785);
        round polys are (c0, c1, c2, c3), block variables first."""
        nb = len(a_blocks)
        pk = 1 << (a_blocks[0].cols - 1).bit_length()
        rounds = (nb.bit_length() - 1) + (pk.bit_length() - 1)
        rp = (GkrQM31 * max(1, 4 * rounds))()
        fa, fb = GkrQM31(), GkrQM31()
        ha = (_P * nb)(*[m.handle for m in a_blocks])
        hb = (_P * len(b_blocks))(*[m.handle for m in b_blocks])
        _check(lib().gkr_prove_matmul_layer_dual_simd(self._h, q_array(claim_point), len(claim_point),
                                                      C.byref(q_to_c(claim_value)), ha, hb, q_array(block_weights),
                                                      nb, ch.handle, proof.handle if proof else None, rp,
                                                      C.byref(fa), C.byref(fb)))
        polys = [tuple(q_from_c(rp[4 * t + i]) for i in range(4)) for t in range(rounds)]
        return {"round_polys": polys, "final_a_eval": q_from_c(fa), "final_b_eval": q_from_c(fb),
                "n_block_vars": nb.bit_length() - 1}

    def qvec_upload(self, vals) -> "QVec":
        a = np.ascontiguousarray(vals, dtype=np.uint32).reshape(-1, 4)
        h = _P()
        _check(lib().gkr_qvec_upload(self._h, a.ctypes.data_as(_PQ), a.shape[0], C.byref(h)))
        return QVec(self, h.value, a.shape[0])

    def qvec_synthetic(self, n: int, seed: int) -> "QVec":
        h = _P()
        _check(lib().gkr_qvec_synthetic(self._h, n, seed, C.byref(h)))
        return QVec(self, h.value, n)

    def sumcheck_product(self, fa: "QVec", fb: "QVec", ch: PoseidonChannel):
        """gkr_sumcheck_product: the matmul round loop over resident QM31 vectors."""
        T = max(0, (fa.n - 1).bit_length())
        rp = (GkrQM31 * max(1, 3 * T))()
        chal = (GkrQM31 * max(1, T))()
        a, b = GkrQM31(), GkrQM31()
        _check(lib().gkr_sumcheck_product(self._h, fa.handle, fb.handle, ch.handle, rp, chal, C.byref(a),
                                          C.byref(b)))
        return {"round_polys": [(q_from_c(rp[3 * t]), q_from_c(rp[3 * t + 1]), q_from_c(rp[3 * t + 2]))
                                for t in range(T)],
                "challenges": [q_from_c(chal[t]) for t in range(T)],
                "final_a_eval": q_from_c(a), "final_b_eval": q_from_c(b)}

    def sumcheck_product_noalloc(self, fa_ptr: int, fb_ptr: int, n: int, ch: PoseidonChannel):
        """gkr_sumcheck_product_noalloc: the same round loop over caller-owned device memory (n canonical
        QM31 at each device pointer), with every device buffer in the library's static scratch array."""
        T = max(0, (n - 1).bit_length())
        rp = (GkrQM31 * max(1, 3 * T))()
        chal = (GkrQM31 * max(1, T))()
        a, b = GkrQM31(), GkrQM31()
        _check(lib().gkr_sumcheck_product_noalloc(self._h, C.cast(C.c_void_p(fa_ptr), _PQ),
                                                  C.cast(C.c_void_p(fb_ptr), _PQ), n, ch.handle, rp, chal,
                                                  C.byref(a), C.byref(b)))
        return {"round_polys": [(q_from_c(rp[3 * t]), q_from_c(rp[3 * t + 1]), q_from_c(rp[3 * t + 2]))
                                for t in range(T)],
                "challenges": [q_from_c(chal[t]) for t in range(T)],
                "final_a_eval": q_from_c(a), "final_b_eval": q_from_c(b)}

    def matmul_forward(self, a: "Matrix", b: "Matrix") -> "Matrix":
        """gkr_matmul_forward: C = A * B mod P as a new resident matrix."""
        h = _P()
        _check(lib().gkr_matmul_forward(self._h, a.handle, b.handle, C.byref(h)))
        return Matrix(self, h.value, a.rows, b.cols)

    def matmul_forward_into(self, a: "Matrix", b: "Matrix", out: "Matrix") -> None:
        """gkr_matmul_forward_into: C = A * B mod P written into an existing matrix."""
        _check(lib().gkr_matmul_forward_into(self._h, a.handle, b.handle, out.handle))

    def weight_commitment(self, b: "Matrix") -> int:
        """gkr_weight_commitment: commit_mle_root_only(matrix_to_mle_col_major_padded(B))."""
        out = GkrFelt()
        _check(lib().gkr_weight_commitment(self._h, b.handle, C.byref(out)))
        return felt_from_c(out)

    def weight_commitments(self, mats: Sequence["Matrix"]) -> List[int]:
        """gkr_weight_commitments: one root per matrix, hashed as one batch."""
        hs = (_P * max(1, len(mats)))(*[m.handle for m in mats])
        out = (GkrFelt * max(1, len(mats)))()
        _check(lib().gkr_weight_commitments(self._h, hs, len(mats), out))
        return [felt_from_c(out[i]) for i in range(len(mats))]

    def mle_commitment(self, evals: "QVec") -> int:
        """gkr_mle_commitment: commit_mle_root_only over resident QM31 values."""
        out = GkrFelt()
        _check(lib().gkr_mle_commitment(self._h, evals.handle, C.byref(out)))
        return felt_from_c(out)

    def prove_weight_opening(self, b: "Matrix", eval_point, ch: PoseidonChannel, proof: "Proof",
                             expected_value=None) -> int:
        """gkr_prove_weight_opening: opening appended to proof; returns the commitment."""
        cm = GkrFelt()
        ev = C.byref(q_to_c(expected_value)) if expected_value is not None else None
        _check(lib().gkr_prove_weight_opening(self._h, b.handle, q_array(eval_point), len(eval_point), ev,
                                              ch.handle, proof.handle, C.byref(cm)))
        return felt_from_c(cm)

    def prove_weight_openings(self, ch: PoseidonChannel, proof: "Proof") -> None:
        """gkr_prove_weight_openings: open every weight claim recorded in proof."""
        _check(lib().gkr_prove_weight_openings(self._h, ch.handle, proof.handle))

    def prove_weight_binding(self, ch: PoseidonChannel, proof: "Proof", mode: int) -> None:
        """gkr_prove_weight_binding: the weight phase in the given transcript mode."""
        _check(lib().gkr_prove_weight_binding(self._h, ch.handle, proof.handle, mode))

    def _mul_result(self, out, eq, nv, claim_point):
        return {"eq_round_polys": [tuple(q_from_c(eq[4 * t + j]) for j in range(4)) for t in range(nv)],
                "lhs_eval": q_from_c(out.lhs_eval), "rhs_eval": q_from_c(out.rhs_eval),
                "alpha": q_from_c(out.alpha), "next_point": [tuple(q) for q in claim_point],
                "next_value": q_from_c(out.next_value)}

    def prove_mul_layer(self, claim_point, claim_value, lhs: "Matrix", rhs: "Matrix", ch: PoseidonChannel,
                        proof: Optional["Proof"] = None):
        """gkr_prove_mul_layer: reduce_mul_layer over two resident matrices (padded to powers of two)."""
        nv = max(0, (_next_pow2(lhs.rows) * _next_pow2(lhs.cols) - 1).bit_length())
        eq = (GkrQM31 * max(1, 4 * nv))()
        out = GkrMulOut()
        out.eq_round_polys = C.cast(eq, _PQ)
        _check(lib().gkr_prove_mul_layer(self._h, q_array(claim_point), len(claim_point),
                                         C.byref(q_to_c(claim_value)), lhs.handle, rhs.handle, ch.handle,
                                         proof.handle if proof else None, C.byref(out)))
        return self._mul_result(out, eq, out.n_vars, claim_point)

    def reduce_mul_layer(self, claim_point, claim_value, lhs_vals, rhs_vals, ch: PoseidonChannel,
                         proof: Optional["Proof"] = None):
        """gkr_reduce_mul_layer: the reference signature, QM31 slices from the host ((n, 4) arrays)."""
        la = np.ascontiguousarray(lhs_vals, dtype=np.uint32).reshape(-1, 4)
        lb = np.ascontiguousarray(rhs_vals, dtype=np.uint32).reshape(-1, 4)
        n = la.shape[0]
        nv = max(0, (n - 1).bit_length())
        eq = (GkrQM31 * max(1, 4 * nv))()
        out = GkrMulOut()
        out.eq_round_polys = C.cast(eq, _PQ)
        _check(lib().gkr_reduce_mul_layer(self._h, q_array(claim_point), len(claim_point),
                                          C.byref(q_to_c(claim_value)), la.ctypes.data_as(_PQ),
                                          lb.ctypes.data_as(_PQ), n, ch.handle, proof.handle if proof else None,
                                          C.byref(out)))
        return self._mul_result(out, eq, out.n_vars, claim_point)

    def mul_output_claim(self, lhs: "Matrix", rhs: "Matrix", point) -> QM31:
        out = GkrQM31()
        _check(lib().gkr_mul_output_claim(self._h, lhs.handle, rhs.handle, q_array(point), len(point),
                                          C.byref(out)))
        return q_from_c(out)

    def prove_norm_layer(self, kind: int, claim_point, claim_value, inp: "Matrix", dim: int, ch: PoseidonChannel,
                         gamma=None, proof: Optional["Proof"] = None) -> dict:
        """gkr_prove_layernorm_layer (kind STEP_LAYERNORM) / gkr_prove_rmsnorm_layer (STEP_RMSNORM): a dict with
        the oracle's norm proof keys."""
        nv = len(claim_point)
        o, keep = _norm_struct(nv, _next_pow2(inp.rows))
        if kind == STEP_LAYERNORM:
            _check(lib().gkr_prove_layernorm_layer(self._h, q_array(claim_point), nv, C.byref(q_to_c(claim_value)),
                                                   inp.handle, dim, ch.handle, proof.handle if proof else None,
                                                   C.byref(o)))
        else:
            g = np.ascontiguousarray(gamma if gamma is not None else np.zeros(1), dtype=np.uint32)
            _check(lib().gkr_prove_rmsnorm_layer(self._h, q_array(claim_point), nv, C.byref(q_to_c(claim_value)),
                                                 inp.handle, dim, g.ctypes.data_as(_U32P),
                                                 0 if gamma is None else len(g), ch.handle,
                                                 proof.handle if proof else None, C.byref(o)))
        return _norm_dict(o, keep, nv)

    def norm_output_claim(self, kind: int, inp: "Matrix", dim: int, point, gamma=None) -> QM31:
        g = np.ascontiguousarray(gamma if gamma is not None else np.zeros(1), dtype=np.uint32)
        v = GkrQM31()
        _check(lib().gkr_norm_output_claim(self._h, kind, inp.handle, dim, g.ctypes.data_as(_U32P),
                                           0 if gamma is None else len(g), q_array(point), len(point), C.byref(v)))
        return q_from_c(v)

    def prove_activation_layer(self, claim_point, claim_value, inp: "Matrix", act_type: int, ch: PoseidonChannel,
                               table_log_size: int = 0, proof: Optional["Proof"] = None):
        if table_log_size == 0:
            table_log_size = 20 if act_type == 4 else 16
        nv = len(claim_point)
        eq = (GkrQM31 * max(1, 4 * nv))()
        mults = (C.c_uint32 * (1 << table_log_size))()
        mrp = (GkrQM31 * (2 * table_log_size))()
        out = GkrLogupOut()
        out.eq_round_polys = C.cast(eq, _PQ)
        out.multiplicities = C.cast(mults, _U32P)
        out.mult_round_polys = C.cast(mrp, _PQ)
        _check(lib().gkr_prove_activation_layer(self._h, q_array(claim_point), nv, C.byref(q_to_c(claim_value)),
                                                inp.handle, act_type, table_log_size, ch.handle,
                                                proof.handle if proof else None, C.byref(out)))
        return {
            "claimed_sum": q_from_c(out.claimed_sum),
            "eq_round_polys": [tuple(q_from_c(eq[4 * t + j]) for j in range(4)) for t in range(nv)],
            "final_evals": (q_from_c(out.w_eval), q_from_c(out.in_eval), q_from_c(out.out_eval)),
            "multiplicities": np.frombuffer(mults, dtype=np.uint32).copy(),
            "mult_round_polys": [(q_from_c(mrp[2 * t]), q_from_c(mrp[2 * t + 1])) for t in range(table_log_size)],
            "mult_final_eval": q_from_c(out.mult_final_eval),
            "mult_claimed_sum": q_from_c(out.mult_claimed_sum),
            "input_eval": q_from_c(out.input_eval),
            "output_eval": q_from_c(out.output_eval),
            "table_commitment": felt_from_c(out.table_commitment),
            "gamma": q_from_c(out.gamma),
            "beta": q_from_c(out.beta),
        }


def make_steps(steps) -> "C.Array":
    """steps: sequence of (kind, claim, a, b, activation_type, table_log_size[, dim]) with Matrix objects."""
    arr = (GkrStep * max(1, len(steps)))()
    for i, st in enumerate(steps):
        kind, claim, a, b, act, tlog = st[:6]
        arr[i].kind, arr[i].claim = kind, claim
        arr[i].a = a.handle if a is not None else None
        arr[i].b = b.handle if b is not None else None
        arr[i].activation_type, arr[i].table_log_size = act, tlog
        arr[i].dim = st[6] if len(st) > 6 else 0
    return arr


def prove_walk(ctx: "Context", ch: PoseidonChannel, steps, proof: "Proof", init_point=None, init_value=None,
               n_steps=None):
    """gkr_prove_walk: run the layer steps in order; returns the final (point, value) claim.

    `steps` is a list of (kind, claim, a, b, activation_type, table_log_size) tuples or an array
    from make_steps (then pass n_steps).
    """
    if isinstance(steps, (list, tuple)):
        arr, n = make_steps(steps), len(steps)
    else:
        arr, n = steps, (n_steps if n_steps is not None else len(steps))
    fp = (GkrQM31 * 64)()
    nf = C.c_uint32()
    fv = GkrQM31()
    ip = q_array(init_point) if init_point is not None else None
    iv = C.byref(q_to_c(init_value)) if init_value is not None else None
    _check(lib().gkr_prove_walk(ctx.handle, ch.handle, arr, n, ip, len(init_point) if init_point else 0, iv,
                                proof.handle if proof else None, fp, C.byref(nf), C.byref(fv)))
    return [q_from_c(fp[i]) for i in range(nf.value)], q_from_c(fv)


# ------------------------------------------------------------------ verifier replay (host only)
def verify_matmul_layer(claim_point, claim_value, m: int, k: int, n: int, round_polys, final_a, final_b,
                        ch: PoseidonChannel):
    """gkr_verify_matmul_layer (verify_matmul_reduction); round_polys: (c0, c1, c2) per round.
    Returns the input claim (point, value); raises GkrError (code 6) when a check fails."""
    rp = q_array([q for t in round_polys for q in t])
    npt = (GkrQM31 * 64)()
    nn = C.c_uint32()
    nv = GkrQM31()
    _check(lib().gkr_verify_matmul_layer(q_array(claim_point), len(claim_point), C.byref(q_to_c(claim_value)), m, k,
                                         n, rp, len(round_polys), C.byref(q_to_c(final_a)),
                                         C.byref(q_to_c(final_b)), ch.handle, npt, C.byref(nn), C.byref(nv)))
    return [q_from_c(npt[i]) for i in range(nn.value)], q_from_c(nv)


def verify_mul_layer(claim_point, claim_value, proof, ch: PoseidonChannel):
    """gkr_verify_mul_layer (verify_mul_reduction) on a proof dict as prove_mul_layer returns it."""
    rp = q_array([q for t in proof["eq_round_polys"] for q in t])
    nv = GkrQM31()
    _check(lib().gkr_verify_mul_layer(q_array(claim_point), len(claim_point), C.byref(q_to_c(claim_value)), rp,
                                      len(proof["eq_round_polys"]), C.byref(q_to_c(proof["lhs_eval"])),
                                      C.byref(q_to_c(proof["rhs_eval"])), ch.handle, C.byref(nv)))
    return q_from_c(nv)


def verify_activation_layer(claim_point, act_type: int, table_log_size: int, proof, ch: PoseidonChannel):
    """gkr_verify_activation_layer (LogUp branch of verify_activation_reduction) on a proof dict as
    prove_activation_layer returns it.  Returns the input claim value."""
    out = GkrLogupOut()
    nr = len(proof["eq_round_polys"])
    eq = q_array([q for t in proof["eq_round_polys"] for q in t])
    mults = np.ascontiguousarray(proof["multiplicities"], dtype=np.uint32)
    mrp = q_array([q for t in proof["mult_round_polys"] for q in t])
    out.claimed_sum = q_to_c(proof["claimed_sum"])
    out.eq_round_polys = C.cast(eq, _PQ)
    out.w_eval, out.in_eval, out.out_eval = (q_to_c(x) for x in proof["final_evals"])
    out.multiplicities = mults.ctypes.data_as(_U32P)
    out.mult_round_polys = C.cast(mrp, _PQ)
    out.mult_final_eval = q_to_c(proof["mult_final_eval"])
    out.mult_claimed_sum = q_to_c(proof["mult_claimed_sum"])
    out.input_eval = q_to_c(proof["input_eval"])
    out.output_eval = q_to_c(proof["output_eval"])
    out.table_commitment = felt_to_c(proof["table_commitment"])
    nv = GkrQM31()
    _check(lib().gkr_verify_activation_layer(q_array(claim_point), len(claim_point), act_type, table_log_size, nr,
                                             C.byref(out), ch.handle, C.byref(nv)))
    return q_from_c(nv)


def _norm_struct(nv: int, prow: int):
    keep = {"p0": (GkrQM31 * max(1, 4 * nv))(), "lin": (GkrQM31 * max(1, 4 * nv))(),
            "lg": (GkrQM31 * max(1, 4 * nv))(), "mult": np.zeros(1 << NORM_TABLE_LOG, dtype=np.uint32),
            "mrp": (GkrQM31 * (2 * NORM_TABLE_LOG))(), "rs0": np.zeros(max(1, prow), dtype=np.uint32),
            "rs1": np.zeros(max(1, prow), dtype=np.uint32)}
    o = GkrNormOut()
    o.p0_round_polys, o.lin_round_polys = C.cast(keep["p0"], C.POINTER(GkrQM31)), C.cast(keep["lin"], C.POINTER(GkrQM31))
    o.logup_round_polys = C.cast(keep["lg"], C.POINTER(GkrQM31))
    o.multiplicities = keep["mult"].ctypes.data_as(_U32P)
    o.mult_round_polys = C.cast(keep["mrp"], C.POINTER(GkrQM31))
    o.row_stats0, o.row_stats1 = keep["rs0"].ctypes.data_as(_U32P), keep["rs1"].ctypes.data_as(_U32P)
    return o, keep


def _norm_dict(o: GkrNormOut, keep, nv: int) -> dict:
    d = {dk: q_from_c(getattr(o, ck)) for ck, dk in NORM_Q_KEYS}
    for key, arr in (("p0_round_polys", "p0"), ("lin_round_polys", "lin"), ("logup_round_polys", "lg")):
        d[key] = [tuple(q_from_c(keep[arr][4 * t + j]) for j in range(4)) for t in range(nv)]
    d["multiplicities"] = keep["mult"].copy()
    d["mult_round_polys"] = [(q_from_c(keep["mrp"][2 * t]), q_from_c(keep["mrp"][2 * t + 1]))
                             for t in range(NORM_TABLE_LOG)]
    d["table_commitment"] = felt_from_c(o.table_commitment)
    d["gamma_commitment"] = felt_from_c(o.gamma_commitment)
    d["n_active"], d["n_rows"] = int(o.n_active), int(o.n_rows)
    d["row_stats0"] = [int(x) for x in keep["rs0"][:o.n_rows]]
    d["row_stats1"] = [int(x) for x in keep["rs1"][:o.n_rows]]
    return d


def verify_norm_layer(kind: int, claim_point, claim_value, dim: int, proof: dict, ch: PoseidonChannel) -> QM31:
    """gkr_verify_layernorm_layer / gkr_verify_rmsnorm_layer on a norm proof dict; returns the input claim value."""
    nv = len(claim_point)
    o, keep = _norm_struct(nv, max(1, proof["n_rows"]))
    for ck, dk in NORM_Q_KEYS:
        setattr(o, ck, q_to_c(proof[dk]))
    for key, arr in (("p0_round_polys", "p0"), ("lin_round_polys", "lin"), ("logup_round_polys", "lg")):
        for t, rp in enumerate(proof[key]):
            for j in range(4):
                keep[arr][4 * t + j] = q_to_c(rp[j])
    keep["mult"][:] = proof["multiplicities"]
    for t, (c0, c1) in enumerate(proof["mult_round_polys"]):
        keep["mrp"][2 * t], keep["mrp"][2 * t + 1] = q_to_c(c0), q_to_c(c1)
    keep["rs0"][:len(proof["row_stats0"])] = proof["row_stats0"]
    keep["rs1"][:len(proof["row_stats1"])] = proof["row_stats1"]
    o.table_commitment = felt_to_c(proof["table_commitment"])
    o.n_active, o.n_rows = proof["n_active"], proof["n_rows"]
    nx = GkrQM31()
    f = lib().gkr_verify_layernorm_layer if kind == STEP_LAYERNORM else lib().gkr_verify_rmsnorm_layer
    _check(f(q_array(claim_point), nv, C.byref(q_to_c(claim_value)), dim, C.byref(o), ch.handle, C.byref(nx)))
    return q_from_c(nx)


def felts_to_words(felts) -> np.ndarray:
    """felt252 ints -> (n, 8) little-endian u32 words."""
    out = np.zeros((len(felts), 8), dtype=np.uint32)
    for i, v in enumerate(felts):
        for j in range(8):
            out[i, j] = (v >> (32 * j)) & 0xFFFFFFFF
    return out


def verify_walk(calldata, shapes, init_point, init_value, ch: PoseidonChannel, fresh_values=()):
    """gkr_verify_walk: a walk from serialized calldata (felt ints, or an (n, 8) u32 word array).
    shapes: sequence of (kind, rows, cols, cols_b, activation_type, table_log_size[, claim]);
    fresh_values: the claim values of the fresh MatMul / Mul layers, in order.  Returns
    (point, value, felts read)."""
    if isinstance(calldata, np.ndarray):
        words = np.ascontiguousarray(calldata, dtype=np.uint32).reshape(-1, 8)
        n_felts = len(words)
        cd = words.ctypes.data_as(C.POINTER(GkrFelt))
    else:
        n_felts = len(calldata)
        cd = (GkrFelt * max(1, n_felts))()
        for i, v in enumerate(calldata):
            cd[i] = felt_to_c(v)
    sh = (GkrLayerShape * max(1, len(shapes)))()
    for i, shp in enumerate(shapes):
        kind, rows, cols, cols_b, act, tlog = shp[:6]
        sh[i].kind, sh[i].rows, sh[i].cols, sh[i].cols_b = kind, rows, cols, cols_b
        sh[i].activation_type, sh[i].table_log_size = act, tlog
        sh[i].claim = shp[6] if len(shp) > 6 else CLAIM_CHAINED
        sh[i].dim = shp[7] if len(shp) > 7 else 0
    fp = (GkrQM31 * 64)()
    nf = C.c_uint32()
    fv = GkrQM31()
    used = C.c_size_t()
    ip = init_point or []
    _check(lib().gkr_verify_walk(cd, n_felts, sh, len(shapes), q_array(ip), len(ip),
                                 C.byref(q_to_c(init_value)) if init_value is not None else None,
                                 q_array(fresh_values), len(fresh_values), ch.handle, fp, C.byref(nf),
                                 C.byref(fv), C.byref(used)))
    return [q_from_c(fp[i]) for i in range(nf.value)], q_from_c(fv), used.value


class Matrix:
    def __init__(self, ctx: Context, handle: int, rows: int, cols: int):
        self.ctx, self._h, self.rows, self.cols = ctx, handle, rows, cols

    @property
    def device_ptr(self) -> int:
        """Device address of the row-major u32 entries (gkr_matrix_device_ptr)."""
        return lib().gkr_matrix_device_ptr(self._h)

    def invalidate(self) -> None:
        """gkr_matrix_invalidate: the entries changed outside the library (wrapped device memory
        written by the caller); the copies derived from them are rebuilt on the next use."""
        _check(lib().gkr_matrix_invalidate(self.ctx.handle, self._h))

    def cached_commitment(self) -> Optional[int]:
        """gkr_matrix_commitment_cached: the weight commitment kept on the matrix, or None."""
        f = GkrFelt()
        cached = C.c_int()
        _check(lib().gkr_matrix_commitment_cached(self._h, C.byref(f), C.byref(cached)))
        return felt_from_c(f) if cached.value else None

    def set_commitment(self, root: int) -> None:
        """gkr_matrix_set_commitment: keep `root` as this weight's commitment."""
        _check(lib().gkr_matrix_set_commitment(self.ctx.handle, self._h, C.byref(felt_to_c(root))))

    @property
    def handle(self) -> int:
        return self._h

    def download(self) -> np.ndarray:
        out = np.empty((self.rows, self.cols), dtype=np.uint32)
        _check(lib().gkr_matrix_download(self.ctx.handle, self._h, out.ctypes.data_as(_U32P)))
        return out

    def free(self):
        if self._h:
            lib().gkr_matrix_free(self._h)
            self._h = None

    def __del__(self):
        if _lib is not None and getattr(self, "_h", None):
            self.free()


class QVec:
    """A resident QM31 vector (gkr_qvec)."""

    def __init__(self, ctx: "Context", handle: int, n: int):
        self.ctx, self._h, self.n = ctx, handle, n

    @property
    def handle(self) -> int:
        return self._h

    def download(self) -> np.ndarray:
        out = np.empty((self.n, 4), dtype=np.uint32)
        _check(lib().gkr_qvec_download(self.ctx.handle, self._h, out.ctypes.data_as(_PQ)))
        return out

    @property
    def device_ptr(self) -> int:
        """Device address of the n QM31 (gkr_qvec_device_ptr)."""
        return lib().gkr_qvec_device_ptr(self._h)

    def __del__(self):
        if self._h and _lib is not None:
            _lib.gkr_qvec_free(self._h)
            self._h = None


class Proof:
    """GKRProof container (engine/src/gkr/types.rs:589-643)."""

    def __init__(self):
        h = C.c_void_p()
        _check(lib().gkr_proof_new(C.byref(h)))
        self._h = h.value

    def __del__(self):
        if _lib is not None and getattr(self, "_h", None):
            _lib.gkr_proof_free(self._h)
            self._h = None

    @property
    def handle(self) -> int:
        return self._h

    def num_layers(self) -> int:
        return int(lib().gkr_proof_num_layers(self._h))

    def set_input_claim(self, point, value):
        _check(lib().gkr_proof_set_input_claim(self._h, q_array(point), len(point), C.byref(q_to_c(value))))

    def add_weight_commitment(self, c: int):
        _check(lib().gkr_proof_add_weight_commitment(self._h, C.byref(felt_to_c(c))))

    def set_io_commitment(self, c: int):
        _check(lib().gkr_proof_set_io_commitment(self._h, C.byref(felt_to_c(c))))

    def serialize(self) -> List[int]:
        n = C.c_size_t()
        rc = lib().gkr_proof_serialize(self._h, None, 0, C.byref(n))
        if rc not in (0, 5):
            _check(rc)
        arr = (GkrFelt * max(1, n.value))()
        _check(lib().gkr_proof_serialize(self._h, arr, n.value, C.byref(n)))
        return [felt_from_c(arr[i]) for i in range(n.value)]

    def stream_to(self, out: Optional[np.ndarray]) -> None:
        """Serialize each layer into out, an (cap, 8) uint32 array of felt words, as the reducers append
        it (gkr_proof_stream_to); serialize_into(out) then writes only the count and the tail.  None
        ends the streaming.  The proof keeps a reference to out."""
        if out is None:
            _check(lib().gkr_proof_stream_to(self._h, None, 0))
            self._stream_buf = None
            return
        assert out.dtype == np.uint32 and out.ndim == 2 and out.shape[1] == 8 and out.flags["C_CONTIGUOUS"]
        self._stream_buf = out
        _check(lib().gkr_proof_stream_to(self._h, out.ctypes.data_as(C.POINTER(GkrFelt)), out.shape[0]))

    def serialize_into(self, out: np.ndarray) -> int:
        """gkr_proof_serialize into out ((cap, 8) uint32); returns the felt count."""
        assert out.dtype == np.uint32 and out.ndim == 2 and out.shape[1] == 8 and out.flags["C_CONTIGUOUS"]
        n = C.c_size_t()
        _check(lib().gkr_proof_serialize(self._h, out.ctypes.data_as(C.POINTER(GkrFelt)), out.shape[0], C.byref(n)))
        return n.value

    def serialize_words(self) -> np.ndarray:
        """The serialized proof as an (n, 8) array of little-endian u32 felt words (no int conversion)."""
        n = C.c_size_t()
        rc = lib().gkr_proof_serialize(self._h, None, 0, C.byref(n))
        if rc not in (0, 5):
            _check(rc)
        out = np.zeros((max(1, n.value), 8), dtype=np.uint32)
        _check(lib().gkr_proof_serialize(self._h, out.ctypes.data_as(C.POINTER(GkrFelt)), n.value, C.byref(n)))
        return out[:n.value]

    def binding_groups(self) -> List[List[int]]:
        """The serialized aggregated binding proofs of GKR_WEIGHT_AGGREGATED_FULL, one per group."""
        out = []
        for g in range(lib().gkr_proof_num_binding_groups(self._h)):
            n = C.c_size_t()
            rc = lib().gkr_proof_binding_group(self._h, g, None, 0, C.byref(n))
            if rc not in (0, 5):
                _check(rc)
            arr = (GkrFelt * max(1, n.value))()
            _check(lib().gkr_proof_binding_group(self._h, g, arr, n.value, C.byref(n)))
            out.append([felt_from_c(arr[i]) for i in range(n.value)])
        return out

    def layer_claim_value(self, layer: int) -> QM31:
        """The output-claim value layer `layer` was proved against (gkr_proof_layer_claim_value)."""
        v = GkrQM31()
        _check(lib().gkr_proof_layer_claim_value(self._h, layer, C.byref(v)))
        return q_from_c(v)


def activation_table(act_type: int, log_size: int) -> np.ndarray:
    out = np.empty(1 << log_size, dtype=np.uint32)
    _check(lib().gkr_activation_table(act_type, log_size, out.ctypes.data_as(_U32P)))
    return out


def synthetic_value(kind: int, seed: int, i: int) -> int:
    return int(lib().gkr_synthetic_value(kind, seed, i))


# ------------------------------------------------------------------ STWO LogUp-GKR batch
LOOKUP_GRAND_PRODUCT, LOOKUP_LOGUP_GENERIC, LOOKUP_LOGUP_MULTIPLICITIES, LOOKUP_LOGUP_SINGLES = 0, 1, 2, 3


class GkrLookupInstance(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("n_vars", C.c_uint32), ("numerators", C.c_void_p),
                ("denominators", C.c_void_p)]


class GkrLookupBatch(C.Structure):
    _fields_ = [("output_claims", _PQ), ("round_polys", _PQ), ("round_poly_lens", _U32P), ("masks", _PQ),
                ("ood_point", _PQ), ("claims_to_verify", _PQ), ("n_layers", C.c_uint32)]


def _lookup_buffers(n_inst: int, n_layers: int):
    n_rounds = max(1, n_layers * (n_layers - 1) // 2)
    keep = {"oc": (GkrQM31 * (2 * n_inst))(), "rp": (GkrQM31 * (4 * n_rounds))(),
            "rl": np.zeros(n_rounds, dtype=np.uint32), "mk": (GkrQM31 * (4 * max(1, n_layers) * n_inst))(),
            "ood": (GkrQM31 * max(1, n_layers))(), "cv": (GkrQM31 * (2 * n_inst))()}
    b = GkrLookupBatch()
    b.output_claims, b.round_polys = C.cast(keep["oc"], _PQ), C.cast(keep["rp"], _PQ)
    b.round_poly_lens = keep["rl"].ctypes.data_as(_U32P)
    b.masks, b.ood_point, b.claims_to_verify = C.cast(keep["mk"], _PQ), C.cast(keep["ood"], _PQ), C.cast(keep["cv"], _PQ)
    return b, keep


def lookup_gate(kind: int) -> int:
    return 0 if kind == LOOKUP_GRAND_PRODUCT else 1


def _lookup_result(keep, kinds, nvs, n_layers) -> dict:
    """The proof as a dict with the oracle's keys (oracle.prove_lookup_batch)."""
    n_inst = len(kinds)
    ncl = [1 if k == LOOKUP_GRAND_PRODUCT else 2 for k in kinds]
    d = {"kinds": list(kinds), "n_vars": list(nvs), "n_layers": n_layers,
         "output_claims": [[q_from_c(keep["oc"][2 * i + c]) for c in range(ncl[i])] for i in range(n_inst)],
         "claims_to_verify": [[q_from_c(keep["cv"][2 * i + c]) for c in range(ncl[i])] for i in range(n_inst)],
         "ood_point": [q_from_c(keep["ood"][k]) for k in range(n_layers)], "round_polys": [], "masks": []}
    r = 0
    for layer in range(n_layers):
        polys = []
        for _ in range(layer):
            polys.append([q_from_c(keep["rp"][4 * r + c]) for c in range(int(keep["rl"][r]))])
            r += 1
        d["round_polys"].append(polys)
    for layer in range(n_layers):
        d["masks"].append([[q_from_c(keep["mk"][4 * (layer * n_inst + i) + c]) for c in range(2 * ncl[i])]
                           if layer >= n_layers - nvs[i] else None for i in range(n_inst)])
    return d


def prove_lookup_batch(ctx: "Context", ch: PoseidonChannel, instances) -> dict:
    """gkr_prove_lookup_batch.  instances: (kind, n_vars, numerators, denominators) with device
    columns given as QVec / Matrix objects or device addresses (None where the kind has none)."""
    arr = (GkrLookupInstance * max(1, len(instances)))()
    n_layers = 0
    ptr = lambda v: None if v is None else (v if isinstance(v, int) else v.device_ptr)  # noqa: E731
    for i, (kind, nv, num, den) in enumerate(instances):
        arr[i].kind, arr[i].n_vars = kind, nv
        arr[i].numerators, arr[i].denominators = ptr(num), ptr(den)
        n_layers = max(n_layers, nv)
    b, keep = _lookup_buffers(len(instances), n_layers)
    _check(lib().gkr_prove_lookup_batch(ctx.handle, ch.handle, arr, len(instances), C.byref(b)))
    return _lookup_result(keep, [x[0] for x in instances], [x[1] for x in instances], n_layers)


def _lookup_fill(d):
    n_inst, n_layers = len(d["kinds"]), d["n_layers"]
    b, keep = _lookup_buffers(n_inst, n_layers)
    b.n_layers = n_layers
    for i in range(n_inst):
        for c, v in enumerate(d["output_claims"][i]):
            keep["oc"][2 * i + c] = q_to_c(v)
    r = 0
    for layer in range(n_layers):
        for poly in d["round_polys"][layer]:
            keep["rl"][r] = len(poly)
            for c, v in enumerate(poly):
                keep["rp"][4 * r + c] = q_to_c(v)
            r += 1
        for i in range(n_inst):
            m = d["masks"][layer][i]
            if m is not None:
                for c, v in enumerate(m):
                    keep["mk"][4 * (layer * n_inst + i) + c] = q_to_c(v)
    gates = np.array([lookup_gate(k) for k in d["kinds"]], dtype=np.uint32)
    nvs = np.array(d["n_vars"], dtype=np.uint32)
    return b, keep, gates, nvs


def verify_lookup_batch(d: dict, ch: PoseidonChannel):
    """gkr_verify_lookup_batch on a proof dict; returns (ood_point, claims_to_verify)."""
    b, keep, gates, nvs = _lookup_fill(d)
    ood = (GkrQM31 * max(1, d["n_layers"]))()
    cv = (GkrQM31 * (2 * len(gates)))()
    _check(lib().gkr_verify_lookup_batch(gates.ctypes.data_as(_U32P), nvs.ctypes.data_as(_U32P), len(gates),
                                         C.byref(b), ch.handle, ood, cv))
    ncl = [1 if g == 0 else 2 for g in gates]
    return ([q_from_c(ood[k]) for k in range(d["n_layers"])],
            [[q_from_c(cv[2 * i + c]) for c in range(ncl[i])] for i in range(len(gates))])


def serialize_lookup_batch(d: dict) -> List[int]:
    """gkr_serialize_lookup_batch (serialize_stwo_gkr_batch_proof) as felt ints."""
    b, keep, gates, nvs = _lookup_fill(d)
    n = C.c_size_t()
    rc = lib().gkr_serialize_lookup_batch(gates.ctypes.data_as(_U32P), nvs.ctypes.data_as(_U32P), len(gates),
                                          C.byref(b), None, 0, C.byref(n))
    if rc not in (0, 5):
        _check(rc)
    out = (GkrFelt * max(1, n.value))()
    _check(lib().gkr_serialize_lookup_batch(gates.ctypes.data_as(_U32P), nvs.ctypes.data_as(_U32P), len(gates),
                                            C.byref(b), out, n.value, C.byref(n)))
    return [felt_from_c(out[i]) for i in range(n.value)]


# ------------------------------------------------------------------ aggregated weight binding
class GkrBindingClaim(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("eval_point", _PQ), ("n_point", C.c_uint32), ("expected_value", GkrQM31),
                ("commitment", GkrFelt)]


def prove_aggregated_binding(ctx: "Context", ch: PoseidonChannel, claims) -> List[int]:
    """gkr_prove_aggregated_binding: claims are (weight Matrix, eval point, expected value, commitment int);
    returns the serialize_aggregated_binding_proof felts."""
    arr = (GkrBindingClaim * max(1, len(claims)))()
    keep = []
    for i, (w, pt, v, cm) in enumerate(claims):
        qa = q_array(pt)
        keep.append(qa)
        arr[i].weight, arr[i].eval_point, arr[i].n_point = w.handle, C.cast(qa, _PQ), len(pt)
        arr[i].expected_value, arr[i].commitment = q_to_c(v), felt_to_c(cm)
    n = C.c_size_t()
    rc = lib().gkr_prove_aggregated_binding(ctx.handle, ch.handle, arr, len(claims), None, 0, C.byref(n))
    if rc != 5:
        _check(rc)
    out = (GkrFelt * max(1, n.value))()
    _check(lib().gkr_prove_aggregated_binding(ctx.handle, ch.handle, arr, len(claims), out, n.value, C.byref(n)))
    return [felt_from_c(out[i]) for i in range(n.value)]
