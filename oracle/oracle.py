"""ctypes wrapper of the CPU oracle (_build/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker and the timed CPU baseline.  QM31 values are 4-tuples,
felts are Python ints, matrices are numpy uint32 arrays.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import List, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
P = (1 << 31) - 1

_lib = None
_U32P = C.POINTER(C.c_uint32)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        L.orc_channel_size.restype = C.c_size_t
        L.orc_synthetic_value.restype = C.c_uint32
        L.orc_synthetic_value.argtypes = [C.c_int, C.c_uint64, C.c_uint64]
        L.orc_synthetic_fill.argtypes = [_U32P, C.c_size_t, C.c_int, C.c_uint64]
        L.orc_mix_u64.argtypes = [C.c_void_p, C.c_uint64]
        L.orc_activation.restype = C.c_uint32
        L.orc_activation.argtypes = [C.c_uint32, C.c_uint32]
        for name in ("orc_m31_add", "orc_m31_sub", "orc_m31_mul"):
            getattr(L, name).restype = C.c_uint32
            getattr(L, name).argtypes = [C.c_uint32, C.c_uint32]
        L.orc_m31_inv.restype = C.c_uint32
        L.orc_m31_inv.argtypes = [C.c_uint32]
        L.orc_reduce_matmul_layer.argtypes = [_U32P, C.c_size_t, C.c_size_t, _U32P, C.c_size_t, _U32P, C.c_int,
                                              _U32P, C.c_int, C.c_size_t, C.c_void_p, _U32P, _U32P, _U32P, _U32P]
        L.orc_prove_matmul_layer.argtypes = [_U32P, C.c_int, _U32P, _U32P, C.c_size_t, C.c_size_t, _U32P,
                                             C.c_size_t, C.c_void_p, _U32P, _U32P, _U32P, _U32P, _U32P]
        L.orc_matmul_output_claim.argtypes = [_U32P, C.c_size_t, C.c_size_t, _U32P, C.c_size_t, _U32P, C.c_int,
                                              _U32P]
        L.orc_matmul_forward.argtypes = [_U32P, C.c_size_t, C.c_size_t, _U32P, C.c_size_t, _U32P]
        L.orc_restrict_cols_fused.argtypes = [_U32P, C.c_size_t, C.c_size_t, _U32P, C.c_int, C.c_size_t, _U32P]
        L.orc_restrict_rows_fused.argtypes = [_U32P, C.c_size_t, C.c_size_t, _U32P, C.c_int, C.c_size_t, _U32P]
        L.orc_restrict_mle.argtypes = [_U32P, C.c_size_t, _U32P, C.c_int, _U32P]
        L.orc_evaluate_mle.argtypes = [_U32P, C.c_int, _U32P, _U32P]
        L.orc_prove_activation_layer.argtypes = [_U32P, C.c_int, _U32P, _U32P, C.c_size_t, C.c_size_t, C.c_uint32,
                                                 C.c_uint32, C.c_void_p] + [_U32P] * 9
        L.orc_verify_matmul_layer.argtypes = [_U32P, C.c_int, _U32P, C.c_size_t, C.c_size_t, C.c_size_t, _U32P,
                                              C.c_int, _U32P, _U32P, C.c_void_p, _U32P, _U32P]
        L.orc_verify_activation_layer.argtypes = [_U32P, C.c_int, _U32P, C.c_uint32, C.c_uint32, _U32P, _U32P,
                                                  C.c_int] + [_U32P] * 6 + [C.c_void_p]
        L.orc_mle_commitment.argtypes = [_U32P, C.c_size_t, _U32P]
        L.orc_mle_opening.restype = C.c_size_t
        L.orc_mle_opening.argtypes = [_U32P, C.c_size_t, _U32P, C.c_size_t, C.c_void_p, _U32P, _U32P, C.c_size_t]
        L.orc_weight_commitment.argtypes = [_U32P, C.c_size_t, C.c_size_t, _U32P]
        L.orc_sumcheck_product.argtypes = [_U32P, _U32P, C.c_size_t, C.c_void_p, _U32P, _U32P, _U32P, _U32P]
        L.orc_reduce_mul_layer.argtypes = [_U32P, C.c_int, _U32P, _U32P, _U32P, C.c_size_t, C.c_void_p] + [_U32P] * 5
        L.orc_verify_mul_layer.argtypes = [_U32P, C.c_int, _U32P, _U32P, C.c_int, _U32P, _U32P, C.c_void_p, _U32P]
        _lib = L
    return _lib


def _qa(qs: Sequence[Sequence[int]]) -> np.ndarray:
    if isinstance(qs, np.ndarray) and qs.dtype == np.uint32 and qs.ndim == 2 and qs.shape[1] == 4 and len(qs):
        return np.ascontiguousarray(qs)
    a = np.zeros((max(1, len(qs)), 4), dtype=np.uint32)
    for i, q in enumerate(qs):
        a[i] = q
    return a


def _p(a: np.ndarray):
    return a.ctypes.data_as(_U32P)


def _q(a: np.ndarray, i: int = 0):
    return tuple(int(x) for x in a.reshape(-1, 4)[i])


def felt_words(v: int) -> np.ndarray:
    return np.array([(v >> (32 * i)) & 0xFFFFFFFF for i in range(8)], dtype=np.uint32)


def felt_int(w) -> int:
    return sum(int(w[i]) << (32 * i) for i in range(8))


# PolicyConfig (engine/src/policy.rs:48-121): its fields in declaration order,
# the presets strict / standard / relaxed (policy.rs:131-203), and
# policy_commitment (policy.rs:236-254): poseidon_hash_many of the domain
# separator "POL" + version 1 (policy.rs:28) and the fields as integers
# (weight_binding_mode: Individual 0, Aggregated 1, TrustlessMode2 2,
# TrustlessMode3 3, policy.rs:30-43).
POLICY_FIELDS = ("allow_missing_norm_proof", "allow_logup_activation", "allow_missing_segment_binding",
                 "skip_rms_sq_proof", "piecewise_activation", "skip_batch_tokens", "skip_unified_stark",
                 "weight_binding_mode", "aggregated_full_binding", "aggregated_rlc_only", "io_packing", "packed_proof",
                 "double_packed_proof", "validate_decode_chain")
POLICY_PRESETS = {
    "strict": dict(allow_missing_norm_proof=0, allow_logup_activation=0, allow_missing_segment_binding=0,
                   skip_rms_sq_proof=0, piecewise_activation=1, skip_batch_tokens=0, skip_unified_stark=0,
                   weight_binding_mode=1, aggregated_full_binding=1, aggregated_rlc_only=0, io_packing=1,
                   packed_proof=1, double_packed_proof=1, validate_decode_chain=1),
    "standard": dict(allow_missing_norm_proof=1, allow_logup_activation=1, allow_missing_segment_binding=0,
                     skip_rms_sq_proof=1, piecewise_activation=0, skip_batch_tokens=1, skip_unified_stark=1,
                     weight_binding_mode=1, aggregated_full_binding=1, aggregated_rlc_only=0, io_packing=1,
                     packed_proof=1, double_packed_proof=1, validate_decode_chain=1),
    "relaxed": dict(allow_missing_norm_proof=1, allow_logup_activation=1, allow_missing_segment_binding=1,
                    skip_rms_sq_proof=1, piecewise_activation=1, skip_batch_tokens=1, skip_unified_stark=1,
                    weight_binding_mode=1, aggregated_full_binding=0, aggregated_rlc_only=0, io_packing=1,
                    packed_proof=1, double_packed_proof=1, validate_decode_chain=0),
}


def policy_commitment(policy: dict) -> int:
    return hash_many([0x504F4C01] + [int(policy[f]) for f in POLICY_FIELDS])


class Channel:
    """Oracle PoseidonChannel (engine/src/crypto/poseidon_channel.rs:83-308)."""

    def __init__(self):
        self.buf = (C.c_uint8 * int(lib().orc_channel_size()))()
        lib().orc_channel_init(self.buf)

    def clone(self) -> "Channel":
        c = Channel()
        C.memmove(c.buf, self.buf, len(self.buf))
        return c

    def mix_u64(self, v: int):
        lib().orc_mix_u64(self.buf, v)

    def mix_felt(self, v: int):
        lib().orc_mix_felt(self.buf, _p(felt_words(v)))

    def mix_secure_field(self, q):
        lib().orc_mix_secure_field(self.buf, _p(_qa([q])))

    def mix_felts(self, qs):
        lib().orc_mix_felts(self.buf, _p(_qa(qs)), C.c_size_t(len(qs)))

    def mix_poly_coeffs(self, c0, c1, c2):
        lib().orc_mix_poly_coeffs(self.buf, _p(_qa([c0, c1, c2])))

    def mix_poly_coeffs_deg3(self, c0, c1, c2, c3):
        lib().orc_mix_poly_coeffs_deg3(self.buf, _p(_qa([c0, c1, c2, c3])))

    def draw_qm31(self):
        out = np.zeros(4, dtype=np.uint32)
        lib().orc_draw_qm31(self.buf, _p(out))
        return _q(out)

    def draw_qm31s(self, n: int):
        return [self.draw_qm31() for _ in range(n)]

    def draw_felt252(self) -> int:
        out = np.zeros(8, dtype=np.uint32)
        lib().orc_draw_felt252(self.buf, _p(out))
        return felt_int(out)

    def digest(self) -> int:
        out = np.zeros(8, dtype=np.uint32)
        lib().orc_digest(self.buf, _p(out))
        return felt_int(out)


def trace_point(ch: "Channel", label: str, index: int = -1) -> None:
    """orc_trace: one line of the ORACLE_CHANNEL_TRACE transcript trace (a walk's step boundaries are
    marked from Python, the layers' own points from C)."""
    lib().orc_trace(ch.buf, label.encode(), C.c_long(index))


def channel_state(ch: "Channel") -> List[int]:
    """The channel in the reference's to_gpu_state layout (poseidon_channel.rs:109-135): 8 LE u32
    words of the canonical digest, n_draws, hash_count lo, hash_count hi."""
    d = ch.digest()
    words = [(d >> (32 * i)) & 0xFFFFFFFF for i in range(8)]
    raw = bytes(ch.buf)
    n_draws = int.from_bytes(raw[32:36], "little")
    hash_count = int.from_bytes(raw[40:48], "little")
    return words + [n_draws, hash_count & 0xFFFFFFFF, hash_count >> 32]


def set_channel_state(ch: "Channel", st) -> None:
    """Load a to_gpu_state layout (11 words, see channel_state) into an oracle channel."""
    lib().orc_channel_set_state(ch.buf, _p(np.ascontiguousarray(st, dtype=np.uint32)))


def hash_many(xs: Sequence[int]) -> int:
    a = np.concatenate([felt_words(x) for x in xs]) if xs else np.zeros(8, dtype=np.uint32)
    out = np.zeros(8, dtype=np.uint32)
    lib().orc_hash_many(_p(a), C.c_size_t(len(xs)), _p(out))
    return felt_int(out)


def hades(state: Sequence[int]) -> List[int]:
    a = np.concatenate([felt_words(x) for x in state])
    lib().orc_hades(_p(a))
    return [felt_int(a[8 * i:8 * i + 8]) for i in range(3)]


def hades_constant(idx: int) -> int:
    out = np.zeros(8, dtype=np.uint32)
    lib().orc_hades_constant(idx, _p(out))
    return felt_int(out)


def qmul(x, y):
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_qm31_mul(_p(_qa([x])), _p(_qa([y])), _p(out))
    return _q(out)


def qadd(x, y):
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_qm31_add(_p(_qa([x])), _p(_qa([y])), _p(out))
    return _q(out)


def qsub(x, y):
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_qm31_sub(_p(_qa([x])), _p(_qa([y])), _p(out))
    return _q(out)


def qinv(x):
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_qm31_inv(_p(_qa([x])), _p(out))
    return _q(out)


def evaluate_mle(evals: Sequence, point: Sequence):
    e = _qa(evals)
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_evaluate_mle(_p(e), len(point), _p(_qa(point)), _p(out))
    return _q(out)


def inner_product_q(fa: np.ndarray, fb: np.ndarray):
    """sum_i fa[i] * fb[i] over two QM31 vectors ((n, 4) arrays)."""
    a = np.ascontiguousarray(fa, dtype=np.uint32).reshape(-1, 4)
    b = np.ascontiguousarray(fb, dtype=np.uint32).reshape(-1, 4)
    assert a.shape == b.shape
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_inner_product_q(_p(a), _p(b), C.c_size_t(a.shape[0]), _p(out))
    return _q(out)


def restrict_mle(evals: Sequence, assign: Sequence):
    e = _qa(evals)
    out = np.zeros((len(evals) >> len(assign), 4), dtype=np.uint32)
    lib().orc_restrict_mle(_p(e), len(evals), _p(_qa(assign)), len(assign), _p(out))
    return [_q(out, i) for i in range(out.shape[0])]


def eq_evals(r: Sequence):
    out = np.zeros((1 << len(r), 4), dtype=np.uint32)
    lib().orc_eq_evals(_p(_qa(r)), len(r), _p(out))
    return out


def lagrange_basis(c: Sequence):
    out = np.zeros((1 << len(c), 4), dtype=np.uint32)
    lib().orc_lagrange_basis(_p(_qa(c)), len(c), _p(out))
    return out


def _next_pow2(v: int) -> int:
    return 1 << max(0, (v - 1).bit_length())


def matmul_forward(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.uint32)
    B = np.ascontiguousarray(B, dtype=np.uint32)
    out = np.zeros((A.shape[0], B.shape[1]), dtype=np.uint32)
    lib().orc_matmul_forward(_p(A), A.shape[0], A.shape[1], _p(B), B.shape[1], _p(out))
    return out


def matmul_output_claim(A: np.ndarray, B: np.ndarray, r_out):
    A = np.ascontiguousarray(A, dtype=np.uint32)
    B = np.ascontiguousarray(B, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_matmul_output_claim(_p(A), A.shape[0], A.shape[1], _p(B), B.shape[1], _p(_qa(r_out)), len(r_out),
                                  _p(out))
    return _q(out)


def restrict_cols_fused(B: np.ndarray, r_j, pk: int):
    B = np.ascontiguousarray(B, dtype=np.uint32)
    out = np.zeros((pk, 4), dtype=np.uint32)
    lib().orc_restrict_cols_fused(_p(B), B.shape[0], B.shape[1], _p(_qa(r_j)), len(r_j), pk, _p(out))
    return out


def restrict_rows_fused(A: np.ndarray, r_i, pk: int):
    A = np.ascontiguousarray(A, dtype=np.uint32)
    out = np.zeros((pk, 4), dtype=np.uint32)
    lib().orc_restrict_rows_fused(_p(A), A.shape[0], A.shape[1], _p(_qa(r_i)), len(r_i), pk, _p(out))
    return out


def reduce_matmul_layer(A: np.ndarray, B: np.ndarray, r_i, r_j, pk: int, ch: Channel):
    """SimdBackend::reduce_matmul_layer (engine/src/backend.rs:111-197)."""
    A = np.ascontiguousarray(A, dtype=np.uint32)
    B = np.ascontiguousarray(B, dtype=np.uint32)
    T = pk.bit_length() - 1
    rp = np.zeros((max(1, 3 * T), 4), dtype=np.uint32)
    chal = np.zeros((max(1, T), 4), dtype=np.uint32)
    fa = np.zeros(4, dtype=np.uint32)
    fb = np.zeros(4, dtype=np.uint32)
    rc = lib().orc_reduce_matmul_layer(_p(A), A.shape[0], A.shape[1], _p(B), B.shape[1], _p(_qa(r_i)), len(r_i),
                                       _p(_qa(r_j)), len(r_j), pk, ch.buf, _p(rp), _p(chal), _p(fa), _p(fb))
    if rc:
        raise ValueError(f"oracle reduce_matmul_layer failed ({rc})")
    return {"round_polys": [(_q(rp, 3 * t), _q(rp, 3 * t + 1), _q(rp, 3 * t + 2)) for t in range(T)],
            "challenges": [_q(chal, t) for t in range(T)], "final_a_eval": _q(fa), "final_b_eval": _q(fb)}


def prove_matmul_layer(claim_point, claim_value, A: np.ndarray, B: np.ndarray, ch: Channel):
    """reduce_matmul_layer_with_backend (engine/src/gkr/prover.rs:5959-6070)."""
    A = np.ascontiguousarray(A, dtype=np.uint32)
    B = np.ascontiguousarray(B, dtype=np.uint32)
    m, k = A.shape
    n = B.shape[1]
    T = _next_pow2(k).bit_length() - 1
    lm = _next_pow2(m).bit_length() - 1
    rp = np.zeros((max(1, 3 * T), 4), dtype=np.uint32)
    fa = np.zeros(4, dtype=np.uint32)
    fb = np.zeros(4, dtype=np.uint32)
    npnt = np.zeros((max(1, lm + T), 4), dtype=np.uint32)
    nv = np.zeros(4, dtype=np.uint32)
    rc = lib().orc_prove_matmul_layer(_p(_qa(claim_point)), len(claim_point), _p(_qa([claim_value])), _p(A), m, k,
                                      _p(B), n, ch.buf, _p(rp), _p(fa), _p(fb), _p(npnt), _p(nv))
    if rc:
        raise ValueError(f"oracle prove_matmul_layer failed ({rc})")
    return {"round_polys": [(_q(rp, 3 * t), _q(rp, 3 * t + 1), _q(rp, 3 * t + 2)) for t in range(T)],
            "final_a_eval": _q(fa), "final_b_eval": _q(fb),
            "next_point": [_q(npnt, i) for i in range(lm + T)], "next_value": _q(nv)}


def prove_activation_layer(claim_point, claim_value, X: np.ndarray, act_type: int, ch: Channel,
                           table_log_size: int = 0):
    """reduce_activation_layer (engine/src/gkr/prover.rs:6400-6600)."""
    if table_log_size == 0:
        table_log_size = 20 if act_type == 4 else 16
    X = np.ascontiguousarray(X, dtype=np.uint32)
    nv = len(claim_point)
    cs = np.zeros(4, dtype=np.uint32)
    eq = np.zeros((max(1, 4 * nv), 4), dtype=np.uint32)
    fe = np.zeros((3, 4), dtype=np.uint32)
    mults = np.zeros(1 << table_log_size, dtype=np.uint32)
    mrp = np.zeros((2 * table_log_size, 4), dtype=np.uint32)
    mfin = np.zeros(4, dtype=np.uint32)
    msum = np.zeros(4, dtype=np.uint32)
    ie = np.zeros(4, dtype=np.uint32)
    tc = np.zeros(8, dtype=np.uint32)
    rc = lib().orc_prove_activation_layer(_p(_qa(claim_point)), nv, _p(_qa([claim_value])), _p(X), X.shape[0],
                                          X.shape[1], act_type, table_log_size, ch.buf, _p(cs), _p(eq), _p(fe),
                                          _p(mults), _p(mrp), _p(mfin), _p(msum), _p(ie), _p(tc))
    if rc:
        raise ValueError(f"oracle prove_activation_layer failed ({rc})")
    return {
        "claimed_sum": _q(cs),
        "eq_round_polys": [tuple(_q(eq, 4 * t + j) for j in range(4)) for t in range(nv)],
        "final_evals": (_q(fe, 0), _q(fe, 1), _q(fe, 2)),
        "multiplicities": mults,
        "mult_round_polys": [(_q(mrp, 2 * t), _q(mrp, 2 * t + 1)) for t in range(table_log_size)],
        "mult_final_eval": _q(mfin),
        "mult_claimed_sum": _q(msum),
        "input_eval": _q(ie),
        "output_eval": tuple(claim_value),
        "table_commitment": felt_int(tc),
    }


def qmul_rows(w, X: np.ndarray) -> np.ndarray:
    """w * X[i] for every QM31 row of X ((n, 4) array), the textbook tower product
    (u^2 = 2 + i) in uint64 numpy arithmetic; rows canonical in, canonical out."""
    X = np.asarray(X, dtype=np.uint64).reshape(-1, 4)
    w0, w1, w2, w3 = (np.uint64(int(v) % P) for v in w)
    p = np.uint64(P)

    def cm(a, b, c, d):  # (a + b i)(c + d i)
        return (a * c % p + (p - b * d % p)) % p, (a * d % p + b * c % p) % p

    x0, x1, x2, x3 = X[:, 0], X[:, 1], X[:, 2], X[:, 3]
    ll = cm(w0, w1, x0, x1)
    hh = cm(w2, w3, x2, x3)
    rh = ((2 * hh[0] % p + (p - hh[1])) % p, (hh[0] + 2 * hh[1]) % p)  # (2 + i) * hh
    lh = cm(w0, w1, x2, x3)
    hl = cm(w2, w3, x0, x1)
    out = np.stack([(ll[0] + rh[0]) % p, (ll[1] + rh[1]) % p, (lh[0] + hl[0]) % p, (lh[1] + hl[1]) % p], axis=1)
    return out.astype(np.uint32)


def prove_matmul_layer_simd(claim_point, claim_value, A_blocks, B: np.ndarray, block_weights, ch: Channel):
    """reduce_matmul_layer_simd_gpu (engine/src/gkr/prover.rs:5422-5600): mix m, k, n and the claim;
    f_a = sum_b w_b restrict_rows(A_b, r_i) (combine_blocks, gpu_sumcheck.rs:1123-1146); f_b =
    restrict_cols(B, r_j); the degree-2 round loop; mix final_a, final_b."""
    A0 = np.asarray(A_blocks[0])
    m, k = A0.shape
    n = B.shape[1]
    pk = _next_pow2(k)
    lm = _next_pow2(m).bit_length() - 1
    ln = _next_pow2(n).bit_length() - 1
    r_i, r_j = list(claim_point[:lm]), list(claim_point[lm:lm + ln])
    ch.mix_u64(m)
    ch.mix_u64(k)
    ch.mix_u64(n)
    ch.mix_secure_field(claim_value)
    fa = np.zeros((pk, 4), dtype=np.uint64)
    for A_b, w in zip(A_blocks, block_weights):
        fa = (fa + qmul_rows(w, restrict_rows_fused(A_b, r_i, pk))) % P
    fb = restrict_cols_fused(B, r_j, pk)
    res = sumcheck_product(fa.astype(np.uint32), fb, ch)
    ch.mix_secure_field(res["final_a_eval"])
    ch.mix_secure_field(res["final_b_eval"])
    return {"round_polys": res["round_polys"], "final_a_eval": res["final_a_eval"],
            "final_b_eval": res["final_b_eval"], "next_point": r_i + res["challenges"],
            "next_value": res["final_a_eval"]}


def _qops():
    p = np.uint64(P)

    def add(x, y):
        return (x + y) % p

    def sub(x, y):
        return (x + (p - y)) % p

    def mul(x, y):  # elementwise QM31 product of (n, 4) uint64 arrays (u^2 = 2 + i)
        def cm(a, b, c, d):
            return (a * c % p + (p - b * d % p)) % p, (a * d % p + b * c % p) % p
        ll = cm(x[:, 0], x[:, 1], y[:, 0], y[:, 1])
        hh = cm(x[:, 2], x[:, 3], y[:, 2], y[:, 3])
        rh = ((2 * hh[0] % p + (p - hh[1])) % p, (hh[0] + 2 * hh[1]) % p)
        lh = cm(x[:, 0], x[:, 1], y[:, 2], y[:, 3])
        hl = cm(x[:, 2], x[:, 3], y[:, 0], y[:, 1])
        return np.stack([(ll[0] + rh[0]) % p, (ll[1] + rh[1]) % p, (lh[0] + hl[0]) % p, (lh[1] + hl[1]) % p], axis=1)
    return add, sub, mul


def sumcheck_3way(w: np.ndarray, a: np.ndarray, b: np.ndarray, ch: Channel):
    """GpuSumcheckExecutor::sumcheck_3way (engine/src/gpu_sumcheck.rs:2597-2681): rounds of
    sum_x w(x) a(x) b(x) evaluated at t = 0..3 on the top variable (MSB first), Newton differences to
    c0..c3, mix_poly_coeffs_deg3, draw, fold all three; numpy over (n, 4) QM31 arrays."""
    add, sub, mul = _qops()
    w, a, b = (np.asarray(v, dtype=np.uint64).reshape(-1, 4) for v in (w, a, b))
    rounds, chals = [], []
    while w.shape[0] > 1:
        mid = w.shape[0] // 2
        lo = (w[:mid], a[:mid], b[:mid])
        dl = tuple(sub(h, l) for h, l in zip((w[mid:], a[mid:], b[mid:]), lo))
        cur = lo
        s = []
        for t in range(4):
            if t:
                cur = tuple(add(x, d) for x, d in zip(cur, dl))
            prod = mul(mul(cur[0], cur[1]), cur[2])
            s.append(tuple(int(v) for v in (prod.sum(axis=0) % P)))
        d1 = qsub(s[1], s[0])
        d2 = qmul(qadd(qsub(qsub(s[2], s[1]), s[1]), s[0]), qinv((2, 0, 0, 0)))
        d3 = qmul(qsub(qsub(s[3], s[0]), qmul((3, 0, 0, 0), qsub(s[2], s[1]))), qinv((6, 0, 0, 0)))
        c0, c1 = s[0], qadd(qsub(d1, d2), qmul((2, 0, 0, 0), d3))
        c2, c3 = qsub(d2, qmul((3, 0, 0, 0), d3)), d3
        rounds.append((c0, c1, c2, c3))
        ch.mix_poly_coeffs_deg3(c0, c1, c2, c3)
        r = ch.draw_qm31()
        chals.append(r)
        rr = np.tile(np.array(r, dtype=np.uint64), (mid, 1))
        w, a, b = (add(l, mul(rr, d)) for l, d in zip(lo, dl))
    fin = tuple(tuple(int(v) for v in x[0]) for x in (w, a, b))
    return {"round_polys": rounds, "challenges": chals, "final_w": fin[0], "final_a": fin[1], "final_b": fin[2]}


def prove_matmul_layer_dual_simd(claim_point, claim_value, A_blocks, B_blocks, block_weights, ch: Channel):
    """reduce_matmul_layer_dual_simd_gpu (engine/src/gkr/prover.rs:5615-5785): mix m, k, n, the block count
    and the claim; ext_w[b pk + x] = w_b, ext_a = restrict_rows(A_b, r_i), ext_b = restrict_cols(B_b, r_j);
    the three-factor sumcheck; mix final_a, final_b."""
    m, k = np.asarray(A_blocks[0]).shape
    n = np.asarray(B_blocks[0]).shape[1]
    nb = len(A_blocks)
    pk = _next_pow2(k)
    lm = _next_pow2(m).bit_length() - 1
    ln = _next_pow2(n).bit_length() - 1
    r_i, r_j = list(claim_point[:lm]), list(claim_point[lm:lm + ln])
    ch.mix_u64(m)
    ch.mix_u64(k)
    ch.mix_u64(n)
    ch.mix_u64(nb)
    ch.mix_secure_field(claim_value)
    ew = np.concatenate([np.tile(np.array(w, dtype=np.uint32), (pk, 1)) for w in block_weights])
    ea = np.concatenate([restrict_rows_fused(A, r_i, pk) for A in A_blocks])
    eb = np.concatenate([restrict_cols_fused(B, r_j, pk) for B in B_blocks])
    res = sumcheck_3way(ew, ea, eb, ch)
    ch.mix_secure_field(res["final_a"])
    ch.mix_secure_field(res["final_b"])
    return {"round_polys": res["round_polys"], "final_a_eval": res["final_a"], "final_b_eval": res["final_b"],
            "n_block_vars": nb.bit_length() - 1, "challenges": res["challenges"], "final_w": res["final_w"]}


def verify_matmul_layer(claim_point, claim_value, m: int, k: int, n: int, round_polys, final_a, final_b,
                        ch: Channel) -> int:
    """verify_matmul_reduction (engine/src/gkr/verifier.rs:2675-2788); 0 = accepted."""
    c0c2 = _qa([q for rp in round_polys for q in (rp[0], rp[2])])
    return int(lib().orc_verify_matmul_layer(_p(_qa(claim_point)), len(claim_point), _p(_qa([claim_value])), m, k,
                                             n, _p(c0c2), len(round_polys), _p(_qa([final_a])), _p(_qa([final_b])),
                                             ch.buf, None, None))


def verify_activation_layer(claim_point, claim_value, act_type: int, table_log: int, proof, ch: Channel) -> int:
    """verify_activation_reduction, LogUp branch (engine/src/gkr/verifier.rs:3058-3290); 0 = accepted."""
    c = _qa([q for rp in proof["eq_round_polys"] for q in (rp[0], rp[2], rp[3])])
    fe = _qa(list(proof["final_evals"]))
    mults = np.ascontiguousarray(proof["multiplicities"], dtype=np.uint32)
    mrp = _qa([q for rp in proof["mult_round_polys"] for q in rp])
    return int(lib().orc_verify_activation_layer(
        _p(_qa(claim_point)), len(claim_point), _p(_qa([claim_value])), act_type, table_log,
        _p(_qa([proof["claimed_sum"]])), _p(c), len(proof["eq_round_polys"]), _p(fe), _p(mults), _p(mrp),
        _p(_qa([proof["mult_final_eval"]])), _p(_qa([proof["mult_claimed_sum"]])), _p(_qa([proof["input_eval"]])),
        ch.buf))


def weight_commitment(B: np.ndarray) -> int:
    """commit_mle_root_only(matrix_to_mle_col_major_padded(B)) (mle_opening.rs:630; prover.rs:1021-1023)."""
    B = np.ascontiguousarray(B, dtype=np.uint32)
    out = np.zeros(8, dtype=np.uint32)
    lib().orc_weight_commitment(_p(B), B.shape[0], B.shape[1], _p(out))
    return felt_int(out)


def mle_commitment(evals: np.ndarray) -> int:
    """commit_mle_root_only over QM31 evaluations given as an (n, 4) array."""
    e = np.ascontiguousarray(evals, dtype=np.uint32).reshape(-1, 4)
    out = np.zeros(8, dtype=np.uint32)
    lib().orc_mle_commitment(_p(e), e.shape[0], _p(out))
    return felt_int(out)


def col_major_mle(B: np.ndarray) -> np.ndarray:
    """matrix_to_mle_col_major_padded (prover.rs:1021-1023): (pk * pn, 4) QM31 array, B[i][j] at j * pk + i."""
    r, c = B.shape
    pk, pn = 1 << max(0, (r - 1).bit_length()), 1 << max(0, (c - 1).bit_length())
    out = np.zeros((pn, pk, 4), dtype=np.uint32)
    out[:c, :r, 0] = (np.asarray(B, dtype=np.uint64) % P).T
    return out.reshape(-1, 4)


def mle_opening(evals: np.ndarray, challenges, ch: Channel, n_queries: int = 10):
    """prove_mle_opening_with_commitment (mle_opening.rs:1654-1915): (commitment, serialized proof felts)."""
    e = np.ascontiguousarray(evals, dtype=np.uint32).reshape(-1, 4)
    chal = _qa(challenges) if len(challenges) else np.zeros(4, dtype=np.uint32)
    cm = np.zeros(8, dtype=np.uint32)
    probe = ch.clone()  # sizing pass on a copy; the real pass advances ch
    n = lib().orc_mle_opening(_p(e), e.shape[0], _p(chal), n_queries, probe.buf, _p(cm), None, 0)
    out = np.zeros((max(1, n), 8), dtype=np.uint32)
    lib().orc_mle_opening(_p(e), e.shape[0], _p(chal), n_queries, ch.buf, _p(cm), _p(out), n)
    return felt_int(cm), [felt_int(out[i]) for i in range(n)]


def synthetic_q(n: int, seed: int) -> np.ndarray:
    """n uniform QM31 values, four consecutive kind-0 draws each: (n, 4) array."""
    out = np.empty((n, 4), dtype=np.uint32)
    lib().orc_synthetic_fill(_p(out), out.size, 0, seed)
    return out


def sumcheck_product(fa: np.ndarray, fb: np.ndarray, ch: Channel):
    """The reduce_matmul_layer round loop (engine/src/backend.rs:146-177) over QM31 vectors."""
    fa = np.ascontiguousarray(fa, dtype=np.uint32).reshape(-1, 4)
    fb = np.ascontiguousarray(fb, dtype=np.uint32).reshape(-1, 4)
    n = fa.shape[0]
    T = max(0, (n - 1).bit_length())
    rp = np.zeros((max(1, 3 * T), 4), dtype=np.uint32)
    chal = np.zeros((max(1, T), 4), dtype=np.uint32)
    a, b = np.zeros(4, dtype=np.uint32), np.zeros(4, dtype=np.uint32)
    if lib().orc_sumcheck_product(_p(fa), _p(fb), n, ch.buf, _p(rp), _p(chal), _p(a), _p(b)):
        raise ValueError("oracle sumcheck_product: length must be a power of two")
    return {"round_polys": [(_q(rp, 3 * t), _q(rp, 3 * t + 1), _q(rp, 3 * t + 2)) for t in range(T)],
            "challenges": [_q(chal, t) for t in range(T)], "final_a_eval": _q(a), "final_b_eval": _q(b)}


def padded_mle(X: np.ndarray) -> np.ndarray:
    """pad_matrix_pow2 + matrix_to_mle (components/matmul.rs:649-664, 174-187): (n, 4) QM31 array."""
    r, c = X.shape
    pr, pc = 1 << max(0, (r - 1).bit_length()), 1 << max(0, (c - 1).bit_length())
    out = np.zeros((pr * pc, 4), dtype=np.uint32)
    out.reshape(pr, pc, 4)[:r, :c, 0] = np.asarray(X, dtype=np.uint64) % P
    return out


def reduce_mul_layer(claim_point, claim_value, lhs: np.ndarray, rhs: np.ndarray, ch: Channel):
    """reduce_mul_layer (engine/src/gkr/prover.rs:6172-6271) over QM31 MLEs given as (n, 4) arrays."""
    lhs = np.ascontiguousarray(lhs, dtype=np.uint32).reshape(-1, 4)
    rhs = np.ascontiguousarray(rhs, dtype=np.uint32).reshape(-1, 4)
    n = lhs.shape[0]
    if rhs.shape[0] != n:
        raise ValueError("lhs and rhs must have the same length")
    nv = max(0, (n - 1).bit_length())
    rp = np.zeros((max(1, 4 * nv), 4), dtype=np.uint32)
    le, re_, al, nx = (np.zeros(4, dtype=np.uint32) for _ in range(4))
    rc = lib().orc_reduce_mul_layer(_p(_qa(claim_point)), len(claim_point), _p(_qa([claim_value])), _p(lhs),
                                    _p(rhs), n, ch.buf, _p(rp), _p(le), _p(re_), _p(al), _p(nx))
    if rc:
        raise ValueError(f"oracle reduce_mul_layer failed ({rc})")
    return {"eq_round_polys": [tuple(_q(rp, 4 * t + j) for j in range(4)) for t in range(nv)],
            "lhs_eval": _q(le), "rhs_eval": _q(re_), "alpha": _q(al),
            "next_point": [tuple(q) for q in claim_point], "next_value": _q(nx)}


def mul_output_claim(lhs: np.ndarray, rhs: np.ndarray, point) -> tuple:
    """MLE of the element-wise product of two padded M31 matrices at `point`."""
    a, b = padded_mle(lhs), padded_mle(rhs)
    prod = np.zeros_like(a)
    prod[:, 0] = (a[:, 0].astype(np.uint64) * b[:, 0].astype(np.uint64)) % P
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_evaluate_mle(_p(prod), len(point), _p(_qa(point)), _p(out))
    return _q(out)


def verify_mul_layer(claim_point, claim_value, proof, ch: Channel):
    """verify_mul_reduction (engine/src/gkr/verifier.rs:2963-3045); returns (status, next_value)."""
    c = _qa([q for rp in proof["eq_round_polys"] for q in (rp[0], rp[2], rp[3])])
    nx = np.zeros(4, dtype=np.uint32)
    rc = lib().orc_verify_mul_layer(_p(_qa(claim_point)), len(claim_point), _p(_qa([claim_value])), _p(c),
                                    len(proof["eq_round_polys"]), _p(_qa([proof["lhs_eval"]])),
                                    _p(_qa([proof["rhs_eval"]])), ch.buf, _p(nx))
    return int(rc), _q(nx)


def activation(tag: int, v: int) -> int:
    return int(lib().orc_activation(tag, v))


def synthetic(rows: int, cols: int, kind: int, seed: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.uint32)
    lib().orc_synthetic_fill(_p(out), out.size, kind, seed)
    return out


def synthetic_value(kind: int, seed: int, i: int) -> int:
    return int(lib().orc_synthetic_value(kind, seed, i))


# ------------------------------------------------------------------ serialization
def _ser_q(out: list, q) -> None:
    out.extend(int(x) for x in q)


def serialize_matmul_layer(out: list, round_polys, final_a, final_b) -> None:
    """LayerProof::MatMul in serialize_gkr_model_proof (engine/src/cairo_serde.rs:1321-1336)."""
    out.append(0)
    out.append(len(round_polys))
    for rp in round_polys:  # c1 omitted
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
    _ser_q(out, final_a)
    _ser_q(out, final_b)


def serialize_activation_layer(out: list, act_type: int, proof) -> None:
    """LayerProof::Activation with a LogUp proof (cairo_serde.rs:1367-1402, 1071-1105, 1138-1156)."""
    out.append(3)
    out.append(act_type)
    _ser_q(out, proof["input_eval"])
    _ser_q(out, proof["output_eval"])
    out.append(int(proof["table_commitment"]))
    out.append(1)  # has LogUp
    _ser_q(out, proof["claimed_sum"])
    out.append(len(proof["eq_round_polys"]))
    for rp in proof["eq_round_polys"]:
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
        _ser_q(out, rp[3])
    for q in proof["final_evals"]:
        _ser_q(out, q)
    mults = list(int(x) for x in proof["multiplicities"])
    out.append(len(mults))
    out.extend(mults)
    out.append(1)  # multiplicity sumcheck present
    out.append(len(proof["mult_round_polys"]))
    for c0, c1 in proof["mult_round_polys"]:
        _ser_q(out, c0)
        _ser_q(out, c1)
    _ser_q(out, proof["mult_final_eval"])
    _ser_q(out, proof["mult_claimed_sum"])
    out.append(0)  # no activation product proof
    out.append(0)  # no piecewise proof


def serialize_mul_layer(out: list, proof) -> None:
    """LayerProof::Mul (cairo_serde.rs:1339-1354): tag 2, rounds, (c0, c2, c3) per round, lhs, rhs."""
    out.append(2)
    out.append(len(proof["eq_round_polys"]))
    for rp in proof["eq_round_polys"]:
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
        _ser_q(out, rp[3])
    _ser_q(out, proof["lhs_eval"])
    _ser_q(out, proof["rhs_eval"])


def serialize_tail(out: list, input_point, input_value, weight_commitments, io_commitment,
                   n_weight_openings: int = 0) -> None:
    """Input claim, weight commitments, opening count, IO commitment (cairo_serde.rs:1740-1771)."""
    out.append(len(input_point))
    for q in input_point:
        _ser_q(out, q)
    _ser_q(out, input_value)
    out.append(len(weight_commitments))
    out.extend(int(c) for c in weight_commitments)
    out.append(n_weight_openings)
    out.append(int(io_commitment))


def parse_mle_opening(felts, pos: int = 0):
    """Read a serialized MleOpeningProof (cairo_serde.rs:341-369) at felts[pos:]; returns (proof, next pos)."""
    def u():
        nonlocal pos
        pos += 1
        return int(felts[pos - 1])

    def q():
        return tuple(u() for _ in range(4))

    roots = [u() for _ in range(u())]
    queries = []
    for _ in range(u()):
        idx, rounds = u(), []
        for _ in range(u()):
            lv, rv = q(), q()
            ls = [u() for _ in range(u())]
            rs = [u() for _ in range(u())]
            rounds.append((lv, rv, ls, rs))
        queries.append((idx, rounds))
    return {"intermediate_roots": roots, "queries": queries, "final_value": q()}, pos


def _securefield_felt(v) -> int:
    a, b, c, d = (int(x) for x in v)
    return (1 << 124) | (a << 93) | (b << 62) | (c << 31) | d


def _merkle_verify(root: int, index: int, leaf: int, siblings) -> bool:
    """PoseidonMerkleTree::verify (poseidon_merkle.rs): hash up the path, left/right by the index bits."""
    cur = leaf
    for s in siblings:
        cur = hades([s, cur, 2])[0] if index & 1 else hades([cur, s, 2])[0]
        index >>= 1
    return cur == root


def verify_mle_opening(commitment: int, proof, challenges, ch: Channel, n_queries: int = 10) -> bool:
    """verify_mle_opening (mle_opening.rs:1918-2028)."""
    ch.mix_felt(commitment)
    for r in proof["intermediate_roots"]:
        ch.mix_felt(r)
    n = len(challenges)
    if n == 0:
        return not proof["queries"]
    half = 1 << (n - 1)
    nq = min(n_queries, half)
    idxs = [(ch.draw_felt252() & ((1 << 64) - 1)) % half for _ in range(nq)]
    if len(proof["queries"]) != nq:
        return False
    roots = [commitment] + list(proof["intermediate_roots"])
    for (pair, rounds), want in zip(proof["queries"], idxs):
        if pair != want or len(rounds) != n:
            return False
        cur, size = pair, 1 << n
        for t, (lv, rv, ls, rs) in enumerate(rounds):
            mid = size // 2
            if t < len(roots):
                if not _merkle_verify(roots[t], cur, _securefield_felt(lv), ls):
                    return False
                if not _merkle_verify(roots[t], mid + cur, _securefield_felt(rv), rs):
                    return False
            folded = qadd(lv, qmul(challenges[t], qsub(rv, lv)))
            if t == n - 1 and tuple(folded) != tuple(proof["final_value"]):
                return False
            cur %= max(mid // 2, 1)
            size = mid
    return True


def rlc_weight_binding(values, ch: Channel):
    """RLC weight binding (prover.rs:1335-1345, 669-699): rho = draw_qm31;
    mix_secure_field(sum_i rho^i * value_i)."""
    rho = ch.draw_qm31()
    pw, combined = (1, 0, 0, 0), (0, 0, 0, 0)
    for v in values:
        combined = qadd(combined, qmul(pw, v))
        pw = qmul(pw, rho)
    ch.mix_secure_field(combined)
    return combined


# ------------------------------------------------------------------ LayerNorm / RMSNorm (norm.c)
NORM_TABLE_LOG = 16


class NormOut(C.Structure):
    """orc_norm_out (oracle.h)."""
    _fields_ = [("input_eval", C.c_uint32 * 4), ("output_eval", C.c_uint32 * 4), ("mean_eval", C.c_uint32 * 4),
                ("rsqrt_eval", C.c_uint32 * 4), ("var_eval", C.c_uint32 * 4), ("n_active", C.c_uint32),
                ("sum0", C.c_uint32 * 4), ("sum1", C.c_uint32 * 4), ("p0_round_polys", _U32P),
                ("p0_final0", C.c_uint32 * 4), ("p0_final1", C.c_uint32 * 4), ("lin_round_polys", _U32P),
                ("lin_final0", C.c_uint32 * 4), ("lin_final1", C.c_uint32 * 4), ("cb_input", C.c_uint32 * 4),
                ("cb_mean", C.c_uint32 * 4), ("claimed_sum", C.c_uint32 * 4), ("logup_round_polys", _U32P),
                ("w_eval", C.c_uint32 * 4), ("in_eval", C.c_uint32 * 4), ("out_eval", C.c_uint32 * 4),
                ("multiplicities", _U32P), ("mult_round_polys", _U32P), ("mult_final", C.c_uint32 * 4),
                ("mult_sum", C.c_uint32 * 4), ("table_commitment", C.c_uint32 * 8), ("n_rows", C.c_uint32),
                ("row_stats0", _U32P), ("row_stats1", _U32P), ("gamma_commitment", C.c_uint32 * 8),
                ("gamma_eval", C.c_uint32 * 4)]


NORM_SCALAR_KEYS = ("input_eval", "output_eval", "mean_eval", "rsqrt_eval", "var_eval", "sum0", "sum1", "p0_final0",
                    "p0_final1", "lin_final0", "lin_final1", "cb_input", "cb_mean", "claimed_sum", "w_eval",
                    "in_eval", "out_eval", "mult_final", "mult_sum", "gamma_eval")


def _norm_lib():
    L = lib()
    if not getattr(L, "_norm_ready", False):
        L.orc_rsqrt.restype = C.c_uint32
        L.orc_rsqrt.argtypes = [C.c_uint32]
        L.orc_layernorm_forward.argtypes = [_U32P, C.c_size_t, C.c_size_t, C.c_size_t, _U32P]
        L.orc_rmsnorm_forward.argtypes = [_U32P, C.c_size_t, C.c_size_t, C.c_size_t, _U32P, C.c_size_t, _U32P]
        L.orc_prove_layernorm_layer.argtypes = [_U32P, C.c_int, _U32P, _U32P, C.c_size_t, C.c_size_t, C.c_size_t,
                                                C.c_void_p, C.POINTER(NormOut)]
        L.orc_prove_rmsnorm_layer.argtypes = [_U32P, C.c_int, _U32P, _U32P, C.c_size_t, C.c_size_t, C.c_size_t,
                                              _U32P, C.c_size_t, C.c_void_p, C.POINTER(NormOut)]
        for name in ("orc_verify_layernorm_layer", "orc_verify_rmsnorm_layer"):
            getattr(L, name).argtypes = [_U32P, C.c_int, _U32P, C.c_size_t, C.POINTER(NormOut), C.c_void_p, _U32P]
        L._norm_ready = True
    return L


def rsqrt_table_value(v: int) -> int:
    return int(_norm_lib().orc_rsqrt(v))


def layernorm_forward(X: np.ndarray, dim: int) -> np.ndarray:
    """The LayerNorm output as reduce_layernorm_layer defines it, on the padded matrix."""
    X = np.ascontiguousarray(X, dtype=np.uint32)
    out = np.zeros((_next_pow2(X.shape[0]), _next_pow2(X.shape[1])), dtype=np.uint32)
    _norm_lib().orc_layernorm_forward(_p(X), X.shape[0], X.shape[1], dim, _p(out))
    return out


def rmsnorm_forward(X: np.ndarray, dim: int, gamma=None) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.uint32)
    g = np.ascontiguousarray(gamma if gamma is not None else np.zeros(1), dtype=np.uint32)
    out = np.zeros((_next_pow2(X.shape[0]), _next_pow2(X.shape[1])), dtype=np.uint32)
    _norm_lib().orc_rmsnorm_forward(_p(X), X.shape[0], X.shape[1], dim, _p(g), 0 if gamma is None else len(g),
                                    _p(out))
    return out


def _norm_buffers(nv: int, prow: int):
    bufs = {"p0": np.zeros(16 * nv, dtype=np.uint32), "lin": np.zeros(16 * nv, dtype=np.uint32),
            "lg": np.zeros(16 * nv, dtype=np.uint32), "mult": np.zeros(1 << NORM_TABLE_LOG, dtype=np.uint32),
            "mrp": np.zeros(8 * NORM_TABLE_LOG, dtype=np.uint32), "rs0": np.zeros(max(1, prow), dtype=np.uint32),
            "rs1": np.zeros(max(1, prow), dtype=np.uint32)}
    o = NormOut()
    o.p0_round_polys, o.lin_round_polys, o.logup_round_polys = _p(bufs["p0"]), _p(bufs["lin"]), _p(bufs["lg"])
    o.multiplicities, o.mult_round_polys = _p(bufs["mult"]), _p(bufs["mrp"])
    o.row_stats0, o.row_stats1 = _p(bufs["rs0"]), _p(bufs["rs1"])
    return o, bufs


def _norm_dict(o: "NormOut", bufs, nv: int) -> dict:
    d = {k: tuple(int(x) for x in getattr(o, k)) for k in NORM_SCALAR_KEYS}
    polys = lambda a: [tuple(tuple(int(x) for x in a[16 * t + 4 * j:16 * t + 4 * j + 4]) for j in range(4))
                       for t in range(nv)]  # noqa: E731
    d["p0_round_polys"], d["lin_round_polys"], d["logup_round_polys"] = (polys(bufs["p0"]), polys(bufs["lin"]),
                                                                         polys(bufs["lg"]))
    d["multiplicities"] = bufs["mult"].copy()
    d["mult_round_polys"] = [(tuple(int(x) for x in bufs["mrp"][8 * t:8 * t + 4]),
                              tuple(int(x) for x in bufs["mrp"][8 * t + 4:8 * t + 8])) for t in range(NORM_TABLE_LOG)]
    d["table_commitment"] = felt_int(o.table_commitment)
    d["gamma_commitment"] = felt_int(o.gamma_commitment)
    d["n_active"], d["n_rows"] = int(o.n_active), int(o.n_rows)
    d["row_stats0"] = [int(x) for x in bufs["rs0"][:o.n_rows]]
    d["row_stats1"] = [int(x) for x in bufs["rs1"][:o.n_rows]]
    return d


def prove_layernorm_layer(claim_point, claim_value, X: np.ndarray, dim: int, ch: Channel) -> dict:
    """reduce_layernorm_layer (engine/src/gkr/prover.rs:7944-8395)."""
    X = np.ascontiguousarray(X, dtype=np.uint32)
    nv = len(claim_point)
    o, bufs = _norm_buffers(nv, _next_pow2(X.shape[0]))
    rc = _norm_lib().orc_prove_layernorm_layer(_p(_qa(claim_point)), nv, _p(_qa([claim_value])), _p(X), X.shape[0],
                                               X.shape[1], dim, ch.buf, C.byref(o))
    if rc:
        raise ValueError(f"oracle prove_layernorm_layer failed ({rc})")
    return _norm_dict(o, bufs, nv)


def prove_rmsnorm_layer(claim_point, claim_value, X: np.ndarray, dim: int, ch: Channel, gamma=None) -> dict:
    """reduce_rmsnorm_layer_with_gamma (engine/src/gkr/prover.rs:8407-8801)."""
    X = np.ascontiguousarray(X, dtype=np.uint32)
    g = np.ascontiguousarray(gamma if gamma is not None else np.zeros(1), dtype=np.uint32)
    nv = len(claim_point)
    o, bufs = _norm_buffers(nv, _next_pow2(X.shape[0]))
    rc = _norm_lib().orc_prove_rmsnorm_layer(_p(_qa(claim_point)), nv, _p(_qa([claim_value])), _p(X), X.shape[0],
                                             X.shape[1], dim, _p(g), 0 if gamma is None else len(g), ch.buf,
                                             C.byref(o))
    if rc:
        raise ValueError(f"oracle prove_rmsnorm_layer failed ({rc})")
    return _norm_dict(o, bufs, nv)


def _norm_struct(proof: dict):
    nv = len(proof["lin_round_polys"])
    o, bufs = _norm_buffers(nv, max(1, proof["n_rows"]))
    for k in NORM_SCALAR_KEYS:
        getattr(o, k)[:] = list(proof[k])
    flat = lambda polys: [x for rp in polys for q in rp for x in q]  # noqa: E731
    bufs["p0"][:] = flat(proof["p0_round_polys"])
    bufs["lin"][:] = flat(proof["lin_round_polys"])
    bufs["lg"][:] = flat(proof["logup_round_polys"])
    bufs["mult"][:] = proof["multiplicities"]
    bufs["mrp"][:] = [x for c0, c1 in proof["mult_round_polys"] for x in (*c0, *c1)]
    bufs["rs0"][:len(proof["row_stats0"])] = proof["row_stats0"]
    bufs["rs1"][:len(proof["row_stats1"])] = proof["row_stats1"]
    o.table_commitment[:] = list(felt_words(proof["table_commitment"]))
    o.n_active, o.n_rows = proof["n_active"], proof["n_rows"]
    return o, bufs, nv


def verify_norm_layer(kind: str, claim_point, claim_value, dim: int, proof: dict, ch: Channel):
    """verify_layernorm_reduction / verify_rmsnorm_reduction (verifier.rs:4153-4690, 4693-5076).
    Returns (status, next_value); status 0 = accepted."""
    o, bufs, nv = _norm_struct(proof)
    nx = np.zeros(4, dtype=np.uint32)
    f = _norm_lib().orc_verify_layernorm_layer if kind == "layernorm" else _norm_lib().orc_verify_rmsnorm_layer
    rc = f(_p(_qa(claim_point)), len(claim_point), _p(_qa([claim_value])), dim, C.byref(o), ch.buf, _p(nx))
    return int(rc), _q(nx)


def _ser_norm_logup(out: list, proof: dict) -> None:
    """serialize_logup_proof with multiplicities (cairo_serde.rs:1071-1105)."""
    out.append(1)
    _ser_q(out, proof["claimed_sum"])
    out.append(len(proof["logup_round_polys"]))
    for rp in proof["logup_round_polys"]:
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
        _ser_q(out, rp[3])
    for k in ("w_eval", "in_eval", "out_eval"):
        _ser_q(out, proof[k])
    out.append(len(proof["multiplicities"]))
    out.extend(int(x) for x in proof["multiplicities"])


def serialize_layernorm_layer(out: list, proof: dict) -> None:
    """LayerProof::LayerNorm in serialize_gkr_model_proof (cairo_serde.rs:1388-1484)."""
    out.append(4)
    for k in ("input_eval", "output_eval", "mean_eval", "rsqrt_eval"):
        _ser_q(out, proof[k])
    out.append(int(proof["table_commitment"]))
    out.append(0)  # simd_combined
    out.append(1)  # has the mean-variance part
    out.append(proof["n_active"])
    _ser_q(out, proof["sum0"])
    _ser_q(out, proof["sum1"])
    out.append(len(proof["p0_round_polys"]))
    for rp in proof["p0_round_polys"]:
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
        _ser_q(out, rp[3])
    _ser_q(out, proof["p0_final0"])
    _ser_q(out, proof["p0_final1"])
    out.append(len(proof["lin_round_polys"]))
    for rp in proof["lin_round_polys"]:
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
        _ser_q(out, rp[3])
    _ser_q(out, proof["lin_final0"])
    _ser_q(out, proof["lin_final1"])
    _ser_q(out, proof["cb_input"])
    _ser_q(out, proof["cb_mean"])
    _ser_norm_logup(out, proof)
    out.append(1)  # multiplicity sumcheck (cairo_serde.rs:1138-1156)
    out.append(len(proof["mult_round_polys"]))
    for c0, c1 in proof["mult_round_polys"]:
        _ser_q(out, c0)
        _ser_q(out, c1)
    _ser_q(out, proof["mult_final"])
    _ser_q(out, proof["mult_sum"])
    _ser_q(out, proof["var_eval"])
    for key in ("row_stats0", "row_stats1"):
        if proof["n_rows"] > 1:
            out.append(1)
            out.append(len(proof[key]))
            out.extend(proof[key])
        else:
            out.append(0)


def serialize_rmsnorm_layer(out: list, proof: dict) -> None:
    """LayerProof::RMSNorm in serialize_gkr_model_proof (cairo_serde.rs:1648-1720): no multiplicity
    sumcheck in this format."""
    out.append(8)
    for k in ("input_eval", "output_eval", "mean_eval", "rsqrt_eval"):
        _ser_q(out, proof[k])
    out.append(int(proof["table_commitment"]))
    out.append(0)  # simd_combined
    out.append(1)  # has the RMS^2 part
    out.append(proof["n_active"])
    _ser_q(out, proof["sum0"])
    out.append(len(proof["p0_round_polys"]))
    for rp in proof["p0_round_polys"]:
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
        _ser_q(out, rp[3])
    _ser_q(out, proof["p0_final0"])
    out.append(len(proof["lin_round_polys"]))
    for rp in proof["lin_round_polys"]:
        _ser_q(out, rp[0])
        _ser_q(out, rp[2])
        _ser_q(out, rp[3])
    _ser_q(out, proof["lin_final0"])
    _ser_q(out, proof["lin_final1"])
    _ser_norm_logup(out, proof)
    if proof["n_rows"] > 1:
        out.append(1)
        out.append(len(proof["row_stats0"]))
        out.extend(proof["row_stats0"])
    else:
        out.append(0)


# ------------------------------------------------------------------ STWO LogUp-GKR batch (lookup_gkr.c)
LOOKUP_GRAND_PRODUCT, LOOKUP_LOGUP_GENERIC, LOOKUP_LOGUP_MULTIPLICITIES, LOOKUP_LOGUP_SINGLES = 0, 1, 2, 3


class LookupLayer(C.Structure):
    """orc_lookup_layer (oracle.h)."""
    _fields_ = [("kind", C.c_uint32), ("n_vars", C.c_uint32), ("num", _U32P), ("den", _U32P)]


class LookupOut(C.Structure):
    """orc_lookup_out (oracle.h)."""
    _fields_ = [("output_claims", _U32P), ("round_polys", _U32P), ("round_poly_lens", _U32P), ("masks", _U32P),
                ("ood_point", _U32P), ("claims_to_verify", _U32P), ("n_layers", C.c_uint32)]


def _lookup_lib():
    L = lib()
    if not getattr(L, "_lookup_ready", False):
        L.orc_prove_lookup_batch.argtypes = [C.c_void_p, C.POINTER(LookupLayer), C.c_size_t, C.POINTER(LookupOut)]
        L.orc_verify_lookup_batch.argtypes = [_U32P, _U32P, C.c_size_t, C.POINTER(LookupOut), C.c_void_p, _U32P,
                                              _U32P]
        L._lookup_ready = True
    return L


def lookup_gate(kind: int) -> int:
    """Gate of an instance: 0 grand product, 1 LogUp."""
    return 0 if kind == LOOKUP_GRAND_PRODUCT else 1


def _lookup_bufs(n_inst: int, n_layers: int):
    n_rounds = max(1, n_layers * (n_layers - 1) // 2)
    return {"oc": np.zeros(8 * n_inst, dtype=np.uint32), "rp": np.zeros(16 * n_rounds, dtype=np.uint32),
            "rl": np.zeros(n_rounds, dtype=np.uint32), "mk": np.zeros(16 * max(1, n_layers) * n_inst, dtype=np.uint32),
            "ood": np.zeros(4 * max(1, n_layers), dtype=np.uint32), "cv": np.zeros(8 * n_inst, dtype=np.uint32)}


def _lookup_struct(b) -> "LookupOut":
    o = LookupOut()
    o.output_claims, o.round_polys, o.round_poly_lens = _p(b["oc"]), _p(b["rp"]), _p(b["rl"])
    o.masks, o.ood_point, o.claims_to_verify = _p(b["mk"]), _p(b["ood"]), _p(b["cv"])
    return o


def prove_lookup_batch(ch: "Channel", instances) -> dict:
    """prove_batch (stwo-gpu/crates/stwo/src/prover/lookups/gkr_prover.rs:396-500).  instances:
    (kind, numerators, denominators) with numerators a QM31 (n, 4) array (generic), an M31 (n,)
    array (multiplicities) or None, denominators a QM31 (n, 4) array (grand product: the column)."""
    arrs, layers = [], (LookupLayer * len(instances))()
    n_layers = 0
    for i, (kind, num, den) in enumerate(instances):
        den = _qa(den)
        nv = max(0, (len(den) - 1).bit_length())
        n_layers = max(n_layers, nv)
        layers[i].kind, layers[i].n_vars, layers[i].den = kind, nv, _p(den)
        arrs.append(den)
        if kind == LOOKUP_LOGUP_GENERIC:
            nq = _qa(num)
            layers[i].num = _p(nq)
            arrs.append(nq)
        elif kind == LOOKUP_LOGUP_MULTIPLICITIES:
            nm = np.ascontiguousarray(num, dtype=np.uint32)
            layers[i].num = _p(nm)
            arrs.append(nm)
    b = _lookup_bufs(len(instances), n_layers)
    o = _lookup_struct(b)
    rc = _lookup_lib().orc_prove_lookup_batch(ch.buf, layers, len(instances), C.byref(o))
    if rc:
        raise ValueError(f"oracle prove_lookup_batch failed ({rc})")
    kinds = [k for k, _, _ in instances]
    nvs = [layers[i].n_vars for i in range(len(instances))]
    return _lookup_dict(b, kinds, nvs, n_layers)


def _lookup_dict(b, kinds, nvs, n_layers) -> dict:
    """The dense proof arrays as a dict: output_claims[i] and claims_to_verify[i] (1 or 2 QM31),
    round_polys[layer] (coefficient lists, leading zeros dropped), masks[layer][i] (2 values per
    column; None before instance i joins), ood_point."""
    n_inst = len(kinds)
    ncl = [1 if k == LOOKUP_GRAND_PRODUCT else 2 for k in kinds]
    q = lambda a, i: tuple(int(x) for x in a[4 * i:4 * i + 4])  # noqa: E731
    d = {"kinds": list(kinds), "n_vars": list(nvs), "n_layers": n_layers,
         "output_claims": [[q(b["oc"], 2 * i + c) for c in range(ncl[i])] for i in range(n_inst)],
         "claims_to_verify": [[q(b["cv"], 2 * i + c) for c in range(ncl[i])] for i in range(n_inst)],
         "ood_point": [q(b["ood"], k) for k in range(n_layers)], "round_polys": [], "masks": []}
    r = 0
    for layer in range(n_layers):
        polys = []
        for _ in range(layer):
            polys.append([q(b["rp"], 4 * r + c) for c in range(int(b["rl"][r]))])
            r += 1
        d["round_polys"].append(polys)
    for layer in range(n_layers):
        d["masks"].append([[q(b["mk"], 4 * (layer * n_inst + i) + c) for c in range(2 * ncl[i])]
                           if layer >= n_layers - nvs[i] else None for i in range(n_inst)])
    return d


def _lookup_arrays(d) -> dict:
    n_inst, n_layers = len(d["kinds"]), d["n_layers"]
    b = _lookup_bufs(n_inst, n_layers)
    for i in range(n_inst):
        for c, v in enumerate(d["output_claims"][i]):
            b["oc"][8 * i + 4 * c:8 * i + 4 * c + 4] = v
    r = 0
    for layer in range(n_layers):
        for poly in d["round_polys"][layer]:
            b["rl"][r] = len(poly)
            for c, v in enumerate(poly):
                b["rp"][16 * r + 4 * c:16 * r + 4 * c + 4] = v
            r += 1
        for i in range(n_inst):
            m = d["masks"][layer][i]
            if m is not None:
                for c, v in enumerate(m):
                    b["mk"][16 * (layer * n_inst + i) + 4 * c:16 * (layer * n_inst + i) + 4 * c + 4] = v
    return b


def verify_lookup_batch(d: dict, ch: "Channel"):
    """partially_verify_batch (gkr_verifier.rs:17-157) on a proof dict.  Returns (status,
    ood_point, claims_to_verify); status 0 = accepted."""
    b = _lookup_arrays(d)
    o = _lookup_struct(b)
    o.n_layers = d["n_layers"]
    gates = np.array([lookup_gate(k) for k in d["kinds"]], dtype=np.uint32)
    nvs = np.array(d["n_vars"], dtype=np.uint32)
    ood = np.zeros(4 * max(1, d["n_layers"]), dtype=np.uint32)
    cv = np.zeros(8 * len(gates), dtype=np.uint32)
    rc = _lookup_lib().orc_verify_lookup_batch(_p(gates), _p(nvs), len(gates), C.byref(o), ch.buf, _p(ood), _p(cv))
    ncl = [1 if g == 0 else 2 for g in gates]
    return (int(rc), [_q(ood, k) for k in range(d["n_layers"])],
            [[_q(cv, 2 * i + c) for c in range(ncl[i])] for i in range(len(gates))])


def serialize_lookup_batch(out: list, d: dict) -> None:
    """serialize_stwo_gkr_batch_proof (engine/src/cairo_serde.rs:3330-3420)."""
    n_inst = len(d["kinds"])
    out.append(n_inst)
    for i in range(n_inst):
        out.append(lookup_gate(d["kinds"][i]))
        out.append(d["n_vars"][i])
        out.append(len(d["output_claims"][i]))
        for v in d["output_claims"][i]:
            _ser_q(out, v)
    out.append(d["n_layers"])
    for layer in range(d["n_layers"]):
        polys = d["round_polys"][layer]
        out.append(len(polys))
        for poly in polys:
            for c in range(4):
                _ser_q(out, poly[c] if c < len(poly) else (0, 0, 0, 0))
            out.append(len(poly))
        # masks: layer_masks_by_instance[i][layer], the instance's own layer index (cairo_serde.rs:3403-3416):
        # instances of different sizes would index past their masks, so the reference only serializes
        # batches of one size
        out.append(n_inst)
        for i in range(n_inst):
            if d["n_vars"][i] != d["n_layers"]:
                raise ValueError("serialize_stwo_gkr_batch_proof indexes masks by layer: instances must share n_vars")
            m = d["masks"][layer][i]
            out.append(len(m))
            for v in m:
                _ser_q(out, v)
            out.append(len(m) // 2)


# ------------------------------------------------------------------ aggregated weight binding
# crypto/aggregated_opening.rs: prove_aggregated_binding(_streaming) (:681-730, :1647-1720),
# verify_aggregated_binding (:1774-1905), serialize_aggregated_binding_proof (cairo_serde.rs:3885-3920).
# Pure Python over the oracle's field, hash and MLE primitives: small cases only.
BINDING_GROUP_SIZE = 4  # gkr/prover.rs:366


def poseidon_hash(a: int, b: int) -> int:
    """starknet_crypto::poseidon_hash(a, b) = hades([a, b, 2])[0]."""
    return hades([a, b, 2])[0]


def binding_config(n_vars):
    """AggregatedBindingConfig::from_claims (:70-95) from the claims' local variable counts."""
    n_max = max(n_vars)
    m_padded = 1 << max(0, (len(n_vars) - 1).bit_length())
    sel = m_padded.bit_length() - 1
    return {"selector_bits": sel, "n_max": n_max, "m_padded": m_padded, "n_global": sel + n_max,
            "n_claims": len(n_vars)}


def compute_zero_tree_root(n_vars: int) -> int:
    """:157-171: the root of 2^n_vars zero leaves (securefield_to_felt(0) = 2^124)."""
    h = 1 << 124
    for _ in range(n_vars):
        h = poseidon_hash(h, h)
    return h


def build_super_root(claims, cfg) -> dict:
    """:181-227: subtree roots (a smaller matrix's root hashed up with zero trees), zero-tree padding to
    m_padded slots, then a Merkle tree over them."""
    zeros = [compute_zero_tree_root(k) for k in range(cfg["n_max"] + 1)]
    subs = []
    for c in claims:
        r = c["commitment"]
        for k in range(cfg["n_max"] - c["n_vars"]):
            r = poseidon_hash(r, zeros[c["n_vars"] + k])
        subs.append(r)
    subs += [zeros[cfg["n_max"]]] * (cfg["m_padded"] - len(subs))
    cur = list(subs)
    while len(cur) > 1:
        cur = [poseidon_hash(cur[2 * i], cur[2 * i + 1]) for i in range(len(cur) // 2)]
    return {"root": cur[0], "subtree_roots": subs}


def _eq1(a, b):
    one = (1, 0, 0, 0)
    return qadd(qmul(a, b), qmul(qsub(one, a), qsub(one, b)))


def _selector_weight(k: int, selector, sel_bits: int):
    """compute_selector_weight (:289-309): bits of k, most significant first."""
    w = (1, 0, 0, 0)
    for j, s in enumerate(selector):
        bit = (k >> (sel_bits - 1 - j)) & 1
        w = qmul(w, _eq1(s, (bit, 0, 0, 0)))
    return w


def _global_point(index: int, n_vars: int, point, cfg):
    """global_point (:328-356): selector bits of the claim's matrix index, zeros, the local point."""
    g = [(((index >> b) & 1), 0, 0, 0) for b in range(cfg["selector_bits"] - 1, -1, -1)]
    g += [(0, 0, 0, 0)] * (cfg["n_max"] - n_vars)
    return g + [tuple(q) for q in point]


def _unified_oracle(t, mles, cfg):
    """eval_unified_oracle (:364-393): sum_k sel_k(t_sel) W_k(t_loc[n_max - n_k ..])."""
    sb = cfg["selector_bits"]
    sel, loc = t[:sb], t[sb:]
    acc = (0, 0, 0, 0)
    for k, mle in enumerate(mles):
        w = _selector_weight(k, sel, sb)
        if w == (0, 0, 0, 0):
            continue
        nk = (len(mle) - 1).bit_length()
        acc = qadd(acc, qmul(w, evaluate_mle([tuple(int(x) for x in v) for v in mle], loc[cfg["n_max"] - nk:])))
    return acc


def prove_aggregated_binding(claims, mles, ch: Channel) -> dict:
    """prove_aggregated_binding_streaming (:1647-1720) / prove_aggregated_binding (:681-730).
    claims: dicts (n_vars, point, value, commitment), one per matrix, in slot order; mles: the
    matrices' MLEs (matrix_to_mle_col_major_padded) as (2^n_vars, 4) arrays."""
    cfg = binding_config([c["n_vars"] for c in claims])
    sr = build_super_root(claims, cfg)
    ch.mix_felt(sr["root"])
    rho = ch.draw_qm31()
    betas, pw = [], (1, 0, 0, 0)
    for _ in claims:
        betas.append(pw)
        pw = qmul(pw, rho)
    gps = [_global_point(i, c["n_vars"], c["point"], cfg) for i, c in enumerate(claims)]
    n = cfg["n_global"]
    eqp = [(1, 0, 0, 0)] * len(claims)
    chal, polys = [], []
    inv2 = qinv((2, 0, 0, 0))
    for rnd in range(n):
        s = []
        for x in range(3):
            xv = (x, 0, 0, 0)
            tot = (0, 0, 0, 0)
            for i, c in enumerate(claims):
                pt = chal + [xv] + gps[i][rnd + 1:]
                mis = qsub(_unified_oracle(pt, mles, cfg), tuple(c["value"]))
                tot = qadd(tot, qmul(qmul(betas[i], eqp[i]), qmul(_eq1(gps[i][rnd], xv), mis)))
            s.append(tot)
        c0 = s[0]
        c2 = qmul(qadd(qsub(s[0], qadd(s[1], s[1])), s[2]), inv2)
        c1 = qsub(qsub(s[1], s[0]), c2)
        ch.mix_poly_coeffs(c0, c1, c2)
        polys.append((c0, c1, c2))
        r = ch.draw_qm31()
        chal.append(r)
        eqp = [qmul(eqp[i], _eq1(r, gps[i][rnd])) for i in range(len(claims))]
    oracle_eval = _unified_oracle(chal, mles, cfg)
    ch.mix_felts([oracle_eval])
    slot = 1 << cfg["n_max"]
    virtual = np.zeros((cfg["m_padded"] * slot, 4), dtype=np.uint32)
    for k, mle in enumerate(mles):
        virtual[k * slot:k * slot + len(mle)] = mle
    cm, felts = mle_opening(virtual, chal, ch)
    return {"config": cfg, "round_polys": polys, "oracle_eval": oracle_eval, "super_root": sr,
            "opening": parse_mle_opening(felts)[0], "opening_felts": felts, "opening_commitment": cm,
            "challenges": chal}


def verify_aggregated_binding(proof, claims, ch: Channel) -> bool:
    """verify_aggregated_binding (:1774-1905), single-opening path."""
    cfg = proof["config"]
    if build_super_root(claims, cfg)["root"] != proof["super_root"]["root"]:
        return False
    ch.mix_felt(proof["super_root"]["root"])
    rho = ch.draw_qm31()
    betas, pw = [], (1, 0, 0, 0)
    for _ in claims:
        betas.append(pw)
        pw = qmul(pw, rho)
    gps = [_global_point(i, c["n_vars"], c["point"], cfg) for i, c in enumerate(claims)]
    if len(proof["round_polys"]) != cfg["n_global"]:
        return False
    cur, chal = (0, 0, 0, 0), []
    for c0, c1, c2 in proof["round_polys"]:
        if qadd(c0, qadd(qadd(c0, c1), c2)) != cur:
            return False
        ch.mix_poly_coeffs(c0, c1, c2)
        r = ch.draw_qm31()
        chal.append(r)
        cur = qadd(c0, qmul(r, qadd(c1, qmul(r, c2))))
    tot = (0, 0, 0, 0)
    for i, c in enumerate(claims):
        e = (1, 0, 0, 0)
        for a, b in zip(gps[i], chal):
            e = qmul(e, _eq1(a, b))
        tot = qadd(tot, qmul(qmul(betas[i], e), qsub(tuple(proof["oracle_eval"]), tuple(c["value"]))))
    if tot != cur:
        return False
    ch.mix_felts([proof["oracle_eval"]])
    return verify_mle_opening(proof["super_root"]["root"], proof["opening"], chal, ch)


def serialize_aggregated_binding_proof(out: list, proof) -> None:
    """serialize_aggregated_binding_proof (cairo_serde.rs:3885-3920)."""
    cfg = proof["config"]
    for k in ("selector_bits", "n_max", "m_padded", "n_global", "n_claims"):
        out.append(cfg[k])
    out.append(len(proof["round_polys"]))
    for c0, c1, c2 in proof["round_polys"]:
        for q in (c0, c1, c2):
            _ser_q(out, q)
    _ser_q(out, proof["oracle_eval"])
    out.append(proof["super_root"]["root"])
    out.append(len(proof["super_root"]["subtree_roots"]))
    out.extend(proof["super_root"]["subtree_roots"])
    out.extend(proof["opening_felts"])
