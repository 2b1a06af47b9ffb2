"""The transcript trace (GKR_CHANNEL_TRACE in the library, ORACLE_CHANNEL_TRACE in the oracle): the
channel digest and draw count at fixed points of every reduction and after every walk step, the
tool for finding where two transcripts part (the reference prints its channel under
STWO_CHANNEL_TRACE, engine/src/gpu_sumcheck.rs:2708-2740, gkr/prover.rs:1523-1541, 6002-6012).

On the CPU: the oracle proves a MatMul -> Mul -> Activation -> MatMul walk and traces it; the
product's walk verifier replays the serialized proof with its own trace; the two traces are equal
line for line, with the points each layer kind defines.  A changed felt in the third layer's
multiplicity sumcheck makes the verifier's trace stop where it parts from the oracle's.  The GPU
prover's trace of the same walk is compared with the oracle's in tests/test_gpu_parity.py."""
import os

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

P = (1 << 31) - 1


def lg(v):
    return max(0, (v - 1).bit_length())


def chained_walk_proof(trace_path=None):
    """The oracle's MatMul -> Mul -> Activation -> MatMul walk (the circuit of
    tests/test_verifier.py's chained walk); with trace_path, the oracle traces it (walk steps marked
    from here).  Returns (calldata, shapes, start channel state, claim point, value, end digest)."""
    rng = np.random.default_rng(5)
    X0 = rng.integers(0, P, size=(4, 12), dtype=np.uint32)
    W0 = rng.integers(0, P, size=(12, 16), dtype=np.uint32)
    H = O.matmul_forward(X0, W0)
    L = np.vectorize(lambda x: O.activation(3, int(x)), otypes=[np.uint32])(H)
    R = rng.integers(0, P, size=(4, 16), dtype=np.uint32)
    X = ((L.astype(np.uint64) * R) % P).astype(np.uint32)
    W = rng.integers(0, P, size=(16, 8), dtype=np.uint32)
    ch = O.Channel()
    ch.mix_u64(11)
    r = ch.draw_qm31s(lg(4) + lg(8))
    v = O.matmul_output_claim(X, W, r)
    ch.mix_secure_field(v)
    start = O.channel_state(ch)
    old = os.environ.get("ORACLE_CHANNEL_TRACE")
    if trace_path:
        os.environ["ORACLE_CHANNEL_TRACE"] = trace_path
    try:
        o1 = O.prove_matmul_layer(r, v, X, W, ch)
        O.trace_point(ch, "walk.step", 0)
        o2 = O.reduce_mul_layer(o1["next_point"], o1["next_value"], O.padded_mle(L), O.padded_mle(R), ch)
        O.trace_point(ch, "walk.step", 1)
        o3 = O.prove_activation_layer(o2["next_point"], o2["next_value"], H, 3, ch, 8)
        O.trace_point(ch, "walk.step", 2)
        o4 = O.prove_matmul_layer(o2["next_point"], o3["input_eval"], X0, W0, ch)
        O.trace_point(ch, "walk.step", 3)
    finally:
        if old is None:
            os.environ.pop("ORACLE_CHANNEL_TRACE", None)
        else:
            os.environ["ORACLE_CHANNEL_TRACE"] = old
    cd = [4]
    O.serialize_matmul_layer(cd, o1["round_polys"], o1["final_a_eval"], o1["final_b_eval"])
    O.serialize_mul_layer(cd, o2)
    O.serialize_activation_layer(cd, 3, o3)
    O.serialize_matmul_layer(cd, o4["round_polys"], o4["final_a_eval"], o4["final_b_eval"])
    O.serialize_tail(cd, o4["next_point"], o4["next_value"], [], 0)
    shapes = [(G.STEP_MATMUL, 4, 16, 8, 0, 0), (G.STEP_MUL, 4, 16, 0, 0, 0), (G.STEP_ACTIVATION, 4, 16, 0, 3, 8),
              (G.STEP_MATMUL, 4, 12, 16, 0, 0)]
    return cd, shapes, start, r, v, ch.digest()


def verify_traced(cd, shapes, start, r, v, path):
    """The product's walk verifier with GKR_CHANNEL_TRACE=path; returns the raised error, if any."""
    gch = G.PoseidonChannel()
    gch.import_state(start)
    old = os.environ.get("GKR_CHANNEL_TRACE")
    os.environ["GKR_CHANNEL_TRACE"] = path
    try:
        G.verify_walk(cd, shapes, r, v, gch)
        return None, gch
    except G.GkrError as e:
        return e, gch
    finally:
        if old is None:
            os.environ.pop("GKR_CHANNEL_TRACE", None)
        else:
            os.environ["GKR_CHANNEL_TRACE"] = old


def read(path):
    with open(path) as f:
        return [line.split() for line in f.read().splitlines()]


EXPECTED_LABELS = ["matmul.rounds", "matmul", "walk.step",
                   "mul.eq", "mul", "walk.step",
                   "logup.gamma_beta", "logup.eq", "logup.mult", "logup", "walk.step",
                   "matmul.rounds", "matmul", "walk.step"]


def test_verifier_trace_equals_oracle_trace(tmp_path):
    ot, vt = str(tmp_path / "oracle.trace"), str(tmp_path / "verifier.trace")
    cd, shapes, start, r, v, end = chained_walk_proof(ot)
    err, gch = verify_traced(cd, shapes, start, r, v, vt)
    assert err is None and gch.digest() == end
    o, g = read(ot), read(vt)
    assert [x[0] for x in o] == EXPECTED_LABELS
    assert o == g
    assert [int(x[2], 16) for x in o if x[0] == "walk.step"][-1] == end
    # nothing is written once the variable is unset
    size = os.path.getsize(vt)
    gch2 = G.PoseidonChannel()
    gch2.import_state(start)
    G.verify_walk(cd, shapes, r, v, gch2)
    assert os.path.getsize(vt) == size


def test_trace_locates_a_changed_layer(tmp_path):
    """A felt changed in the Activation layer's multiplicity rounds: the verifier's trace equals the
    oracle's up to that layer's eq-sumcheck and stops before its multiplicity point."""
    ot, vt = str(tmp_path / "oracle.trace"), str(tmp_path / "verifier.trace")
    cd, shapes, start, r, v, end = chained_walk_proof(ot)
    o = read(ot)
    # the first multiplicity round's c0 of layer 2, found by walking the serialized layout
    pos = 1
    nr = cd[pos + 1]
    pos += 2 + nr * 8 + 8  # MatMul: tag, n rounds, (c0, c2) per round, final a, b
    nr = cd[pos + 1]
    pos += 2 + nr * 12 + 8  # Mul: tag, n rounds, (c0, c2, c3) per round, lhs, rhs
    assert cd[pos] == 3
    p2 = pos + 2 + 8 + 1 + 1 + 4  # tag, act type, in/out evals, table commitment, has LogUp, claimed sum
    nr = cd[p2]
    p2 += 1 + nr * 12 + 12  # rounds, (c0, c2, c3) per round, w / in / out evals
    nm = cd[p2]
    p2 += 1 + nm + 1  # multiplicities, has multiplicity sumcheck
    assert cd[p2] == 8  # multiplicity rounds of a 2^8 table
    bad = list(cd)
    bad[p2 + 1] = (bad[p2 + 1] + 1) % P  # first round's c0
    err, _ = verify_traced(bad, shapes, start, r, v, vt)
    assert err is not None and err.code == 6
    g = read(vt)
    n_ok = len(g)
    assert g == o[:n_ok]
    assert [x[0] for x in g][-1] == "logup.eq"  # parted at the multiplicity sumcheck of step 2
    assert o[n_ok][0] == "logup.mult"
