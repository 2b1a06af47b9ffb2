"""The product's verifier replay (host code of the C ABI, no GPU needed) against the reference's
SP3 calldata and against proofs the CPU oracle produces: honest proofs are accepted with the same
next claims and transcript as the oracle's verifier; tampered ones are rejected with
GKR_ERR_VERIFY."""
import random

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest
import qm31_py as Q

P = (1 << 31) - 1


def lg(v):
    return max(0, (v - 1).bit_length())


def test_sp3_calldata_walk(golden):
    """The reference's SP3 proof (engine/tests/artifacts/sp3_matmul_only_proof.json): the layer
    section and input claim of its calldata verify as a one-layer chained walk; the transcript ends
    at the fixture's post-walk digest; the remaining felts are the commitments and openings."""
    sp3 = golden["sp3"]
    cd = [int(x, 16) for x in sp3["calldata_hex"]]
    ch = G.PoseidonChannel()
    ch.seed_gkr(1, 1, 4)
    r_out = ch.draw_qm31s(1)
    value = O.evaluate_mle([(50, 0, 0, 0), (60, 0, 0, 0)], r_out)
    ch.mix_secure_field(value)
    pt, val, used = G.verify_walk(cd, [(G.STEP_MATMUL, 1, 4, 2, 0, 0)], r_out, value, ch)
    assert ch.digest() == int(sp3["post_walk_digest"], 16)
    assert [list(q) for q in pt] == sp3["input_claim_point"]
    # layer count + MatMul proof + input claim
    assert used == 1 + (2 + 2 * 8 + 8) + (1 + 4 * len(pt) + 4)
    assert cd[used] == 1 and cd[used + 1] == int(sp3["weight_commitments"][0], 16)
    # a changed round coefficient, final evaluation or stated input claim is rejected
    for idx in (3, 10, 20, 27, used - 1):
        bad = list(cd)
        bad[idx] = (bad[idx] + 1) % P
        ch2 = G.PoseidonChannel()
        ch2.seed_gkr(1, 1, 4)
        ch2.draw_qm31s(1)
        ch2.mix_secure_field(value)
        with pytest.raises(G.GkrError) as e:
            G.verify_walk(bad, [(G.STEP_MATMUL, 1, 4, 2, 0, 0)], r_out, value, ch2)
        assert e.value.code == 6
    # the circuit must match the proof
    ch3 = G.PoseidonChannel()
    with pytest.raises(G.GkrError, match="expected an Activation"):
        G.verify_walk(cd, [(G.STEP_ACTIVATION, 1, 4, 0, 5, 0)], r_out, value, ch3)


@pytest.mark.parametrize("m,k,n", [(1, 4, 2), (3, 17, 5), (8, 64, 16), (5, 100, 7)])
def test_matmul_layer_verifier(m, k, n):
    rng = np.random.default_rng(m * 100 + k)
    A = rng.integers(0, P, size=(m, k), dtype=np.uint32)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    ch = O.Channel()
    ch.mix_u64(k)
    r = ch.draw_qm31s(lg(m) + lg(n))
    v = O.matmul_output_claim(A, B, r)
    start = ch.clone()
    proof = O.prove_matmul_layer(r, v, A, B, ch)
    gch = G.PoseidonChannel()
    gch.import_state(_export(start))
    pt, val = G.verify_matmul_layer(r, v, m, k, n, proof["round_polys"], proof["final_a_eval"],
                                    proof["final_b_eval"], gch)
    assert (pt, val) == (proof["next_point"], proof["next_value"])
    assert gch.digest() == ch.digest()
    # tampering: final evaluation, a round coefficient, the claim, the round count
    for mutate in ("final_b", "c0", "claim", "rounds"):
        g2 = G.PoseidonChannel()
        g2.import_state(_export(start))
        rp = [list(t) for t in proof["round_polys"]]
        fa, fb, cv = proof["final_a_eval"], proof["final_b_eval"], v
        if mutate == "final_b":
            fb = Q.qadd(fb, (1, 0, 0, 0))
        elif mutate == "c0":
            rp[0][0] = Q.qadd(rp[0][0], (0, 1, 0, 0))
        elif mutate == "claim":
            cv = Q.qadd(cv, (0, 0, 1, 0))
        else:
            rp = rp[:-1]
        with pytest.raises(G.GkrError) as e:
            G.verify_matmul_layer(r, cv, m, k, n, [tuple(t) for t in rp], fa, fb, g2)
        assert e.value.code == 6


def _export(oracle_channel):
    """Oracle channel state in the 11-word to_gpu_state layout."""
    return O.channel_state(oracle_channel)


@pytest.mark.parametrize("rows,cols,tag,tlog", [(4, 64, 5, 10), (3, 5, 3, 8), (8, 8, 4, 6), (2, 8, 2, 8)])
def test_activation_layer_verifier(rows, cols, tag, tlog):
    rng = np.random.default_rng(rows * 31 + cols)
    X = rng.integers(0, P, size=(rows, cols), dtype=np.uint32)
    nv = lg(rows) + lg(cols)
    ch = O.Channel()
    ch.mix_u64(tag)
    r = ch.draw_qm31s(nv)
    v = ch.draw_qm31()
    start = ch.clone()
    proof = O.prove_activation_layer(r, v, X, tag, ch, tlog)
    vch = start.clone()
    assert O.verify_activation_layer(r, v, tag, tlog, proof, vch) == 0
    gch = G.PoseidonChannel()
    gch.import_state(_export(start))
    assert G.verify_activation_layer(r, tag, tlog, proof, gch) == proof["input_eval"]
    assert gch.digest() == ch.digest() == vch.digest()
    for field in ("claimed_sum", "w_eval", "mult_final_eval", "commitment", "mult"):
        bad = dict(proof)
        if field == "w_eval":
            fe = list(proof["final_evals"])
            fe[0] = Q.qadd(fe[0], (1, 0, 0, 0))
            bad["final_evals"] = tuple(fe)
        elif field == "commitment":
            bad["table_commitment"] = proof["table_commitment"] ^ 1
        elif field == "mult":
            m = np.array(proof["multiplicities"], copy=True)
            j = int(np.argmax(m))
            m[j] -= 1
            m[(j + 1) % len(m)] += 1
            bad["multiplicities"] = m
        else:
            bad[field] = Q.qadd(proof[field], (0, 0, 0, 1))
        g2 = G.PoseidonChannel()
        g2.import_state(_export(start))
        with pytest.raises(G.GkrError) as e:
            G.verify_activation_layer(r, tag, tlog, bad, g2)
        assert e.value.code == 6


def test_activation_verifier_refuses_relu():
    """ReLU is proved algebraically by the reference (prover.rs:1770-1776); the LogUp replay and the
    walk verifier refuse a LogUp proof of it."""
    X = np.arange(15, dtype=np.uint32).reshape(3, 5)
    ch = O.Channel()
    r = ch.draw_qm31s(lg(3) + lg(5))
    v = ch.draw_qm31()
    start = ch.clone()
    proof = O.prove_activation_layer(r, v, X, 1, ch, 8)
    gch = G.PoseidonChannel()
    gch.import_state(_export(start))
    with pytest.raises(G.GkrError) as e:
        G.verify_activation_layer(r, 1, 8, proof, gch)
    assert e.value.code == 1
    cd = [1]
    O.serialize_activation_layer(cd, 1, proof)
    O.serialize_tail(cd, r, proof["input_eval"], [], 0)
    g2 = G.PoseidonChannel()
    g2.import_state(_export(start))
    with pytest.raises(G.GkrError, match="algebraically"):
        G.verify_walk(cd, [(G.STEP_ACTIVATION, 3, 5, 0, 1, 8)], r, v, g2)


@pytest.mark.parametrize("rows,cols", [(1, 2), (3, 5), (8, 16)])
def test_mul_layer_verifier(rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    A = rng.integers(0, P, size=(rows, cols), dtype=np.uint32)
    B = rng.integers(0, P, size=(rows, cols), dtype=np.uint32)
    nv = lg(rows) + lg(cols)
    ch = O.Channel()
    ch.mix_u64(cols)
    r = ch.draw_qm31s(nv + 1)
    v = O.mul_output_claim(A, B, r[:nv])
    start = ch.clone()
    proof = O.reduce_mul_layer(r, v, O.padded_mle(A), O.padded_mle(B), ch)
    gch = G.PoseidonChannel()
    gch.import_state(_export(start))
    assert G.verify_mul_layer(r, v, proof, gch) == proof["next_value"]
    assert gch.digest() == ch.digest()
    bad = dict(proof)
    bad["rhs_eval"] = Q.qadd(proof["rhs_eval"], (1, 0, 0, 0))
    g2 = G.PoseidonChannel()
    g2.import_state(_export(start))
    with pytest.raises(G.GkrError) as e:
        G.verify_mul_layer(r, v, bad, g2)
    assert e.value.code == 6


def test_serialized_chained_walk():
    """A MatMul -> Mul -> Activation -> MatMul walk (output to input) proved by the oracle and
    serialized as the reference does; the product's walk verifier accepts it and rejects any
    changed felt among a sample of positions."""
    rng = np.random.default_rng(5)
    # circuit (input to output): H = X0 . W0; L = sigmoid(H); X = L (.) R; Y = X . W
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
    start = ch.clone()
    o1 = O.prove_matmul_layer(r, v, X, W, ch)
    o2 = O.reduce_mul_layer(o1["next_point"], o1["next_value"], O.padded_mle(L), O.padded_mle(R), ch)
    o3 = O.prove_activation_layer(o2["next_point"], o2["next_value"], H, 3, ch, 8)
    o4 = O.prove_matmul_layer(o2["next_point"], o3["input_eval"], X0, W0, ch)
    cd = [4]
    O.serialize_matmul_layer(cd, o1["round_polys"], o1["final_a_eval"], o1["final_b_eval"])
    O.serialize_mul_layer(cd, o2)
    O.serialize_activation_layer(cd, 3, o3)
    O.serialize_matmul_layer(cd, o4["round_polys"], o4["final_a_eval"], o4["final_b_eval"])
    O.serialize_tail(cd, o4["next_point"], o4["next_value"], [], 0)
    shapes = [(G.STEP_MATMUL, 4, 16, 8, 0, 0), (G.STEP_MUL, 4, 16, 0, 0, 0), (G.STEP_ACTIVATION, 4, 16, 0, 3, 8),
              (G.STEP_MATMUL, 4, 12, 16, 0, 0)]
    gch = G.PoseidonChannel()
    gch.import_state(_export(start))
    pt, val, used = G.verify_walk(cd, shapes, r, v, gch)
    assert (pt, val) == (o4["next_point"], o4["next_value"])
    assert gch.digest() == ch.digest()
    assert used == len(cd) - 3  # weight-commitment count, opening count, IO commitment follow
    pick = random.Random(1)
    for idx in pick.sample(range(1, used), 40):
        bad = list(cd)
        bad[idx] = (bad[idx] + 1) % P
        g2 = G.PoseidonChannel()
        g2.import_state(_export(start))
        with pytest.raises(G.GkrError):
            G.verify_walk(bad, shapes, r, v, g2)


def test_fresh_claim_walk_verifier():
    """A fresh-claim walk (the configs 3-5 driver: every layer draws its output point; a MatMul or Mul
    takes MLE(output) there and mixes it, an Activation draws its value) proved by the oracle and
    serialized; the walk verifier replays it from the fresh values alone and ends at the same
    transcript; a changed fresh value or felt is rejected."""
    rng = np.random.default_rng(9)
    A1, B1 = rng.integers(0, P, size=(3, 20), dtype=np.uint32), rng.integers(0, P, size=(20, 6), dtype=np.uint32)
    S = rng.integers(0, P, size=(4, 12), dtype=np.uint32)
    L, R = rng.integers(0, P, size=(2, 9), dtype=np.uint32), rng.integers(0, P, size=(2, 9), dtype=np.uint32)
    ch = O.Channel()
    ch.mix_u64(3)
    start = ch.clone()
    cd = [4]
    fresh = []
    r = ch.draw_qm31s(lg(3) + lg(6))
    v = O.matmul_output_claim(A1, B1, r)
    fresh.append(v)
    ch.mix_secure_field(v)
    o = O.prove_matmul_layer(r, v, A1, B1, ch)
    O.serialize_matmul_layer(cd, o["round_polys"], o["final_a_eval"], o["final_b_eval"])
    r = ch.draw_qm31s(lg(4) + lg(12))
    v = ch.draw_qm31()
    o = O.prove_activation_layer(r, v, S, 2, ch, 8)
    O.serialize_activation_layer(cd, 2, o)
    r = ch.draw_qm31s(lg(2) + lg(9))
    v = O.mul_output_claim(L, R, r)
    fresh.append(v)
    ch.mix_secure_field(v)
    o = O.reduce_mul_layer(r, v, O.padded_mle(L), O.padded_mle(R), ch)
    O.serialize_mul_layer(cd, o)
    r = ch.draw_qm31s(lg(3) + lg(6))
    v = O.matmul_output_claim(A1, B1, r)
    fresh.append(v)
    ch.mix_secure_field(v)
    o = O.prove_matmul_layer(r, v, A1, B1, ch)
    O.serialize_matmul_layer(cd, o["round_polys"], o["final_a_eval"], o["final_b_eval"])
    O.serialize_tail(cd, o["next_point"], o["next_value"], [], 0)
    F = G.CLAIM_FRESH
    shapes = [(G.STEP_MATMUL, 3, 20, 6, 0, 0, F), (G.STEP_ACTIVATION, 4, 12, 0, 2, 8, F),
              (G.STEP_MUL, 2, 9, 0, 0, 0, F), (G.STEP_MATMUL, 3, 20, 6, 0, 0, F)]
    gch = G.PoseidonChannel()
    gch.import_state(_export(start))
    pt, val, used = G.verify_walk(cd, shapes, None, None, gch, fresh)
    assert (pt, val) == (o["next_point"], o["next_value"])
    assert gch.digest() == ch.digest()
    bad_fresh = list(fresh)
    bad_fresh[1] = Q.qadd(bad_fresh[1], (1, 0, 0, 0))
    g2 = G.PoseidonChannel()
    g2.import_state(_export(start))
    with pytest.raises(G.GkrError) as e:
        G.verify_walk(cd, shapes, None, None, g2, bad_fresh)
    assert e.value.code == 6
    g3 = G.PoseidonChannel()
    g3.import_state(_export(start))
    with pytest.raises(G.GkrError) as e:
        G.verify_walk(cd, shapes, None, None, g3, fresh[:2])
    assert e.value.code == 1
