"""GPU weight openings (gkr_prove_weight_opening / gkr_prove_weight_openings) against the
reference's SP3 calldata (the whole proof, felt for felt, and the transcript digest after the
openings), against the oracle's opening on random shapes, and at Qwen shapes through the
oracle's restatement of verify_mle_opening."""
import sys
import time

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

pytestmark = pytest.mark.gpu
P = (1 << 31) - 1


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def lg(v):
    return max(0, (v - 1).bit_length())


def test_sp3_full_calldata(gpu_ctx, golden):
    sp3 = golden["sp3"]
    A = np.array([[1, 2, 3, 4]], dtype=np.uint32)
    B = np.array([[2 * i + j + 1 for j in range(2)] for i in range(4)], dtype=np.uint32)
    a, b = gpu_ctx.upload(A), gpu_ctx.upload(B)
    ch = G.PoseidonChannel()
    ch.seed_gkr(1, 1, 4)
    r_out = ch.draw_qm31s(1)
    value = gpu_ctx.matmul_output_claim(a, b, r_out)
    ch.mix_secure_field(value)
    proof = G.Proof()
    res = gpu_ctx.prove_matmul_layer(r_out, value, a, b, ch, proof)
    proof.set_input_claim(res["next_point"], res["next_value"])
    assert ch.digest() == int(sp3["post_walk_digest"], 16)
    gpu_ctx.prove_weight_openings(ch, proof)
    assert ch.digest() == int(sp3["final_channel_digest_after_openings"], 16)
    proof.set_io_commitment(int(sp3["io_commitment"], 16))
    assert proof.serialize() == [int(x, 16) for x in sp3["calldata_hex"]]


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 2), (2, 1), (3, 5), (4, 4), (17, 33), (100, 7), (64, 256),
                                       (5, 1000), (1000, 3)])
def test_opening_matches_oracle(gpu_ctx, rows, cols):
    log(f"opening {rows}x{cols}")
    rng = np.random.default_rng(rows * 7919 + cols)
    B = rng.integers(0, P, size=(rows, cols), dtype=np.uint32)
    nv = lg(rows) + lg(cols)
    och = O.Channel()
    och.mix_u64(rows + cols)
    point = och.draw_qm31s(nv)
    gch = G.PoseidonChannel()
    gch.import_state(O.channel_state(och))
    cm_o, felts_o = O.mle_opening(O.col_major_mle(B), point, och)
    proof = G.Proof()
    cm_g = gpu_ctx.prove_weight_opening(gpu_ctx.upload(B), point, gch, proof)
    assert cm_g == cm_o == O.weight_commitment(B)
    assert gch.digest() == och.digest()
    expected = O.evaluate_mle([tuple(v) for v in O.col_major_mle(B)], point) if nv else (int(B[0, 0]), 0, 0, 0)
    got = proof.serialize()
    # 0 layers, empty input point, zero input value, [1, cm], [1, record], io commitment
    head = [0, 0, 0, 0, 0, 0, 1, cm_o, 1, nv] + [x for q in point for x in q] + list(expected)
    assert got == head + felts_o + [0]


def test_expected_value_is_checked(gpu_ctx):
    B = np.arange(12, dtype=np.uint32).reshape(3, 4)
    ch = G.PoseidonChannel()
    point = ch.draw_qm31s(4)
    with pytest.raises(G.GkrError):
        gpu_ctx.prove_weight_opening(gpu_ctx.upload(B), point, ch, G.Proof(), expected_value=(1, 2, 3, 4))
    with pytest.raises(G.GkrError):  # wrong number of variables
        gpu_ctx.prove_weight_opening(gpu_ctx.upload(B), point[:3], G.PoseidonChannel(), G.Proof())


def _openings_from_calldata(cd, n_layers_felts):
    """Split the weight-opening section of serialized calldata (cairo_serde.rs:1750-1767)."""
    pos = n_layers_felts
    n_pt = cd[pos]
    pos += 1 + 4 * n_pt + 4
    n_cm = cd[pos]
    cms = cd[pos + 1:pos + 1 + n_cm]
    pos += 1 + n_cm
    out = []
    for _ in range(cd[pos]):
        pos += 1
        nv = cd[pos]
        point = [tuple(cd[pos + 1 + 4 * i:pos + 5 + 4 * i]) for i in range(nv)]
        pos += 1 + 4 * nv
        expected = tuple(cd[pos:pos + 4])
        pos += 4
        proof, pos = O.parse_mle_opening(cd, pos)
        out.append((point, expected, proof))
        pos -= 1
    return cms, out


@pytest.mark.parametrize("m,k,n", [(1, 5120, 13824), (2, 13824, 5120), (3, 5120, 1024)])
def test_qwen_shape_opening_verifies(gpu_ctx, m, k, n):
    """A MatMul layer at a Qwen2.5-14B weight shape, then its weight opening: the oracle's
    verify_mle_opening accepts it on the same transcript, the commitment equals the root-only
    commitment, and the opened value is final_b (checked inside the opening)."""
    log(f"qwen opening {m}x{k} . {k}x{n}")
    a = gpu_ctx.synthetic(m, k, 0, 3)
    b = gpu_ctx.synthetic(k, n, 0, 4)
    ch = G.PoseidonChannel()
    ch.mix_u64(k)
    r_out = ch.draw_qm31s(lg(m) + lg(n))
    value = gpu_ctx.matmul_output_claim(a, b, r_out)
    ch.mix_secure_field(value)
    proof = G.Proof()
    res = gpu_ctx.prove_matmul_layer(r_out, value, a, b, ch, proof)
    proof.set_input_claim(res["next_point"], res["next_value"])
    st = ch.export_state()  # the oracle verifier continues from the product's state after the walk
    t = time.perf_counter()
    gpu_ctx.prove_weight_openings(ch, proof)
    log(f"  opening took {time.perf_counter() - t:.3f} s")
    cd = proof.serialize()
    n_layer = 1 + 2 + 8 * lg(k) + 8
    cms, ops = _openings_from_calldata(cd, n_layer)
    assert len(ops) == 1 and cms == [gpu_ctx.weight_commitment(b)]
    point, expected, op = ops[0]
    assert expected == tuple(res["final_b_eval"])
    assert tuple(op["final_value"]) == expected
    vch = _oracle_channel_from_state(st)
    assert O.verify_mle_opening(cms[0], op, point, vch)
    assert vch.digest() == ch.digest()


def _oracle_channel_from_state(st):
    """An oracle channel holding the product channel's exported state (digest, n_draws, hash_count)."""
    och = O.Channel()
    words = np.array(st, dtype=np.uint32)
    O.set_channel_state(och, words)
    return och


@pytest.mark.parametrize("mode", [G.WEIGHT_SEQUENTIAL, G.WEIGHT_AGGREGATED_RLC, G.WEIGHT_RLC_DIRECT])
def test_weight_binding_modes(gpu_ctx, mode):
    """Three MatMul layers (one weight used twice), then the weight phase in each of the
    reference's transcript modes: commitments in claim order (AGGREGATED_RLC) or none
    (RLC_DIRECT), rho drawn and sum rho^i * final_b_i mixed (oracle replay), or the
    sequential openings."""
    rng = np.random.default_rng(11)
    W1 = rng.integers(0, P, size=(24, 40), dtype=np.uint32)
    W2 = rng.integers(0, P, size=(40, 9), dtype=np.uint32)
    X = rng.integers(0, P, size=(3, 24), dtype=np.uint32)
    x, w1, w2 = gpu_ctx.upload(X), gpu_ctx.upload(W1), gpu_ctx.upload(W2)
    H = gpu_ctx.upload(O.matmul_forward(X, W1))
    ch = G.PoseidonChannel()
    ch.mix_u64(3)
    proof = G.Proof()
    finals = []
    for a, b in [(H, w2), (x, w1), (x, w1)]:
        r = ch.draw_qm31s(lg(a.rows) + lg(b.cols))
        v = gpu_ctx.matmul_output_claim(a, b, r)
        ch.mix_secure_field(v)
        finals.append(gpu_ctx.prove_matmul_layer(r, v, a, b, ch, proof)["final_b_eval"])
    och = O.Channel()
    O.set_channel_state(och, ch.export_state())
    n_before = len(proof.serialize())
    gpu_ctx.prove_weight_binding(ch, proof, mode)
    cd = proof.serialize()
    if mode == G.WEIGHT_SEQUENTIAL:
        assert cd[n_before - 3] == 3  # three commitments, then three openings
        assert cd[n_before - 3 + 4] == 3
        return
    O.rlc_weight_binding(finals, och)
    assert ch.digest() == och.digest()
    # [.., input point len 0, value, n_commitments, commitments..., 0 openings, io]
    want = [O.weight_commitment(W2), O.weight_commitment(W1), O.weight_commitment(W1)]
    if mode == G.WEIGHT_AGGREGATED_RLC:
        assert cd[n_before - 3:n_before - 3 + 4] == [3] + want and cd[-2] == 0
    else:
        assert cd[n_before - 3] == 0 and cd[-2] == 0


@pytest.mark.parametrize("mode", [G.WEIGHT_AGGREGATED_RLC, G.WEIGHT_AGGREGATED_FULL])
def test_weight_phase_with_cached_commitments(gpu_ctx, mode):
    """Three proofs of the same MatMul layers and weight phase on the same resident weights: the
    first computes the commitments, the second takes them from the matrices (the weight cache of
    weight_cache.rs:283-327), the third recomputes them after invalidate.  All three proofs (and
    binding groups) are identical, and the cached roots equal the oracle's."""
    print(f"case weight phase with cached commitments, mode {mode}", flush=True)
    rng = np.random.default_rng(12)
    W1 = rng.integers(0, P, size=(24, 40), dtype=np.uint32)
    W2 = rng.integers(0, P, size=(40, 9), dtype=np.uint32)
    X = rng.integers(0, P, size=(3, 24), dtype=np.uint32)
    x, w1, w2 = gpu_ctx.upload(X), gpu_ctx.upload(W1), gpu_ctx.upload(W2)
    H = gpu_ctx.upload(O.matmul_forward(X, W1))

    def prove():
        ch = G.PoseidonChannel()
        ch.mix_u64(4)
        proof = G.Proof()
        for a, b in [(H, w2), (x, w1), (x, w1)]:
            r = ch.draw_qm31s(lg(a.rows) + lg(b.cols))
            v = gpu_ctx.matmul_output_claim(a, b, r)
            ch.mix_secure_field(v)
            gpu_ctx.prove_matmul_layer(r, v, a, b, ch, proof)
        gpu_ctx.prove_weight_binding(ch, proof, mode)
        return proof.serialize(), proof.binding_groups(), ch.digest()

    first = prove()
    assert w1.cached_commitment() == O.weight_commitment(W1) and w2.cached_commitment() == O.weight_commitment(W2)
    assert prove() == first
    w1.invalidate()
    w2.invalidate()
    assert w1.cached_commitment() is None
    assert prove() == first
