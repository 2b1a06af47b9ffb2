"""Aggregated weight binding (prove_aggregated_binding_streaming, engine/src/crypto/aggregated_opening.rs:
1647-1720) on the HIP path against the CPU oracle: the serialized AggregatedWeightBindingProof (config,
mismatch-sumcheck round polynomials, oracle value, super root, subtree roots, the opening of the virtual
MLE) felt for felt and the channel digest, for groups of 1 to 8 claims with equal and mixed sizes, ragged
matrices, a 1 x 1 weight and a tampered claim; the oracle's verifier accepts the proofs of honest
claims (the proofs are the same felts)."""
import sys

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

pytestmark = pytest.mark.gpu
P = (1 << 31) - 1


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _claims(rng, shapes, tamper=None):
    out = []
    for i, (r, c) in enumerate(shapes):
        B = O.synthetic(r, c, 1, int(rng.integers(1, 1 << 30)))
        mle = O.col_major_mle(B)
        nv = (len(mle) - 1).bit_length()
        pt = [tuple(int(x) for x in rng.integers(0, P, size=4)) for _ in range(nv)]
        v = O.evaluate_mle([tuple(int(x) for x in row) for row in mle], pt)
        if tamper == i:
            v = O.qadd(v, (1, 0, 0, 0))
        out.append((B, mle, pt, v, O.weight_commitment(B)))
    return out


def _check(ctx, shapes, seed, tamper=None):
    rng = np.random.default_rng(seed)
    cl = _claims(rng, shapes, tamper)
    gch, och = G.PoseidonChannel(), O.Channel()
    gch.mix_u64(seed)
    och.mix_u64(seed)
    vch = och.clone()
    mats = [ctx.upload(B) for B, *_ in cl]
    got = G.prove_aggregated_binding(ctx, gch, [(m, pt, v, cm) for m, (B, mle, pt, v, cm) in zip(mats, cl)])
    oclaims = [{"n_vars": (len(mle) - 1).bit_length(), "point": pt, "value": v, "commitment": cm}
               for B, mle, pt, v, cm in cl]
    proof = O.prove_aggregated_binding(oclaims, [mle for _, mle, *_ in cl], och)
    ref = []
    O.serialize_aggregated_binding_proof(ref, proof)
    assert got == ref
    assert gch.digest() == och.digest()
    # a 1 x 1 weight's commitment is the root of its leaf padded to two (a zero felt), while the
    # super root extends it with zero-leaf subtrees: the reference's super root then differs from
    # the virtual MLE's root and its own verifier rejects the opening
    consistent = all(c["n_vars"] > 0 for c in oclaims)
    assert (proof["opening_commitment"] == proof["super_root"]["root"]) == consistent
    assert O.verify_aggregated_binding(proof, oclaims, vch) == (tamper is None and consistent)


@pytest.mark.parametrize("shapes", [[(4, 8)], [(8, 8), (8, 8)], [(4, 8), (8, 8), (3, 5)],
                                    [(16, 32), (2, 2), (7, 9), (16, 16)], [(1, 1), (4, 4)],
                                    [(5, 3)] * 5, [(8, 4), (4, 8), (2, 16), (16, 2), (1, 32), (32, 1), (3, 3), (6, 6)],
                                    [(64, 256), (256, 64), (100, 100), (128, 128)]])
def test_aggregated_binding_matches_oracle(gpu_ctx, shapes):
    log(f"case binding {shapes}")
    _check(gpu_ctx, shapes, len(shapes) * 7 + shapes[0][0])


def test_aggregated_binding_tampered_claim(gpu_ctx):
    log("case binding tampered")
    _check(gpu_ctx, [(8, 8), (4, 8)], 5, tamper=0)


def test_aggregated_binding_errors(gpu_ctx):
    log("case binding errors")
    m = gpu_ctx.upload(np.ones((4, 4), dtype=np.uint32))
    ch = G.PoseidonChannel()
    pt = [(1, 0, 0, 0)] * 4
    with pytest.raises(G.GkrError):  # point of the wrong length
        G.prove_aggregated_binding(gpu_ctx, ch, [(m, pt[:3], (0, 0, 0, 0), 0)])
    with pytest.raises(G.GkrError):  # too many claims
        G.prove_aggregated_binding(gpu_ctx, ch, [(m, pt, (0, 0, 0, 0), 0)] * 9)
    with pytest.raises(G.GkrError):
        G.prove_aggregated_binding(gpu_ctx, ch, [])


def lg(v):
    return max(0, (v - 1).bit_length())


def test_weight_phase_full_binding(gpu_ctx):
    """GKR_WEIGHT_AGGREGATED_FULL after five MatMul layers (two weights claimed twice): the
    commitments in claim order, then groups of 4 and 1 claims proved on the channel, each group's
    serialized proof equal to the oracle's over the same claims (points r_j || challenges, values
    final_b) and the same transcript."""
    log("case weight phase full binding")
    rng = np.random.default_rng(21)
    shapes = [(3, 24, 40), (3, 40, 9), (2, 16, 16), (3, 24, 40), (5, 9, 12)]
    Ws = {}
    mats = []
    for m, k, n in shapes:
        if (k, n) not in Ws:
            Ws[(k, n)] = rng.integers(0, P, size=(k, n), dtype=np.uint32)
        X = rng.integers(0, P, size=(m, k), dtype=np.uint32)
        mats.append((X, Ws[(k, n)]))
    dev = {key: gpu_ctx.upload(W) for key, W in Ws.items()}
    ch = G.PoseidonChannel()
    ch.mix_u64(21)
    proof = G.Proof()
    claims = []
    for (X, W), (m, k, n) in zip(mats, shapes):
        a = gpu_ctx.upload(X)
        r = ch.draw_qm31s(lg(m) + lg(n))
        v = gpu_ctx.matmul_output_claim(a, dev[(k, n)], r)
        ch.mix_secure_field(v)
        o = gpu_ctx.prove_matmul_layer(r, v, a, dev[(k, n)], ch, proof)
        pt = list(r[lg(m):]) + list(o["next_point"][lg(m):])
        claims.append({"n_vars": lg(k) + lg(n), "point": pt, "value": o["final_b_eval"],
                       "commitment": O.weight_commitment(W), "mle": O.col_major_mle(W)})
    och = O.Channel()
    O.set_channel_state(och, ch.export_state())
    gpu_ctx.prove_weight_binding(ch, proof, G.WEIGHT_AGGREGATED_FULL)
    groups = proof.binding_groups()
    assert len(groups) == 2
    for g, start in enumerate((0, 4)):
        part = claims[start:start + 4]
        p = O.prove_aggregated_binding(part, [c["mle"] for c in part], och)
        ref = []
        O.serialize_aggregated_binding_proof(ref, p)
        assert groups[g] == ref, g
    assert ch.digest() == och.digest()
