"""LayerNorm and RMSNorm layers (reduce_layernorm_layer, reduce_rmsnorm_layer_with_gamma,
engine/src/gkr/prover.rs:7944-8801) on the HIP path against the CPU oracle: bit-exact evaluations,
round polynomials of the three parts, multiplicities, row statistics, transcript and serialized
LayerProof::LayerNorm / ::RMSNorm; the library's verifiers on the GPU proofs; norms inside
gkr_prove_walk (chained and fresh claims) and gkr_verify_walk over their calldata."""
import sys

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

pytestmark = pytest.mark.gpu
P = (1 << 31) - 1
ONE = (1, 0, 0, 0)


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def lg(v):
    return max(0, (v - 1).bit_length())


def _channels(seed):
    g, o = G.PoseidonChannel(), O.Channel()
    g.mix_u64(seed)
    o.mix_u64(seed)
    return g, o


def _shift_rows(rows, cols, seed, hi=200):
    """Rows that are shifts of one row: equal variances, the case the reference's multi-row
    variance binding accepts (verifier.rs:4428-4462)."""
    rng = np.random.default_rng(seed)
    base = rng.integers(0, hi, size=cols)
    return np.array([base + 37 * i for i in range(rows)], dtype=np.uint32)


def _ser(kind, proof):
    out = [1]
    (O.serialize_layernorm_layer if kind == G.STEP_LAYERNORM else O.serialize_rmsnorm_layer)(out, proof)
    return out


def _check_layer(ctx, kind, X, dim, seed, gamma=None):
    rows, cols = X.shape
    nv = lg(rows) + lg(cols)
    x = ctx.upload(X)
    gch, och = _channels(seed)
    r = gch.draw_qm31s(nv)
    assert r == och.draw_qm31s(nv)
    v = ctx.norm_output_claim(kind, x, dim, r, gamma)
    gch.mix_secure_field(v)
    och.mix_secure_field(v)
    vch_o, vch_g = och.clone(), gch.clone()
    proof = G.Proof()
    got = ctx.prove_norm_layer(kind, r, v, x, dim, gch, gamma, proof)
    if kind == G.STEP_LAYERNORM:
        ref = O.prove_layernorm_layer(r, v, X, dim, och)
    else:
        ref = O.prove_rmsnorm_layer(r, v, X, dim, och, gamma)
    assert ref["output_eval"] == v  # the output claim is the MLE of the forward output
    mg, mo = got.pop("multiplicities"), ref.pop("multiplicities")
    assert np.array_equal(mg, mo)
    assert got == ref
    assert gch.digest() == och.digest()
    ref["multiplicities"] = mo
    proof.set_input_claim(r, ref["input_eval"])
    ser = _ser(kind, ref)
    O.serialize_tail(ser, r, ref["input_eval"], [], 0)
    assert proof.serialize() == ser
    name = "layernorm" if kind == G.STEP_LAYERNORM else "rmsnorm"
    st, nxt = O.verify_norm_layer(name, r, v, dim, ref, vch_o)
    # the reference's multi-row LayerNorm variance binding holds only when every padded row has one
    # variance (zero padding rows included)
    if kind == G.STEP_RMSNORM or ref["n_rows"] == 1 or len(set(ref["row_stats1"])) == 1:
        assert st == 0 and nxt == ref["input_eval"]
        assert G.verify_norm_layer(kind, r, v, dim, dict(ref), vch_g) == ref["input_eval"]
        assert vch_g.digest() == gch.digest()
    else:
        assert st == 7
        with pytest.raises(G.GkrError):
            G.verify_norm_layer(kind, r, v, dim, dict(ref), vch_g)
    return ref


@pytest.mark.parametrize("rows,cols,dim", [(1, 2, 2), (2, 4, 4), (1, 8, 8), (3, 5, 5), (4, 4, 4), (2, 8, 6),
                                           (7, 33, 33), (16, 64, 64), (1, 1024, 1024), (8, 1000, 1000)])
def test_layernorm_layer(gpu_ctx, rows, cols, dim):
    log(f"case layernorm {rows}x{cols} dim {dim}")
    _check_layer(gpu_ctx, G.STEP_LAYERNORM, _shift_rows(rows, cols, rows * 100 + cols), dim, rows * 1000 + cols)


@pytest.mark.parametrize("rows,cols,dim,hi", [(4, 16, 16, 5000), (5, 96, 96, 1 << 20), (64, 5120, 5120, 2000)])
def test_layernorm_distinct_variances(gpu_ctx, rows, cols, dim, hi):
    """Independent rows (distinct variances; the last case is the Qwen hidden width): prover parity
    holds and both verifiers reject, as the reference's does."""
    log(f"case layernorm distinct {rows}x{cols}")
    X = np.random.default_rng(rows + cols).integers(0, hi, size=(rows, cols), dtype=np.uint32)
    ref = _check_layer(gpu_ctx, G.STEP_LAYERNORM, X, dim, 77 + rows)
    assert len(set(ref["row_stats1"])) > 1


@pytest.mark.parametrize("rows,cols,dim,gamma", [(2, 1, 1, None), (2, 4, 4, None), (1, 8, 8, None),
                                                 (3, 6, 6, None), (2, 4, 4, [3, 5, 7, 11]),
                                                 (4, 5, 5, [2, 3, 4, 5, 6]), (7, 40, 40, None),
                                                 (16, 128, 128, "rand"), (64, 5120, 5120, "rand"),
                                                 (3, 100, 100, [9])])
def test_rmsnorm_layer(gpu_ctx, rows, cols, dim, gamma):
    log(f"case rmsnorm {rows}x{cols} dim {dim} gamma {'rand' if isinstance(gamma, str) else gamma}")
    rng = np.random.default_rng(rows * 7 + cols)
    X = rng.integers(0, 300, size=(rows, cols), dtype=np.uint32)
    if isinstance(gamma, str):
        gamma = rng.integers(1, 1 << 12, size=cols, dtype=np.uint32)
    g = None if gamma is None else np.array(gamma, dtype=np.uint32)
    _check_layer(gpu_ctx, G.STEP_RMSNORM, X, dim, rows * 1000 + cols, g)


def test_norm_errors(gpu_ctx):
    log("case norm errors")
    x = gpu_ctx.upload(_shift_rows(2, 4, 1))
    ch = G.PoseidonChannel()
    with pytest.raises(G.GkrError):  # claim point of the wrong length
        gpu_ctx.prove_norm_layer(G.STEP_LAYERNORM, [ONE] * 2, ONE, x, 4, ch)
    with pytest.raises(G.GkrError):  # dim 0
        gpu_ctx.prove_norm_layer(G.STEP_RMSNORM, [ONE] * 3, ONE, x, 0, ch)
    with pytest.raises(G.GkrError):  # a single entry: no sumcheck rounds (the oracle refuses it too)
        gpu_ctx.prove_norm_layer(G.STEP_LAYERNORM, [], ONE, gpu_ctx.upload(np.ones((1, 1), dtype=np.uint32)), 1, ch)


def test_walk_matmul_layernorm_matmul(gpu_ctx):
    """gkr_prove_walk over Y = LN(X0 . W0) . W1 with chained claims, then a fresh RMSNorm, against
    the oracle call by call; the calldata without the RMSNorm verifies in gkr_verify_walk."""
    log("case walk matmul-layernorm-matmul")
    rng = np.random.default_rng(31)
    X0 = _shift_rows(4, 24, 5, 40)
    # equal column sums in W0 keep H's rows shifts of one another (one variance)
    W0 = rng.integers(0, 10, size=(24, 32), dtype=np.uint32)
    W0[23] = 240 - W0[:23].sum(axis=0)
    H = O.matmul_forward(X0, W0)
    Z = O.layernorm_forward(H, 32)
    W1 = rng.integers(0, P, size=(32, 16), dtype=np.uint32)
    M = rng.integers(0, 500, size=(3, 20), dtype=np.uint32)
    gm = rng.integers(1, 100, size=20, dtype=np.uint32)
    gz, g1, gh, gx0, gw0, gmm, ggm = (gpu_ctx.upload(A) for A in (Z, W1, H, X0, W0, M, gm.reshape(1, -1)))
    steps = [(G.STEP_MATMUL, G.CLAIM_FRESH, gz, g1, 0, 0), (G.STEP_LAYERNORM, G.CLAIM_CHAINED, gh, None, 0, 0, 32),
             (G.STEP_MATMUL, G.CLAIM_CHAINED, gx0, gw0, 0, 0)]
    gch, och = _channels(9)
    start = gch.export_state()
    proof = G.Proof()
    fp, fv = G.prove_walk(gpu_ctx, gch, steps, proof)
    ser = [3]
    r = och.draw_qm31s(lg(4) + lg(16))
    v = O.matmul_output_claim(Z, W1, r)
    och.mix_secure_field(v)
    o1 = O.prove_matmul_layer(r, v, Z, W1, och)
    O.serialize_matmul_layer(ser, o1["round_polys"], o1["final_a_eval"], o1["final_b_eval"])
    o2 = O.prove_layernorm_layer(o1["next_point"], o1["next_value"], H, 32, och)
    O.serialize_layernorm_layer(ser, o2)
    o3 = O.prove_matmul_layer(o1["next_point"], o2["input_eval"], X0, W0, och)
    O.serialize_matmul_layer(ser, o3["round_polys"], o3["final_a_eval"], o3["final_b_eval"])
    assert (fp, fv) == (o3["next_point"], o3["next_value"])
    assert gch.digest() == och.digest()
    proof.set_input_claim(fp, fv)
    O.serialize_tail(ser, fp, fv, [], 0)
    cd = proof.serialize()
    assert cd == ser
    shapes = [(G.STEP_MATMUL, 4, 32, 16, 0, 0, G.CLAIM_FRESH), (G.STEP_LAYERNORM, 4, 32, 0, 0, 0, 0, 32),
              (G.STEP_MATMUL, 4, 24, 32, 0, 0)]
    vch = G.PoseidonChannel()
    vch.import_state(start)
    pt, val, used = G.verify_walk(cd, shapes, None, None, vch, [proof.layer_claim_value(0)])
    assert (pt, val) == (fp, fv) and vch.digest() == gch.digest()
    mm = []
    O.serialize_matmul_layer(mm, o1["round_polys"], o1["final_a_eval"], o1["final_b_eval"])
    bad = list(cd)
    at = 1 + len(mm) + 6  # inside the LayerNorm section's input evaluation
    bad[at] = (bad[at] + 1) % P
    vch2 = G.PoseidonChannel()
    vch2.import_state(start)
    with pytest.raises(G.GkrError):
        G.verify_walk(bad, shapes, None, None, vch2, [proof.layer_claim_value(0)])
    # a fresh RMSNorm (with its scale) after the walk, on the same channel
    proof2 = G.Proof()
    fp2, fv2 = G.prove_walk(gpu_ctx, gch, [(G.STEP_RMSNORM, G.CLAIM_FRESH, gmm, ggm, 0, 0, 20)], proof2)
    r4 = och.draw_qm31s(lg(3) + lg(20))
    o4v = O.evaluate_mle([(int(x), 0, 0, 0) for x in O.rmsnorm_forward(M, 20, gm).reshape(-1)], r4)
    assert proof2.layer_claim_value(0) == o4v
    och.mix_secure_field(o4v)
    o4 = O.prove_rmsnorm_layer(r4, o4v, M, 20, och, gm)
    assert (fp2, fv2) == (r4, o4["input_eval"]) and gch.digest() == och.digest()
    proof2.set_input_claim(fp2, fv2)
    ser2 = [1]
    O.serialize_rmsnorm_layer(ser2, o4)
    O.serialize_tail(ser2, fp2, fv2, [], 0)
    cd2 = proof2.serialize()
    assert cd2 == ser2
    with pytest.raises(G.GkrError, match="RMSNorm"):  # the format drops its multiplicity sumcheck
        G.verify_walk(cd2, [(G.STEP_RMSNORM, 3, 20, 0, 0, 0, G.CLAIM_FRESH, 20)], None, None, G.PoseidonChannel(),
                      [o4v])


def test_walk_fresh_layernorm(gpu_ctx):
    """A fresh LayerNorm step: point drawn, output MLE taken from the witness and mixed; the walk
    verifier replays it with the prover's claim value."""
    log("case walk fresh layernorm")
    X = _shift_rows(8, 64, 12, 1000)
    gx = gpu_ctx.upload(X)
    gch, och = _channels(21)
    start = gch.export_state()
    proof = G.Proof()
    fp, fv = G.prove_walk(gpu_ctx, gch, [(G.STEP_LAYERNORM, G.CLAIM_FRESH, gx, None, 0, 0)], proof)
    r = och.draw_qm31s(lg(8) + lg(64))
    v = O.evaluate_mle([(int(x), 0, 0, 0) for x in O.layernorm_forward(X, 64).reshape(-1)], r)
    och.mix_secure_field(v)
    o = O.prove_layernorm_layer(r, v, X, 64, och)
    assert (fp, fv) == (r, o["input_eval"]) and gch.digest() == och.digest()
    proof.set_input_claim(fp, fv)
    cd = proof.serialize()
    vch = G.PoseidonChannel()
    vch.import_state(start)
    pt, val, _ = G.verify_walk(cd, [(G.STEP_LAYERNORM, 8, 64, 0, 0, 0, G.CLAIM_FRESH)], None, None, vch,
                               [proof.layer_claim_value(0)])
    assert (pt, val) == (fp, fv) and vch.digest() == gch.digest()
