"""Mul layer (reduce_mul_layer, element-wise product) on the HIP path against the CPU oracle:
bit-exact round polynomials, final evals, combiner, transcript and serialized LayerProof::Mul."""
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


def lg(v):
    return max(0, (v - 1).bit_length())


def _channels(seed):
    g, o = G.PoseidonChannel(), O.Channel()
    g.mix_u64(seed)
    o.mix_u64(seed)
    return g, o


@pytest.mark.parametrize("rows,cols,kind", [(1, 1, 0), (1, 2, 0), (3, 5, 0), (4, 4, 1), (7, 33, 0), (16, 64, 1),
                                            (64, 96, 0), (33, 1000, 0), (64, 1024, 1)])
def test_mul_layer_matrices(gpu_ctx, rows, cols, kind):
    log(f"case mul {rows}x{cols} kind {kind}")
    A = O.synthetic(rows, cols, kind, 1000 + rows)
    B = O.synthetic(rows, cols, kind, 2000 + cols)
    a, b = gpu_ctx.upload(A), gpu_ctx.upload(B)
    nv = lg(rows) + lg(cols)
    gch, och = _channels(rows * 1000 + cols)
    r = gch.draw_qm31s(nv)
    assert r == och.draw_qm31s(nv)
    v = gpu_ctx.mul_output_claim(a, b, r)
    assert v == O.mul_output_claim(A, B, r)
    gch.mix_secure_field(v)
    och.mix_secure_field(v)
    vch = och.clone()
    proof = G.Proof()
    got = gpu_ctx.prove_mul_layer(r, v, a, b, gch, proof)
    ref = O.reduce_mul_layer(r, v, O.padded_mle(A), O.padded_mle(B), och)
    assert got == ref
    assert gch.digest() == och.digest()
    st, nxt = O.verify_mul_layer(r, v, got, vch)
    assert st == 0 and nxt == got["next_value"]
    proof.set_input_claim(r, got["next_value"])
    ser = [1]
    O.serialize_mul_layer(ser, ref)
    O.serialize_tail(ser, r, ref["next_value"], [], 0)
    assert proof.serialize() == ser


@pytest.mark.parametrize("n,extra", [(1, 0), (2, 1), (64, 0), (4096, 3)])
def test_reduce_mul_layer_host_slices(gpu_ctx, n, extra):
    """The reference signature: full QM31 (not only M31-lifted) slices, a claim point longer than
    log2 n (its first log2 n coordinates feed the eq table; the next claim keeps all of it)."""
    log(f"case reduce_mul host slices n={n}")
    rng = np.random.default_rng(n + extra)
    la = rng.integers(0, P, size=(n, 4), dtype=np.uint32)
    lb = rng.integers(0, P, size=(n, 4), dtype=np.uint32)
    gch, och = _channels(n)
    r = gch.draw_qm31s(lg(n) + extra)
    assert r == och.draw_qm31s(lg(n) + extra)
    v = gch.draw_qm31()
    assert v == och.draw_qm31()
    got = gpu_ctx.reduce_mul_layer(r, v, la, lb, gch)
    ref = O.reduce_mul_layer(r, v, la, lb, och)
    assert got == ref
    assert gch.digest() == och.digest()


def test_mul_layer_errors(gpu_ctx):
    log("case mul errors")
    a = gpu_ctx.upload(O.synthetic(4, 8, 0, 1))
    b = gpu_ctx.upload(O.synthetic(4, 16, 0, 2))
    ch = G.PoseidonChannel()
    with pytest.raises(G.GkrError, match="same length"):
        gpu_ctx.prove_mul_layer([(1, 0, 0, 0)] * 6, (0, 0, 0, 0), a, b, ch)
    c = gpu_ctx.upload(O.synthetic(8, 4, 0, 3))  # same padded length as a: accepted (reference semantics)
    gpu_ctx.prove_mul_layer([(1, 0, 0, 0)] * 5, (0, 0, 0, 0), a, c, G.PoseidonChannel())
    with pytest.raises(G.GkrError, match="too short"):
        gpu_ctx.prove_mul_layer([(1, 0, 0, 0)] * 4, (0, 0, 0, 0), a, c, G.PoseidonChannel())
    with pytest.raises(G.GkrError, match="power of 2"):
        gpu_ctx.reduce_mul_layer([], (0, 0, 0, 0), np.zeros((3, 4), np.uint32), np.zeros((3, 4), np.uint32),
                                 G.PoseidonChannel())
    with pytest.raises(G.GkrError, match="canonical"):
        gpu_ctx.reduce_mul_layer([(1, 0, 0, 0)], (0, 0, 0, 0), np.full((2, 4), P, np.uint32),
                                 np.zeros((2, 4), np.uint32), G.PoseidonChannel())


def test_mul_layer_swiglu_shape(gpu_ctx):
    """Qwen2.5-14B SwiGLU product (SiLU(gate) * up, 64 x 13824 -> 2^20): bit-exact against the oracle."""
    rows, cols = 64, 13824
    log(f"case mul swiglu {rows}x{cols}")
    A = O.synthetic(rows, cols, 0, 77)
    B = O.synthetic(rows, cols, 1, 78)
    a, b = gpu_ctx.upload(A), gpu_ctx.upload(B)
    gch, och = _channels(14)
    r = gch.draw_qm31s(20)
    assert r == och.draw_qm31s(20)
    v = gpu_ctx.mul_output_claim(a, b, r)
    gch.mix_secure_field(v)
    och.mix_secure_field(v)
    vch = och.clone()
    got = gpu_ctx.prove_mul_layer(r, v, a, b, gch)
    ref = O.reduce_mul_layer(r, v, O.padded_mle(A), O.padded_mle(B), och)
    assert got == ref and gch.digest() == och.digest()
    assert O.verify_mul_layer(r, v, got, vch)[0] == 0


def test_walk_with_mul_step(gpu_ctx):
    """gkr_prove_walk: fresh MatMul on X . W, chained Mul (X = L (.) R), chained Activation on L,
    and a fresh Mul, against the oracle call by call."""
    log("case walk with mul")
    L, R = O.synthetic(4, 64, 1, 51), O.synthetic(4, 64, 1, 52)
    X = ((L.astype(np.uint64) * R.astype(np.uint64)) % P).astype(np.uint32)  # X = L (.) R
    W = O.synthetic(64, 32, 1, 53)
    M1, M2 = O.synthetic(3, 20, 0, 54), O.synthetic(3, 20, 0, 55)
    gx, gw, gl, gr, g1, g2 = (gpu_ctx.upload(M) for M in (X, W, L, R, M1, M2))
    steps = [(G.STEP_MATMUL, G.CLAIM_FRESH, gx, gw, 0, 0), (G.STEP_MUL, G.CLAIM_CHAINED, gl, gr, 0, 0),
             (G.STEP_ACTIVATION, G.CLAIM_CHAINED, gl, None, 5, 10), (G.STEP_MUL, G.CLAIM_FRESH, g1, g2, 0, 0)]
    gch, och = _channels(3)
    proof = G.Proof()
    fp, fv = G.prove_walk(gpu_ctx, gch, steps, proof)
    ser = [4]
    r = och.draw_qm31s(lg(4) + lg(32))
    v = O.matmul_output_claim(X, W, r)
    och.mix_secure_field(v)
    o1 = O.prove_matmul_layer(r, v, X, W, och)
    O.serialize_matmul_layer(ser, o1["round_polys"], o1["final_a_eval"], o1["final_b_eval"])
    o2 = O.reduce_mul_layer(o1["next_point"], o1["next_value"], O.padded_mle(L), O.padded_mle(R), och)
    O.serialize_mul_layer(ser, o2)
    o3 = O.prove_activation_layer(o2["next_point"], o2["next_value"], L, 5, och, 10)
    O.serialize_activation_layer(ser, 5, o3)
    r4 = och.draw_qm31s(lg(3) + lg(20))
    v4 = O.mul_output_claim(M1, M2, r4)
    och.mix_secure_field(v4)
    o4 = O.reduce_mul_layer(r4, v4, O.padded_mle(M1), O.padded_mle(M2), och)
    O.serialize_mul_layer(ser, o4)
    assert (fp, fv) == (o4["next_point"], o4["next_value"])
    assert gch.digest() == och.digest()
    proof.set_input_claim(fp, fv)
    O.serialize_tail(ser, fp, fv, [], 0)
    assert proof.serialize() == ser


def test_native_walk_proof_verifies(gpu_ctx):
    """A chained walk proved on the GPU over a consistent circuit (H = X0 . W0, L = sigmoid(H),
    X = L (.) R, Y = X . W), serialized, then verified by the library's walk verifier from the same
    starting transcript; a changed felt is rejected."""
    log("case native walk verifies")
    rng = np.random.default_rng(8)
    X0 = rng.integers(0, P, size=(8, 40), dtype=np.uint32)
    W0 = rng.integers(0, P, size=(40, 32), dtype=np.uint32)
    H = O.matmul_forward(X0, W0)
    L = np.vectorize(lambda x: O.activation(3, int(x)), otypes=[np.uint32])(H)
    R = rng.integers(0, P, size=(8, 32), dtype=np.uint32)
    X = ((L.astype(np.uint64) * R) % P).astype(np.uint32)
    W = rng.integers(0, P, size=(32, 24), dtype=np.uint32)
    gx0, gw0, gh, gl, gr, gx, gw = (gpu_ctx.upload(M) for M in (X0, W0, H, L, R, X, W))
    ch = G.PoseidonChannel()
    ch.seed_gkr(4, 8, 40)
    start = ch.export_state()
    r = ch.draw_qm31s(lg(8) + lg(24))
    v = gpu_ctx.matmul_output_claim(gx, gw, r)
    ch.mix_secure_field(v)
    after_claim = ch.export_state()
    steps = [(G.STEP_MATMUL, G.CLAIM_CHAINED, gx, gw, 0, 0), (G.STEP_MUL, G.CLAIM_CHAINED, gl, gr, 0, 0),
             (G.STEP_ACTIVATION, G.CLAIM_CHAINED, gh, None, 3, 12), (G.STEP_MATMUL, G.CLAIM_CHAINED, gx0, gw0, 0, 0)]
    proof = G.Proof()
    fp, fv = G.prove_walk(gpu_ctx, ch, steps, proof, init_point=r, init_value=v)
    proof.set_input_claim(fp, fv)
    cd = proof.serialize()
    shapes = [(G.STEP_MATMUL, 8, 32, 24, 0, 0), (G.STEP_MUL, 8, 32, 0, 0, 0), (G.STEP_ACTIVATION, 8, 32, 0, 3, 12),
              (G.STEP_MATMUL, 8, 40, 32, 0, 0)]
    vch = G.PoseidonChannel()
    vch.import_state(after_claim)
    pt, val, used = G.verify_walk(cd, shapes, r, v, vch)
    assert (pt, val) == (fp, fv) and vch.digest() == ch.digest()
    assert used == len(cd) - 3
    assert start != after_claim
    bad = list(cd)
    bad[used // 2] = (bad[used // 2] + 1) % P
    vch2 = G.PoseidonChannel()
    vch2.import_state(after_claim)
    with pytest.raises(G.GkrError):
        G.verify_walk(bad, shapes, r, v, vch2)


def test_cairo_mul_case_gpu_prover(gpu_ctx):
    """The reference's hand-built one-variable Mul proof (elo-cairo-verifier/tests/
    test_layer_verifiers.cairo:143-214): the GPU prover, from a fresh channel, gives exactly its
    round polynomial and its lhs/rhs evaluations at the challenge drawn after mix_u64(0x4D554C),
    the claim value and the round polynomial."""
    from test_reference_cases import cairo_mul_case
    log("case cairo mul")
    c = cairo_mul_case()
    lhs = np.array(c["lhs_mle"], dtype=np.uint32)
    rhs = np.array(c["rhs_mle"], dtype=np.uint32)
    g = gpu_ctx.reduce_mul_layer(c["point"], c["value"], lhs, rhs, G.PoseidonChannel())
    assert g["eq_round_polys"] == [c["poly"]]
    assert (g["lhs_eval"], g["rhs_eval"]) == (c["lhs"], c["rhs"])
