"""HIP path (through the C ABI) against the CPU oracle: bit-exact parity.

Small and mid sizes compare every output word with the oracle on the same
seeded inputs; the Qwen2.5-14B up-projection shape is checked through
size-independent properties (verifier replay, final evaluations equal the
MLEs of A and B at the challenge point).
"""
import os
import random
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


def npow2(v):
    return 1 << max(0, (v - 1).bit_length())


def lg(v):
    return npow2(v).bit_length() - 1


def test_sp3_fixture_on_gpu(gpu_ctx, golden):
    sp3 = golden["sp3"]
    log("case sp3 1x4 . 4x2")
    A = np.array([[1, 2, 3, 4]], dtype=np.uint32)
    B = np.array([[2 * i + j + 1 for j in range(2)] for i in range(4)], dtype=np.uint32)
    a, b = gpu_ctx.upload(A), gpu_ctx.upload(B)
    ch = G.PoseidonChannel()
    ch.seed_gkr(1, 1, 4)
    r_out = ch.draw_qm31s(1)
    value = gpu_ctx.matmul_output_claim(a, b, r_out)
    assert value == O.evaluate_mle([(50, 0, 0, 0), (60, 0, 0, 0)], r_out)
    ch.mix_secure_field(value)
    proof = G.Proof()
    res = gpu_ctx.prove_matmul_layer(r_out, value, a, b, ch, proof)
    assert ch.digest() == int(sp3["post_walk_digest"], 16)
    assert [list(q) for q in res["next_point"]] == sp3["input_claim_point"]
    proof.set_input_claim(res["next_point"], res["next_value"])
    proof.add_weight_commitment(int(sp3["weight_commitments"][0], 16))
    felts = proof.serialize()
    cd = [int(x, 16) for x in sp3["calldata_hex"]]
    # num_layers, MatMul proof, input claim, weight commitments: the first 42 felts
    assert felts[:42] == cd[:42]


def _random_point(rng, n):
    return [tuple(rng.randrange(P) for _ in range(4)) for _ in range(n)]


def _compare_layer(ctx, A, B, seed, label, a=None, b=None):
    """One matmul layer (fresh output claim, then the reduction) on the GPU against the oracle; a, b:
    resident matrices holding A and B (uploaded here when absent, and then freed)."""
    log(f"case {label} A{A.shape} B{B.shape}")
    own = a is None
    if own:
        a, b = ctx.upload(A), ctx.upload(B)
    m, k = A.shape
    n = B.shape[1]
    gch, och = G.PoseidonChannel(), O.Channel()
    gch.mix_u64(seed)
    och.mix_u64(seed)
    nv = lg(m) + lg(n)
    r_g, r_o = gch.draw_qm31s(nv), och.draw_qm31s(nv)
    assert r_g == r_o
    v_g = ctx.matmul_output_claim(a, b, r_g)
    v_o = O.matmul_output_claim(A, B, r_o)
    assert v_g == v_o
    gch.mix_secure_field(v_g)
    och.mix_secure_field(v_o)
    rg = ctx.prove_matmul_layer(r_g, v_g, a, b, gch)
    ro = O.prove_matmul_layer(r_o, v_o, A, B, och)
    assert rg["round_polys"] == ro["round_polys"]
    assert rg["final_a_eval"] == ro["final_a_eval"] and rg["final_b_eval"] == ro["final_b_eval"]
    assert rg["next_point"] == ro["next_point"] and rg["next_value"] == ro["next_value"]
    assert gch.digest() == och.digest()
    if own:
        a.free()
        b.free()


def test_config1_uniform_256(gpu_ctx):
    """A, B 256x256 uniform M31 (A seed 0, B seed 1), channel new()."""
    A = O.synthetic(256, 256, 0, 0)
    B = O.synthetic(256, 256, 0, 1)
    log("case config1 256x256x256")
    a, b = gpu_ctx.synthetic(256, 256, 0, 0), gpu_ctx.synthetic(256, 256, 0, 1)
    assert (a.download() == A).all() and (b.download() == B).all()
    gch, och = G.PoseidonChannel(), O.Channel()
    r = gch.draw_qm31s(16)
    assert r == och.draw_qm31s(16)
    v = gpu_ctx.matmul_output_claim(a, b, r)
    assert v == O.matmul_output_claim(A, B, r)
    rg = gpu_ctx.prove_matmul_layer(r, v, a, b, gch)
    ro = O.prove_matmul_layer(r, v, A, B, och)
    assert len(rg["round_polys"]) == 8
    assert rg == ro
    assert gch.digest() == och.digest()


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (1, 4, 2), (2, 3, 5), (7, 13, 3), (1, 64, 1), (16, 1, 8),
                                   (33, 100, 70), (64, 300, 257), (5, 1024, 12), (64, 576, 192), (3, 2048, 4)])
def test_matmul_layer_random_shapes(gpu_ctx, m, k, n):
    rng = np.random.default_rng(m * 10007 + k * 101 + n)
    A = rng.integers(0, P, size=(m, k), dtype=np.uint32)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    _compare_layer(gpu_ctx, A, B, m + k + n, "random")


@pytest.fixture(scope="module")
def int8_ctx():
    """A context created with GKR_INT8_WEIGHTS=1: int8-range weights take the int8 restriction."""
    old = os.environ.get("GKR_INT8_WEIGHTS")
    os.environ["GKR_INT8_WEIGHTS"] = "1"
    try:
        ctx = G.Context(0)
    finally:
        if old is None:
            del os.environ["GKR_INT8_WEIGHTS"]
        else:
            os.environ["GKR_INT8_WEIGHTS"] = old
    yield ctx
    ctx.close()


@pytest.fixture(scope="module")
def u32_ctx():
    """A context created with GKR_INT8_WEIGHTS=0: every weight takes the u32 restriction."""
    old = os.environ.get("GKR_INT8_WEIGHTS")
    os.environ["GKR_INT8_WEIGHTS"] = "0"
    try:
        ctx = G.Context(0)
    finally:
        if old is None:
            del os.environ["GKR_INT8_WEIGHTS"]
        else:
            os.environ["GKR_INT8_WEIGHTS"] = old
    yield ctx
    ctx.close()


@pytest.mark.parametrize("m,k,n", [(1, 576, 576), (1, 1536, 576), (64, 512, 1024)])
def test_matmul_layer_int8_range(gpu_ctx, m, k, n):
    A = O.synthetic(m, k, 1, 11)
    B = O.synthetic(k, n, 1, 12)
    _compare_layer(gpu_ctx, A, B, 3, "int8")


@pytest.mark.parametrize("m,k,n", [(1, 576, 576), (64, 512, 1024), (3, 700, 3000), (64, 5120, 1024)])
def test_matmul_layer_u32_restriction(u32_ctx, m, k, n):
    """int8-range weights under GKR_INT8_WEIGHTS=0 take the u32 restriction (k_restrict_cols)."""
    A = O.synthetic(m, k, 1, 13)
    B = O.synthetic(k, n, 1, 14)
    _compare_layer(u32_ctx, A, B, 4, "u32 path")


@pytest.mark.parametrize("m,k,n", [(1, 576, 576), (1, 1536, 576), (64, 512, 1024), (3, 700, 3000), (2, 33, 5),
                                   (5, 4100, 2048), (1, 16, 9000)])
def test_matmul_layer_int8_weight_path(int8_ctx, m, k, n):
    """The int8 weight copy (16 x 64 tiles, digit blocks, MFMA restriction) gives the same proof as
    the oracle, including ragged row tiles, partial column steps and several chunks."""
    A = O.synthetic(m, k, 1, 21)
    B = O.synthetic(k, n, 1, 22)
    _compare_layer(int8_ctx, A, B, 5, "int8 path")


@pytest.mark.parametrize("m,k,n", [(2, 40, 70), (4, 300, 1100)])
def test_int8_context_full_range_weights(int8_ctx, m, k, n):
    """Weights outside the int8 range fall back to the u32 restriction under an int8 context."""
    rng = np.random.default_rng(m + k + n)
    A = rng.integers(0, P, size=(m, k), dtype=np.uint32)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    B[0, 0] = 200  # out of int8 range even if the rest were small
    _compare_layer(int8_ctx, A, B, 7, "int8 ctx, full range")


def test_wrapped_weight_changed_and_invalidated(gpu_ctx):
    """A weight borrowed with gkr_matrix_wrap_device, proved once (which builds its int8 copy), then
    written by the caller: the library keeps the copy it derived until gkr_matrix_invalidate, after
    which the proof is the oracle's proof of the new entries."""
    m, k, n = 8, 640, 512
    A, B1, B2 = O.synthetic(m, k, 1, 31), O.synthetic(k, n, 1, 32), O.synthetic(k, n, 1, 33)
    a, store = gpu_ctx.upload(A), gpu_ctx.upload(B1)
    w = gpu_ctx.wrap_device(store.device_ptr, k, n)
    _compare_layer(gpu_ctx, A, B1, 40, "wrapped weight", a, w)
    # the caller writes new int8-range entries into the borrowed memory (B2 = I . B2)
    ident, b2 = gpu_ctx.upload(np.eye(k, dtype=np.uint32)), gpu_ctx.upload(B2)
    gpu_ctx.matmul_forward_into(ident, b2, store)
    assert np.array_equal(w.download(), B2)
    # as documented, the derived int8 copy still holds B1 until the caller invalidates it
    _compare_layer(gpu_ctx, A, B1, 41, "wrapped weight, changed, not invalidated", a, w)
    w.invalidate()
    _compare_layer(gpu_ctx, A, B2, 42, "wrapped weight, invalidated", a, w)
    _compare_layer(gpu_ctx, A, B2, 43, "wrapped weight, copy rebuilt", a, w)
    assert G.lib().gkr_matrix_invalidate(None, w.handle) == 1  # GKR_ERR_INVALID


def test_boundary_values(gpu_ctx):
    # extremes of M31: 0 and P - 1 everywhere
    A = np.full((4, 8), P - 1, dtype=np.uint32)
    B = np.full((8, 4), P - 1, dtype=np.uint32)
    B[::2] = 0
    _compare_layer(gpu_ctx, A, B, 1, "extremes")


def test_zkmlops_reduce_matmul_layer(gpu_ctx):
    rng = random.Random(4)
    for (m, k, n) in [(4, 8, 4), (3, 17, 9), (1, 32, 1), (8, 1, 2)]:
        log(f"case zkmlops {m}x{k}x{n}")
        nprng = np.random.default_rng(k)
        A = nprng.integers(0, P, size=(m, k), dtype=np.uint32)
        B = nprng.integers(0, P, size=(k, n), dtype=np.uint32)
        r_i, r_j = _random_point(rng, lg(m)), _random_point(rng, lg(n))
        gch, och = G.PoseidonChannel(), O.Channel()
        a, b = gpu_ctx.upload(A), gpu_ctx.upload(B)
        rg = gpu_ctx.reduce_matmul_layer(a, b, r_i, r_j, npow2(k), gch)
        ro = O.reduce_matmul_layer(A, B, r_i, r_j, npow2(k), och)
        assert rg == ro
        assert gch.digest() == och.digest()


def test_zkmlops_shape_errors(gpu_ctx):
    a = gpu_ctx.upload(np.ones((2, 3), dtype=np.uint32))
    b = gpu_ctx.upload(np.ones((4, 2), dtype=np.uint32))
    ch = G.PoseidonChannel()
    with pytest.raises(G.GkrError):
        gpu_ctx.reduce_matmul_layer(a, b, [(1, 0, 0, 0)], [(1, 0, 0, 0)], 4, ch)
    b2 = gpu_ctx.upload(np.ones((3, 2), dtype=np.uint32))
    with pytest.raises(G.GkrError):  # wrong pk
        gpu_ctx.reduce_matmul_layer(a, b2, [(1, 0, 0, 0)], [(1, 0, 0, 0)], 8, ch)
    with pytest.raises(G.GkrError):  # non-canonical upload
        gpu_ctx.upload(np.full((2, 2), P, dtype=np.uint32))


def test_mle_ops(gpu_ctx):
    rng = random.Random(9)
    for n in (0, 1, 3, 6, 11):
        log(f"case mle n={n}")
        evals = _random_point(rng, 1 << n)
        point = _random_point(rng, n)
        assert gpu_ctx.evaluate_mle_at_point(evals, point) == O.evaluate_mle(evals, point)
        for s in range(0, n + 1, max(1, n // 2)):
            assign = _random_point(rng, s)
            assert gpu_ctx.restrict_mle(evals, assign) == O.restrict_mle(evals, assign)


# 48 x 1500 (2^17 padded entries) and 20 x 50000 (2^21): the prepare pass fused with the
# eq-sumcheck's first trip (two rounds, then one), ragged rows and columns
@pytest.mark.parametrize("rows,cols,tag,tlog", [(1, 8, 5, 8), (4, 16, 5, 10), (3, 5, 3, 6), (2, 32, 4, 8),
                                                (1, 1536, 5, 16), (8, 96, 2, 12), (16, 64, 3, 16),
                                                (48, 1500, 5, 12), (20, 50000, 3, 10)])
def test_activation_layer_parity(gpu_ctx, rows, cols, tag, tlog):
    log(f"case logup {rows}x{cols} tag={tag} table=2^{tlog}")
    X = O.synthetic(rows, cols, 0, rows * 1000 + cols)
    nv = lg(rows) + lg(cols)
    gch, och = G.PoseidonChannel(), O.Channel()
    pt = gch.draw_qm31s(nv)
    val = gch.draw_qm31()
    assert pt == och.draw_qm31s(nv) and val == och.draw_qm31()
    x = gpu_ctx.upload(X)
    gp = G.Proof()
    pg = gpu_ctx.prove_activation_layer(pt, val, x, tag, gch, tlog, gp)
    po = O.prove_activation_layer(pt, val, X, tag, och, tlog)
    for key in ("claimed_sum", "eq_round_polys", "final_evals", "mult_round_polys", "mult_final_eval",
                "mult_claimed_sum", "input_eval", "output_eval", "table_commitment"):
        assert pg[key] == po[key], key
    assert (pg["multiplicities"] == po["multiplicities"]).all()
    assert gch.digest() == och.digest()
    # serialized layer equals the oracle's serialization
    gp.set_input_claim(pt, pg["input_eval"])
    felts = gp.serialize()
    ref = [1]
    O.serialize_activation_layer(ref, tag, po)
    O.serialize_tail(ref, pt, po["input_eval"], [], 0)
    assert felts == ref


def test_relu_is_not_a_logup_activation(gpu_ctx):
    """The reference proves ReLU algebraically (prover.rs:1770-1776), never with LogUp: the LogUp
    reducer and a walk step refuse it before any device work or transcript change."""
    log("case relu refused")
    X = O.synthetic(3, 5, 0, 35)
    x = gpu_ctx.upload(X)
    gch = G.PoseidonChannel()
    pt = gch.draw_qm31s(lg(3) + lg(5))
    val = gch.draw_qm31()
    d0 = gch.digest()
    with pytest.raises(G.GkrError) as e:
        gpu_ctx.prove_activation_layer(pt, val, x, 1, gch, 6)
    assert e.value.code == 1 and "algebraically" in str(e.value)
    with pytest.raises(G.GkrError) as e:
        G.prove_walk(gpu_ctx, gch, [(G.STEP_ACTIVATION, G.CLAIM_CHAINED, x, None, 1, 6)], G.Proof(), pt, val)
    assert e.value.code == 1
    assert gch.digest() == d0


def test_two_layer_walk_and_serialization(gpu_ctx):
    """MatMul -> SiLU(LogUp) -> MatMul walk on one channel, claims chained as in the GKR loop."""
    log("case walk")
    X = O.synthetic(4, 64, 1, 21)
    W1 = O.synthetic(64, 32, 1, 22)
    H = O.matmul_forward(X, W1)
    W2 = O.synthetic(32, 16, 1, 23)
    gx, gw1, gh, gw2 = gpu_ctx.upload(X), gpu_ctx.upload(W1), gpu_ctx.upload(H), gpu_ctx.upload(W2)
    gch, och = G.PoseidonChannel(), O.Channel()
    for ch in (gch, och):
        ch.mix_u64(3); ch.mix_u64(4); ch.mix_u64(64)
    r = gch.draw_qm31s(lg(4) + lg(16))
    assert r == och.draw_qm31s(lg(4) + lg(16))
    # output layer claim on W2's product (the walk's last matmul consumes H directly here)
    v = gpu_ctx.matmul_output_claim(gh, gw2, r)
    assert v == O.matmul_output_claim(H, W2, r)
    gch.mix_secure_field(v); och.mix_secure_field(v)
    proof = G.Proof()
    l1 = gpu_ctx.prove_matmul_layer(r, v, gh, gw2, gch, proof)
    o1 = O.prove_matmul_layer(r, v, H, W2, och)
    assert l1 == o1
    l2 = gpu_ctx.prove_activation_layer(l1["next_point"], l1["next_value"], gh, 5, gch, 12, proof)
    o2 = O.prove_activation_layer(o1["next_point"], o1["next_value"], H, 5, och, 12)
    assert l2["eq_round_polys"] == o2["eq_round_polys"] and gch.digest() == och.digest()
    l3 = gpu_ctx.prove_matmul_layer(l1["next_point"], l2["input_eval"], gx, gw1, gch, proof)
    o3 = O.prove_matmul_layer(o1["next_point"], o2["input_eval"], X, W1, och)
    assert l3 == o3 and gch.digest() == och.digest()
    proof.set_input_claim(l3["next_point"], l3["next_value"])
    ref = [3]
    O.serialize_matmul_layer(ref, o1["round_polys"], o1["final_a_eval"], o1["final_b_eval"])
    O.serialize_activation_layer(ref, 5, o2)
    O.serialize_matmul_layer(ref, o3["round_polys"], o3["final_a_eval"], o3["final_b_eval"])
    O.serialize_tail(ref, o3["next_point"], o3["next_value"], [], 0)
    assert proof.serialize() == ref


def test_native_walk_chained(gpu_ctx):
    """gkr_prove_walk over MatMul -> SiLU(LogUp) -> MatMul with chained claims equals the oracle's
    layer-by-layer walk (final claim, transcript and serialized proof)."""
    log("case native walk chained")
    X = O.synthetic(4, 64, 1, 31)
    W1 = O.synthetic(64, 32, 1, 32)
    H = O.matmul_forward(X, W1)
    W2 = O.synthetic(32, 16, 1, 33)
    gx, gw1, gh, gw2 = gpu_ctx.upload(X), gpu_ctx.upload(W1), gpu_ctx.upload(H), gpu_ctx.upload(W2)
    och = O.Channel()
    och.mix_u64(9)
    r = och.draw_qm31s(lg(4) + lg(16))
    v = O.matmul_output_claim(H, W2, r)
    och.mix_secure_field(v)
    gch = G.PoseidonChannel()
    gch.mix_u64(9)
    assert gch.draw_qm31s(lg(4) + lg(16)) == r
    gch.mix_secure_field(v)
    proof = G.Proof()
    C_ = G.CLAIM_CHAINED
    steps = [(G.STEP_MATMUL, C_, gh, gw2, 0, 0), (G.STEP_ACTIVATION, C_, gh, None, 5, 12),
             (G.STEP_MATMUL, C_, gx, gw1, 0, 0)]
    fp, fv = G.prove_walk(gpu_ctx, gch, steps, proof, init_point=r, init_value=v)
    o1 = O.prove_matmul_layer(r, v, H, W2, och)
    o2 = O.prove_activation_layer(o1["next_point"], o1["next_value"], H, 5, och, 12)
    o3 = O.prove_matmul_layer(o1["next_point"], o2["input_eval"], X, W1, och)
    assert (fp, fv) == (o3["next_point"], o3["next_value"])
    assert gch.digest() == och.digest()
    proof.set_input_claim(fp, fv)
    ref = [3]
    O.serialize_matmul_layer(ref, o1["round_polys"], o1["final_a_eval"], o1["final_b_eval"])
    O.serialize_activation_layer(ref, 5, o2)
    O.serialize_matmul_layer(ref, o3["round_polys"], o3["final_a_eval"], o3["final_b_eval"])
    O.serialize_tail(ref, o3["next_point"], o3["next_value"], [], 0)
    assert proof.serialize() == ref


def test_native_walk_fresh_claims(gpu_ctx):
    """gkr_prove_walk with fresh claims (draw point, claim, mix) equals the same sequence driven
    call by call from the host and the oracle's transcript; ragged shapes, two activations."""
    log("case native walk fresh")
    A1, B1 = O.synthetic(3, 50, 1, 41), O.synthetic(50, 20, 1, 42)
    A2, B2 = O.synthetic(5, 20, 1, 43), O.synthetic(20, 7, 1, 44)
    S = O.synthetic(6, 40, 0, 45)
    gs = [gpu_ctx.upload(M) for M in (A1, B1, A2, B2, S)]
    F = G.CLAIM_FRESH
    steps = [(G.STEP_MATMUL, F, gs[0], gs[1], 0, 0), (G.STEP_ACTIVATION, F, gs[4], None, 4, 10),
             (G.STEP_MATMUL, F, gs[2], gs[3], 0, 0), (G.STEP_ACTIVATION, F, gs[4], None, 2, 0)]
    gch = G.PoseidonChannel()
    gch.mix_u64(77)
    proof = G.Proof()
    fp, fv = G.prove_walk(gpu_ctx, gch, steps, proof)
    och = O.Channel()
    och.mix_u64(77)
    ref = [4]
    for kind, _, a, b, act, tlog in [(0, 0, A1, B1, 0, 0), (3, 0, S, None, 4, 10), (0, 0, A2, B2, 0, 0),
                                     (3, 0, S, None, 2, 0)]:
        if kind == 0:
            r = och.draw_qm31s(lg(a.shape[0]) + lg(b.shape[1]))
            v = O.matmul_output_claim(a, b, r)
            och.mix_secure_field(v)
            o = O.prove_matmul_layer(r, v, a, b, och)
            O.serialize_matmul_layer(ref, o["round_polys"], o["final_a_eval"], o["final_b_eval"])
            last = (o["next_point"], o["next_value"])
        else:
            r = och.draw_qm31s(lg(a.shape[0]) + lg(a.shape[1]))
            v = och.draw_qm31()
            o = O.prove_activation_layer(r, v, a, act, och, tlog or 16)
            O.serialize_activation_layer(ref, act, o)
            last = (r, o["input_eval"])
    assert (fp, fv) == last
    assert gch.digest() == och.digest()
    proof.set_input_claim(fp, fv)
    O.serialize_tail(ref, fp, fv, [], 0)
    assert proof.serialize() == ref


def test_walk_cancel_with_restriction_launched_ahead(gpu_ctx):
    """A walk that fails after the next matmul's restriction was launched ahead of its claim point
    (step 0's hand-over left by the test hook) cancels that queued wait: the context stays usable
    and the same walk then gives the same proof as before, equal to the oracle's."""
    log("case walk cancel with restriction launched ahead")
    A1, B1 = O.synthetic(4, 64, 1, 51), O.synthetic(64, 32, 1, 52)
    A2, B2 = O.synthetic(4, 32, 1, 53), O.synthetic(32, 16, 1, 54)
    gs = [gpu_ctx.upload(M) for M in (A1, B1, A2, B2)]
    F = G.CLAIM_FRESH
    steps = [(G.STEP_MATMUL, F, gs[0], gs[1], 0, 0), (G.STEP_MATMUL, F, gs[2], gs[3], 0, 0)]

    def run():
        ch = G.PoseidonChannel()
        ch.mix_u64(5)
        proof = G.Proof()
        fp, fv = G.prove_walk(gpu_ctx, ch, steps, proof)
        proof.set_input_claim(fp, fv)
        return ch.digest(), proof.serialize()

    first = run()  # sizes the context's buffers, so the next walks launch step 1's restriction ahead
    gpu_ctx.debug(G.DEBUG_HANDOVER_CANCEL, 0)
    with pytest.raises(G.GkrError):
        run()
    assert run() == first
    och = O.Channel()
    och.mix_u64(5)
    ref = [2]
    for a, b in ((A1, B1), (A2, B2)):
        r = och.draw_qm31s(lg(a.shape[0]) + lg(b.shape[1]))
        v = O.matmul_output_claim(a, b, r)
        och.mix_secure_field(v)
        o = O.prove_matmul_layer(r, v, a, b, och)
        O.serialize_matmul_layer(ref, o["round_polys"], o["final_a_eval"], o["final_b_eval"])
        last = (o["next_point"], o["next_value"])
    O.serialize_tail(ref, last[0], last[1], [], 0)
    assert first == (och.digest(), ref)


def test_walk_retries_a_step_whose_wait_expired(gpu_ctx):
    """A walk step whose hand-over wait expires before the host posts (the test hook cuts the bounded
    wait to 4 polls: a host held up longer than the wait) is proved again from the channel and
    claim it started from: the walk succeeds with the same proof and transcript as an undisturbed
    walk, and the retry is counted (timer id 19).  Steps: fresh MatMul (its hand-over expires, with
    the next MatMul's restriction already launched ahead), MatMul, SiLU activation, chained MatMul."""
    log("case walk retry after an expired wait")
    A1, B1 = O.synthetic(4, 64, 1, 61), O.synthetic(64, 32, 1, 62)
    A2, B2 = O.synthetic(4, 32, 1, 63), O.synthetic(32, 16, 1, 64)
    X = O.synthetic(4, 16, 0, 65)
    A3, B3 = O.synthetic(4, 8, 1, 66), O.synthetic(8, 16, 1, 67)
    gs = [gpu_ctx.upload(M) for M in (A1, B1, A2, B2, X, A3, B3)]
    F, Ch = G.CLAIM_FRESH, G.CLAIM_CHAINED
    steps = [(G.STEP_MATMUL, F, gs[0], gs[1], 0, 0), (G.STEP_MATMUL, F, gs[2], gs[3], 0, 0),
             (G.STEP_ACTIVATION, F, gs[4], None, 5, 10), (G.STEP_MATMUL, Ch, gs[5], gs[6], 0, 0)]

    def run():
        ch = G.PoseidonChannel()
        ch.mix_u64(6)
        proof = G.Proof()
        fp, fv = G.prove_walk(gpu_ctx, ch, steps, proof)
        proof.set_input_claim(fp, fv)
        return ch.digest(), proof.serialize()

    first = run()
    gpu_ctx.reset_timing()
    gpu_ctx.debug(G.DEBUG_HANDOVER_EXPIRE, 4)
    assert run() == first
    assert gpu_ctx.kernel_time(19)[1] == 1
    assert run() == first
    assert gpu_ctx.kernel_time(19)[1] == 1


ACT_KEYS = ("claimed_sum", "eq_round_polys", "final_evals", "mult_round_polys", "mult_final_eval",
            "mult_claimed_sum", "input_eval", "output_eval", "table_commitment")


def test_activation_layer_launched_ahead():
    """An activation layer of a size its context has proved before has its first kernels (eq tables,
    the table's inversion, the prepare pass, the eq-sumcheck's first trip) launched before the host
    draws gamma and beta; they wait on the device for the posted claim point and gamma, beta.  Five
    layers in a row on one context (two sizes of table, different inputs and claims): every output
    and the transcript equal the oracle's, and counter id 20 counts the three launched ahead."""
    log("case activation layer launched ahead")
    ctx = G.Context(0)
    try:
        for i, (tag, tlog) in enumerate([(5, 12), (5, 12), (5, 12), (3, 10), (3, 10)]):
            X = O.synthetic(12, 40, 0, 700 + i)
            nv = lg(12) + lg(40)
            gch, och = G.PoseidonChannel(), O.Channel()
            gch.mix_u64(i)
            och.mix_u64(i)
            pt = gch.draw_qm31s(nv)
            val = gch.draw_qm31()
            assert pt == och.draw_qm31s(nv) and val == och.draw_qm31()
            pg = ctx.prove_activation_layer(pt, val, ctx.upload(X), tag, gch, tlog)
            po = O.prove_activation_layer(pt, val, X, tag, och, tlog)
            for key in ACT_KEYS:
                assert pg[key] == po[key], (i, key)
            assert (pg["multiplicities"] == po["multiplicities"]).all()
            assert gch.digest() == och.digest()
        assert ctx.kernel_time(20)[1] == 3
    finally:
        ctx.close()


def test_walk_activation_launched_ahead():
    """Walk steps MatMul, activation (fresh claim), MatMul, activation (chained claim), MatMul: once
    the context has proved an activation of that size, an activation step's first kernels are
    launched at the previous step's last launch and wait on the device for the claim point and
    gamma, beta, which the step posts.  Two walks on one context (one and two steps launched ahead,
    counter id 20) both equal the oracle's transcript and serialized proof."""
    log("case walk activation launched ahead")
    A1, B1 = O.synthetic(4, 64, 1, 81), O.synthetic(64, 32, 1, 82)
    A2, B2 = O.synthetic(4, 32, 1, 83), O.synthetic(32, 16, 1, 84)
    A3, B3 = O.synthetic(2, 48, 1, 85), O.synthetic(48, 8, 1, 86)
    S = O.synthetic(8, 16, 0, 87)  # 2^7 entries, as A2
    och = O.Channel()
    och.mix_u64(21)
    ref = [5]
    last = None
    for kind, a, b in [(0, A1, B1), (3, S, None), (0, A2, B2), (4, A2, None), (0, A3, B3)]:
        if kind == 0:
            r = och.draw_qm31s(lg(a.shape[0]) + lg(b.shape[1]))
            v = O.matmul_output_claim(a, b, r)
            och.mix_secure_field(v)
            o = O.prove_matmul_layer(r, v, a, b, och)
            O.serialize_matmul_layer(ref, o["round_polys"], o["final_a_eval"], o["final_b_eval"])
            last = (o["next_point"], o["next_value"])
        else:
            if kind == 3:
                r = och.draw_qm31s(lg(a.shape[0]) + lg(a.shape[1]))
                v = och.draw_qm31()
            else:
                r, v = last
            o = O.prove_activation_layer(r, v, a, 5, och, 12)
            O.serialize_activation_layer(ref, 5, o)
            last = (r, o["input_eval"])
    O.serialize_tail(ref, last[0], last[1], [], 0)
    ctx = G.Context(0)
    try:
        gs = [ctx.upload(M) for M in (A1, B1, A2, B2, A3, B3, S)]
        F, Ch = G.CLAIM_FRESH, G.CLAIM_CHAINED
        steps = [(G.STEP_MATMUL, F, gs[0], gs[1], 0, 0), (G.STEP_ACTIVATION, F, gs[6], None, 5, 12),
                 (G.STEP_MATMUL, F, gs[2], gs[3], 0, 0), (G.STEP_ACTIVATION, Ch, gs[2], None, 5, 12),
                 (G.STEP_MATMUL, F, gs[4], gs[5], 0, 0)]
        for ahead in (1, 3):
            ch = G.PoseidonChannel()
            ch.mix_u64(21)
            proof = G.Proof()
            fp, fv = G.prove_walk(ctx, ch, steps, proof)
            assert (fp, fv) == last
            assert ch.digest() == och.digest()
            proof.set_input_claim(fp, fv)
            assert proof.serialize() == ref
            assert ctx.kernel_time(20)[1] == ahead
    finally:
        ctx.close()


def test_activation_values_wait_expired():
    """An activation layer whose first kernels were launched ahead, with the test hook cutting the
    bounded wait for its gamma and beta to 4 polls (it expires before the host posts them): a walk
    proves that step again (counter id 19) and gives the same proof as an undisturbed walk; a direct
    call fails with GKR_ERR_DEVICE, and the next call equals the oracle's layer."""
    log("case activation values wait expired")
    S = O.synthetic(8, 16, 0, 91)
    A, B = O.synthetic(4, 32, 1, 92), O.synthetic(32, 16, 1, 93)
    ctx = G.Context(0)
    try:
        gs, ga, gb = ctx.upload(S), ctx.upload(A), ctx.upload(B)
        F = G.CLAIM_FRESH
        steps = [(G.STEP_ACTIVATION, F, gs, None, 5, 12), (G.STEP_MATMUL, F, ga, gb, 0, 0)]

        def walk():
            ch = G.PoseidonChannel()
            ch.mix_u64(31)
            proof = G.Proof()
            fp, fv = G.prove_walk(ctx, ch, steps, proof)
            proof.set_input_claim(fp, fv)
            return ch.digest(), proof.serialize()

        first = walk()  # the context's first activation of this size: proved the ordinary way
        assert walk() == first and ctx.kernel_time(20)[1] == 1
        ctx.reset_timing()
        ctx.debug(G.DEBUG_TRIP_EXPIRE, 4)
        assert walk() == first
        assert ctx.kernel_time(19)[1] == 1
        assert walk() == first
        assert ctx.kernel_time(19)[1] == 1
        nv = lg(8) + lg(16)
        for expire in (True, False):
            gch, och = G.PoseidonChannel(), O.Channel()
            pt = gch.draw_qm31s(nv)
            val = gch.draw_qm31()
            assert pt == och.draw_qm31s(nv) and val == och.draw_qm31()
            if expire:
                ctx.debug(G.DEBUG_TRIP_EXPIRE, 4)
                with pytest.raises(G.GkrError) as e:
                    ctx.prove_activation_layer(pt, val, gs, 5, gch, 12)
                assert e.value.code == 2 and "posted values" in str(e.value)
                continue
            pg = ctx.prove_activation_layer(pt, val, gs, 5, gch, 12)
            po = O.prove_activation_layer(pt, val, S, 5, och, 12)
            for key in ACT_KEYS:
                assert pg[key] == po[key], key
            assert gch.digest() == och.digest()
    finally:
        ctx.close()


def _trip_walk(ctx, mats):
    """Fresh MatMul (k = 4096: its second trip is launched ahead), SiLU LogUp over 2^16 entries (eq and
    multiplicity trips launched ahead), MatMul; returns (digest, serialized proof)."""
    gs = [ctx.upload(M) for M in mats]
    F = G.CLAIM_FRESH
    steps = [(G.STEP_MATMUL, F, gs[0], gs[1], 0, 0), (G.STEP_ACTIVATION, F, gs[2], None, 5, 16),
             (G.STEP_MATMUL, F, gs[3], gs[4], 0, 0)]
    ch = G.PoseidonChannel()
    ch.mix_u64(12)
    proof = G.Proof()
    fp, fv = G.prove_walk(ctx, ch, steps, proof)
    proof.set_input_claim(fp, fv)
    return ch.digest(), proof.serialize()


TRIP_MATS = [O.synthetic(4, 4096, 1, 71), O.synthetic(4096, 16, 1, 72), O.synthetic(64, 1024, 0, 73),
             O.synthetic(8, 2048, 1, 74), O.synthetic(2048, 64, 1, 75)]


def test_walk_retries_a_step_whose_trip_wait_expired(gpu_ctx):
    """The first trip launched ahead in a walk (the MatMul's second trip, behind k_mailbox_wait) stops
    waiting after 4 polls, before the host posts its challenges (test hook): the step is proved
    again and the walk gives the same proof as an undisturbed one; the retry is counted (timer id
    19), and the next walk runs undisturbed."""
    log("case walk retry after an expired trip wait")
    first = _trip_walk(gpu_ctx, TRIP_MATS)
    gpu_ctx.reset_timing()
    gpu_ctx.debug(G.DEBUG_TRIP_EXPIRE, 4)
    assert _trip_walk(gpu_ctx, TRIP_MATS) == first
    assert gpu_ctx.kernel_time(19)[1] == 1
    assert _trip_walk(gpu_ctx, TRIP_MATS) == first
    assert gpu_ctx.kernel_time(19)[1] == 1


def test_walk_without_launcher_thread(gpu_ctx):
    """A context created with GKR_ASYNC_LAUNCH=0 (the calling thread issues every launch) proves
    the same fresh-claim walk, bit for bit, as the default context (launches issued by the
    context's launcher thread)."""
    log("case walk without launcher thread")
    old = os.environ.get("GKR_ASYNC_LAUNCH")
    os.environ["GKR_ASYNC_LAUNCH"] = "0"
    try:
        sctx = G.Context(0)
    finally:
        if old is None:
            del os.environ["GKR_ASYNC_LAUNCH"]
        else:
            os.environ["GKR_ASYNC_LAUNCH"] = old
    try:
        mats = [O.synthetic(4, 96, 1, 61), O.synthetic(96, 40, 1, 62), O.synthetic(4, 40, 1, 63),
                O.synthetic(40, 24, 1, 64), O.synthetic(8, 40, 0, 65)]
        F = G.CLAIM_FRESH
        proofs = []
        for ctx in (gpu_ctx, sctx):
            gs = [ctx.upload(M) for M in mats]
            steps = [(G.STEP_MATMUL, F, gs[0], gs[1], 0, 0), (G.STEP_ACTIVATION, F, gs[4], None, 5, 10),
                     (G.STEP_MATMUL, F, gs[2], gs[3], 0, 0), (G.STEP_MATMUL, F, gs[2], gs[3], 0, 0)]
            for _ in range(2):  # the second walk launches restrictions ahead of their points
                ch = G.PoseidonChannel()
                ch.mix_u64(9)
                proof = G.Proof()
                fp, fv = G.prove_walk(ctx, ch, steps, proof)
                proof.set_input_claim(fp, fv)
                proofs.append((ch.digest(), proof.serialize()))
        assert proofs[0] == proofs[1] == proofs[2] == proofs[3]
    finally:
        sctx.close()


def test_native_walk_errors(gpu_ctx):
    """A chained first step without an initial claim and an unknown step kind are rejected."""
    log("case native walk errors")
    a = gpu_ctx.upload(O.synthetic(2, 4, 1, 1))
    b = gpu_ctx.upload(O.synthetic(4, 2, 1, 2))
    with pytest.raises(G.GkrError, match="no previous claim"):
        G.prove_walk(gpu_ctx, G.PoseidonChannel(), [(G.STEP_MATMUL, G.CLAIM_CHAINED, a, b, 0, 0)], G.Proof())
    with pytest.raises(G.GkrError, match="unknown kind"):
        G.prove_walk(gpu_ctx, G.PoseidonChannel(), [(7, G.CLAIM_FRESH, a, b, 0, 0)], G.Proof())


@pytest.mark.parametrize("path", ["u32", "int8"])
def test_qwen_up_projection_properties(gpu_ctx, int8_ctx, path):
    """Qwen2.5-14B MLP up projection (64 x 5120 . 5120 x 13824, int8-range): verifier replay and
    final evaluations equal MLE_A / MLE_B^T at the challenge point (oracle on the CPU)."""
    gpu_ctx = int8_ctx if path == "int8" else gpu_ctx
    m, k, n = 64, 5120, 13824
    log("case qwen up 64x5120x13824 " + path)
    a = gpu_ctx.synthetic(m, k, 1, 101)
    b = gpu_ctx.synthetic(k, n, 1, 102)
    ch = G.PoseidonChannel()
    ch.mix_u64(42)
    vch = O.Channel()
    vch.mix_u64(42)
    nv = lg(m) + lg(n)
    r = ch.draw_qm31s(nv)
    assert r == vch.draw_qm31s(nv)
    v = gpu_ctx.matmul_output_claim(a, b, r)
    res = gpu_ctx.prove_matmul_layer(r, v, a, b, ch)
    assert len(res["round_polys"]) == 13
    assert O.verify_matmul_layer(r, v, m, k, n, res["round_polys"], res["final_a_eval"], res["final_b_eval"],
                                 vch) == 0
    assert vch.digest() == ch.digest()
    A = O.synthetic(m, k, 1, 101)
    lm = lg(m)
    fa = O.restrict_rows_fused(A, r[:lm], npow2(k))
    assert O.evaluate_mle([tuple(int(x) for x in row) for row in fa], res["next_point"][lm:]) == res["final_a_eval"]
    B = b.download()
    assert B[7, 11] == O.synthetic_value(1, 102, 7 * n + 11)
    fb = O.restrict_cols_fused(B, r[lm:], npow2(k))
    assert O.evaluate_mle([tuple(int(x) for x in row) for row in fb], res["next_point"][lm:]) == res["final_b_eval"]
    # the claim is MLE_C(r) = sum_l f_a[l] f_b[l]
    s = (0, 0, 0, 0)
    for x, y in zip(fa, fb):
        s = O.qadd(s, O.qmul(tuple(int(t) for t in x), tuple(int(t) for t in y)))
    assert v == s


def test_matrix_outlives_context():
    """Freeing a matrix after its context was destroyed is safe; using it is an error."""
    ctx = G.Context(0)
    a = ctx.upload(np.ones((2, 2), dtype=np.uint32))
    b = ctx.upload(np.ones((2, 2), dtype=np.uint32))
    ctx.close()
    a.free()
    other = G.Context(0)
    ch = G.PoseidonChannel()
    with pytest.raises(G.GkrError):
        other.reduce_matmul_layer(b, b, [(1, 0, 0, 0)], [(1, 0, 0, 0)], 2, ch)
    b.free()
    other.close()


def test_walk_trace_equals_oracle_trace(gpu_ctx, tmp_path):
    """GKR_CHANNEL_TRACE on the GPU prover: the chained MatMul -> Mul -> Activation -> MatMul walk of
    tests/test_trace.py proved by gkr_prove_walk writes the same trace, line for line, as the oracle
    proving it (ORACLE_CHANNEL_TRACE)."""
    import test_trace as T
    log("case walk transcript trace")
    ot, gt = str(tmp_path / "oracle.trace"), str(tmp_path / "gpu.trace")
    cd, shapes, start, r, v, end = T.chained_walk_proof(ot)
    rng = np.random.default_rng(5)  # the walk's matrices, as chained_walk_proof draws them
    X0 = rng.integers(0, P, size=(4, 12), dtype=np.uint32)
    W0 = rng.integers(0, P, size=(12, 16), dtype=np.uint32)
    H = O.matmul_forward(X0, W0)
    L = np.vectorize(lambda x: O.activation(3, int(x)), otypes=[np.uint32])(H)
    R = rng.integers(0, P, size=(4, 16), dtype=np.uint32)
    X = ((L.astype(np.uint64) * R) % P).astype(np.uint32)
    W = rng.integers(0, P, size=(16, 8), dtype=np.uint32)
    dev = {k: gpu_ctx.upload(m) for k, m in dict(X0=X0, W0=W0, H=H, L=L, R=R, X=X, W=W).items()}
    Ch = G.CLAIM_CHAINED
    arr = G.make_steps([(G.STEP_MATMUL, Ch, dev["X"], dev["W"], 0, 0), (G.STEP_MUL, Ch, dev["L"], dev["R"], 0, 0),
                        (G.STEP_ACTIVATION, Ch, dev["H"], None, 3, 8), (G.STEP_MATMUL, Ch, dev["X0"], dev["W0"], 0, 0)])
    gch = G.PoseidonChannel()
    gch.import_state(start)
    old = os.environ.get("GKR_CHANNEL_TRACE")
    os.environ["GKR_CHANNEL_TRACE"] = gt
    try:
        G.prove_walk(gpu_ctx, gch, arr, G.Proof(), n_steps=4, init_point=r, init_value=v)
    finally:
        if old is None:
            os.environ.pop("GKR_CHANNEL_TRACE", None)
        else:
            os.environ["GKR_CHANNEL_TRACE"] = old
    assert gch.digest() == end
    assert T.read(gt) == T.read(ot)
    assert [x[0] for x in T.read(gt)] == T.EXPECTED_LABELS
