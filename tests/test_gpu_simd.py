"""Shared-weight SIMD matmul layer on the GPU (gkr_prove_matmul_layer_simd =
reduce_matmul_layer_simd_gpu, engine/src/gkr/prover.rs:5422-5600) against the oracle:
round polynomials, final evaluations, next claim and channel digest bit-exact."""
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


def lg(v):
    return max(0, (v - 1).bit_length())


def _compare(ctx, As, B, ws, seed, label):
    log(f"case simd {label}: {len(As)} blocks A{As[0].shape} B{B.shape}")
    m, k = As[0].shape
    n = B.shape[1]
    a = [ctx.upload(A) for A in As]
    b = ctx.upload(B)
    gch, och = G.PoseidonChannel(), O.Channel()
    gch.mix_u64(seed)
    och.mix_u64(seed)
    r = gch.draw_qm31s(lg(m) + lg(n))
    assert r == och.draw_qm31s(lg(m) + lg(n))
    v = (0, 0, 0, 0)
    for A, w in zip(As, ws):
        v = O.qadd(v, O.qmul(w, O.matmul_output_claim(A, B, r)))
    proof = G.Proof()
    rg = ctx.prove_matmul_layer_simd(r, v, a, ws, b, gch, proof)
    ro = O.prove_matmul_layer_simd(r, v, As, B, ws, och)
    assert rg == ro
    assert gch.digest() == och.digest()
    for x in a:
        x.free()
    b.free()
    return proof


@pytest.mark.parametrize("m,k,n,nb", [(1, 1, 1, 1), (1, 4, 2, 2), (3, 37, 11, 3), (2, 1, 3, 5), (8, 300, 70, 4),
                                      (64, 512, 256, 8), (5, 2048, 9, 64), (16, 1000, 513, 2)])
def test_simd_layer_matches_oracle(gpu_ctx, m, k, n, nb):
    rng = np.random.default_rng(m * 7 + k * 3 + n + nb)
    prng = random.Random(nb * 1000 + k)
    As = [rng.integers(0, P, size=(m, k), dtype=np.uint32) for _ in range(nb)]
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    ws = [tuple(prng.randrange(P) for _ in range(4)) for _ in range(nb)]
    _compare(gpu_ctx, As, B, ws, nb + 1, "random")


def test_simd_layer_int8_range_and_proof_record(gpu_ctx):
    As = [O.synthetic(64, 1024, 1, 40 + i) for i in range(4)]
    B = O.synthetic(1024, 2048, 1, 50)
    prng = random.Random(9)
    ws = [tuple(prng.randrange(P) for _ in range(4)) for _ in range(4)]
    proof = _compare(gpu_ctx, As, B, ws, 3, "int8 range")
    felts = proof.serialize()
    assert felts[0] == 1 and felts[1] == 0  # one layer, tag 0 (MatMul)


def test_simd_layer_errors(gpu_ctx):
    A = gpu_ctx.upload(np.ones((2, 4), dtype=np.uint32))
    A2 = gpu_ctx.upload(np.ones((2, 5), dtype=np.uint32))
    B = gpu_ctx.upload(np.ones((4, 2), dtype=np.uint32))
    r = [(1, 0, 0, 0), (2, 0, 0, 0)]
    ch = G.PoseidonChannel()
    with pytest.raises(G.GkrError):
        gpu_ctx.prove_matmul_layer_simd(r, (0, 0, 0, 0), [A, A2], [(1, 0, 0, 0)] * 2, B, ch)  # shape mismatch
    with pytest.raises(G.GkrError):
        gpu_ctx.prove_matmul_layer_simd(r, (0, 0, 0, 0), [A], [(P, 0, 0, 0)], B, ch)  # weight not canonical
    with pytest.raises(G.GkrError):
        gpu_ctx.prove_matmul_layer_simd(r, (0, 0, 0, 0), [A] * 65, [(1, 0, 0, 0)] * 65, B, ch)  # too many blocks
    with pytest.raises(G.GkrError):
        gpu_ctx.prove_matmul_layer_simd(r[:1], (0, 0, 0, 0), [A], [(1, 0, 0, 0)], B, ch)  # claim size
    for x in (A, A2, B):
        x.free()


@pytest.mark.parametrize("m,k,n,nb", [(1, 1, 1, 1), (2, 3, 2, 2), (3, 37, 11, 4), (8, 300, 70, 8), (64, 256, 128, 16),
                                      (4, 64, 8, 64), (16, 1000, 513, 2)])
def test_dual_simd_layer_matches_oracle(gpu_ctx, m, k, n, nb):
    log(f"case dual simd {nb} blocks A({m},{k}) B({k},{n})")
    rng = np.random.default_rng(m * 5 + k + n * 3 + nb)
    prng = random.Random(nb * 77 + k)
    As = [rng.integers(0, P, size=(m, k), dtype=np.uint32) for _ in range(nb)]
    Bs = [rng.integers(0, P, size=(k, n), dtype=np.uint32) for _ in range(nb)]
    ws = [tuple(prng.randrange(P) for _ in range(4)) for _ in range(nb)]
    a = [gpu_ctx.upload(A) for A in As]
    b = [gpu_ctx.upload(B) for B in Bs]
    gch, och = G.PoseidonChannel(), O.Channel()
    gch.mix_u64(nb)
    och.mix_u64(nb)
    r = gch.draw_qm31s(lg(m) + lg(n))
    assert r == och.draw_qm31s(lg(m) + lg(n))
    v = (0, 0, 0, 0)
    for A, B, w in zip(As, Bs, ws):
        v = O.qadd(v, O.qmul(w, O.matmul_output_claim(A, B, r)))
    proof = G.Proof()
    rg = gpu_ctx.prove_matmul_layer_dual_simd(r, v, a, b, ws, gch, proof)
    ro = O.prove_matmul_layer_dual_simd(r, v, As, Bs, ws, och)
    assert rg["round_polys"] == ro["round_polys"]
    assert (rg["final_a_eval"], rg["final_b_eval"], rg["n_block_vars"]) == \
        (ro["final_a_eval"], ro["final_b_eval"], ro["n_block_vars"])
    assert gch.digest() == och.digest()
    felts = proof.serialize()
    rounds = len(ro["round_polys"])
    assert felts[:4] == [1, 7, ro["n_block_vars"], rounds]  # one layer: MatMulDualSimd, n_block_vars, rounds
    body = [x for (c0, _c1, c2, c3) in ro["round_polys"] for q in (c0, c2, c3) for x in q]
    body += list(ro["final_a_eval"]) + list(ro["final_b_eval"])
    assert felts[4:4 + len(body)] == body  # c1 omitted (cairo_serde.rs:1629-1646)
    for x in a + b:
        x.free()


def test_dual_simd_errors(gpu_ctx):
    A = gpu_ctx.upload(np.ones((2, 4), dtype=np.uint32))
    B = gpu_ctx.upload(np.ones((4, 2), dtype=np.uint32))
    r = [(1, 0, 0, 0), (2, 0, 0, 0)]
    ch = G.PoseidonChannel()
    with pytest.raises(G.GkrError):  # not a power of two
        gpu_ctx.prove_matmul_layer_dual_simd(r, (0, 0, 0, 0), [A] * 3, [B] * 3, [(1, 0, 0, 0)] * 3, ch)
    with pytest.raises(G.GkrError):  # weight not canonical
        gpu_ctx.prove_matmul_layer_dual_simd(r, (0, 0, 0, 0), [A], [B], [(0, P, 0, 0)], ch)
    for x in (A, B):
        x.free()
