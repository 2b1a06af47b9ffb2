"""The oracle's SIMD matmul reductions: the shared-weight one (reduce_matmul_layer_simd_gpu,
engine/src/gkr/prover.rs:5422-5600) pinned on the CPU: one block with weight 1 is
the plain matmul reduction (itself pinned by the SP3 fixture); the block combine
against the pure-Python QM31 tower; for several blocks the sumcheck identities,
final_a = sum_b w_b MLE_{A_b} and final_b = MLE_{B^T} by brute force, and the
restated MatMul verifier accepting the proof of the claim sum_b w_b MLE_{A_b B}(r).
"""
import random

import numpy as np
import oracle as O
import pytest
import qm31_py as Q

P = (1 << 31) - 1


def rq(rng):
    return tuple(rng.randrange(P) for _ in range(4))


def test_block_combine_against_tower():
    rng = random.Random(3)
    w = rq(rng)
    X = np.array([rq(rng) for _ in range(64)], dtype=np.uint32)
    Y = O.qmul_rows(w, X)
    for i in range(64):
        assert tuple(int(v) for v in Y[i]) == Q.qmul(w, tuple(int(v) for v in X[i]))


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 37, 11), (4, 64, 8)])
def test_one_block_is_the_matmul_reduction(m, k, n):
    rng = np.random.default_rng(m + k + n)
    A = rng.integers(0, P, size=(m, k), dtype=np.uint32)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    c1, c2 = O.Channel(), O.Channel()
    c1.mix_u64(7)
    c2.mix_u64(7)
    nv = (max(0, (m - 1).bit_length())) + (max(0, (n - 1).bit_length()))
    r = c1.draw_qm31s(nv)
    assert c2.draw_qm31s(nv) == r
    v = O.matmul_output_claim(A, B, r)
    assert O.prove_matmul_layer_simd(r, v, [A], B, [(1, 0, 0, 0)], c2) == O.prove_matmul_layer(r, v, A, B, c1)
    assert c1.digest() == c2.digest()


@pytest.mark.parametrize("m,k,n,nb", [(3, 6, 5, 2), (2, 8, 4, 3), (4, 5, 3, 4)])
def test_blocks_identities_bruteforce_and_verifier(m, k, n, nb):
    rng = np.random.default_rng(100 * nb + k)
    prng = random.Random(nb)
    As = [rng.integers(0, P, size=(m, k), dtype=np.uint32) for _ in range(nb)]
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    ws = [rq(prng) for _ in range(nb)]
    ch = O.Channel()
    ch.mix_u64(11)
    pm, pk, pn = [1 << max(0, (v - 1).bit_length()) for v in (m, k, n)]
    lm = pm.bit_length() - 1
    r = ch.draw_qm31s(lm + pn.bit_length() - 1)
    claim = (0, 0, 0, 0)
    for A, w in zip(As, ws):
        claim = Q.qadd(claim, Q.qmul(w, O.matmul_output_claim(A, B, r)))
    vch = ch.clone()
    res = O.prove_matmul_layer_simd(r, claim, As, B, ws, ch)
    cur = claim
    for (c0, c1, c2), rr in zip(res["round_polys"], res["next_point"][lm:]):
        assert Q.qadd(c0, Q.qadd(Q.qadd(c0, c1), c2)) == cur
        cur = Q.qadd(Q.qadd(c0, Q.qmul(c1, rr)), Q.qmul(Q.qmul(c2, rr), rr))
    assert cur == Q.qmul(res["final_a_eval"], res["final_b_eval"])
    fa = (0, 0, 0, 0)
    for A, w in zip(As, ws):
        Ap = np.zeros((pm, pk), dtype=np.uint32)
        Ap[:m, :k] = A
        fa = Q.qadd(fa, Q.qmul(w, O.evaluate_mle([(int(v), 0, 0, 0) for v in Ap.reshape(-1)], res["next_point"])))
    assert fa == res["final_a_eval"]
    Bp = np.zeros((pk, pn), dtype=np.uint32)
    Bp[:k, :n] = B
    assert O.evaluate_mle([(int(v), 0, 0, 0) for v in Bp.T.reshape(-1)], r[lm:] + res["next_point"][lm:]) == \
        res["final_b_eval"]
    assert O.verify_matmul_layer(r, claim, m, k, n, res["round_polys"], res["final_a_eval"], res["final_b_eval"],
                                 vch) == 0
    assert vch.digest() == ch.digest()


def _bruteforce_rounds(w, a, b, chals):
    """Round values s(t), t = 0..3, of sum w a b with the top variables bound to chals (pure Python)."""
    vals = [list(map(tuple, v)) for v in (w, a, b)]
    out = []
    for r in chals:
        mid = len(vals[0]) // 2
        s = []
        for t in range(4):
            tt = (t, 0, 0, 0)
            acc = (0, 0, 0, 0)
            for i in range(mid):
                e = [Q.qadd(v[i], Q.qmul(tt, Q.qsub(v[mid + i], v[i]))) for v in vals]
                acc = Q.qadd(acc, Q.qmul(Q.qmul(e[0], e[1]), e[2]))
            s.append(acc)
        out.append(s)
        vals = [[Q.qadd(v[i], Q.qmul(r, Q.qsub(v[mid + i], v[i]))) for i in range(mid)] for v in vals]
    return out, [v[0] for v in vals]


def _poly(c, x):
    return Q.qadd(Q.qadd(c[0], Q.qmul(c[1], x)), Q.qadd(Q.qmul(Q.qmul(c[2], x), x),
                                                         Q.qmul(Q.qmul(Q.qmul(c[3], x), x), x)))


@pytest.mark.parametrize("n", [1, 2, 8, 16])
def test_sumcheck_3way_bruteforce(n):
    rng = random.Random(n)
    w, a, b = ([rq(rng) for _ in range(n)] for _ in range(3))
    ch = O.Channel()
    ch.mix_u64(n)
    res = O.sumcheck_3way(np.array(w, dtype=np.uint32), np.array(a, dtype=np.uint32), np.array(b, dtype=np.uint32),
                          ch)
    svals, fins = _bruteforce_rounds(w, a, b, res["challenges"])
    for c, s in zip(res["round_polys"], svals):
        for t in range(4):
            assert _poly(c, (t, 0, 0, 0)) == s[t]
    assert (res["final_w"], res["final_a"], res["final_b"]) == tuple(fins)


@pytest.mark.parametrize("m,k,n,nb", [(2, 3, 2, 1), (3, 6, 5, 2), (2, 8, 4, 4)])
def test_dual_simd_identities_and_bruteforce(m, k, n, nb):
    rng = np.random.default_rng(31 * nb + k)
    prng = random.Random(nb + 7)
    As = [rng.integers(0, P, size=(m, k), dtype=np.uint32) for _ in range(nb)]
    Bs = [rng.integers(0, P, size=(k, n), dtype=np.uint32) for _ in range(nb)]
    ws = [rq(prng) for _ in range(nb)]
    ch = O.Channel()
    ch.mix_u64(5)
    pm, pk, pn = [1 << max(0, (v - 1).bit_length()) for v in (m, k, n)]
    lm = pm.bit_length() - 1
    r = ch.draw_qm31s(lm + pn.bit_length() - 1)
    claim = (0, 0, 0, 0)
    for A, B, w in zip(As, Bs, ws):
        claim = Q.qadd(claim, Q.qmul(w, O.matmul_output_claim(A, B, r)))
    res = O.prove_matmul_layer_dual_simd(r, claim, As, Bs, ws, ch)
    cur = claim
    for c, x in zip(res["round_polys"], res["challenges"]):
        assert Q.qadd(_poly(c, (0, 0, 0, 0)), _poly(c, (1, 0, 0, 0))) == cur
        cur = _poly(c, x)
    assert cur == Q.qmul(Q.qmul(res["final_w"], res["final_a_eval"]), res["final_b_eval"])
    nbv = res["n_block_vars"]
    rb, rk = res["challenges"][:nbv], res["challenges"][nbv:]
    fa = fb = fw = (0, 0, 0, 0)
    for i, (A, B, w) in enumerate(zip(As, Bs, ws)):
        e = O.evaluate_mle([(1 if j == i else 0, 0, 0, 0) for j in range(nb)], rb) if nbv else (1, 0, 0, 0)
        Ap = np.zeros((pm, pk), dtype=np.uint32)
        Ap[:m, :k] = A
        Bp = np.zeros((pk, pn), dtype=np.uint32)
        Bp[:k, :n] = B
        fa = Q.qadd(fa, Q.qmul(e, O.evaluate_mle([(int(v), 0, 0, 0) for v in Ap.reshape(-1)], r[:lm] + rk)))
        fb = Q.qadd(fb, Q.qmul(e, O.evaluate_mle([(int(v), 0, 0, 0) for v in Bp.T.reshape(-1)], r[lm:] + rk)))
        fw = Q.qadd(fw, Q.qmul(e, w))
    assert (fa, fb, fw) == (res["final_a_eval"], res["final_b_eval"], res["final_w"])
