"""The CPU oracle pinned by what the mathematics fixes (no GPU).

Brute-force MLE sums on tiny inputs (pure-Python third implementation),
fused == naive restriction (the equality the reference relies on in
components/matmul.rs:2045-2218), sumcheck and LogUp identities, and the
restated verifier accepting honest proofs and rejecting tampered ones.
"""
import random

import numpy as np
import oracle as O
import pytest
import qm31_py as Q

P = (1 << 31) - 1


def rq(rng):
    return tuple(rng.randrange(P) for _ in range(4))


def test_qm31_field_axioms():
    rng = random.Random(1)
    for _ in range(50):
        x, y, z = rq(rng), rq(rng), rq(rng)
        assert O.qmul(x, y) == Q.qmul(x, y)
        assert O.qmul(O.qmul(x, y), z) == O.qmul(x, O.qmul(y, z))
        assert O.qmul(x, O.qadd(y, z)) == O.qadd(O.qmul(x, y), O.qmul(x, z))
        assert O.qmul(x, O.qinv(x)) == (1, 0, 0, 0)
    # u^2 = 2 + i
    assert O.qmul((0, 0, 1, 0), (0, 0, 1, 0)) == (2, 1, 0, 0)
    # inverse through Fermat in the full extension (pure Python)
    x = rq(rng)
    assert O.qinv(x) == Q.qinv(x)


@pytest.mark.parametrize("n", [0, 1, 2, 3, 5])
def test_evaluate_mle_bruteforce(n):
    rng = random.Random(n)
    evals = [rq(rng) for _ in range(1 << n)]
    point = [rq(rng) for _ in range(n)]
    assert O.evaluate_mle(evals, point) == Q.mle_bruteforce(evals, point)


def test_eq_tables_agree_and_bruteforce():
    rng = random.Random(7)
    r = [rq(rng) for _ in range(5)]
    eq = O.eq_evals(r)
    lg = O.lagrange_basis(r)
    assert (eq == lg).all()
    for x in range(32):
        assert tuple(int(v) for v in eq[x]) == Q.eq_weight(r, x, 5)
    s = (0, 0, 0, 0)
    for x in range(32):
        s = Q.qadd(s, tuple(int(v) for v in eq[x]))
    assert s == (1, 0, 0, 0)  # sum of eq over the hypercube


def test_restrict_mle_bruteforce():
    rng = random.Random(3)
    n, s = 5, 2
    evals = [rq(rng) for _ in range(1 << n)]
    assign = [rq(rng) for _ in range(s)]
    out = O.restrict_mle(evals, assign)
    rest = 1 << (n - s)
    for y in range(rest):
        want = (0, 0, 0, 0)
        for x in range(1 << s):
            want = Q.qadd(want, Q.qmul(Q.eq_weight(assign, x, s), evals[x * rest + y]))
        assert out[y] == want


@pytest.mark.parametrize("m,k,n", [(1, 4, 2), (3, 5, 7), (8, 16, 4), (5, 1, 3), (16, 33, 9)])
def test_fused_restrict_equals_naive(m, k, n):
    rng = np.random.default_rng(m * 100 + k * 10 + n)
    A = rng.integers(0, P, size=(m, k), dtype=np.uint32)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    pm, pk, pn = [1 << max(0, (v - 1).bit_length()) for v in (m, k, n)]
    r = random.Random(m + k + n)
    r_i = [rq(r) for _ in range(pm.bit_length() - 1)]
    r_j = [rq(r) for _ in range(pn.bit_length() - 1)]
    # naive: pad -> MLE -> restrict (backend.rs:127-134)
    Ap = np.zeros((pm, pk), dtype=np.uint32)
    Ap[:m, :k] = A
    a_mle = [(int(v), 0, 0, 0) for v in Ap.reshape(-1)]
    fa = O.restrict_mle(a_mle, r_i)
    Bp = np.zeros((pk, pn), dtype=np.uint32)
    Bp[:k, :n] = B
    b_mle = [(int(v), 0, 0, 0) for v in Bp.T.reshape(-1)]  # column-major
    fb = O.restrict_mle(b_mle, r_j)
    fa2 = O.restrict_rows_fused(A, r_i, pk)
    fb2 = O.restrict_cols_fused(B, r_j, pk)
    assert [tuple(int(x) for x in row) for row in fa2] == fa
    assert [tuple(int(x) for x in row) for row in fb2] == fb
    # MLE_C(r_i || r_j) == sum_l f_a[l] f_b[l]   (C = A B)
    claim = O.matmul_output_claim(A, B, r_i + r_j)
    s = (0, 0, 0, 0)
    for x, y in zip(fa, fb):
        s = Q.qadd(s, Q.qmul(x, y))
    assert s == claim


@pytest.mark.parametrize("m,k,n", [(1, 4, 2), (4, 8, 4), (3, 7, 5), (1, 1, 1), (2, 1, 3), (6, 3, 1)])
def test_matmul_sumcheck_identities_and_verifier(m, k, n):
    rng = np.random.default_rng(k * 31 + m)
    A = rng.integers(0, P, size=(m, k), dtype=np.uint32)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    ch = O.Channel()
    ch.mix_u64(99)
    pm, pk, pn = [1 << max(0, (v - 1).bit_length()) for v in (m, k, n)]
    nv = (pm.bit_length() - 1) + (pn.bit_length() - 1)
    r = ch.draw_qm31s(nv)
    claim = O.matmul_output_claim(A, B, r)
    vch = ch.clone()
    res = O.prove_matmul_layer(r, claim, A, B, ch)
    # each round: p(0) + p(1) = running claim; last: p(r) = final_a * final_b
    cur = claim
    for (c0, c1, c2), rr in zip(res["round_polys"], res["next_point"][pm.bit_length() - 1:]):
        assert Q.qadd(c0, Q.qadd(Q.qadd(c0, c1), c2)) == cur
        cur = Q.qadd(Q.qadd(c0, Q.qmul(c1, rr)), Q.qmul(Q.qmul(c2, rr), rr))
    assert cur == Q.qmul(res["final_a_eval"], res["final_b_eval"])
    # final_a = MLE_A(r_i || challenges), final_b = MLE_B^T(r_j || challenges)
    Ap = np.zeros((pm, pk), dtype=np.uint32)
    Ap[:m, :k] = A
    assert O.evaluate_mle([(int(v), 0, 0, 0) for v in Ap.reshape(-1)], res["next_point"]) == res["final_a_eval"]
    Bp = np.zeros((pk, pn), dtype=np.uint32)
    Bp[:k, :n] = B
    lm = pm.bit_length() - 1
    bpt = r[lm:] + res["next_point"][lm:]
    assert O.evaluate_mle([(int(v), 0, 0, 0) for v in Bp.T.reshape(-1)], bpt) == res["final_b_eval"]
    assert O.verify_matmul_layer(r, claim, m, k, n, res["round_polys"], res["final_a_eval"], res["final_b_eval"],
                                 vch) == 0
    assert vch.digest() == ch.digest()


def test_activation_functions():
    # fixed-point scale 2^16; values above P/2 are negative (lookup_table.rs:192-342)
    assert O.activation(5, 0) == 0
    big = 20 << 16
    assert O.activation(5, big) == big  # silu(20) = 20 / (1 + e^-20) rounds to 20
    assert O.activation(1, 5) == 5 and O.activation(1, P - 5) == 0
    assert O.activation(3, 0) == 1 << 15 and O.activation(3, 7) == 1 << 16 and O.activation(3, P - 1) == 0
    assert O.activation(4, 0) == 1 << 16 and O.activation(4, 3 << 16) == 1 << 19
    assert O.activation(4, P - 1) == 1 << 16  # neg = 0 -> decay 0
    prev = -1
    for x in range(0, 1 << 16, 97):  # silu is increasing on x >= 0
        v = O.activation(5, x)
        assert v >= prev
        prev = v


@pytest.mark.parametrize("rows,cols,tag,tlog", [(1, 8, 5, 8), (4, 16, 5, 10), (3, 5, 1, 6), (2, 32, 4, 8),
                                                (1, 1, 2, 4)])
def test_logup_identities_and_verifier(rows, cols, tag, tlog):
    rng = np.random.default_rng(rows * 7 + cols)
    X = rng.integers(0, P, size=(rows, cols), dtype=np.uint32)
    n = (1 << max(0, (rows - 1).bit_length())) * (1 << max(0, (cols - 1).bit_length()))
    nv = n.bit_length() - 1
    ch = O.Channel()
    ch.mix_u64(5)
    pt = ch.draw_qm31s(nv)
    val = ch.draw_qm31()
    vch = ch.clone()
    if nv == 0:
        # the reference prover handles a single element (no eq rounds) but its
        # verifier rejects a 0-round eq-sumcheck (verifier.rs: "has 0 rounds")
        proof = O.prove_activation_layer(pt, val, X, tag, ch, tlog)
        assert proof["eq_round_polys"] == []
        assert O.verify_activation_layer(pt, val, tag, tlog, proof, vch) != 0
        return
    proof = O.prove_activation_layer(pt, val, X, tag, ch, tlog)
    assert int(proof["multiplicities"].sum()) == n
    assert proof["mult_claimed_sum"] == (n % P, 0, 0, 0)
    # multiplicity final eval = MLE of the multiplicities at the round challenges (checked via chain)
    assert O.verify_activation_layer(pt, val, tag, tlog, proof, vch) == 0
    assert vch.digest() == ch.digest()
    # input_eval is MLE(padded input) at the claim point
    pr, pc = 1 << max(0, (rows - 1).bit_length()), 1 << max(0, (cols - 1).bit_length())
    Xp = np.zeros((pr, pc), dtype=np.uint32)
    Xp[:rows, :cols] = X
    assert O.evaluate_mle([(int(v), 0, 0, 0) for v in Xp.reshape(-1)], pt) == proof["input_eval"]
    assert proof["table_commitment"] == O.hash_many([tag, tlog])
    # tampering with the LogUp sum or a round poly is rejected
    bad = dict(proof)
    bad["claimed_sum"] = Q.qadd(proof["claimed_sum"], (1, 0, 0, 0))
    ch2 = O.Channel()
    ch2.mix_u64(5)
    ch2.draw_qm31s(nv)
    ch2.draw_qm31()
    assert O.verify_activation_layer(pt, val, tag, tlog, bad, ch2) != 0
    bad = dict(proof)
    rp = list(proof["eq_round_polys"])
    rp[0] = (rp[0][0], rp[0][1], Q.qadd(rp[0][2], (1, 0, 0, 0)), rp[0][3])
    bad["eq_round_polys"] = rp
    ch3 = O.Channel()
    ch3.mix_u64(5)
    ch3.draw_qm31s(nv)
    ch3.draw_qm31()
    assert O.verify_activation_layer(pt, val, tag, tlog, bad, ch3) != 0


def _poly3(c, t):
    """c0 + c1 t + c2 t^2 + c3 t^3 over QM31."""
    t2 = Q.qmul(t, t)
    return Q.qadd(Q.qadd(c[0], Q.qmul(c[1], t)), Q.qadd(Q.qmul(c[2], t2), Q.qmul(c[3], Q.qmul(t2, t))))


def test_mul_layer_reference_case_and_bruteforce():
    """The reference's own test case (prover.rs:10629-10680: a = [2..5], b = [1..4], mix_u64(77),
    r = draw_qm31s(2)), checked against brute force: each round polynomial evaluated at 0..3 equals
    the direct sum over the hypercube of eq_t * a_t * b_t; the final evals are MLE_a / MLE_b at the
    replayed challenges; the combiner is drawn after mixing lhs, rhs; the verifier accepts."""
    a = [(v, 0, 0, 0) for v in range(2, 6)]
    b = [(v, 0, 0, 0) for v in range(1, 5)]
    ch = O.Channel()
    ch.mix_u64(77)
    r = ch.draw_qm31s(2)
    c = [Q.qmul(x, y) for x, y in zip(a, b)]
    claim = Q.mle_bruteforce(c, r)
    assert claim == O.evaluate_mle(c, r)
    replay = ch.clone()
    vch = ch.clone()
    proof = O.reduce_mul_layer(r, claim, np.array(a, dtype=np.uint32), np.array(b, dtype=np.uint32), ch)
    assert len(proof["eq_round_polys"]) == 2
    # replay the transcript in Python: tag, claim, per-round deg-3 mix + draw
    replay.mix_u64(0x4D554C)
    replay.mix_secure_field(claim)
    eqv = [Q.eq_weight(r, i, 2) for i in range(4)]
    fa, fb = list(a), list(b)
    s = []
    cur = claim
    for rp in proof["eq_round_polys"]:
        mid = len(fa) // 2
        for t in range(4):
            tq = (t, 0, 0, 0)
            omt = Q.qsub((1, 0, 0, 0), tq)
            brute = (0, 0, 0, 0)
            for i in range(mid):
                lin = lambda v: Q.qadd(Q.qmul(omt, v[i]), Q.qmul(tq, v[mid + i]))  # noqa: E731
                brute = Q.qadd(brute, Q.qmul(Q.qmul(lin(eqv), lin(fa)), lin(fb)))
            assert _poly3(rp, tq) == brute
        assert Q.qadd(_poly3(rp, (0, 0, 0, 0)), _poly3(rp, (1, 0, 0, 0))) == cur
        replay.mix_poly_coeffs_deg3(*rp)
        x = replay.draw_qm31()
        s.append(x)
        cur = _poly3(rp, x)
        fold = lambda v: [Q.qadd(Q.qmul(Q.qsub((1, 0, 0, 0), x), v[i]), Q.qmul(x, v[mid + i]))  # noqa: E731
                          for i in range(mid)]
        eqv, fa, fb = fold(eqv), fold(fa), fold(fb)
    assert proof["lhs_eval"] == Q.mle_bruteforce(a, s)
    assert proof["rhs_eval"] == Q.mle_bruteforce(b, s)
    eq_rs = (1, 0, 0, 0)
    for ri, si in zip(r, s):
        eq_rs = Q.qmul(eq_rs, Q.qadd(Q.qmul(Q.qsub((1, 0, 0, 0), ri), Q.qsub((1, 0, 0, 0), si)), Q.qmul(ri, si)))
    assert cur == Q.qmul(Q.qmul(eq_rs, proof["lhs_eval"]), proof["rhs_eval"])
    replay.mix_secure_field(proof["lhs_eval"])
    replay.mix_secure_field(proof["rhs_eval"])
    alpha = replay.draw_qm31()
    assert proof["alpha"] == alpha
    assert proof["next_value"] == Q.qadd(Q.qmul(alpha, proof["lhs_eval"]),
                                         Q.qmul(Q.qsub((1, 0, 0, 0), alpha), proof["rhs_eval"]))
    assert replay.digest() == ch.digest()
    st, nxt = O.verify_mul_layer(r, claim, proof, vch)
    assert st == 0 and nxt == proof["next_value"] and vch.digest() == ch.digest()


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (8, 8), (7, 33)])
def test_mul_layer_matrices_verifier_and_tamper(rows, cols):
    """Padded-matrix Mul layers (pad_matrix_pow2 + matrix_to_mle) of uniform M31 values: the
    verifier accepts; a longer claim point uses its first log2(n) entries; tampered evals and
    claims are rejected."""
    rng = np.random.default_rng(rows * 131 + cols)
    A = rng.integers(0, P, size=(rows, cols), dtype=np.uint32)
    B = rng.integers(0, P, size=(rows, cols), dtype=np.uint32)
    la, lb = O.padded_mle(A), O.padded_mle(B)
    nv = la.shape[0].bit_length() - 1
    ch = O.Channel()
    ch.mix_u64(rows)
    r = ch.draw_qm31s(nv + 2)  # two extra trailing coordinates, ignored by the eq table
    claim = O.mul_output_claim(A, B, r[:nv])
    vch, tch = ch.clone(), ch.clone()
    proof = O.reduce_mul_layer(r, claim, la, lb, ch)
    assert proof["next_point"] == [tuple(q) for q in r]
    st, nxt = O.verify_mul_layer(r, claim, proof, vch)
    assert st == 0 and nxt == proof["next_value"] and vch.digest() == ch.digest()
    if nv > 0:
        bad = dict(proof)
        bad["lhs_eval"] = Q.qadd(proof["lhs_eval"], (1, 0, 0, 0))
        assert O.verify_mul_layer(r, claim, bad, tch.clone())[0] != 0
        bad_claim = Q.qadd(claim, (0, 0, 1, 0))
        assert O.verify_mul_layer(r, bad_claim, proof, tch.clone())[0] != 0


@pytest.mark.parametrize("n", [1, 2, 16, 64])
def test_sumcheck_product_identities(n):
    """The round loop over QM31 vectors: p_0(0) + p_0(1) = sum f_a f_b, p_t(0) + p_t(1) = p_{t-1}(r),
    the last value equals final_a * final_b, the final evals are the brute-force MLEs at the
    replayed challenges, and the transcript replays in Python."""
    fa, fb = O.synthetic_q(n, 5), O.synthetic_q(n, 6)
    A = [tuple(int(x) for x in row) for row in fa]
    B = [tuple(int(x) for x in row) for row in fb]
    ch = O.Channel()
    ch.mix_u64(n)
    rep = ch.clone()
    res = O.sumcheck_product(fa, fb, ch)
    cur = (0, 0, 0, 0)
    for x, y in zip(A, B):
        cur = Q.qadd(cur, Q.qmul(x, y))
    assert O.inner_product_q(fa, fb) == cur  # the parallel sum the 2^28 GPU test starts from
    for (c0, c1, c2), r in zip(res["round_polys"], res["challenges"]):
        assert Q.qadd(c0, Q.qadd(Q.qadd(c0, c1), c2)) == cur
        rep.mix_poly_coeffs(c0, c1, c2)
        assert rep.draw_qm31() == r
        cur = Q.qadd(Q.qadd(c0, Q.qmul(c1, r)), Q.qmul(c2, Q.qmul(r, r)))
    assert res["final_a_eval"] == Q.mle_bruteforce(A, res["challenges"])
    assert res["final_b_eval"] == Q.mle_bruteforce(B, res["challenges"])
    assert cur == Q.qmul(res["final_a_eval"], res["final_b_eval"])
    assert rep.digest() == ch.digest()


def _tree_root(leaves):
    n = 2
    while n < len(leaves):
        n *= 2
    level = list(leaves) + [0] * (n - len(leaves))
    while len(level) > 1:
        level = [O.hades([level[i], level[i + 1], 2])[0] for i in range(0, len(level), 2)]
    return level[0]


@pytest.mark.parametrize("k,n", [(1, 1), (1, 2), (3, 1), (3, 5), (4, 4), (6, 3)])
def test_weight_commitment_bruteforce(k, n):
    """Merkle root spelled out: leaf (1 << 124) | (v << 93) at index j * pk + i, zero leaves and
    zero MLE padding, node = hades([l, r, 2])[0]."""
    rng = np.random.default_rng(k * 10 + n)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    pk = 1 << max(0, (k - 1).bit_length())
    pn = 1 << max(0, (n - 1).bit_length())
    leaves = [1 << 124] * (pk * pn)
    for i in range(k):
        for j in range(n):
            leaves[j * pk + i] = (1 << 124) | (int(B[i, j]) << 93)
    assert O.weight_commitment(B) == _tree_root(leaves)
    q = rng.integers(0, P, size=(5, 4), dtype=np.uint32)
    packed = [(1 << 124) | (int(a) << 93) | (int(b) << 62) | (int(c) << 31) | int(d) for a, b, c, d in q]
    assert O.mle_commitment(q) == _tree_root(packed)


def test_channel_state_round_trip():
    a = O.Channel()
    a.mix_u64(99)
    a.draw_qm31()
    b = O.Channel()
    O.set_channel_state(b, O.channel_state(a))
    assert b.digest() == a.digest() and O.channel_state(b) == O.channel_state(a)
    assert b.draw_felt252() == a.draw_felt252()
