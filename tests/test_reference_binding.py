"""The aggregated weight binding's transcript by the reference's second statement of it: the Cairo
verifier's verify_aggregated_binding (elo-cairo-verifier/src/aggregated_binding.cairo:270-421, with
verify_super_root :98-104, compute_zero_tree_root :111-128, verify_subtree_commitments :214-266,
channel_mix_poly_coeffs channel.cairo:154+), spelled out in Python and run over the oracle's
binding proofs (CPU only).  Step 7, the MLE opening against the super root, is the oracle's
verify_mle_opening, which the reference's SP3 opening pins.

What it pins beyond the restated Rust verifier: the order of the transcript (super root mixed,
rho drawn, n_global degree-2 rounds from sum 0 with (c0, c1, c2) mixed as two packed felts, the
oracle value mixed as a one-element mix_felts, then the opening), the global points (selector bits
most significant first, zero padding, the local point), beta_i = rho^i, and the subtree roots
(a commitment hashed up with zero-tree roots, zero-tree padding slots)."""
import numpy as np
import oracle as O
import pytest

from test_oracle_binding import mle_claim

ONE, ZERO = (1, 0, 0, 0), (0, 0, 0, 0)


def _zero_root(n):
    """compute_zero_tree_root (aggregated_binding.cairo:111-128): leaf pack(0) = 2^124, then one
    hash of a node with itself per level."""
    h = 1 << 124
    if n == 0:
        return h
    h = O.poseidon_hash(h, h)
    for _ in range(1, n):
        h = O.poseidon_hash(h, h)
    return h


def _merkle(leaves):
    cur = list(leaves)
    while len(cur) > 1:
        cur = [O.poseidon_hash(cur[i], cur[i + 1]) for i in range(0, len(cur), 2)]
    return cur[0]


def cairo_verify_aggregated_binding(proof, claims, ch):
    """verify_aggregated_binding (aggregated_binding.cairo:270-421); raises AssertionError with the
    Cairo panic message.  claims: dicts (point, value, commitment) in slot order."""
    cfg = proof["config"]
    subs = proof["super_root"]["subtree_roots"]
    assert _merkle(subs) == proof["super_root"]["root"], "BINDING_SUPER_ROOT_FAILED"
    ok = len(subs) == cfg["m_padded"]
    for i, c in enumerate(claims):  # verify_subtree_commitments (:214-266)
        r = c["commitment"]
        for k in range(len(c["point"]), cfg["n_max"]):
            r = O.poseidon_hash(r, _zero_root(k))
        ok = ok and subs[i] == r
    for i in range(cfg["n_claims"], cfg["m_padded"]):
        ok = ok and subs[i] == _zero_root(cfg["n_max"])
    assert ok, "BINDING_SUBTREE_COMMITMENTS_FAILED"
    ch.mix_felt(proof["super_root"]["root"])
    rho = ch.draw_qm31()
    assert len(proof["round_polys"]) == cfg["n_global"], "BINDING_ROUND_POLY_COUNT_MISMATCH"
    cur, s = ZERO, []
    for c0, c1, c2 in proof["round_polys"]:
        assert O.qadd(c0, O.qadd(c0, O.qadd(c1, c2))) == cur, "BINDING_SUMCHECK_ROUND_FAILED"
        ch.mix_poly_coeffs(c0, c1, c2)
        r = ch.draw_qm31()
        s.append(r)
        cur = O.qadd(c0, O.qmul(r, O.qadd(c1, O.qmul(r, c2))))
    total, rho_pow = ZERO, ONE
    sb = cfg["selector_bits"]
    for i, c in enumerate(claims):
        g = [(((i >> b) & 1), 0, 0, 0) for b in range(sb - 1, -1, -1)]
        g += [ZERO] * (cfg["n_max"] - len(c["point"])) + [tuple(q) for q in c["point"]]
        e = ONE
        for a, b in zip(g, s):
            e = O.qmul(e, O.qadd(O.qmul(a, b), O.qmul(O.qsub(ONE, a), O.qsub(ONE, b))))
        total = O.qadd(total, O.qmul(rho_pow, O.qmul(e, O.qsub(tuple(proof["oracle_eval"]), tuple(c["value"])))))
        rho_pow = O.qmul(rho_pow, rho)
    assert cur == total, "BINDING_FINAL_SUM_MISMATCH"
    ch.mix_felts([tuple(proof["oracle_eval"])])
    assert O.verify_mle_opening(proof["super_root"]["root"], proof["opening"], s, ch), "BINDING_MLE_OPENING_FAILED"
    return True


def _case(sizes, seed, honest=True):
    rng = np.random.default_rng(seed)
    cl = [mle_claim(rng, n) for n in sizes]
    if not honest:
        cl[0] = mle_claim(rng, sizes[0], honest=False)
    claims, mles = [c for c, _ in cl], [m for _, m in cl]
    ch = O.Channel()
    ch.mix_u64(seed)
    start = ch.clone()
    return claims, O.prove_aggregated_binding(claims, mles, ch), start, ch


@pytest.mark.parametrize("sizes", [[4], [3, 3], [3, 5, 4], [3, 4, 5, 3, 4]])
def test_cairo_statement_accepts_oracle_binding(sizes):
    """Accepted, ending on the prover's channel state (the opening's transcript included)."""
    claims, p, start, end = _case(sizes, 10 + len(sizes))
    ch = start.clone()
    assert cairo_verify_aggregated_binding(p, claims, ch)
    assert ch.digest() == end.digest()


def test_cairo_statement_rejections():
    """A claim whose value is off by one (its mismatch sum is not 0: BINDING_SUMCHECK_ROUND_FAILED at
    the first round), a changed round coefficient (BINDING_SUMCHECK_ROUND_FAILED), a wrong commitment
    (BINDING_SUBTREE_COMMITMENTS_FAILED), a changed subtree root (BINDING_SUPER_ROOT_FAILED) and a
    changed oracle value, which the final sum rejects."""
    claims, p, start, _ = _case([3, 4], 5, honest=False)
    with pytest.raises(AssertionError, match="BINDING_SUMCHECK_ROUND_FAILED"):
        cairo_verify_aggregated_binding(p, claims, start.clone())
    claims, p, start, _ = _case([3, 4], 6)
    bad = dict(p, round_polys=list(p["round_polys"]))
    c0, c1, c2 = bad["round_polys"][1]
    bad["round_polys"][1] = (O.qadd(c0, ONE), c1, c2)
    with pytest.raises(AssertionError, match="BINDING_SUMCHECK_ROUND_FAILED"):
        cairo_verify_aggregated_binding(bad, claims, start.clone())
    wrong = [dict(claims[0], commitment=12345)] + claims[1:]
    with pytest.raises(AssertionError, match="BINDING_SUBTREE_COMMITMENTS_FAILED"):
        cairo_verify_aggregated_binding(p, wrong, start.clone())
    sr = dict(p["super_root"], subtree_roots=[p["super_root"]["subtree_roots"][0] + 1] +
              p["super_root"]["subtree_roots"][1:])
    with pytest.raises(AssertionError, match="BINDING_SUPER_ROOT_FAILED"):
        cairo_verify_aggregated_binding(dict(p, super_root=sr), claims, start.clone())
    with pytest.raises(AssertionError, match="BINDING_FINAL_SUM_MISMATCH"):
        cairo_verify_aggregated_binding(dict(p, oracle_eval=O.qadd(tuple(p["oracle_eval"]), ONE)), claims,
                                        start.clone())
