"""The oracle's aggregated weight binding (prove_aggregated_binding, engine/src/crypto/
aggregated_opening.rs:681-730 and the streaming variant :1647-1720) pinned on the CPU:

* the reference's own tests (:1981-2176): zero-tree roots, the configuration of three claims of
  5, 7 and 3 variables, the unified oracle equal to the dense virtual MLE for equal sizes,
  proofs of 1, 2 and 10 (varying-size) matrices accepted by the restated verifier, a tampered
  claim and a wrong commitment rejected;
* the super root equal to the Merkle root of the virtual MLE (slots of 2^n_max entries, smaller
  matrices zero-extended) computed independently by the oracle's commitment;
* every round polynomial of a small case against the definition: sum over the remaining
  hypercube of R(t) = sum_i beta_i eq(g_i, t) (W(t) - v_i), W the unified oracle, with the
  transcript replayed in Python;
* the serialization layout (config, round polynomials, oracle value, roots, opening).
No reference vector covers this protocol; the transcript is pinned by the reference's Cairo statement
of the verifier (tests/test_reference_binding.py)."""
import numpy as np
import oracle as O
import pytest

P = (1 << 31) - 1
ONE, ZERO = (1, 0, 0, 0), (0, 0, 0, 0)


def rq(rng):
    return tuple(int(x) for x in rng.integers(0, P, size=4))


def mle_claim(rng, nv, honest=True):
    mle = rng.integers(0, P, size=(1 << nv, 4), dtype=np.uint32)
    pt = [rq(rng) for _ in range(nv)]
    v = O.evaluate_mle([tuple(int(x) for x in r) for r in mle], pt)
    if not honest:
        v = O.qadd(v, ONE)
    return {"n_vars": nv, "point": pt, "value": v, "commitment": O.mle_commitment(mle)}, mle


def test_zero_tree_root():
    z = 1 << 124
    h1 = O.poseidon_hash(z, z)
    assert O.compute_zero_tree_root(0) == z
    assert O.compute_zero_tree_root(1) == h1
    assert O.compute_zero_tree_root(2) == O.poseidon_hash(h1, h1)
    assert O.compute_zero_tree_root(3) == O.mle_commitment(np.zeros((8, 4), dtype=np.uint32))


def test_config_from_claims():
    assert O.binding_config([5, 7, 3]) == {"selector_bits": 2, "n_max": 7, "m_padded": 4, "n_global": 9,
                                           "n_claims": 3}
    assert O.binding_config([4]) == {"selector_bits": 0, "n_max": 4, "m_padded": 1, "n_global": 4, "n_claims": 1}


@pytest.mark.parametrize("sizes", [[3, 3], [2, 3, 4], [4, 2, 2, 3], [5]])
def test_super_root_is_virtual_mle_root(sizes):
    rng = np.random.default_rng(sum(sizes))
    cl = [mle_claim(rng, n) for n in sizes]
    claims, mles = [c for c, _ in cl], [m for _, m in cl]
    cfg = O.binding_config(sizes)
    slot = 1 << cfg["n_max"]
    virtual = np.zeros((cfg["m_padded"] * slot, 4), dtype=np.uint32)
    for k, m in enumerate(mles):
        virtual[k * slot:k * slot + len(m)] = m
    assert O.build_super_root(claims, cfg)["root"] == O.mle_commitment(virtual)


def test_sparse_matches_dense():
    """Equal sizes: the unified oracle is the virtual MLE; a smaller matrix is not zero-extended by
    the unified oracle (its leading local coordinates are dropped), so the two differ."""
    rng = np.random.default_rng(4)
    for sizes, equal in (([3, 3], True), ([2, 3], False)):
        cl = [mle_claim(rng, n) for n in sizes]
        mles = [m for _, m in cl]
        cfg = O.binding_config(sizes)
        slot = 1 << cfg["n_max"]
        virtual = np.zeros((cfg["m_padded"] * slot, 4), dtype=np.uint32)
        for k, m in enumerate(mles):
            virtual[k * slot:k * slot + len(m)] = m
        pt = [rq(rng) for _ in range(cfg["n_global"])]
        dense = O.evaluate_mle([tuple(int(x) for x in r) for r in virtual], pt)
        assert (O._unified_oracle(pt, mles, cfg) == dense) == equal


@pytest.mark.parametrize("sizes", [[5], [3, 3], [3, 4, 5, 3, 4, 5, 6, 3, 4, 5]])
def test_reference_flows_verify(sizes):
    rng = np.random.default_rng(len(sizes))
    cl = [mle_claim(rng, n) for n in sizes]
    claims, mles = [c for c, _ in cl], [m for _, m in cl]
    ch = O.Channel()
    ch.mix_u64(42)
    vch = ch.clone()
    p = O.prove_aggregated_binding(claims, mles, ch)
    assert p["opening_commitment"] == p["super_root"]["root"]
    assert O.verify_aggregated_binding(p, claims, vch) and vch.digest() == ch.digest()


def test_tampered_claim_and_wrong_commitment_fail():
    rng = np.random.default_rng(7)
    cl = [mle_claim(rng, 3, honest=False), mle_claim(rng, 3)]
    claims, mles = [c for c, _ in cl], [m for _, m in cl]
    ch = O.Channel()
    ch.mix_u64(42)
    vch = ch.clone()
    p = O.prove_aggregated_binding(claims, mles, ch)
    assert not O.verify_aggregated_binding(p, claims, vch)
    cl = [mle_claim(rng, 3), mle_claim(rng, 3)]
    claims, mles = [c for c, _ in cl], [m for _, m in cl]
    claims[0]["commitment"] = 9999
    ch = O.Channel()
    vch = ch.clone()
    p = O.prove_aggregated_binding(claims, mles, ch)
    assert not O.verify_aggregated_binding(p, claims, vch)


def test_round_polys_against_definition():
    rng = np.random.default_rng(11)
    sizes = [2, 1, 2]
    cl = [mle_claim(rng, n) for n in sizes]
    claims, mles = [c for c, _ in cl], [m for _, m in cl]
    ch = O.Channel()
    rep = ch.clone()
    p = O.prove_aggregated_binding(claims, mles, ch)
    cfg = p["config"]
    n = cfg["n_global"]
    rep.mix_felt(p["super_root"]["root"])
    rho = rep.draw_qm31()
    betas = [ONE]
    for _ in claims[1:]:
        betas.append(O.qmul(betas[-1], rho))
    gps = [O._global_point(i, c["n_vars"], c["point"], cfg) for i, c in enumerate(claims)]

    def R(t):
        w = O._unified_oracle(t, mles, cfg)
        acc = ZERO
        for i, c in enumerate(claims):
            e = ONE
            for a, b in zip(gps[i], t):
                e = O.qmul(e, O._eq1(a, b))
            acc = O.qadd(acc, O.qmul(O.qmul(betas[i], e), O.qsub(w, tuple(c["value"]))))
        return acc
    chal = []
    for j, (c0, c1, c2) in enumerate(p["round_polys"]):
        for x in range(3):
            acc = ZERO
            k = n - j - 1
            for rest in range(1 << k):
                t = chal + [(x, 0, 0, 0)] + [(((rest >> (k - 1 - b)) & 1), 0, 0, 0) for b in range(k)]
                acc = O.qadd(acc, R(t))
            xv = (x, 0, 0, 0)
            assert O.qadd(c0, O.qmul(xv, O.qadd(c1, O.qmul(xv, c2)))) == acc, (j, x)
        rep.mix_poly_coeffs(c0, c1, c2)
        chal.append(rep.draw_qm31())
    assert chal == p["challenges"]
    assert p["oracle_eval"] == O._unified_oracle(chal, mles, cfg)


def test_serialization_layout():
    rng = np.random.default_rng(13)
    cl = [mle_claim(rng, 3), mle_claim(rng, 2)]
    claims, mles = [c for c, _ in cl], [m for _, m in cl]
    p = O.prove_aggregated_binding(claims, mles, O.Channel())
    out = []
    O.serialize_aggregated_binding_proof(out, p)
    assert out[:5] == [1, 3, 2, 4, 2]
    assert out[5] == 4 and len(out) > 6 + 48 + 4 + 1 + 1 + 2
    at = 6 + 48 + 4
    assert out[at] == p["super_root"]["root"] and out[at + 1] == 2
    assert out[at + 4:] == p["opening_felts"]
