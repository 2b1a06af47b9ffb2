"""The oracle's STWO LogUp-GKR / grand-product batch prover (prove_batch,
stwo-gpu/crates/stwo/src/prover/lookups/gkr_prover.rs:396-500) pinned on the CPU:

* the reference's own tests (backend/cpu/lookups/gkr.rs:323-452): the output claims equal the
  fraction sum (or the product) of the whole column, and the artifact's claims equal the input
  columns' multilinear extensions at the OOD point (each instance on the last n_vars coordinates),
  for the grand-product, generic, singles and multiplicities layers, alone and batched;
* every round polynomial of a one-instance proof against brute-force sums over the hypercube of
  eq((r, t, x), y) (num + lambda den)(r, t, x) at t = 0..3, from the input layer's MLE with the
  transcript replayed in Python (mix claims, draw alpha then lambda, mix the coefficients with the
  leading zeros dropped, masks, the layer challenge), including a zero round polynomial mixed as
  an empty slice (an all-zero grand-product column);
* the restated partially_verify_batch accepts and ends on the prover's transcript; changed round
  polynomials, masks, output claims and gates are rejected.
No reference-held vector covers this protocol (its tests run on the Blake2s channel and assert the
properties above); the Poseidon transcript is pinned by the reference's Cairo statement of the
verifier (tests/test_reference_lookup_gkr.py)."""
import numpy as np
import oracle as O
import pytest
import qm31_py as Q

P = (1 << 31) - 1
ONE, ZERO = (1, 0, 0, 0), (0, 0, 0, 0)


def qv(x):
    return (int(x) % P, 0, 0, 0)


def rq(rng, n):
    return rng.integers(0, P, size=(n, 4), dtype=np.uint32)


def tq(a):
    return [tuple(int(v) for v in row) for row in a]


def frac_sum(nums, dens):
    """Fraction sum from zero, left to right, as the reference's tests compute it."""
    n, d = ZERO, ONE
    for a, b in zip(nums, dens):
        n, d = Q.qadd(Q.qmul(n, b), Q.qmul(a, d)), Q.qmul(d, b)
    return n, d


def columns(kind, num, den):
    """(numerator column, denominator column) as QM31 lists; grand product: (column, None)."""
    dq = tq(den)
    if kind == O.LOOKUP_GRAND_PRODUCT:
        return dq, None
    if kind == O.LOOKUP_LOGUP_GENERIC:
        return tq(num), dq
    if kind == O.LOOKUP_LOGUP_MULTIPLICITIES:
        return [qv(x) for x in num], dq
    return [ONE] * len(dq), dq


def make(rng, spec):
    out = []
    for kind, nv in spec:
        n = 1 << nv
        num = rq(rng, n) if kind == O.LOOKUP_LOGUP_GENERIC else (
            rng.integers(0, P, size=n, dtype=np.uint32) if kind == O.LOOKUP_LOGUP_MULTIPLICITIES else None)
        out.append((kind, num, rq(rng, n)))
    return out


SPECS = [[(O.LOOKUP_GRAND_PRODUCT, 5)], [(O.LOOKUP_LOGUP_GENERIC, 5)], [(O.LOOKUP_LOGUP_SINGLES, 5)],
         [(O.LOOKUP_LOGUP_MULTIPLICITIES, 5)], [(O.LOOKUP_LOGUP_GENERIC, 1)], [(O.LOOKUP_GRAND_PRODUCT, 1)],
         [(O.LOOKUP_LOGUP_MULTIPLICITIES, 2)],
         [(O.LOOKUP_LOGUP_GENERIC, 5), (O.LOOKUP_LOGUP_MULTIPLICITIES, 3), (O.LOOKUP_LOGUP_SINGLES, 4),
          (O.LOOKUP_GRAND_PRODUCT, 2)],
         [(O.LOOKUP_LOGUP_MULTIPLICITIES, 4)] * 3 + [(O.LOOKUP_LOGUP_SINGLES, 4)]]


@pytest.mark.parametrize("si", range(len(SPECS)))
def test_lookup_batch_reference_properties(si):
    rng = np.random.default_rng(si)
    inst = make(rng, SPECS[si])
    ch = O.Channel()
    ch.mix_u64(si)
    vch = ch.clone()
    d = O.prove_lookup_batch(ch, inst)
    n_layers = d["n_layers"]
    assert n_layers == max(nv for _, nv in SPECS[si])
    for i, (kind, num, den) in enumerate(inst):
        nc, dc = columns(kind, num, den)
        nv = SPECS[si][i][1]
        pt = d["ood_point"][n_layers - nv:]
        if kind == O.LOOKUP_GRAND_PRODUCT:
            prod = ONE
            for v in nc:
                prod = Q.qmul(prod, v)
            assert d["output_claims"][i] == [prod]
            assert d["claims_to_verify"][i] == [Q.mle_bruteforce(nc, pt)]
        else:
            assert d["output_claims"][i] == list(frac_sum(nc, dc))
            assert d["claims_to_verify"][i] == [Q.mle_bruteforce(nc, pt), Q.mle_bruteforce(dc, pt)]
    st, ood, cv = O.verify_lookup_batch(d, vch)
    assert st == 0 and ood == d["ood_point"] and cv == d["claims_to_verify"]
    assert vch.digest() == ch.digest()


def _fold_point(vals, nv, pt_prefix, t, rest_bits, last):
    """MLE of vals at (prefix, t, rest bits, last) (first variable most significant)."""
    k = nv - len(pt_prefix) - 2
    pt = list(pt_prefix) + [qv(t)] + [qv((rest_bits >> (k - 1 - j)) & 1) for j in range(k)] + [qv(last)]
    return Q.mle_bruteforce(vals, pt)


def stwo_mix(ch, qs):
    """Poseidon252Channel::mix_felts (stwo core/channel/poseidon252.rs:70-84) on a replay channel:
    digest = poseidon_hash_many([digest, packed pairs...]) with n_draws reset.  An empty slice
    still hashes [digest], unlike PoseidonChannel::mix_felts (poseidon_channel.rs:261-264), which
    returns at once; the empty case is spelled out here from hash_many."""
    if qs:
        ch.mix_felts(qs)
        return
    st = O.channel_state(ch)
    d = O.hash_many([ch.digest()])
    hc = (st[9] | (st[10] << 32)) + 1
    O.set_channel_state(ch, [(d >> (32 * i)) & 0xFFFFFFFF for i in range(8)] + [0, hc & 0xFFFFFFFF, hc >> 32])


@pytest.mark.parametrize("kind,zero", [(O.LOOKUP_GRAND_PRODUCT, False), (O.LOOKUP_LOGUP_GENERIC, False),
                                       (O.LOOKUP_LOGUP_SINGLES, False), (O.LOOKUP_LOGUP_MULTIPLICITIES, False),
                                       (O.LOOKUP_GRAND_PRODUCT, True)])
def test_lookup_round_polys_brute_force(kind, zero):
    """One instance of 4 variables: replay the transcript in Python and check every round polynomial
    at t = 0..3 against sum_x eq((c, t, x), y) * (num(c,t,x) + lambda den(c,t,x)) where num/den are
    the fraction sum (or product) of the layer below at (c, t, x, 0) and (c, t, x, 1).  zero: a
    grand product over an all-zero column, so every round polynomial is zero and is mixed as an
    empty slice (the transcript then depends on the empty-slice rule of the STWO channel)."""
    nv = 4
    rng = np.random.default_rng(40 + kind)
    inst = make(rng, [(kind, nv)])
    if zero:
        inst = [(kind, None, np.zeros_like(inst[0][2]))]
    ch = O.Channel()
    rep = ch.clone()
    d = O.prove_lookup_batch(ch, inst)
    nc, dc = columns(kind, inst[0][1], inst[0][2])
    # the circuit's layers, by variables (layer k has k variables)
    layers = {nv: (nc, dc)}
    for k in range(nv - 1, -1, -1):
        a, b = layers[k + 1]
        if kind == O.LOOKUP_GRAND_PRODUCT:
            layers[k] = ([Q.qmul(a[2 * i], a[2 * i + 1]) for i in range(1 << k)], None)
        else:
            layers[k] = ([Q.qadd(Q.qmul(a[2 * i], b[2 * i + 1]), Q.qmul(a[2 * i + 1], b[2 * i])) for i in range(1 << k)],
                         [Q.qmul(b[2 * i], b[2 * i + 1]) for i in range(1 << k)])
    gp = kind == O.LOOKUP_GRAND_PRODUCT
    claims = [layers[0][0][0]] if gp else [layers[0][0][0], layers[0][1][0]]
    assert d["output_claims"][0] == claims
    ood = []
    for layer in range(nv):
        rep.mix_felts(claims)
        rep.draw_qm31()  # alpha (one instance: unused)
        lam = rep.draw_qm31()
        a, b = layers[layer + 1]
        lv = layer + 1
        claim = claims[0] if gp else Q.qadd(claims[0], Q.qmul(lam, claims[1]))
        chal = []
        for r, poly in enumerate(d["round_polys"][layer]):
            pre = chal[:r]
            for t in range(4):
                acc = ZERO
                k = lv - r - 2
                for rest in range(1 << k):
                    xb = pre + [qv(t)] + [qv((rest >> (k - 1 - j)) & 1) for j in range(k)]
                    e = ONE
                    for xv, yv in zip(xb, ood):
                        e = Q.qmul(e, Q.qadd(Q.qmul(xv, yv), Q.qmul(Q.qsub(ONE, xv), Q.qsub(ONE, yv))))
                    if gp:
                        term = Q.qmul(_fold_point(a, lv, pre, t, rest, 0), _fold_point(a, lv, pre, t, rest, 1))
                    else:
                        n0, n1 = _fold_point(a, lv, pre, t, rest, 0), _fold_point(a, lv, pre, t, rest, 1)
                        d0, d1 = _fold_point(b, lv, pre, t, rest, 0), _fold_point(b, lv, pre, t, rest, 1)
                        term = Q.qadd(Q.qadd(Q.qmul(n0, d1), Q.qmul(n1, d0)), Q.qmul(lam, Q.qmul(d0, d1)))
                    acc = Q.qadd(acc, Q.qmul(e, term))
                val = ZERO
                for c in reversed(poly):
                    val = Q.qadd(Q.qmul(val, qv(t)), c)
                assert val == acc, (layer, r, t)
            assert not poly or poly[-1] != ZERO  # leading zeros dropped
            assert not zero or poly == []
            stwo_mix(rep, poly)
            chal.append(rep.draw_qm31())
        mask = d["masks"][layer][0]
        rep.mix_felts(mask)
        c = rep.draw_qm31()
        ood = chal + [c]
        claims = [Q.qadd(mask[2 * k], Q.qmul(c, Q.qsub(mask[2 * k + 1], mask[2 * k]))) for k in range(len(mask) // 2)]
    assert ood == d["ood_point"] and claims == d["claims_to_verify"][0]
    assert rep.digest() == ch.digest()
    if zero:  # the restated verifier takes the same transcript
        vch = O.Channel()
        st, vood, _ = O.verify_lookup_batch(d, vch)
        assert st == 0 and vood == d["ood_point"] and vch.digest() == ch.digest()


def test_lookup_verifier_rejects():
    rng = np.random.default_rng(7)
    inst = make(rng, [(O.LOOKUP_LOGUP_GENERIC, 4), (O.LOOKUP_LOGUP_MULTIPLICITIES, 3), (O.LOOKUP_GRAND_PRODUCT, 2)])
    ch = O.Channel()
    start = ch.clone()
    d = O.prove_lookup_batch(ch, inst)
    assert O.verify_lookup_batch(d, start.clone())[0] == 0
    bad = dict(d, round_polys=[list(p) for p in d["round_polys"]])
    bad["round_polys"][2] = [list(q) for q in bad["round_polys"][2]]
    bad["round_polys"][2][1][0] = Q.qadd(bad["round_polys"][2][1][0], ONE)
    assert O.verify_lookup_batch(bad, start.clone())[0] != 0
    bad = dict(d, masks=[list(m) for m in d["masks"]])
    bad["masks"][3][1] = [Q.qadd(bad["masks"][3][1][0], ONE)] + bad["masks"][3][1][1:]
    assert O.verify_lookup_batch(bad, start.clone())[0] != 0
    bad = dict(d, output_claims=[list(c) for c in d["output_claims"]])
    bad["output_claims"][0][0] = Q.qadd(bad["output_claims"][0][0], ONE)
    assert O.verify_lookup_batch(bad, start.clone())[0] != 0
    bad = dict(d, kinds=[O.LOOKUP_LOGUP_GENERIC] * 3)  # a LogUp gate over a grand-product mask
    assert O.verify_lookup_batch(bad, start.clone())[0] != 0


def test_lookup_refusals():
    """Cases where the reference panics: a 1-variable multiplicities layer (try_into_mask is
    unimplemented for it), an empty batch, a 0-variable instance."""
    rng = np.random.default_rng(3)
    with pytest.raises(ValueError):
        O.prove_lookup_batch(O.Channel(), make(rng, [(O.LOOKUP_LOGUP_MULTIPLICITIES, 1)]))
    with pytest.raises(ValueError):
        O.prove_lookup_batch(O.Channel(), [])
    with pytest.raises(ValueError):
        O.prove_lookup_batch(O.Channel(), [(O.LOOKUP_LOGUP_SINGLES, None, rq(rng, 1))])


def test_lookup_serialization_layout():
    """serialize_stwo_gkr_batch_proof (cairo_serde.rs:3330-3420) on equal-size instances; mixed sizes
    are refused (the reference indexes each instance's masks by the global layer)."""
    rng = np.random.default_rng(9)
    inst = make(rng, [(O.LOOKUP_LOGUP_MULTIPLICITIES, 3), (O.LOOKUP_LOGUP_SINGLES, 3)])
    d = O.prove_lookup_batch(O.Channel(), inst)
    out = []
    O.serialize_lookup_batch(out, d)
    assert out[:3] == [2, 1, 3] and out[3] == 2
    n_head = 1 + 2 * (3 + 2 * 4)
    assert out[n_head] == 3  # layers
    # layer 0: no rounds, two masks of 4 QM31
    assert out[n_head + 1] == 0 and out[n_head + 2] == 2 and out[n_head + 3] == 4
    assert out[n_head + 3 + 1 + 16] == 2
    with pytest.raises(ValueError):
        O.serialize_lookup_batch([], O.prove_lookup_batch(O.Channel(), make(rng, [(1, 3), (1, 2)])))
