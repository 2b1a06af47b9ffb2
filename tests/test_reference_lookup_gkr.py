"""The STWO LogUp-GKR batch transcript on the Poseidon channel, by the reference's second statement
of it: the Cairo verifier's partially_verify_batch (elo-cairo-verifier/src/gkr.cairo:171-400, with
verify_gkr_sumcheck :97-165, the gates and mask reduction :36-95, random_linear_combination
field.cairo:905-920 and channel_mix_felts channel.cairo:199-227), spelled out in Python and run over
the oracle's batch proofs (CPU only).

The reference's batch prover runs on STWO's Poseidon252Channel (engine/src/aggregation.rs:3930,
4047), whose mix_felts hashes [digest] for an empty slice (poseidon252.rs:70-84), while the Cairo
channel returns at once for it (channel.cairo:200-202).  The two statements therefore agree on every
proof whose mixed slices are all non-empty (a zero round polynomial, whose coefficients are all
dropped, is the only empty slice); the oracle and the product follow the prover's channel, and the
test below shows the two statements parting on an all-zero grand-product column."""
import numpy as np
import oracle as O
import pytest
import qm31_py as Q

from test_oracle_lookup_gkr import make

ONE, ZERO = (1, 0, 0, 0), (0, 0, 0, 0)


def _rlc(values, alpha):
    """random_linear_combination (field.cairo:905-920): Horner from the last value."""
    acc = ZERO
    for v in reversed(values):
        acc = Q.qadd(Q.qmul(acc, alpha), v)
    return acc


def _fold(r, v0, v1):
    return Q.qadd(v0, Q.qmul(r, Q.qsub(v1, v0)))


def _eq(a, b):
    e = ONE
    for x, y in zip(a, b):
        e = Q.qmul(e, Q.qadd(Q.qmul(x, y), Q.qmul(Q.qsub(ONE, x), Q.qsub(ONE, y))))
    return e


def _gate(kind, mask):
    """eval_gate (gkr.cairo:36-73): grand product a * b; LogUp (n_a d_b + n_b d_a, d_a d_b)."""
    if kind == O.LOOKUP_GRAND_PRODUCT:
        assert len(mask) == 2, "GrandProduct mask needs 2 values"
        return [Q.qmul(mask[0], mask[1])]
    assert len(mask) == 4, "LogUp mask needs 4 values"
    n_a, n_b, d_a, d_b = mask
    return [Q.qadd(Q.qmul(n_a, d_b), Q.qmul(n_b, d_a)), Q.qmul(d_a, d_b)]


def _mix_felts_cairo(ch, values):
    """channel_mix_felts (channel.cairo:199-227): nothing for an empty slice."""
    if values:
        ch.mix_felts(values)


def cairo_partially_verify_batch(d, ch, swap_draws=False):
    """partially_verify_batch (gkr.cairo:180-400) on a proof dict of the oracle (instances' kinds,
    n_vars and output claims; per layer the round polynomials, leading zeros dropped, and the
    active instances' masks).  Raises AssertionError with the Cairo panic message.  Returns
    (ood_point, claims_to_verify)."""
    n_inst = len(d["kinds"])
    assert n_inst > 0, "GKR: no instances"
    n_layers = max(d["n_vars"])
    assert len(d["round_polys"]) == n_layers, "GKR: layer count mismatch"
    claims = [None] * n_inst
    ood = []
    for layer in range(n_layers):
        remaining = n_layers - layer
        for i in range(n_inst):  # step 1: instances whose output layer is this one
            if d["n_vars"][i] == remaining:
                claims[i] = list(d["output_claims"][i])
        for i in range(n_inst):  # step 2
            if claims[i] is not None:
                _mix_felts_cairo(ch, claims[i])
        alpha = ch.draw_qm31()  # step 3
        lam = ch.draw_qm31()
        if swap_draws:
            alpha, lam = lam, alpha
        active = [i for i in range(n_inst) if claims[i] is not None]
        sc = [Q.qmul(_rlc(claims[i], lam), (1 << (n_layers - d["n_vars"][i]), 0, 0, 0)) for i in active]  # step 4
        expected = _rlc(sc, alpha)  # step 5
        point = []
        for poly in d["round_polys"][layer]:  # step 6: verify_gkr_sumcheck (:105-165)
            c = list(poly) + [ZERO] * (4 - len(poly))
            assert Q.qadd(c[0], Q.qadd(Q.qadd(c[0], c[1]), Q.qadd(c[2], c[3]))) == expected, \
                "GKR sumcheck round sum mismatch"
            _mix_felts_cairo(ch, list(poly))
            x = ch.draw_qm31()
            point.append(x)
            expected = Q.qadd(c[0], Q.qmul(x, Q.qadd(c[1], Q.qmul(x, Q.qadd(c[2], Q.qmul(x, c[3]))))))
        evals = []
        for i in active:  # step 7
            n_unused = n_layers - d["n_vars"][i]
            mask = d["masks"][layer][i]
            evals.append(Q.qmul(_eq(ood[n_unused:], point[n_unused:]), _rlc(_gate(d["kinds"][i], mask), lam)))
        assert expected == _rlc(evals, alpha), "GKR: circuit check failure"  # step 8
        for i in active:  # step 9
            _mix_felts_cairo(ch, list(d["masks"][layer][i]))
        r = ch.draw_qm31()
        ood = point + [r]  # step 10
        for i in active:  # step 11
            m = d["masks"][layer][i]
            claims[i] = [_fold(r, m[2 * c], m[2 * c + 1]) for c in range(len(m) // 2)]
    return ood, claims


SPECS = [[(O.LOOKUP_LOGUP_GENERIC, 5)], [(O.LOOKUP_GRAND_PRODUCT, 4)], [(O.LOOKUP_LOGUP_SINGLES, 3)],
         [(O.LOOKUP_LOGUP_MULTIPLICITIES, 4)],
         [(O.LOOKUP_LOGUP_GENERIC, 5), (O.LOOKUP_LOGUP_MULTIPLICITIES, 3), (O.LOOKUP_LOGUP_SINGLES, 4),
          (O.LOOKUP_GRAND_PRODUCT, 2)],
         [(O.LOOKUP_LOGUP_MULTIPLICITIES, 4)] * 3 + [(O.LOOKUP_LOGUP_SINGLES, 4)]]


@pytest.mark.parametrize("si", range(len(SPECS)))
def test_cairo_statement_accepts_oracle_batch(si):
    """The Cairo statement accepts the oracle's batch proof (every slice non-empty), reaches the
    same OOD point and claims, and ends on the prover's channel state."""
    rng = np.random.default_rng(40 + si)
    ch = O.Channel()
    ch.mix_u64(si)
    start = ch.clone()
    d = O.prove_lookup_batch(ch, make(rng, SPECS[si]))
    assert all(len(p) > 0 for polys in d["round_polys"] for p in polys)
    vch = start.clone()
    ood, claims = cairo_partially_verify_batch(d, vch)
    assert ood == d["ood_point"] and claims == d["claims_to_verify"]
    assert vch.digest() == ch.digest()


def test_cairo_statement_rejections():
    """A changed round-polynomial coefficient, a changed mask value, a changed output claim and a
    swapped alpha / lambda draw order are each caught by the Cairo statement."""
    rng = np.random.default_rng(77)
    ch = O.Channel()
    start = ch.clone()
    d = O.prove_lookup_batch(ch, make(rng, [(O.LOOKUP_LOGUP_GENERIC, 4), (O.LOOKUP_LOGUP_MULTIPLICITIES, 3),
                                            (O.LOOKUP_GRAND_PRODUCT, 2)]))
    bad = dict(d, round_polys=[[list(p) for p in polys] for polys in d["round_polys"]])
    bad["round_polys"][2][1][0] = Q.qadd(bad["round_polys"][2][1][0], ONE)
    with pytest.raises(AssertionError, match="round sum mismatch"):
        cairo_partially_verify_batch(bad, start.clone())
    bad = dict(d, masks=[[None if m is None else list(m) for m in ms] for ms in d["masks"]])
    bad["masks"][3][1][0] = Q.qadd(bad["masks"][3][1][0], ONE)
    with pytest.raises(AssertionError, match="circuit check failure"):
        cairo_partially_verify_batch(bad, start.clone())
    bad = dict(d, output_claims=[list(c) for c in d["output_claims"]])
    bad["output_claims"][0][0] = Q.qadd(bad["output_claims"][0][0], ONE)
    with pytest.raises(AssertionError):
        cairo_partially_verify_batch(bad, start.clone())
    with pytest.raises(AssertionError):
        cairo_partially_verify_batch(d, start.clone(), swap_draws=True)


def test_statements_part_on_an_empty_slice():
    """An all-zero grand-product column: its round polynomials are zero and mixed as empty slices.
    The prover (STWO's Poseidon252Channel rule: hash [digest]) and the Cairo statement (return at
    once) then draw different challenges, so the Cairo statement rejects the proof; the restated
    STWO verifier (the Rust partially_verify_batch on the prover's channel) accepts it."""
    n = 8
    d_col = np.zeros((n, 4), dtype=np.uint32)
    ch = O.Channel()
    start = ch.clone()
    d = O.prove_lookup_batch(ch, [(O.LOOKUP_GRAND_PRODUCT, None, d_col)])
    assert any(len(p) == 0 for polys in d["round_polys"] for p in polys)
    st, ood, _ = O.verify_lookup_batch(d, start.clone())
    assert st == 0 and ood == d["ood_point"]
    vch = start.clone()
    try:
        ood2, _ = cairo_partially_verify_batch(d, vch)
        parted = ood2 != d["ood_point"] or vch.digest() != ch.digest()
    except AssertionError:
        parted = True
    assert parted
