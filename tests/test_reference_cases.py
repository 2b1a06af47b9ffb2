"""Cases the reference itself holds for the LogUp and Mul transcripts and the activation tables,
ported to this build's verifier (the C ABI's host replay), the oracle's verifier and the provers.

* Mul layer: elo-cairo-verifier/tests/test_layer_verifiers.cairo:143-241 — a one-variable Mul
  proof written out by hand: c0..c3 from the eq / lhs / rhs coefficients, the challenge drawn after
  mix_u64(0x4D554C), mix(claim value), mix_poly_coeffs_deg3, and lhs_eval = a0 + (a1 - a0) s.  The
  verifiers must accept it (and reject the case's bad round polynomial), and the provers must
  produce exactly those coefficients and evaluations on the same inputs.
* Activation (LogUp) layer: test_layer_verifiers.cairo:443-580 — a one-variable eq-sumcheck whose
  round polynomial is eq(r0, X) itself (sum 1), with gamma and beta drawn after
  mix_u64(0x4C4F47), mix_u64(type tag), the claimed sum mixed before the round, and
  final_w_eval = 1 / gamma with zero input and output evaluations.  The Cairo verifier checks no
  table side; the reference's Rust verifier (verifier.rs:3058-3290) and this build's do, so the
  port takes all-zero multiplicities (table-side sum 0 = the claimed sum) and the matching
  all-zero multiplicity sumcheck; everything the Cairo case's acceptance depends on is kept.
* The LogUp tail (multiplicity sumcheck and final mixes), which no reference vector covers: the
  Cairo verifier's statement of it (layer_verifiers.cairo:53-95, :282-344, :431-485, parsed per
  model_verifier.cairo:158-215, :298-372) spelled out in Python and run over the oracle's
  serialized proof of a layer with a 4-entry table (two multiplicity rounds): accepted, ending on
  the prover's channel state; a changed c1 rejected; the final mixes' order pinned.
* RMSNorm layer: the Cairo verifier's statement of it (dispatch_rmsnorm, model_verifier.cairo:483-573,
  then verify_rmsnorm_layer, layer_verifiers.cairo:605-680 with verify_linear_eq_sumcheck :358-410,
  verify_logup_eq_sumcheck :282-344 and verify_multiplicity_sumcheck :53-95), replayed over the
  oracle's serialized RMSNorm layer: Part 0 ("RQ", n_active, sum of squares, its rounds, the
  final evaluation), Part 1 ("RN", rms^2 and rsqrt evaluations, the claim value, the linear
  eq-sumcheck, both finals), the rsqrt LogUp ("LOG", "RN", gamma, beta, claimed sum, rounds), the
  multiplicity sumcheck, then input and output evaluations: accepted, ending on the prover's
  channel state; a changed Part-0 or linear round and two swapped Part-1 mixes rejected or parted.
  The reference's Rust serializer writes no multiplicity sumcheck for RMSNorm
  (cairo_serde.rs:1648-1720) while the Cairo dispatcher reads an optional one before the per-row
  statistics; the replay reads the Rust layout and takes the multiplicity rounds from the proof
  record, where that optional field would carry them.
* Activation tables: engine/src/gadgets/lookup_table.rs:466-633 (GELU against its f64 formula
  at 200 points, known values, limits, monotonicity; SiLU(0) and SiLU(1.0))."""
import math

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest
import qm31_py as Q

P = (1 << 31) - 1
ONE, ZERO = (1, 0, 0, 0), (0, 0, 0, 0)


def _q(v):
    return (v % P, 0, 0, 0)


def cairo_mul_case():
    """test_verify_mul_layer_single_var: the hand-built proof and its channel replay."""
    r0 = _q(3)
    a0, a1, b0, b1 = _q(2), _q(5), _q(3), _q(7)
    eq0, eq1 = Q.qsub(ONE, r0), r0
    v = Q.qadd(Q.qmul(eq0, Q.qmul(a0, b0)), Q.qmul(eq1, Q.qmul(a1, b1)))
    eqc0 = Q.qsub(ONE, r0)
    eqc1 = Q.qsub(Q.qadd(r0, r0), ONE)
    da, db = Q.qsub(a1, a0), Q.qsub(b1, b0)
    ea0 = Q.qmul(eqc0, a0)
    ea1 = Q.qadd(Q.qmul(eqc0, da), Q.qmul(eqc1, a0))
    ea2 = Q.qmul(eqc1, da)
    c0 = Q.qmul(ea0, b0)
    c1 = Q.qadd(Q.qmul(ea0, db), Q.qmul(ea1, b0))
    c2 = Q.qadd(Q.qmul(ea1, db), Q.qmul(ea2, b0))
    c3 = Q.qmul(ea2, db)
    assert c0 == Q.qmul(eq0, Q.qmul(a0, b0))
    assert Q.qadd(Q.qadd(Q.qadd(c0, c1), c2), c3) == Q.qmul(eq1, Q.qmul(a1, b1))
    ch = G.PoseidonChannel()  # the prover's Fiat-Shamir, replayed as the case does
    ch.mix_u64(0x4D554C)
    ch.mix_secure_field(v)
    ch.mix_poly_coeffs_deg3(c0, c1, c2, c3)
    s0 = ch.draw_qm31()
    lhs = Q.qadd(a0, Q.qmul(da, s0))
    rhs = Q.qadd(b0, Q.qmul(db, s0))
    return {"point": [r0], "value": v, "poly": (c0, c1, c2, c3), "lhs": lhs, "rhs": rhs,
            "lhs_mle": [a0, a1], "rhs_mle": [b0, b1]}


def test_cairo_mul_case_accepted_by_both_verifiers():
    c = cairo_mul_case()
    proof = {"eq_round_polys": [c["poly"]], "lhs_eval": c["lhs"], "rhs_eval": c["rhs"]}
    G.verify_mul_layer(c["point"], c["value"], proof, G.PoseidonChannel())
    rc, _ = O.verify_mul_layer(c["point"], c["value"], proof, O.Channel())
    assert rc == 0


def test_cairo_mul_case_bad_round_poly_rejected():
    """test_verify_mul_layer_bad_round_poly: c1 is rebuilt from the claim, so the round sum holds,
    and the final check (MUL_FINAL_MISMATCH) fails."""
    v = _q(100)
    bad = {"eq_round_polys": [(_q(10), ZERO, _q(30), _q(40))], "lhs_eval": ZERO, "rhs_eval": ZERO}
    with pytest.raises(G.GkrError) as e:
        G.verify_mul_layer([_q(3)], v, bad, G.PoseidonChannel())
    assert e.value.code == 6
    rc, _ = O.verify_mul_layer([_q(3)], v, bad, O.Channel())
    assert rc != 0


def test_cairo_mul_case_oracle_prover():
    """The oracle's reduce_mul_layer on the case's operands gives the case's coefficients and
    evaluations (the round polynomial is unique; the transcript order fixes s0)."""
    c = cairo_mul_case()
    lhs = np.array(c["lhs_mle"], dtype=np.uint32)
    rhs = np.array(c["rhs_mle"], dtype=np.uint32)
    o = O.reduce_mul_layer(c["point"], c["value"], lhs, rhs, O.Channel())
    assert o["eq_round_polys"] == [c["poly"]]
    assert (o["lhs_eval"], o["rhs_eval"]) == (c["lhs"], c["rhs"])


def cairo_activation_case(tag, table_log, r0=_q(5), poly=None, claimed_sum=ZERO):
    """test_verify_activation_layer_single_var / test_activation_channel_state_changes, with the
    table side made consistent (zero multiplicities: table sum 0 = claimed sum; a zero multiplicity
    sumcheck).  Returns the claim point and the proof dict in prove_activation_layer's layout."""
    sim = G.PoseidonChannel()
    sim.mix_u64(0x4C4F47)
    sim.mix_u64(tag)
    gamma = sim.draw_qm31()
    sim.draw_qm31()  # beta
    if poly is None:  # the eq polynomial of the one variable: (1 - r0) + (2 r0 - 1) X
        poly = (Q.qsub(ONE, r0), Q.qsub(Q.qadd(r0, r0), ONE), ZERO, ZERO)
    sim.mix_secure_field(claimed_sum)
    sim.mix_poly_coeffs_deg3(*poly)
    sim.draw_qm31()
    mult_rounds = [(ZERO, ZERO)] * table_log
    return [r0], {
        "claimed_sum": claimed_sum, "eq_round_polys": [poly],
        "final_evals": (Q.qinv(gamma), ZERO, ZERO),
        "multiplicities": np.zeros(1 << table_log, dtype=np.uint32),
        "mult_round_polys": mult_rounds, "mult_final_eval": ZERO, "mult_claimed_sum": ZERO,
        "input_eval": _q(42), "output_eval": _q(99),
        "table_commitment": O.hash_many([tag, table_log]),
    }


@pytest.mark.parametrize("tag,table_log", [(5, 4), (2, 6), (4, 5)])
def test_cairo_activation_case_accepted(tag, table_log):
    pt, proof = cairo_activation_case(tag, table_log)
    ch = G.PoseidonChannel()
    d0 = ch.digest()
    assert G.verify_activation_layer(pt, tag, table_log, proof, ch) == _q(42)
    assert ch.digest() != d0
    assert O.verify_activation_layer(pt, ZERO, tag, table_log, proof, O.Channel()) == 0


def test_cairo_activation_case_zero_point():
    """test_activation_channel_state_changes: r0 = 0, round polynomial (1, -1, 0, 0)."""
    pt, proof = cairo_activation_case(3, 4, r0=ZERO, poly=(ONE, Q.qsub(ZERO, ONE), ZERO, ZERO))
    assert G.verify_activation_layer(pt, 3, 4, proof, G.PoseidonChannel()) == _q(42)
    assert O.verify_activation_layer(pt, ZERO, 3, 4, proof, O.Channel()) == 0


def test_cairo_activation_case_rejections():
    """test_verify_activation_layer_bad_round_poly (LOGUP_FINAL_MISMATCH), and the case with gamma
    drawn in another order (tag mixed once) or w = 1 / beta: all rejected."""
    pt, proof = cairo_activation_case(5, 4)
    bad = dict(proof)
    bad["eq_round_polys"] = [(_q(10), ZERO, _q(30), _q(40))]
    for p in (bad,):
        with pytest.raises(G.GkrError) as e:
            G.verify_activation_layer(pt, 5, 4, p, G.PoseidonChannel())
        assert e.value.code == 6
        assert O.verify_activation_layer(pt, ZERO, 5, 4, p, O.Channel()) != 0
    # w = 1 / gamma' with gamma' from a transcript that skips the type tag
    sim = G.PoseidonChannel()
    sim.mix_u64(0x4C4F47)
    g_wrong = sim.draw_qm31()
    wrong = dict(proof)
    wrong["final_evals"] = (Q.qinv(g_wrong), ZERO, ZERO)
    with pytest.raises(G.GkrError) as e:
        G.verify_activation_layer(pt, 5, 4, wrong, G.PoseidonChannel())
    assert e.value.code == 6
    assert O.verify_activation_layer(pt, ZERO, 5, 4, wrong, O.Channel()) != 0


# ------------------------------------------------------------------ lookup_table.rs cases
SCALE = 1 << 16


def _tables():
    return {2: G.activation_table(2, 17), 5: G.activation_table(5, 17)}


def test_gelu_matches_f64_reference():
    """lookup_table.rs test_gelu_matches_f64_reference: exact equality at i = 0, 500, ..., 99500
    with the test's own f64 formula (x_real.powi(3) = (x * x) * x)."""
    gelu = _tables()[2]
    k = math.sqrt(2.0 / math.pi)
    for i in range(0, 200 * 500, 500):
        x = i / SCALE
        inner = k * (x + 0.044715 * (x * x * x))
        expected = round(0.5 * x * (1.0 + math.tanh(inner)) * SCALE)
        assert int(gelu[i]) == expected == O.activation(2, i), i


def test_gelu_known_values_and_limits():
    """test_gelu_known_values (1% tolerance), test_gelu_converges_to_identity_for_large_x,
    test_gelu_negative_returns_near_zero, test_gelu_monotonic_positive, GELU vs ReLU at 0.5/1.0."""
    for x, y in [(0.0, 0.0), (0.5, 0.3457), (1.0, 0.8412), (2.0, 1.9545), (3.0, 2.9964)]:
        out = O.activation(2, round(x * SCALE))
        assert abs(out - round(y * SCALE)) <= round(0.01 * SCALE), x
    big = 5 * SCALE
    assert abs(O.activation(2, big) - big) <= SCALE // 100
    assert O.activation(2, P - 5 * SCALE) == 0
    r3 = O.activation(2, P - 3 * SCALE)
    assert r3 == 0 or r3 > P - SCALE
    prev = 0
    for i in range(100):
        out = O.activation(2, i * (SCALE // 10))
        assert out >= prev
        prev = out
    assert O.activation(2, SCALE // 2) < SCALE // 2 and O.activation(2, SCALE) < SCALE


def test_silu_cases():
    """test_silu_zero and test_silu_positive (SiLU(1.0) within 1 of round(2^16 / (1 + e^-1)))."""
    silu = _tables()[5]
    assert int(silu[0]) == 0 == O.activation(5, 0)
    expected = round(1.0 / (1.0 + math.exp(-1.0)) * 65536.0)
    assert abs(int(silu[65536]) - expected) <= 1
    assert O.activation(5, 65536) == int(silu[65536])


# ------------------------------------------------------------------ the LogUp tail, Cairo statement
class _Reader:
    """ProofReader over serialized felts (model_verifier.cairo: read_u32 / read_u64 / read_qm31 /
    read_felt); a QM31 is four felts (a, b, c, d)."""

    def __init__(self, felts, pos=0):
        self.f, self.pos = felts, pos

    def u(self):
        v = int(self.f[self.pos])
        self.pos += 1
        return v

    def q(self):
        return tuple(self.u() for _ in range(4))


def _eq_eval(r, s):
    """eq(r, s) = prod_i (r_i s_i + (1 - r_i)(1 - s_i))."""
    e = ONE
    for a, b in zip(r, s):
        e = Q.qmul(e, Q.qadd(Q.qmul(a, b), Q.qmul(Q.qsub(ONE, a), Q.qsub(ONE, b))))
    return e


def _poly3(c, x):
    return Q.qadd(c[0], Q.qmul(x, Q.qadd(c[1], Q.qmul(x, Q.qadd(c[2], Q.qmul(x, c[3]))))))


def cairo_dispatch_activation(felts, claim_point, ch, swap_final_mix=False):
    """The Cairo verifier's statement of a tag-3 layer, spelled out step by step:
    dispatch_activation's parse (elo-cairo-verifier/src/model_verifier.cairo:298-372, with
    read_optional_logup :158-185 and read_optional_multiplicity_sumcheck :191-215), then
    verify_activation_layer (layer_verifiers.cairo:431-485): mix 0x4C4F47 and the type tag, draw
    gamma and beta, verify_logup_eq_sumcheck (:282-344: mix the claimed sum, degree-3 rounds from
    sum 1 with c1 rebuilt, final eq * w * (gamma - in - beta out)), verify_multiplicity_sumcheck
    (:53-95: per round p(0) + p(1) = sum, mix c0, mix c1, draw, sum = c0 + c1 r; final == sum),
    then mix input_eval and output_eval.  Raises AssertionError with the Cairo panic message.
    swap_final_mix mixes output_eval before input_eval (a transcript the reference does not use).
    Returns (next claim value, felts read)."""
    rd = _Reader(felts)
    assert rd.u() == 3, "tag"
    act_type = rd.u()
    input_eval, output_eval = rd.q(), rd.q()
    rd.u()  # table commitment (checked outside the walk)
    assert rd.u() == 1, "has_logup"
    claimed = rd.q()
    polys = [(rd.q(), rd.q(), rd.q()) for _ in range(rd.u())]  # (c0, c2, c3)
    w_e, in_e, out_e = rd.q(), rd.q(), rd.q()
    for _ in range(rd.u()):
        rd.u()  # multiplicities: consumed, not used
    ms_has = rd.u() == 1
    ms = [(rd.q(), rd.q()) for _ in range(rd.u())] if ms_has else []
    ms_final, ms_claimed = (rd.q(), rd.q()) if ms_has else (ZERO, ZERO)
    assert rd.u() == 0, "has_act_proof"
    assert rd.u() == 0, "has_piecewise"
    ch.mix_u64(0x4C4F47)
    ch.mix_u64(act_type)
    gamma = ch.draw_qm31()
    beta = ch.draw_qm31()
    ch.mix_secure_field(claimed)
    cur, chal = ONE, []
    for c0, c2, c3 in polys:
        c1 = Q.qsub(Q.qsub(Q.qsub(cur, Q.qadd(c0, c0)), c2), c3)
        ch.mix_poly_coeffs_deg3(c0, c1, c2, c3)
        s = ch.draw_qm31()
        chal.append(s)
        cur = _poly3((c0, c1, c2, c3), s)
    d_e = Q.qsub(Q.qsub(gamma, in_e), Q.qmul(beta, out_e))
    assert cur == Q.qmul(_eq_eval(claim_point[:len(polys)], chal), Q.qmul(w_e, d_e)), "LOGUP_FINAL_MISMATCH"
    if ms_has:
        cur = ms_claimed
        for c0, c1 in ms:
            assert Q.qadd(c0, Q.qadd(c0, c1)) == cur, "MULT_SUMCHECK_ROUND_FAIL"
            ch.mix_secure_field(c0)
            ch.mix_secure_field(c1)
            r = ch.draw_qm31()
            cur = Q.qadd(c0, Q.qmul(c1, r))
        assert cur == ms_final, "MULT_SUMCHECK_FINAL_EVAL_MISMATCH"
    first, second = (output_eval, input_eval) if swap_final_mix else (input_eval, output_eval)
    ch.mix_secure_field(first)
    ch.mix_secure_field(second)
    return input_eval, rd.pos


def _activation_tail_case(tag=5, table_log=2, rows=2, cols=4, seed=61):
    """A small activation layer whose multiplicity sumcheck has table_log rounds: the oracle's
    reduce_activation_layer over a rows x cols input with a 2^table_log table, the claim value
    the output MLE at a drawn point.  Returns (point, value, start channel, proof, end channel)."""
    X = O.synthetic(rows, cols, 0, seed)
    out = [[O.activation(tag, int(x) & ((1 << table_log) - 1)) for x in row] for row in X]
    ch = O.Channel()
    ch.mix_u64(seed)
    nv = (rows - 1).bit_length() + (cols - 1).bit_length()
    pt = ch.draw_qm31s(nv)
    val = Q.mle_bruteforce([_q(v) for row in out for v in row], pt)
    start = ch.clone()
    proof = O.prove_activation_layer(pt, val, X, tag, ch, table_log)
    return pt, val, start, proof, ch


def test_logup_tail_cairo_statement_accepts_oracle_proof():
    """The reference's second statement of the LogUp tail (the Cairo verifier: multiplicity
    sumcheck after the eq-sumcheck, c0 and c1 mixed per round, then input_eval and output_eval
    mixed) replayed over the oracle's serialized proof: accepted, ending on the prover's channel
    state; two multiplicity rounds (a 4-entry table) with nonzero multiplicities.  The product's
    walk verifier accepts the same calldata and ends on the same state."""
    pt, val, start, proof, end = _activation_tail_case()
    assert len(proof["mult_round_polys"]) == 2 and int(np.count_nonzero(proof["multiplicities"])) >= 2
    assert proof["output_eval"] == val
    cd = []
    O.serialize_activation_layer(cd, 5, proof)
    ch = start.clone()
    nxt, used = cairo_dispatch_activation(cd, pt, ch)
    assert used == len(cd) and nxt == proof["input_eval"]
    assert ch.digest() == end.digest()
    # the same layer as walk calldata, through the product's verifier
    full = [1] + cd
    O.serialize_tail(full, pt, proof["input_eval"], [], 0)
    gch = G.PoseidonChannel()
    gch.import_state(O.channel_state(start))
    p2, v2, _ = G.verify_walk(full, [(G.STEP_ACTIVATION, 2, 4, 0, 5, 2)], pt, val, gch)
    assert (p2, v2) == (pt, proof["input_eval"]) and gch.digest() == end.digest()


def test_logup_tail_cairo_statement_rejections():
    """A changed c1 of a multiplicity round is rejected by the Cairo statement
    (MULT_SUMCHECK_ROUND_FAIL), by the product's verifier and by the oracle's; a prover that mixed
    output_eval before input_eval ends on another channel state than the Cairo statement's, so the
    final-mix order is pinned (the two evaluations differ here)."""
    pt, val, start, proof, end = _activation_tail_case()
    assert proof["input_eval"] != proof["output_eval"]
    bad = dict(proof)
    c0, c1 = proof["mult_round_polys"][1]
    bad["mult_round_polys"] = [proof["mult_round_polys"][0], (c0, Q.qadd(c1, ONE))]
    cd = []
    O.serialize_activation_layer(cd, 5, bad)
    with pytest.raises(AssertionError, match="MULT_SUMCHECK_ROUND_FAIL"):
        cairo_dispatch_activation(cd, pt, start.clone())
    full = [1] + cd
    O.serialize_tail(full, pt, proof["input_eval"], [], 0)
    gch = G.PoseidonChannel()
    gch.import_state(O.channel_state(start))
    with pytest.raises(G.GkrError) as e:
        G.verify_walk(full, [(G.STEP_ACTIVATION, 2, 4, 0, 5, 2)], pt, val, gch)
    assert e.value.code == 6
    assert O.verify_activation_layer(pt, val, 5, 2, bad, start.clone()) != 0
    good = []
    O.serialize_activation_layer(good, 5, proof)
    swapped = start.clone()
    cairo_dispatch_activation(good, pt, swapped, swap_final_mix=True)
    assert swapped.digest() != end.digest()
    straight = start.clone()
    cairo_dispatch_activation(good, pt, straight)
    assert straight.digest() == end.digest()


# ------------------------------------------------------------------ RMSNorm, Cairo statement
def cairo_rmsnorm(felts, claim_point, claim_value, mult, ch, swap_part1_mix=False):
    """The Cairo verifier's statement of a tag-8 layer, spelled out step by step over the Rust
    layout of LayerProof::RMSNorm (cairo_serde.rs:1648-1720):
    dispatch_rmsnorm (model_verifier.cairo:483-573): Part 0 -- mix_u64(0x5251), mix_u64(n_active),
    mix(sum of squares), per round c1 rebuilt from the running sum, mix_poly_coeffs_deg3, draw,
    sum = p(challenge); then mix(final evaluation);
    verify_rmsnorm_layer (layer_verifiers.cairo:605-680): mix_u64(0x524E), mix(rms_sq_eval),
    mix(rsqrt_eval), mix(claim value); verify_linear_eq_sumcheck (:358-410: rounds from the claim
    value, final == eq(r, s) * input_final * rsqrt_final, LINEAR_FINAL_MISMATCH); mix both finals;
    with a LogUp part: mix_u64(0x4C4F47), mix_u64(0x524E), draw gamma, beta,
    verify_logup_eq_sumcheck (:282-344); verify_multiplicity_sumcheck (:53-95) over `mult`
    ((rounds, final, claimed sum), the multiplicity sumcheck the Rust format does not write);
    mix(input_eval), mix(output_eval).  Returns (next claim value, felts read)."""
    rd = _Reader(felts)
    assert rd.u() == 8, "tag"
    input_eval, output_eval, rms_sq, rsqrt_eval = rd.q(), rd.q(), rd.q(), rd.q()
    rd.u()  # rsqrt table commitment (checked outside the walk)
    assert rd.u() == 0, "simd_combined"
    if rd.u() == 1:  # Part 0b
        n_active = rd.u()
        sq_sum = rd.q()
        rounds = [(rd.q(), rd.q(), rd.q()) for _ in range(rd.u())]
        ch.mix_u64(0x5251)
        ch.mix_u64(n_active)
        ch.mix_secure_field(sq_sum)
        cur = sq_sum
        for c0, c2, c3 in rounds:
            c1 = Q.qsub(Q.qsub(Q.qsub(cur, Q.qadd(c0, c0)), c2), c3)
            ch.mix_poly_coeffs_deg3(c0, c1, c2, c3)
            cur = _poly3((c0, c1, c2, c3), ch.draw_qm31())
        ch.mix_secure_field(rd.q())  # rms_sq_final
    lin = [(rd.q(), rd.q(), rd.q()) for _ in range(rd.u())]
    in_final, rsqrt_final = rd.q(), rd.q()
    has_logup = rd.u() == 1
    if has_logup:
        claimed = rd.q()
        lpolys = [(rd.q(), rd.q(), rd.q()) for _ in range(rd.u())]
        w_e, in_e, out_e = rd.q(), rd.q(), rd.q()
        for _ in range(rd.u()):
            rd.u()  # multiplicities: consumed, not used
    if rd.u() == 1:  # per-row statistics: consumed
        for _ in range(rd.u()):
            rd.u()
    first = [rms_sq, rsqrt_eval] if not swap_part1_mix else [rsqrt_eval, rms_sq]
    ch.mix_u64(0x524E)
    for v in first:
        ch.mix_secure_field(v)
    ch.mix_secure_field(claim_value)
    cur, chal = claim_value, []
    for c0, c2, c3 in lin:
        c1 = Q.qsub(Q.qsub(Q.qsub(cur, Q.qadd(c0, c0)), c2), c3)
        ch.mix_poly_coeffs_deg3(c0, c1, c2, c3)
        x = ch.draw_qm31()
        chal.append(x)
        cur = _poly3((c0, c1, c2, c3), x)
    assert cur == Q.qmul(_eq_eval(claim_point[:len(lin)], chal), Q.qmul(in_final, rsqrt_final)), \
        "LINEAR_FINAL_MISMATCH"
    ch.mix_secure_field(in_final)
    ch.mix_secure_field(rsqrt_final)
    if has_logup:
        ch.mix_u64(0x4C4F47)
        ch.mix_u64(0x524E)
        gamma = ch.draw_qm31()
        beta = ch.draw_qm31()
        ch.mix_secure_field(claimed)
        cur, chal = ONE, []
        for c0, c2, c3 in lpolys:
            c1 = Q.qsub(Q.qsub(Q.qsub(cur, Q.qadd(c0, c0)), c2), c3)
            ch.mix_poly_coeffs_deg3(c0, c1, c2, c3)
            x = ch.draw_qm31()
            chal.append(x)
            cur = _poly3((c0, c1, c2, c3), x)
        d_e = Q.qsub(Q.qsub(gamma, in_e), Q.qmul(beta, out_e))
        assert cur == Q.qmul(_eq_eval(claim_point[:len(lpolys)], chal), Q.qmul(w_e, d_e)), "LOGUP_FINAL_MISMATCH"
    ms_rounds, ms_final, ms_claimed = mult
    cur = ms_claimed
    for c0, c1 in ms_rounds:
        assert Q.qadd(c0, Q.qadd(c0, c1)) == cur, "MULT_SUMCHECK_ROUND_FAIL"
        ch.mix_secure_field(c0)
        ch.mix_secure_field(c1)
        cur = Q.qadd(c0, Q.qmul(c1, ch.draw_qm31()))
    assert cur == ms_final, "MULT_SUMCHECK_FINAL_EVAL_MISMATCH"
    ch.mix_secure_field(input_eval)
    ch.mix_secure_field(output_eval)
    return input_eval, rd.pos


def _rmsnorm_case(rows=2, cols=8, dim=8, seed=71):
    """The oracle's RMSNorm reduction of a rows x cols input, claim = the output MLE at a drawn point.
    Returns (point, value, start channel, proof, end channel, serialized layer)."""
    X = O.synthetic(rows, cols, 1, seed)
    out = O.rmsnorm_forward(X, dim)
    ch = O.Channel()
    ch.mix_u64(seed)
    flat = [_q(int(x)) for x in out.reshape(-1)]
    pt = ch.draw_qm31s((len(flat) - 1).bit_length())
    val = O.evaluate_mle(flat, pt)
    start = ch.clone()
    proof = O.prove_rmsnorm_layer(pt, val, X, dim, ch)
    cd = []
    O.serialize_rmsnorm_layer(cd, proof)
    return pt, val, start, proof, ch, cd


def _mult(proof):
    return proof["mult_round_polys"], proof["mult_final"], proof["mult_sum"]


def test_rmsnorm_cairo_statement_accepts_oracle_proof():
    """The reference's Cairo statement of the RMSNorm layer, replayed over the oracle's serialized
    proof (two padded rows, so the per-row statistics are present), accepts it and ends on the
    prover's channel state; the whole layer is read.  The product's RMSNorm verifier accepts the
    same proof and ends on the same state (its walk verifier refuses RMSNorm calldata, which lacks
    the multiplicity sumcheck)."""
    pt, val, start, proof, end, cd = _rmsnorm_case()
    ch = start.clone()
    nxt, used = cairo_rmsnorm(cd, pt, val, _mult(proof), ch)
    assert used == len(cd) and nxt == proof["input_eval"]
    assert ch.digest() == end.digest()
    gch = G.PoseidonChannel()
    gch.import_state(O.channel_state(start))
    assert G.verify_norm_layer(G.STEP_RMSNORM, pt, val, 8, dict(proof), gch) == proof["input_eval"]
    assert gch.digest() == end.digest()
    full = [1] + cd
    O.serialize_tail(full, pt, proof["input_eval"], [], 0)
    with pytest.raises(G.GkrError, match="multiplicity sumcheck"):
        G.verify_walk(full, [(G.STEP_RMSNORM, 2, 8, 0, 0, 8)], pt, val, G.PoseidonChannel())


def test_rmsnorm_cairo_statement_rejections():
    """A changed c0 of the linear eq-sumcheck's last round fails LINEAR_FINAL_MISMATCH.  A changed
    Part-0 round (Part 0 is replayed, not checked, by the Cairo statement; the Rust verifier checks
    it) changes every later challenge, and so does mixing rsqrt_eval before rms_sq_eval: the
    linear or LogUp eq-sumcheck's final check then fails, so Part 0's transcript and the Part-1
    mix order are pinned."""
    pt, val, start, proof, end, cd = _rmsnorm_case()
    bad = dict(proof)
    lr = list(proof["lin_round_polys"])
    c0, c1, c2, c3 = lr[-1]
    lr[-1] = (Q.qadd(c0, ONE), c1, c2, c3)
    bad["lin_round_polys"] = lr
    bcd = []
    O.serialize_rmsnorm_layer(bcd, bad)
    with pytest.raises(AssertionError, match="LINEAR_FINAL_MISMATCH"):
        cairo_rmsnorm(bcd, pt, val, _mult(proof), start.clone())
    bad0 = dict(proof)
    p0 = list(proof["p0_round_polys"])
    c0, c1, c2, c3 = p0[0]
    p0[0] = (Q.qadd(c0, ONE), c1, c2, c3)
    bad0["p0_round_polys"] = p0
    b0 = []
    O.serialize_rmsnorm_layer(b0, bad0)
    ch = start.clone()
    with pytest.raises(AssertionError):
        cairo_rmsnorm(b0, pt, val, _mult(proof), ch)
    sw = start.clone()
    with pytest.raises(AssertionError):
        cairo_rmsnorm(cd, pt, val, _mult(proof), sw, swap_part1_mix=True)


# ------------------------------------------------------------------ RLC weight binding, verifier statement
def rust_verify_batched_rlc(claims, weights, ch):
    """The Rust verifier's batched RLC weight binding (engine/src/gkr/verifier.rs:1170-1223, no
    deferred proofs): draw rho; combined_expected = sum rho^i expected_i and combined_actual =
    sum rho^i MLE_i(point_i), each weight's MLE the column-major padded matrix
    (evaluate_weight_claim_against_matrix); mix combined_expected; the two must be equal."""
    rho = ch.draw_qm31()
    pw, exp, act = ONE, ZERO, ZERO
    for (point, expected), W in zip(claims, weights):
        mle = [tuple(int(x) for x in v) for v in O.col_major_mle(W)]
        exp = Q.qadd(exp, Q.qmul(pw, expected))
        act = Q.qadd(act, Q.qmul(pw, O.evaluate_mle(mle, point)))
        pw = Q.qmul(pw, rho)
    ch.mix_secure_field(exp)
    assert exp == act, "batched RLC weight-binding mismatch"


def _rlc_walk(seed=11):
    """Three MatMul layers by the oracle (one weight used twice); returns the weight claims (point =
    r_j followed by the reduction's challenges, value = final_b), the weights, the channel before the
    binding and after the prover's RLC binding."""
    rng = np.random.default_rng(seed)
    W1 = rng.integers(0, P, size=(24, 40), dtype=np.uint32)
    W2 = rng.integers(0, P, size=(40, 9), dtype=np.uint32)
    X = rng.integers(0, P, size=(3, 24), dtype=np.uint32)
    H = O.matmul_forward(X, W1)
    ch = O.Channel()
    ch.mix_u64(3)
    claims, weights = [], []
    for a, b in [(H, W2), (X, W1), (X, W1)]:
        lm = (a.shape[0] - 1).bit_length()
        r = ch.draw_qm31s(lm + (b.shape[1] - 1).bit_length())
        v = O.matmul_output_claim(a, b, r)
        ch.mix_secure_field(v)
        o = O.prove_matmul_layer(r, v, a, b, ch)
        claims.append((list(r[lm:]) + list(o["next_point"][lm:]), o["final_b_eval"]))
        weights.append(b)
    before = ch.clone()
    O.rlc_weight_binding([c[1] for c in claims], ch)
    return claims, weights, before, ch


def test_rlc_weight_binding_by_the_rust_verifier_statement():
    """The oracle's RLC binding after three MatMul layers: the Rust verifier's statement accepts the
    claims (every final_b is the weight's MLE at its point), ends on the prover's channel state, and
    rejects a changed claim value."""
    claims, weights, before, after = _rlc_walk()
    ch = before.clone()
    rust_verify_batched_rlc(claims, weights, ch)
    assert ch.digest() == after.digest()
    bad = [claims[0], (claims[1][0], Q.qadd(claims[1][1], ONE)), claims[2]]
    with pytest.raises(AssertionError, match="batched RLC weight-binding mismatch"):
        rust_verify_batched_rlc(bad, weights, before.clone())
