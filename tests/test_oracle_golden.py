"""The CPU oracle against the reference's own golden vectors (no GPU)."""
import hashlib
import random

import numpy as np
import oracle as O

P = (1 << 31) - 1


def test_field_kats(golden):
    f = golden["fields"]
    k = f["qm31_mul"]
    assert O.qmul(k["x"], k["y"]) == tuple(k["xy"])
    assert O.qadd(f["qm31_add"]["x"], f["qm31_add"]["y"]) == tuple(f["qm31_add"]["sum"])
    assert O.qsub(f["qm31_sub"]["x"], f["qm31_sub"]["y"]) == tuple(f["qm31_sub"]["diff"])
    assert O.qsub((0, 0, 0, 0), f["qm31_neg"]["x"]) == tuple(f["qm31_neg"]["neg"])
    # qm0_x_qm1 / qm1 == qm0 (qm31.rs:169)
    assert O.qmul(k["xy"], O.qinv(k["y"])) == tuple(k["x"])
    cm = f["cm31_mul"]
    assert O.qmul(cm["x"] + [0, 0], cm["y"] + [0, 0]) == tuple(cm["xy"] + [0, 0])
    assert O.qmul([0, 1, 0, 0], [0, 1, 0, 0]) == tuple(f["cm31_i_squared"]["xx"] + [0, 0])
    assert O.lib().orc_m31_inv(2) == f["m31_inv2"]["inv"]


def test_hades_constants_match_reference_table(golden):
    g = golden["hades_round_constants"]
    consts = [str(O.hades_constant(i)) for i in range(g["count"])]
    assert consts[0] == g["first"] and consts[-1] == g["last"]
    assert hashlib.sha256(",".join(consts).encode()).hexdigest() == g["sha256_of_decimal_list"]


def test_product_constant_table_matches(golden):
    # the product's generated table (stwo-ml_amd/csrc/hades_constants.inc) holds the same values
    import os
    import re
    path = os.path.join(os.path.dirname(__file__), "..", "stwo-ml_amd", "csrc", "hades_constants.inc")
    limbs = re.findall(r"\{(0x[0-9a-f]+)ull, (0x[0-9a-f]+)ull, (0x[0-9a-f]+)ull, (0x[0-9a-f]+)ull\}", open(path).read())
    vals = [sum(int(l, 16) << (64 * i) for i, l in enumerate(row)) for row in limbs]
    assert len(vals) == golden["hades_round_constants"]["count"]
    digest = hashlib.sha256(",".join(str(v) for v in vals).encode()).hexdigest()
    assert digest == golden["hades_round_constants"]["sha256_of_decimal_list"]


def test_poseidon_kats(golden):
    g = golden["poseidon"]
    ch = O.Channel()
    ch.mix_u64(g["mix_u64"]["value"])
    assert ch.digest() == int(g["mix_u64"]["digest"], 16)
    ch = O.Channel()
    ch.mix_felts([g["mix_felts_qm31_1234"]["value"]])
    assert ch.digest() == int(g["mix_felts_qm31_1234"]["digest"], 16)
    assert O.hash_many([0, int(g["mix_felts_qm31_1234"]["packed"], 16)]) == int(g["mix_felts_qm31_1234"]["digest"], 16)
    # Poseidon252Channel::mix_u32s packs 7 u32 per felt, pads, and injects the
    # length into bits [248:251] of the last felt (poseidon252.rs:82-104, vcs/utils.rs:32-35)
    vals = g["mix_u32s"]["values"]
    pad = 6 - ((len(vals) + 6) % 7)
    data = vals + [0] * pad
    felts = []
    for c in range(0, len(data), 7):
        v = 0
        for y in data[c:c + 7]:
            v = v * 2**32 + y
        felts.append(v)
    if pad:
        felts[-1] += (7 - pad) * 2**248
    assert O.hash_many([0] + felts) == int(g["mix_u32s"]["digest"], 16)


def _sp3_prove():
    ch = O.Channel()
    # GKR seeding without policy commitment: depth 1, input 1x4 (prover.rs:1527-1537)
    for v in (1, 1, 4):
        ch.mix_u64(v)
    r_out = ch.draw_qm31s(1)
    value = O.evaluate_mle([(50, 0, 0, 0), (60, 0, 0, 0)], r_out)
    ch.mix_secure_field(value)
    A = np.array([[1, 2, 3, 4]], dtype=np.uint32)
    B = np.array([[2 * i + j + 1 for j in range(2)] for i in range(4)], dtype=np.uint32)
    assert (O.matmul_forward(A, B) == np.array([[50, 60]])).all()
    assert O.matmul_output_claim(A, B, r_out) == value
    res = O.prove_matmul_layer(r_out, value, A, B, ch)
    return ch, r_out, value, res


def test_sp3_transcript_and_proof(golden):
    sp3 = golden["sp3"]
    ch, r_out, value, res = _sp3_prove()
    cd = [int(x, 16) for x in sp3["calldata_hex"]]
    out = [1]
    O.serialize_matmul_layer(out, res["round_polys"], res["final_a_eval"], res["final_b_eval"])
    assert out == cd[:len(out)]  # num_layers + MatMul layer proof (27 felts)
    # input claim = (r_i || challenges, final_a) (prover.rs:6054-6067)
    assert [list(q) for q in res["next_point"]] == sp3["input_claim_point"]
    tail = []
    O.serialize_tail(tail, res["next_point"], res["next_value"], [int(sp3["weight_commitments"][0], 16)], 0)
    n = len(out)
    assert tail[:-2] == cd[n:n + len(tail) - 2]  # input claim + weight commitment list
    assert ch.digest() == int(sp3["post_walk_digest"], 16)
    # weight claim: B evaluated at (r_j || challenges) equals final_b (prover.rs:2059-2200)
    wc = sp3["weight_claims"][0]
    assert [list(q) for q in wc["eval_point"]] == [list(r_out[0])] + sp3["input_claim_point"]
    assert list(res["final_b_eval"]) == wc["expected_value"]


def test_sp3_verifier_replay(golden):
    sp3 = golden["sp3"]
    cd = [int(x, 16) for x in sp3["calldata_hex"]]
    rp = [((cd[3:7]), None, (cd[7:11])), ((cd[11:15]), None, (cd[15:19]))]
    fa, fb = cd[19:23], cd[23:27]
    ch = O.Channel()
    for v in (1, 1, 4):
        ch.mix_u64(v)
    r_out = ch.draw_qm31s(1)
    value = O.evaluate_mle([(50, 0, 0, 0), (60, 0, 0, 0)], r_out)
    ch.mix_secure_field(value)
    ok = O.verify_matmul_layer(r_out, value, 1, 4, 2, rp, fa, fb, ch)
    assert ok == 0
    assert ch.digest() == int(sp3["post_walk_digest"], 16)


def test_sp3_tamper_rejected(golden):
    """Tampered round polys / final evals fail the final check (test_sp3_cross_language.cairo:222-302)."""
    sp3 = golden["sp3"]
    cd = [int(x, 16) for x in sp3["calldata_hex"]]
    for pos in (3, 7, 11, 19, 23):
        bad = list(cd)
        bad[pos] = (bad[pos] + 1) % P
        rp = [((bad[3:7]), None, (bad[7:11])), ((bad[11:15]), None, (bad[15:19]))]
        ch = O.Channel()
        for v in (1, 1, 4):
            ch.mix_u64(v)
        r_out = ch.draw_qm31s(1)
        value = O.evaluate_mle([(50, 0, 0, 0), (60, 0, 0, 0)], r_out)
        ch.mix_secure_field(value)
        assert O.verify_matmul_layer(r_out, value, 1, 4, 2, rp, bad[19:23], bad[23:27], ch) != 0


def test_synthetic_generator_is_splitmix64():
    # counter mode equals the sequential SplitMix64 stream
    seed = 12345
    state = seed
    mask = (1 << 64) - 1
    for i in range(64):
        state = (state + 0x9E3779B97F4A7C15) & mask
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        z ^= z >> 31
        assert O.synthetic_value(0, seed, i) == (z >> 33)  # P is never hit in this range
        s = (z >> 32) % 255 - 127
        assert O.synthetic_value(1, seed, i) == (s if s >= 0 else P + s)


def test_sp3_weight_commitment(golden):
    """commit_mle_root_only(matrix_to_mle_col_major_padded(W)) for the SP3 weight (4 x 2,
    w[i][j] = 2i + j + 1; engine/tests/artifacts/sp3_matmul_only_proof.json)."""
    B = np.array([[2 * i + j + 1 for j in range(2)] for i in range(4)], dtype=np.uint32)
    assert O.weight_commitment(B) == int(golden["sp3"]["weight_commitments"][0], 16)
    # the row-major layout of the same matrix commits to something else
    assert O.weight_commitment(np.ascontiguousarray(B.T)) != int(golden["sp3"]["weight_commitments"][0], 16)


def test_sp3_weight_opening(golden):
    """The oracle's MLE opening of the SP3 weight at its claim point reproduces the calldata's
    opening section felt for felt and the transcript digest after the openings
    (prove_mle_opening_with_commitment, mle_opening.rs:1654-1915; serialization
    cairo_serde.rs:341-369, 1756-1767)."""
    sp3 = golden["sp3"]
    ch, r_out, value, res = _sp3_prove()
    assert ch.digest() == int(sp3["post_walk_digest"], 16)
    cd = [int(x, 16) for x in sp3["calldata_hex"]]
    W = np.array([[2 * i + j + 1 for j in range(2)] for i in range(4)], dtype=np.uint32)
    wc = sp3["weight_claims"][0]
    point = [tuple(q) for q in wc["eval_point"]]
    cm, felts = O.mle_opening(O.col_major_mle(W), point, ch)
    assert cm == int(sp3["weight_commitments"][0], 16)
    assert ch.digest() == int(sp3["final_channel_digest_after_openings"], 16)
    section = [1, len(point)] + [x for q in point for x in q] + list(wc["expected_value"]) + felts
    start = cd.index(int(sp3["weight_commitments"][0], 16)) + 1
    assert cd[start:] == section + [int(sp3["io_commitment"], 16)]


def test_sp3_io_commitment_is_hash_many_of_twelve(golden):
    """compute_io_commitment (engine/src/aggregation.rs:235-252) hashes rows, cols, len and the data
    of the input, then the same of the output, with poseidon_hash_many: the SP3 fixture's
    io_commitment pins hash_many on 12 inputs (input [[1, 2, 3, 4]], output [[50, 60]])."""
    sp3 = golden["sp3"]
    xs = [1, 4, 4] + sp3["input_data"] + [1, 2, 2] + sp3["output_data"]
    assert xs == [1, 4, 4, 1, 2, 3, 4, 1, 2, 2, 50, 60]
    want = int(sp3["io_commitment"], 16)
    assert O.hash_many(xs) == want
    assert O.hash_many(xs[:-1] + [61]) != want


def test_sp3_opening_verifies_and_tampering_fails(golden):
    """verify_mle_opening (mle_opening.rs:1918-2028) restated in the oracle accepts the
    reference's own SP3 opening (read from its calldata) and rejects changed values,
    siblings, roots, indices and final values."""
    sp3 = golden["sp3"]
    cd = [int(x, 16) for x in sp3["calldata_hex"]]
    ch, _, _, _ = _sp3_prove()
    start = cd.index(int(sp3["weight_commitments"][0], 16)) + 1
    assert cd[start] == 1 and cd[start + 1] == 3
    point = [tuple(cd[start + 2 + 4 * i:start + 6 + 4 * i]) for i in range(3)]
    proof, end = O.parse_mle_opening(cd, start + 2 + 12 + 4)
    assert end == len(cd) - 1
    commitment = int(sp3["weight_commitments"][0], 16)
    assert O.verify_mle_opening(commitment, proof, point, ch.clone())
    import copy

    def tampered(edit):
        b = copy.deepcopy(proof)
        edit(b)
        return b

    def bump_left_value(b):  # query 0, round 1: left value + 1
        idx, rounds = b["queries"][0]
        lv, rv, ls, rs = rounds[1]
        rounds[1] = ((lv[0] + 1,) + tuple(lv[1:]), rv, ls, rs)

    def flip_sibling(b):  # query 2, round 0: a right sibling
        lv, rv, ls, rs = b["queries"][2][1][0]
        rs = list(rs)
        rs[1] ^= 1
        b["queries"][2][1][0] = (lv, rv, ls, rs)

    def flip_root(b):
        b["intermediate_roots"][0] ^= 1

    def flip_index(b):
        b["queries"][3] = (b["queries"][3][0] ^ 1, b["queries"][3][1])

    def change_final(b):
        b["final_value"] = (1, 2, 3, 4)

    for edit in (bump_left_value, flip_sibling, flip_root, flip_index, change_final):
        b = tampered(edit)
        assert not O.verify_mle_opening(commitment, b, point, ch.clone())


def test_oracle_opening_round_trip():
    rng = np.random.default_rng(2)
    for r, c in [(1, 1), (1, 2), (3, 5), (16, 16), (7, 100)]:
        B = rng.integers(0, P, size=(r, c), dtype=np.uint32)
        mle = O.col_major_mle(B)
        nv = (len(mle) - 1).bit_length()
        ch = O.Channel()
        ch.mix_u64(r * 1000 + c)
        point = ch.draw_qm31s(nv)
        start = ch.clone()
        cm, felts = O.mle_opening(mle, point, ch)
        assert cm == O.weight_commitment(B)
        proof, end = O.parse_mle_opening(felts)
        assert end == len(felts)
        assert tuple(proof["final_value"]) == tuple(O.evaluate_mle([tuple(v) for v in mle], point))
        vch = start.clone()
        assert O.verify_mle_opening(cm, proof, point, vch)
        assert vch.digest() == ch.digest()


def test_policy_commitments_of_the_presets(golden):
    """PolicyConfig::policy_commitment (policy.rs:236-254) of the strict / standard / relaxed presets
    equals the values the reference records (deployment script, env-var docs, Cairo contract tests);
    a flipped field, a changed binding mode or a field order swapped gives another value."""
    want = {k: int(v, 16) for k, v in golden["policy"]["commitments"].items()}
    for name, pol in O.POLICY_PRESETS.items():
        assert O.policy_commitment(pol) == want[name], name
    s = dict(O.POLICY_PRESETS["strict"])
    assert O.policy_commitment(dict(s, validate_decode_chain=0)) != want["strict"]
    assert O.policy_commitment(dict(s, weight_binding_mode=2)) != want["strict"]
    swapped = [0x504F4C01] + [int(s[f]) for f in O.POLICY_FIELDS]
    swapped[5], swapped[6] = swapped[6], swapped[5]  # piecewise_activation <-> skip_batch_tokens
    assert O.hash_many(swapped) != want["strict"]
