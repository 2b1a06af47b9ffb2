"""The BASELINE configurations at their full shapes on the GPU, checked against the CPU oracle
(the reference's CPU algorithm): config 5 (the 48-layer Qwen2.5-14B proof, every layer against the
oracle's proof in tests/golden/config5_oracle.json), config 4 (one Qwen2.5-14B layer, the bench's
workload), config 3 (the 30-layer SmolLM2-135M walk), config 2 at 2^28, and the reference-default
2^20 softmax table on the Qwen score shape.  Inputs come from the bench's own generator (bench.LayerWeights), so these
tests prove exactly what bench.py times."""
import os
import sys
import time

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest
import qm31_py as Q

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def lg(v):
    return max(0, (v - 1).bit_length())


def oracle_layer(och, cfg, layer, out, seed_base=0):
    """bench.oracle_layer: the bench's per-layer sequence on the oracle."""
    bench.oracle_layer(O, och, cfg, layer, out, seed_base)


def gpu_walk(ctx, layers, seed=7):
    """bench.prove_model_walk: one gkr_prove_walk over the layers' steps; returns the serialized proof
    (without the input-claim tail) and the channel."""
    arr, n = bench.model_steps(layers)
    ch = G.PoseidonChannel()
    ch.mix_u64(seed)
    proof = G.Proof()
    G.prove_walk(ctx, ch, arr, proof, n_steps=n)
    return proof, ch


def test_config4_qwen_layer_matches_oracle(gpu_ctx):
    """Config 4: one Qwen2.5-14B layer, 64 tokens (q/o 5120x5120, k/v 5120x1024, gate/up 5120x13824,
    down 13824x5120; SiLU LogUp over 64x13824 -> 2^20 with a 2^16 table; softmax-exp over 2560x64 ->
    2^18).  Every serialized felt (round polynomials, final evaluations, LogUp sums, multiplicities,
    multiplicity rounds, table commitments) and the final digest equal the oracle's."""
    log("case config4 qwen layer")
    layers = [bench.LayerWeights(gpu_ctx, bench.QWEN, 0, 0)]
    proof, gch = gpu_walk(gpu_ctx, layers)
    felts = proof.serialize()
    t0 = time.time()
    och = O.Channel()
    och.mix_u64(7)
    ref = [9]
    oracle_layer(och, bench.QWEN, 0, ref)
    log(f"  oracle layer {time.time() - t0:.1f} s")
    n = len(ref)
    assert felts[:n] == ref
    assert gch.digest() == och.digest()


def test_config3_smollm_30_layers_matches_oracle(gpu_ctx):
    """Config 3: the 30-layer SmolLM2-135M decode walk (1 token; q 576x576, k/v 576x192, o 576x576,
    gate/up 576x1536, down 1536x576; SiLU LogUp over 1x1536 with a 2^16 table): the whole serialized
    proof and the digest equal the oracle's."""
    log("case config3 smollm 30 layers")
    layers = [bench.LayerWeights(gpu_ctx, bench.SMOL, l, 0) for l in range(30)]
    proof, gch = gpu_walk(gpu_ctx, layers)
    felts = proof.serialize()
    och = O.Channel()
    och.mix_u64(7)
    ref = [30 * 8]
    for l in range(30):
        oracle_layer(och, bench.SMOL, l, ref)
    assert felts[:len(ref)] == ref
    assert gch.digest() == och.digest()


def test_config2_product_sumcheck_2_28_chain(gpu_ctx):
    """Config 2 at its largest size: f_a, f_b of 2^28 QM31 each (4 GiB per vector).  The verifier's
    chain with the transcript replayed on the CPU: p_0(0) + p_0(1) = sum_x f_a(x) f_b(x) (the
    oracle's sum over the downloaded vectors), p_t(0) + p_t(1) = p_{t-1}(r_{t-1}), ending at
    final_a * final_b; final_a and final_b equal the oracle's MLEs of the downloaded f_a and f_b at
    the challenges."""
    n = 1 << 28
    log("case config2 2^28 chain")
    fa, fb = gpu_ctx.qvec_synthetic(n, 28), gpu_ctx.qvec_synthetic(n, 29)
    gch = G.PoseidonChannel()
    gch.mix_u64(28)
    rep = O.Channel()
    rep.mix_u64(28)
    got = gpu_ctx.sumcheck_product(fa, fb, gch)
    assert len(got["round_polys"]) == 28
    ha, hb = fa.download(), fb.download()
    del fa, fb
    t0 = time.time()
    cur = O.inner_product_q(ha, hb)
    log(f"  oracle sum {time.time() - t0:.1f} s")
    for (c0, c1, c2), r in zip(got["round_polys"], got["challenges"]):
        assert Q.qadd(c0, Q.qadd(Q.qadd(c0, c1), c2)) == cur
        rep.mix_poly_coeffs(c0, c1, c2)
        assert rep.draw_qm31() == r
        cur = Q.qadd(Q.qadd(c0, Q.qmul(c1, r)), Q.qmul(c2, Q.qmul(r, r)))
    assert cur == Q.qmul(got["final_a_eval"], got["final_b_eval"])
    assert rep.digest() == gch.digest()
    assert tuple(O.evaluate_mle(ha, got["challenges"])) == got["final_a_eval"]
    assert tuple(O.evaluate_mle(hb, got["challenges"])) == got["final_b_eval"]
    log(f"  oracle sum and MLEs {time.time() - t0:.1f} s")


def test_softmax_reference_table_qwen_scores(gpu_ctx):
    """The reference-default softmax-exp table (2^20 entries, table_log_size 0) over the Qwen score
    tensor 2560x64 (2^18 inputs): 20 multiplicity rounds, the 2^20 table commitment, bit-exact."""
    log("case softmax 2^20 table")
    X = O.synthetic(2560, 64, 0, 4)
    x = gpu_ctx.upload(X)
    gch, och = G.PoseidonChannel(), O.Channel()
    pt = gch.draw_qm31s(18)
    val = gch.draw_qm31()
    assert pt == och.draw_qm31s(18) and val == och.draw_qm31()
    gp = G.Proof()
    pg = gpu_ctx.prove_activation_layer(pt, val, x, 4, gch, 0, gp)
    po = O.prove_activation_layer(pt, val, X, 4, och, 0)
    assert len(po["mult_round_polys"]) == 20
    for key in ("claimed_sum", "eq_round_polys", "final_evals", "mult_round_polys", "mult_final_eval",
                "mult_claimed_sum", "input_eval", "output_eval", "table_commitment"):
        assert pg[key] == po[key], key
    assert (pg["multiplicities"] == po["multiplicities"]).all()
    assert gch.digest() == och.digest()


def layer_shapes(cfg):
    """The circuit of one bench layer for gkr_verify_walk (fresh claims, bench.model_steps order)."""
    h, i, q, kv, m = cfg["hidden"], cfg["inter"], cfg["q"], cfg["kv"], cfg["tokens"]
    F, MM, ACT = G.CLAIM_FRESH, G.STEP_MATMUL, G.STEP_ACTIVATION
    out = [(MM, m, h, q, 0, 0, F), (MM, m, h, kv, 0, 0, F), (MM, m, h, kv, 0, 0, F), (MM, m, q, h, 0, 0, F),
           (MM, m, h, i, 0, 0, F), (MM, m, h, i, 0, 0, F), (ACT, m, i, 0, 5, 16, F), (MM, m, i, h, 0, 0, F)]
    if m > 1:
        out.append((ACT, cfg["heads"] * m, m, 0, 4, 16, F))
    return out


def test_config5_qwen_48_layers(gpu_ctx):
    """Config 5: the bench's 48-layer Qwen2.5-14B proof (52.9 GB of weights resident) against the CPU
    oracle's proof of the same inputs (tests/golden/config5_oracle.json, written by
    tests/golden/make_config5_fixture.py): every layer's serialized felts (SHA-256 of their words) and
    the channel state after every layer equal the oracle's, and so does the whole proof's SHA-256.
    Layer 23 is also proved again by the oracle on the box from the exported channel state.  The
    whole proof is replayed by the host verifier with the fresh-claim rule, and a changed felt in
    layer 30 is rejected."""
    import hashlib
    import json
    log("case config5 48 layers")
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config5_oracle.json")) as f:
        ref = json.load(f)
    assert ref["n_layers"] == 48 and ref["seed"] == 7
    layers = [bench.LayerWeights(gpu_ctx, bench.QWEN, l, 0) for l in range(48)]
    live = 23
    ch = G.PoseidonChannel()
    ch.mix_u64(7)
    proof = G.Proof()
    states = {}
    for l, L in enumerate(layers):
        if l == live:
            states[l] = ch.export_state()
        arr, n = bench.model_steps([L])
        fp, fv = G.prove_walk(gpu_ctx, ch, arr, proof, n_steps=n)
        states[l + 1] = ch.export_state()
    words = proof.serialize_words()
    assert len(words) == ref["n_felts"]
    # layer count, then 48 equal layers, then the tail: input claim (no point: 1 + 4 felts), commitment
    # count, opening count, IO commitment
    per, rem = divmod(len(words) - 1 - 8, 48)
    assert rem == 0
    for l in range(48):
        want = ref["layers"][l]
        assert per == want["felts"], f"layer {l} length"
        got = hashlib.sha256(words[1 + l * per:1 + (l + 1) * per].tobytes()).hexdigest()
        assert got == want["sha256"], f"layer {l} differs from the oracle's"
        assert list(states[l + 1]) == want["state_after"], f"channel after layer {l}"
    assert hashlib.sha256(words.tobytes()).hexdigest() == ref["proof_sha256"]
    assert list(states[48]) == ref["final_state"]
    log("  48 layers equal the oracle fixture")
    t0 = time.time()
    och = O.Channel()
    O.set_channel_state(och, states[live])
    out = []
    oracle_layer(och, bench.QWEN, live, out)
    log(f"  oracle layer {live}: {time.time() - t0:.1f} s")
    assert np.array_equal(words[1 + live * per:1 + (live + 1) * per], G.felts_to_words(out))
    assert O.channel_state(och) == list(states[live + 1])
    # host replay of the whole proof
    proof.set_input_claim(fp, fv)
    full = proof.serialize_words()
    shapes = layer_shapes(bench.QWEN) * 48
    fresh = [proof.layer_claim_value(i) for i, s in enumerate(shapes) if s[0] == G.STEP_MATMUL]
    vch = G.PoseidonChannel()
    vch.mix_u64(7)
    t0 = time.time()
    pt, val, used = G.verify_walk(full, shapes, None, None, vch, fresh)
    log(f"  host verifier: {time.time() - t0:.1f} s")
    assert (pt, val) == (fp, fv) and vch.digest() == ch.digest()
    bad = full.copy()
    pos = 1 + 30 * per + 5  # a round-polynomial word of layer 30's q matmul
    bad[pos, 0] ^= 1
    v2 = G.PoseidonChannel()
    v2.mix_u64(7)
    with pytest.raises(G.GkrError) as e:
        G.verify_walk(bad, shapes, None, None, v2, fresh)
    assert e.value.code == 6
