"""C ABI of the product library: symbols, host-side channel and tables (no GPU)."""
import os
import random
import re

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
P = (1 << 31) - 1


def header_symbols():
    text = open(os.path.join(ROOT, "include", "gkr_mi355x.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gkr_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = G.lib()
    syms = header_symbols()
    assert len(syms) >= 40
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python binding declares every one of them
    bound = {name for name, _, _ in G.SIGNATURES}
    assert set(syms) <= bound, set(syms) - bound


def test_poseidon_kats_through_abi(golden):
    g = golden["poseidon"]
    ch = G.PoseidonChannel()
    ch.mix_u64(g["mix_u64"]["value"])
    assert ch.digest() == int(g["mix_u64"]["digest"], 16)
    ch = G.PoseidonChannel()
    ch.mix_felts([g["mix_felts_qm31_1234"]["value"]])
    assert ch.digest() == int(g["mix_felts_qm31_1234"]["digest"], 16)


def rq(rng):
    return tuple(rng.randrange(P) for _ in range(4))


def test_channel_matches_oracle_on_random_transcripts():
    rng = random.Random(11)
    for trial in range(20):
        a, b = G.PoseidonChannel(), O.Channel()
        for step in range(25):
            op = rng.randrange(8)
            if op == 0:
                v = rng.getrandbits(64)
                a.mix_u64(v); b.mix_u64(v)
            elif op == 1:
                q = rq(rng)
                a.mix_secure_field(q); b.mix_secure_field(q)
            elif op == 2:
                cs = [rq(rng) for _ in range(3)]
                a.mix_poly_coeffs(*cs); b.mix_poly_coeffs(*cs)
            elif op == 3:
                cs = [rq(rng) for _ in range(4)]
                a.mix_poly_coeffs_deg3(*cs); b.mix_poly_coeffs_deg3(*cs)
            elif op == 4:
                qs = [rq(rng) for _ in range(rng.randrange(0, 6))]
                a.mix_felts(qs); b.mix_felts(qs)
            elif op == 5:
                assert a.draw_qm31() == b.draw_qm31()
            elif op == 6:
                assert a.draw_felt252() == b.draw_felt252()
            else:
                v = rng.randrange(O_P252())
                a.mix_felt(v); b.mix_felt(v)
            assert a.digest() == b.digest()


def O_P252():
    return 2**251 + 17 * 2**192 + 1


def test_channel_state_export_import_and_clone():
    ch = G.PoseidonChannel()
    ch.mix_u64(7)
    ch.draw_qm31()
    st = ch.export_state()
    assert st[8] == 1 and st[9] == 2 and st[10] == 0  # n_draws, hash_count
    other = G.PoseidonChannel()
    other.import_state(st)
    assert other.digest() == ch.digest() and other.draw_qm31() == ch.clone().draw_qm31()
    words = [(ch.digest() >> (32 * i)) & 0xFFFFFFFF for i in range(8)]
    assert st[:8] == words


def test_hash_many_and_permutation_match_oracle():
    rng = random.Random(5)
    for n in range(0, 7):
        xs = [rng.randrange(O_P252()) for _ in range(n)]
        assert G.poseidon_hash_many(xs) == O.hash_many(xs)
    st = [rng.randrange(O_P252()) for _ in range(3)]
    assert G.hades_permute(st) == O.hades(st)
    assert G.poseidon_hash(st[0], st[1]) == O.hades([st[0], st[1], 2])[0]


def test_hash_many_of_twelve_matches_sp3_io_commitment(golden):
    """The product's hash_many on the SP3 io_commitment preimage (compute_io_commitment,
    engine/src/aggregation.rs:235-252): rows, cols, len, data of input then output."""
    sp3 = golden["sp3"]
    xs = [1, 4, 4] + sp3["input_data"] + [1, 2, 2] + sp3["output_data"]
    assert G.poseidon_hash_many(xs) == int(sp3["io_commitment"], 16)


def test_permutation_matches_oracle_on_many_states():
    """The product's permutation (lazy [0, 2p) arithmetic inside) against the oracle's independent
    Montgomery implementation on random states and on edge values (0, 1, p - 1, 2^251, limb
    boundaries)."""
    p = O_P252()
    rng = random.Random(11)
    edges = [0, 1, 2, p - 1, p - 2, 1 << 251, (1 << 251) - 1, (1 << 192) - 1, (1 << 64) - 1, 1 << 128,
             p - (1 << 192), 17 << 192]
    states = [[a, b, c] for a in edges[:4] for b in edges[4:8] for c in edges[8:]]
    states += [[rng.randrange(p) for _ in range(3)] for _ in range(300)]
    for st in states:
        assert G.hades_permute(st) == O.hades(st), st


def test_batched_draws_equal_sequential_draws():
    """draw_qm31s(n) runs its independent permutations in lockstep; it must equal n single draws
    (the oracle draws one at a time) for every remainder modulo the batch width, and leave the
    same channel state."""
    for n in range(0, 11):
        g, o = G.PoseidonChannel(), O.Channel()
        g.mix_u64(n + 1)
        o.mix_u64(n + 1)
        g.draw_qm31()
        o.draw_qm31()
        assert g.draw_qm31s(n) == [o.draw_qm31() for _ in range(n)]
        assert g.draw_qm31() == o.draw_qm31()
        assert g.digest() == o.digest()
        st = g.export_state()
        assert st[8] == n + 2 and (st[9] | (st[10] << 32)) == g.hash_count()


def test_gkr_seeding_with_and_without_policy():
    a, b = G.PoseidonChannel(), O.Channel()
    a.seed_gkr(3, 1, 4)
    for v in (3, 1, 4):
        b.mix_u64(v)
    assert a.digest() == b.digest()
    a.seed_gkr(1, 2, 3, policy_commitment=0)  # zero commitment is skipped
    for v in (1, 2, 3):
        b.mix_u64(v)
    assert a.digest() == b.digest()
    a.seed_gkr(1, 2, 3, policy_commitment=12345)
    for v in (1, 2, 3):
        b.mix_u64(v)
    b.mix_felt(12345)
    assert a.digest() == b.digest()


@pytest.mark.parametrize("tag", [1, 2, 3, 4, 5])
def test_activation_tables_match_oracle(tag):
    t = G.activation_table(tag, 16)
    ref = np.array([O.activation(tag, j) for j in range(0, 1 << 16)], dtype=np.uint32)
    assert (t == ref).all()


def test_synthetic_generator_matches_oracle():
    for kind in (0, 1):
        for seed in (0, 1, 2**63 + 5):
            for i in list(range(100)) + [10**9, 2**40 + 3]:
                assert G.synthetic_value(kind, seed, i) == O.synthetic_value(kind, seed, i)


def test_errors_are_reported():
    ch = G.PoseidonChannel()
    with pytest.raises(G.GkrError) as e:
        ch.mix_secure_field((P, 0, 0, 0))  # not canonical
    assert "canonical" in str(e.value)
    with pytest.raises(G.GkrError):
        ch.mix_felt(O_P252())
    with pytest.raises(G.GkrError):
        G.activation_table(9, 8)


def test_parallel_draw_batches_equal_sequential_draws():
    """draw_qm31s of 4+ values runs on the draw pool's threads; it must equal single draws, also
    with several Python threads drawing at once (one of them takes the pool, the others draw
    alone)."""
    import threading
    rng = random.Random(17)
    for trial in range(300):
        n = rng.choice([4, 5, 8, 19, 20, 64, 257])
        a = G.PoseidonChannel()
        a.mix_u64(trial)
        b = a.clone()
        assert a.draw_qm31s(n) == [b.draw_qm31() for _ in range(n)]
        assert a.export_state() == b.export_state()
    errs = []

    def worker(seed):
        r = random.Random(seed)
        for t in range(100):
            n = r.choice([4, 7, 19, 33])
            a = G.PoseidonChannel()
            a.mix_u64(seed * 1000 + t)
            b = a.clone()
            if a.draw_qm31s(n) != [b.draw_qm31() for _ in range(n)]:
                errs.append((seed, t))
    ts = [threading.Thread(target=worker, args=(s,)) for s in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs


def test_policy_presets_and_commitment(golden):
    """gkr_policy_preset / gkr_policy_commitment: the presets equal the oracle's restatement of
    policy.rs:131-203 and their commitments the reference's recorded values; 60 random policies
    equal the oracle; names are case-insensitive; out-of-range fields and unknown names are
    rejected; seeding with the strict commitment mixes it like the oracle."""
    want = {k: int(v, 16) for k, v in golden["policy"]["commitments"].items()}
    for name in ("strict", "standard", "relaxed"):
        p = G.policy_preset(name)
        assert p == O.POLICY_PRESETS[name]
        assert G.policy_preset(name.upper()) == p
        assert G.policy_commitment(p) == want[name]
    rng = random.Random(3)
    for _ in range(60):
        p = {f: rng.randrange(4 if f == "weight_binding_mode" else 2) for f in G.POLICY_FIELDS}
        assert G.policy_commitment(p) == O.policy_commitment(p)
    with pytest.raises(G.GkrError):
        G.policy_preset("paranoid")
    bad = dict(G.policy_preset("strict"), weight_binding_mode=4)
    with pytest.raises(G.GkrError):
        G.policy_commitment(bad)
    with pytest.raises(G.GkrError):
        G.policy_commitment(dict(G.policy_preset("strict"), io_packing=2))
    a, b = G.PoseidonChannel(), O.Channel()
    a.seed_gkr(48, 64, 5120, policy_commitment=want["strict"])
    for v in (48, 64, 5120):
        b.mix_u64(v)
    b.mix_felt(want["strict"])
    assert a.digest() == b.digest()
