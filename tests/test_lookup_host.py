"""The library's host side of the STWO LogUp-GKR batch on oracle proofs (no GPU):
gkr_verify_lookup_batch replays partially_verify_batch (gkr_verifier.rs:17-157) to the oracle's
artifact and transcript and rejects changed proofs; gkr_serialize_lookup_batch writes the felts of
serialize_stwo_gkr_batch_proof (cairo_serde.rs:3330-3420) as the oracle's serializer does."""
import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest
import qm31_py as Q

P = (1 << 31) - 1
ONE = (1, 0, 0, 0)


def _inst(rng, spec):
    out = []
    for kind, nv in spec:
        n = 1 << nv
        num = (rng.integers(0, P, size=(n, 4), dtype=np.uint32) if kind == O.LOOKUP_LOGUP_GENERIC else
               rng.integers(0, P, size=n, dtype=np.uint32) if kind == O.LOOKUP_LOGUP_MULTIPLICITIES else None)
        out.append((kind, num, rng.integers(0, P, size=(n, 4), dtype=np.uint32)))
    return out


@pytest.mark.parametrize("spec", [[(0, 4)], [(1, 5), (2, 3), (3, 4), (0, 2)], [(2, 6)] * 3 + [(3, 6)], [(1, 1)]])
def test_library_verifier_on_oracle_proofs(spec):
    rng = np.random.default_rng(len(spec))
    och = O.Channel()
    och.mix_u64(7)
    gch = G.PoseidonChannel()
    gch.mix_u64(7)
    d = O.prove_lookup_batch(och, _inst(rng, spec))
    ood, cv = G.verify_lookup_batch(d, gch)
    assert ood == d["ood_point"] and cv == d["claims_to_verify"] and gch.digest() == och.digest()
    if d["n_layers"] > 1:
        bad = dict(d, round_polys=[[list(p) for p in polys] for polys in d["round_polys"]])
        bad["round_polys"][-1][0][0] = Q.qadd(bad["round_polys"][-1][0][0], ONE)
        with pytest.raises(G.GkrError):
            G.verify_lookup_batch(bad, G.PoseidonChannel())
    bad = dict(d, masks=[list(m) for m in d["masks"]])
    bad["masks"][-1][0] = [Q.qadd(bad["masks"][-1][0][0], ONE)] + bad["masks"][-1][0][1:]
    with pytest.raises(G.GkrError):
        G.verify_lookup_batch(bad, G.PoseidonChannel())


def test_library_serializer():
    rng = np.random.default_rng(5)
    d = O.prove_lookup_batch(O.Channel(), _inst(rng, [(2, 5), (3, 5), (0, 5)]))
    ref = []
    O.serialize_lookup_batch(ref, d)
    assert G.serialize_lookup_batch(d) == ref
    d2 = O.prove_lookup_batch(O.Channel(), _inst(rng, [(1, 4), (1, 3)]))
    with pytest.raises(G.GkrError):
        G.serialize_lookup_batch(d2)
