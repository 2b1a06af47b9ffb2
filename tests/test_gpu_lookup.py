"""STWO LogUp-GKR / grand-product batch (prove_batch, stwo-gpu/crates/stwo/src/prover/lookups/
gkr_prover.rs:396-500) on the HIP path against the CPU oracle: output claims, every round
polynomial and its coefficient count, masks, OOD point, artifact claims and the channel digest
bit-exact, for the four layer kinds alone and batched with mixed sizes, up to a 2^20 table; the
library verifier accepts the GPU proofs; serialization equals the oracle's."""
import sys

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

pytestmark = pytest.mark.gpu
P = (1 << 31) - 1


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _make(rng, spec, mult_range=P):
    out = []
    for kind, nv in spec:
        n = 1 << nv
        num = (rng.integers(0, P, size=(n, 4), dtype=np.uint32) if kind == O.LOOKUP_LOGUP_GENERIC else
               rng.integers(0, mult_range, size=n, dtype=np.uint32) if kind == O.LOOKUP_LOGUP_MULTIPLICITIES else None)
        out.append((kind, num, rng.integers(0, P, size=(n, 4), dtype=np.uint32)))
    return out


def _upload(ctx, inst):
    dev, keep = [], []
    for kind, num, den in inst:
        nv = (len(den) - 1).bit_length()
        d = ctx.qvec_upload(den)
        n = None
        if kind == O.LOOKUP_LOGUP_GENERIC:
            n = ctx.qvec_upload(num)
        elif kind == O.LOOKUP_LOGUP_MULTIPLICITIES:
            n = ctx.upload(np.asarray(num, dtype=np.uint32).reshape(1, -1))
        keep += [d, n]
        dev.append((kind, nv, n, d))
    return dev, keep


def _check(ctx, inst, seed):
    dev, keep = _upload(ctx, inst)
    gch, och = G.PoseidonChannel(), O.Channel()
    gch.mix_u64(seed)
    och.mix_u64(seed)
    vch = gch.clone()
    got = G.prove_lookup_batch(ctx, gch, dev)
    ref = O.prove_lookup_batch(och, inst)
    for key in ("n_layers", "output_claims", "ood_point", "claims_to_verify"):
        assert got[key] == ref[key], key
    for layer in range(ref["n_layers"]):
        assert got["round_polys"][layer] == ref["round_polys"][layer], ("round_polys", layer)
        assert got["masks"][layer] == ref["masks"][layer], ("masks", layer)
    assert got == ref
    assert gch.digest() == och.digest()
    ood, cv = G.verify_lookup_batch(got, vch)
    assert ood == got["ood_point"] and cv == got["claims_to_verify"] and vch.digest() == gch.digest()
    return got


def test_lookup_zero_grand_product(gpu_ctx):
    """A grand product over an all-zero column beside a LogUp instance: every round polynomial of
    the grand product is zero, so the batch polynomial of the layers before the smaller LogUp
    instance joins is mixed as an empty slice, which STWO's Poseidon252 channel still hashes."""
    log("case lookup zero grand product")
    rng = np.random.default_rng(77)
    inst = [(0, None, np.zeros((1 << 6, 4), dtype=np.uint32))]
    _check(gpu_ctx, inst, 77)
    inst = _make(rng, [(1, 3)]) + inst
    _check(gpu_ctx, inst, 78)


SPECS = [[(0, 1)], [(1, 1)], [(3, 1)], [(2, 2)], [(0, 5)], [(1, 5)], [(2, 5)], [(3, 5)],
         [(1, 5), (2, 3), (3, 4), (0, 2)], [(2, 12)], [(3, 13), (0, 13)], [(1, 14), (2, 9), (3, 1)],
         [(2, 16)] * 6 + [(3, 16), (0, 10)]]


@pytest.mark.parametrize("si", range(len(SPECS)))
def test_lookup_batch_matches_oracle(gpu_ctx, si):
    log(f"case lookup batch {SPECS[si]}")
    _check(gpu_ctx, _make(np.random.default_rng(100 + si), SPECS[si]), si)


def test_lookup_batch_table_2_20(gpu_ctx):
    """One 2^20-entry table (the reference-default softmax table size) with small multiplicities as
    prove_logup_gkr builds them (numerators: counts, denominators alpha - table value), next to a
    2^16 activation table."""
    log("case lookup batch 2^20 table")
    rng = np.random.default_rng(20)
    alpha = tuple(int(x) for x in rng.integers(0, P, size=4))
    inst = []
    for nv in (20, 16):
        n = 1 << nv
        mult = rng.integers(0, 4, size=n, dtype=np.uint32)
        table = rng.integers(0, P, size=n, dtype=np.uint64)
        den = np.zeros((n, 4), dtype=np.uint32)
        den[:, 0] = (alpha[0] + P - table) % P
        den[:, 1:] = alpha[1:]
        inst.append((O.LOOKUP_LOGUP_MULTIPLICITIES, mult, den))
    got = _check(gpu_ctx, inst, 99)
    assert got["n_layers"] == 20 and sum(len(p) for p in got["round_polys"]) == 190


def test_lookup_batch_serialization(gpu_ctx):
    log("case lookup batch serialization")
    inst = _make(np.random.default_rng(3), [(2, 8), (3, 8), (0, 8), (1, 8)])
    got = _check(gpu_ctx, inst, 3)
    ref = []
    O.serialize_lookup_batch(ref, got)
    assert G.serialize_lookup_batch(got) == ref


def test_lookup_batch_errors(gpu_ctx):
    log("case lookup batch errors")
    d = gpu_ctx.qvec_upload(np.ones((4, 4), dtype=np.uint32))
    m = gpu_ctx.upload(np.ones((1, 2), dtype=np.uint32))
    ch = G.PoseidonChannel()
    for bad in ([(7, 2, None, d)], [(1, 0, d, d)], [(2, 1, m, d)], [(1, 2, None, d)], [(0, 2, None, None)], []):
        with pytest.raises(G.GkrError):
            G.prove_lookup_batch(gpu_ctx, ch, bad)
