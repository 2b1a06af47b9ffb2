"""The allocation-free product sumcheck (gkr_sumcheck_product_noalloc) against the allocating entry
point (gkr_sumcheck_product) on the same vectors: identical round polynomials, challenges, final
evaluations and transcript, on two calls in a row (the second shorter, so the shared static scratch
still holds the first call's contents), plus its size and pointer checks."""
import sys

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_noalloc_matches_allocating_entry_point(gpu_ctx):
    for rep, logn in enumerate([14, 9]):
        n = 1 << logn
        log(f"case noalloc call {rep}: 2^{logn}")
        ha, hb = O.synthetic_q(n, 500 + logn), O.synthetic_q(n, 600 + logn)
        va, vb = gpu_ctx.qvec_upload(ha), gpu_ctx.qvec_upload(hb)
        gch = G.PoseidonChannel()
        gch.mix_u64(logn)
        got = gpu_ctx.sumcheck_product_noalloc(va.device_ptr, vb.device_ptr, n, gch)
        ref_ch = G.PoseidonChannel()
        ref_ch.mix_u64(logn)
        ref = gpu_ctx.sumcheck_product(va, vb, ref_ch)
        assert got == ref
        assert gch.digest() == ref_ch.digest()
        assert got == O.sumcheck_product(ha, hb, _mixed(logn))
        # the caller's vectors are only read
        assert np.array_equal(va.download(), ha) and np.array_equal(vb.download(), hb)


def _mixed(v):
    ch = O.Channel()
    ch.mix_u64(v)
    return ch


def test_noalloc_limits(gpu_ctx):
    log("case noalloc limits")
    n = 1 << 21
    big = gpu_ctx.qvec_synthetic(n, 3)
    with pytest.raises(G.GkrError, match="maximum") as e:
        gpu_ctx.sumcheck_product_noalloc(big.device_ptr, big.device_ptr, n, G.PoseidonChannel())
    assert e.value.code == 1
    with pytest.raises(G.GkrError, match="power of two"):
        gpu_ctx.sumcheck_product_noalloc(big.device_ptr, big.device_ptr, 3, G.PoseidonChannel())
    host = np.zeros((4, 4), dtype=np.uint32)
    with pytest.raises(G.GkrError, match="not device memory"):
        gpu_ctx.sumcheck_product_noalloc(host.ctypes.data, host.ctypes.data, 4, G.PoseidonChannel())
    # the largest allowed length, against the allocating entry point
    m = 1 << 20
    fa, fb = gpu_ctx.qvec_synthetic(m, 5), gpu_ctx.qvec_synthetic(m, 6)
    got = gpu_ctx.sumcheck_product_noalloc(fa.device_ptr, fb.device_ptr, m, G.PoseidonChannel())
    assert got == gpu_ctx.sumcheck_product(fa, fb, G.PoseidonChannel())
    # one entry: no rounds, the values themselves
    one = gpu_ctx.qvec_upload(O.synthetic_q(1, 9))
    r = gpu_ctx.sumcheck_product_noalloc(one.device_ptr, one.device_ptr, 1, G.PoseidonChannel())
    assert r["final_a_eval"] == r["final_b_eval"] == tuple(int(x) for x in O.synthetic_q(1, 9)[0])
