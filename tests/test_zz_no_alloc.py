"""The allocation-free product sumcheck (gkr_sumcheck_product_noalloc) against the allocating entry
point (gkr_sumcheck_product) on the same vectors: identical round polynomials, challenges, final
evaluations and transcript, on two calls in a row (the second shorter, so the shared static scratch
still holds the first call's contents), plus its size and pointer checks, and two threads on two
contexts of one GPU calling it at once (the calls take turns on the GPU's scratch array)."""
import sys
import threading

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


def test_noalloc_two_threads_take_turns(gpu_ctx):
    """Two threads, each with its own context on the same GPU, call the allocation-free sumcheck
    four times each at the same time on vectors of different lengths; every call equals the
    allocating entry point's result for its vectors (the per-GPU lock keeps them from sharing the
    scratch array at once)."""
    log("case noalloc two threads")
    ctx2 = G.Context(0)
    try:
        jobs = []
        for ctx, logn in ((gpu_ctx, 16), (ctx2, 13)):
            n = 1 << logn
            va, vb = ctx.qvec_synthetic(n, 700 + logn), ctx.qvec_synthetic(n, 800 + logn)
            ch = G.PoseidonChannel()
            ch.mix_u64(logn)
            jobs.append((ctx, va, vb, n, logn, ctx.sumcheck_product(va, vb, ch)))
        results = {0: [], 1: []}
        errors = []

        def run(i):
            ctx, va, vb, n, logn, _ = jobs[i]
            try:
                for _ in range(4):
                    ch = G.PoseidonChannel()
                    ch.mix_u64(logn)
                    results[i].append(ctx.sumcheck_product_noalloc(va.device_ptr, vb.device_ptr, n, ch))
            except Exception as e:  # reported below, in the main thread
                errors.append(e)

        th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join(120)
        assert not any(t.is_alive() for t in th), "a thread did not finish"
        assert not errors, errors
        for i in range(2):
            assert len(results[i]) == 4
            for r in results[i]:
                assert r == jobs[i][5]
    finally:
        ctx2.close()
