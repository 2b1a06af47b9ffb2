"""Product sumcheck alone (gkr_sumcheck_product: the reduce_matmul_layer round loop over resident
QM31 vectors; the config-2 workload) against the CPU oracle."""
import sys

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest
import qm31_py as Q

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("logn", [0, 1, 2, 9, 10, 11, 15, 16, 17, 20, 21, 24])
def test_sumcheck_product_parity(gpu_ctx, logn):
    n = 1 << logn
    log(f"case sumcheck_product 2^{logn}")
    fa = gpu_ctx.qvec_synthetic(n, 100 + logn)
    fb = gpu_ctx.qvec_synthetic(n, 200 + logn)
    ha, hb = O.synthetic_q(n, 100 + logn), O.synthetic_q(n, 200 + logn)
    assert np.array_equal(fa.download(), ha) and np.array_equal(fb.download(), hb)
    gch, och = G.PoseidonChannel(), O.Channel()
    gch.mix_u64(logn)
    och.mix_u64(logn)
    got = gpu_ctx.sumcheck_product(fa, fb, gch)
    ref = O.sumcheck_product(ha, hb, och)
    assert got == ref
    assert gch.digest() == och.digest()
    # the caller's vectors are left unchanged, and a second run repeats the proof
    assert np.array_equal(fa.download(), ha) and np.array_equal(fb.download(), hb)
    gch2 = G.PoseidonChannel()
    gch2.mix_u64(logn)
    assert gpu_ctx.sumcheck_product(fa, fb, gch2) == got


def test_sumcheck_product_uploaded_and_errors(gpu_ctx):
    log("case sumcheck_product upload/errors")
    rng = np.random.default_rng(3)
    ha = rng.integers(0, (1 << 31) - 1, size=(4096, 4), dtype=np.uint32)
    hb = rng.integers(0, (1 << 31) - 1, size=(4096, 4), dtype=np.uint32)
    fa, fb = gpu_ctx.qvec_upload(ha), gpu_ctx.qvec_upload(hb)
    assert gpu_ctx.sumcheck_product(fa, fb, G.PoseidonChannel()) == O.sumcheck_product(ha, hb, O.Channel())
    with pytest.raises(G.GkrError, match="not canonical"):
        gpu_ctx.qvec_upload(np.full((2, 4), (1 << 31) - 1, dtype=np.uint32))
    odd = gpu_ctx.qvec_upload(ha[:3])
    with pytest.raises(G.GkrError, match="power of two"):
        gpu_ctx.sumcheck_product(odd, odd, G.PoseidonChannel())
    with pytest.raises(G.GkrError, match="entries"):
        gpu_ctx.sumcheck_product(fa, odd, G.PoseidonChannel())


def test_sumcheck_product_2_26_chain(gpu_ctx):
    """2^26 entries (1 GiB per vector): the verifier's chain p_t(0) + p_t(1) = p_{t-1}(r_t-1) with
    the transcript replayed on the CPU, ending at final_a * final_b."""
    n = 1 << 26
    log("case sumcheck_product 2^26 chain")
    fa, fb = gpu_ctx.qvec_synthetic(n, 7), gpu_ctx.qvec_synthetic(n, 8)
    gch = G.PoseidonChannel()
    gch.mix_u64(26)
    rep = O.Channel()
    rep.mix_u64(26)
    got = gpu_ctx.sumcheck_product(fa, fb, gch)
    cur = None
    for (c0, c1, c2), r in zip(got["round_polys"], got["challenges"]):
        if cur is not None:
            assert Q.qadd(c0, Q.qadd(Q.qadd(c0, c1), c2)) == cur
        rep.mix_poly_coeffs(c0, c1, c2)
        assert rep.draw_qm31() == r
        cur = Q.qadd(Q.qadd(c0, Q.qmul(c1, r)), Q.qmul(c2, Q.qmul(r, r)))
    assert cur == Q.qmul(got["final_a_eval"], got["final_b_eval"])
    assert rep.digest() == gch.digest()


@pytest.mark.parametrize("op,arg", [(G.DEBUG_HANDOVER_CANCEL, 0), (G.DEBUG_HANDOVER_EXPIRE, 4)])
def test_handover_failure_leaves_context_usable(gpu_ctx, op, arg):
    """A hand-over the host cancels before posting its challenges (the error path), or whose
    bounded wait expires before the post, fails the call with a device error while every kernel
    exits normally; the next proofs on the same context are correct (no stale cancel code in the
    mailbox, no timeout code in the shared result flag)."""
    log(f"case handover failure op={op}")
    n = 1 << 12
    fa, fb = gpu_ctx.qvec_synthetic(n, 31), gpu_ctx.qvec_synthetic(n, 32)
    ha, hb = O.synthetic_q(n, 31), O.synthetic_q(n, 32)
    gpu_ctx.debug(op, arg)
    with pytest.raises(G.GkrError) as e:
        gpu_ctx.sumcheck_product(fa, fb, G.PoseidonChannel())
    assert e.value.code == 2
    for rep in range(2):
        assert gpu_ctx.sumcheck_product(fa, fb, G.PoseidonChannel()) == O.sumcheck_product(ha, hb, O.Channel())
    # a matmul layer (restriction, trips, hand-over) on the same context
    A, B = O.synthetic(8, 96, 0, 41), O.synthetic(96, 16, 0, 42)
    a, b = gpu_ctx.upload(A), gpu_ctx.upload(B)
    gch, och = G.PoseidonChannel(), O.Channel()
    r = gch.draw_qm31s(3 + 4)
    assert r == och.draw_qm31s(7)
    v = gpu_ctx.matmul_output_claim(a, b, r)
    assert gpu_ctx.prove_matmul_layer(r, v, a, b, gch) == O.prove_matmul_layer(r, v, A, B, och)
    assert gch.digest() == och.digest()


def test_bounded_wait_wall_clock(gpu_ctx):
    """The wall-clock length of the device-side bounded wait (kWaitSpinLimit = 2^22 polls of the host
    mailbox): hand-overs whose wait is cut to 2^12 and 2^15 polls expire before the host posts, and
    the difference of the two failing calls' times gives the time per poll.  The full limit must
    end well inside the host's own 60 s wait limit (so a waiting kernel always gives up first) and
    last long enough (over 0.5 s) that a host thread descheduled for a moment does not lose the
    proof."""
    import time
    log("case bounded wait wall clock")
    n = 1 << 12
    fa, fb = gpu_ctx.qvec_synthetic(n, 31), gpu_ctx.qvec_synthetic(n, 32)
    times = {}
    for spins in (1 << 12, 1 << 15):
        gpu_ctx.debug(G.DEBUG_HANDOVER_EXPIRE, spins)
        t0 = time.perf_counter()
        with pytest.raises(G.GkrError):
            gpu_ctx.sumcheck_product(fa, fb, G.PoseidonChannel())
        times[spins] = time.perf_counter() - t0
    per_poll = (times[1 << 15] - times[1 << 12]) / ((1 << 15) - (1 << 12))
    full = per_poll * (1 << 22)
    log(f"  {per_poll * 1e9:.0f} ns per poll; 2^22 polls = {full:.2f} s")
    assert 0.5 < full < 30.0
    ha, hb = O.synthetic_q(n, 31), O.synthetic_q(n, 32)
    assert gpu_ctx.sumcheck_product(fa, fb, G.PoseidonChannel()) == O.sumcheck_product(ha, hb, O.Channel())
