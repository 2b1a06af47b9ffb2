"""Serialization while proving (gkr_proof_stream_to): a thread of the proof writes each layer record
into the caller's buffer as the reducers append it, and gkr_proof_serialize with that buffer writes
only the layer count and the tail.  The bytes must equal those of serializing the finished proof
(serialize_gkr_model_proof's layout, which the other tests pin against the reference's SP3 calldata
and the oracle), whatever the buffer, its size, or a walk step proved again."""
import sys

import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _tail_only_proof():
    p = G.Proof()
    p.set_input_claim([(1, 2, 3, 4), (5, 6, 7, 8)], (9, 10, 11, 12))
    p.add_weight_commitment(0x1234)
    p.set_io_commitment(0xABCDEF)
    return p


def test_stream_without_layers():
    """No GPU: a proof without layers streamed into a buffer serializes (count and tail) to the same
    words as without streaming; a short buffer is reported with the full length; None ends it."""
    ref = _tail_only_proof().serialize_words()
    p = _tail_only_proof()
    buf = np.zeros((64, 8), dtype=np.uint32)
    p.stream_to(buf)
    n = p.serialize_into(buf)
    assert n == len(ref) and (buf[:n] == ref).all()
    short = np.zeros((3, 8), dtype=np.uint32)
    p.stream_to(short)
    with pytest.raises(G.GkrError) as e:
        p.serialize_into(short)
    assert e.value.code == 5
    p.stream_to(None)
    assert (p.serialize_words() == ref).all()


MATS = [O.synthetic(4, 4096, 1, 81), O.synthetic(4096, 16, 1, 82), O.synthetic(64, 1024, 0, 83),
        O.synthetic(8, 2048, 1, 84), O.synthetic(2048, 64, 1, 85)]


def _walk(ctx, proof):
    gs = [ctx.upload(M) for M in MATS]
    F = G.CLAIM_FRESH
    steps = [(G.STEP_MATMUL, F, gs[0], gs[1], 0, 0), (G.STEP_ACTIVATION, F, gs[2], None, 5, 16),
             (G.STEP_MATMUL, F, gs[3], gs[4], 0, 0)]
    ch = G.PoseidonChannel()
    ch.mix_u64(13)
    fp, fv = G.prove_walk(ctx, ch, steps, proof)
    proof.set_input_claim(fp, fv)
    proof.set_io_commitment(77)
    return ch.digest()


@pytest.mark.gpu
def test_streamed_walk_equals_serialized_walk(gpu_ctx):
    """A walk (MatMul, SiLU LogUp with 2^16 multiplicities, MatMul) streamed into a large buffer
    serializes to the words of the same walk serialized afterwards; serializing the streamed proof
    into another buffer gives them too; a stream buffer too short for the second layer ends the
    streaming and the proof still serializes in full into a large enough buffer."""
    log("case streamed walk")
    plain = G.Proof()
    d0 = _walk(gpu_ctx, plain)
    ref = plain.serialize_words()
    buf = np.zeros((len(ref) + 100, 8), dtype=np.uint32)
    p = G.Proof()
    p.stream_to(buf)
    assert _walk(gpu_ctx, p) == d0
    n = p.serialize_into(buf)
    assert n == len(ref) and (buf[:n] == ref).all()
    other = np.zeros((len(ref), 8), dtype=np.uint32)
    assert p.serialize_into(other) == len(ref) and (other == ref).all()
    short = np.zeros((2000, 8), dtype=np.uint32)  # the MatMul layer fits, the LogUp layer does not
    q = G.Proof()
    q.stream_to(short)
    _walk(gpu_ctx, q)
    with pytest.raises(G.GkrError) as e:
        q.serialize_into(short)
    assert e.value.code == 5
    assert (q.serialize_words() == ref).all()


@pytest.mark.gpu
def test_streamed_walk_with_a_step_proved_again(gpu_ctx):
    """The walk's first trip launched ahead stops waiting before the host posts (test hook), so its
    step is proved again: the records of the failed attempt were already streamed and are dropped,
    and the streamed proof equals an undisturbed one."""
    log("case streamed walk with retry")
    plain = G.Proof()
    _walk(gpu_ctx, plain)
    ref = plain.serialize_words()
    buf = np.zeros((len(ref), 8), dtype=np.uint32)
    gpu_ctx.reset_timing()
    gpu_ctx.debug(G.DEBUG_TRIP_EXPIRE, 4)
    p = G.Proof()
    p.stream_to(buf)
    _walk(gpu_ctx, p)
    assert gpu_ctx.kernel_time(19)[1] == 1
    assert p.serialize_into(buf) == len(ref) and (buf == ref).all()


@pytest.mark.gpu
def test_streamed_walk_multiplicity_slots(gpu_ctx):
    """Six SiLU LogUp steps (2^16 multiplicities each) in one streamed walk: each layer's
    multiplicities go from a ring of four pinned slots into its record on the stream's thread, so the
    ring comes round while records are still being written; the streamed words equal those of the
    same walk without a stream.  A proof whose stream is ended, and a proof freed, right after their
    walks give their slots back (their records are copied on the way): the next walk on the context
    neither waits for a slot nor differs."""
    import time
    log("case streamed walk, multiplicity slots")
    g = gpu_ctx.upload(MATS[2])
    steps = [(G.STEP_ACTIVATION, G.CLAIM_FRESH, g, None, 5, 16)] * 6

    def run(proof):
        ch = G.PoseidonChannel()
        ch.mix_u64(29)
        fp, fv = G.prove_walk(gpu_ctx, ch, steps, proof)
        proof.set_input_claim(fp, fv)
        return ch.digest()

    plain = G.Proof()
    d0 = run(plain)
    ref = plain.serialize_words()
    buf = np.zeros((len(ref), 8), dtype=np.uint32)
    p = G.Proof()
    p.stream_to(buf)
    assert run(p) == d0
    assert p.serialize_into(buf) == len(ref) and (buf == ref).all()
    buf_q = np.zeros((len(ref), 8), dtype=np.uint32)
    q = G.Proof()
    q.stream_to(buf_q)
    assert run(q) == d0
    q.stream_to(None)  # ends the stream with records possibly unwritten
    assert (q.serialize_words() == ref).all()
    buf_r = np.zeros((len(ref), 8), dtype=np.uint32)
    r = G.Proof()
    r.stream_to(buf_r)
    assert run(r) == d0
    del r  # freed with records possibly unwritten
    t0 = time.time()
    s = G.Proof()
    assert run(s) == d0
    assert time.time() - t0 < 30
    assert (s.serialize_words() == ref).all()
