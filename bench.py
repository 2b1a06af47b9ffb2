#!/usr/bin/env python3
"""Benchmark of the MI355X GKR matmul / LogUp sumcheck prover.

A step is one complete proof of the configured workload over synthetic,
HBM-resident inputs (weights uploaded once before timing):
  qwen48 (default): 48 Qwen2.5-14B-shaped layers, 64 tokens;
  qwen1 (config 4): one such layer;  smollm (config 3): 30 SmolLM2-135M layers,
  1 token;  cfg1 (config 1): one 256x256x256 matmul layer.
Per layer, on one Poseidon channel and in this order: q, k, v, o, gate, up
matmuls, SiLU LogUp, down matmul, softmax-exp LogUp (Qwen only).  Each matmul
gets a fresh output claim (r_out drawn from the channel, value = MLE of A*B at
r_out, mixed), then the reference's matmul reduction; each LogUp layer gets a
drawn claim point and value, then the reference's activation reduction.  The
proof is serialized at the end of every step.

Prints one JSON line.  value = matmul elements (weights k*n plus activations
m*k) proved per second, in Melem/s; proved tokens/s and the HBM roofline of the
dominant kernel (weight-side restriction) are reported beside it, with the CPU
oracle (the reference's CPU algorithm) timed on a bounded sample.
"""
import argparse
import ctypes as C
import hashlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "stwo-ml_amd"))

# Kernel completions raise no host interrupts: the HSA runtime polls its
# signals instead.  The prover's host thread computes the transcript between
# device results, and interrupt handling on the host delays it and the result
# waits (104 ms against 109 ms per 48-layer proof, same proof).  It must be set
# before the HIP runtime starts; a setting in the environment wins.
os.environ.setdefault("HSA_ENABLE_INTERRUPT", "0")

import gkr_mi355x as G  # noqa: E402

METRIC = "GKR matmul-sumcheck Melem/s + % HBM peak; proved tokens/s, Qwen2.5-14B shape"
HBM_PEAK_GBS = 8000.0
P = (1 << 31) - 1  # M31
(K_RESTRICT_COLS, K_RESTRICT_ROWS, K_MM_ROUND, K_EQ3_ROUND, K_LOGUP_PREP, K_EQ_TABLE, K_HOST_FS, K_HOST_WAIT,
 K_HOST_WAIT_TAIL, K_MERKLE, K_HOST_DRAW, K_HOST_LAUNCH, K_HOST_FINISH, K_NORM, K_LOOKUP, K_HOST_GRAM,
 K_HOST_PROOF, K_HOST_WALK_MM, K_HOST_WALK_ACT, K_WALK_RETRY, K_ACT_AHEAD) = range(21)

QWEN = dict(hidden=5120, inter=13824, q=40 * 128, kv=8 * 128, heads=40, tokens=64)
SMOL = dict(hidden=576, inter=1536, q=9 * 64, kv=3 * 64, heads=9, tokens=1)


def lg(v):
    return max(0, (v - 1).bit_length())


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class LayerWeights:
    def __init__(self, ctx, cfg, layer, seed_base):
        h, i, q, kv, m = cfg["hidden"], cfg["inter"], cfg["q"], cfg["kv"], cfg["tokens"]
        s = seed_base + 1000 * layer
        # int8-range weights and activations (kind 1), resident in HBM
        self.mats = {
            "q": (ctx.synthetic(m, h, 1, s + 1), ctx.synthetic(h, q, 1, s + 2)),
            "k": (None, ctx.synthetic(h, kv, 1, s + 3)),
            "v": (None, ctx.synthetic(h, kv, 1, s + 4)),
            "o": (ctx.synthetic(m, q, 1, s + 5), ctx.synthetic(q, h, 1, s + 6)),
            "gate": (ctx.synthetic(m, h, 1, s + 7), ctx.synthetic(h, i, 1, s + 8)),
            "up": (None, ctx.synthetic(h, i, 1, s + 9)),
            "down": (ctx.synthetic(m, i, 1, s + 10), ctx.synthetic(i, h, 1, s + 11)),
        }
        # k, v share the attention input with q; up shares gate's input
        self.mats["k"] = (self.mats["q"][0], self.mats["k"][1])
        self.mats["v"] = (self.mats["q"][0], self.mats["v"][1])
        self.mats["up"] = (self.mats["gate"][0], self.mats["up"][1])
        # LogUp inputs: gate pre-activation (m x inter) and, for multi-token
        # configs, the attention score tensor (heads*m x m); uniform M31 values
        self.silu_in = ctx.synthetic(m, i, 0, s + 12)
        self.scores = ctx.synthetic(cfg["heads"] * m, m, 0, s + 13) if m > 1 else None


def matmul_elems(cfg):
    h, i, q, kv, m = cfg["hidden"], cfg["inter"], cfg["q"], cfg["kv"], cfg["tokens"]
    shapes = [(m, h, q), (m, h, kv), (m, h, kv), (m, q, h), (m, h, i), (m, h, i), (m, i, h)]
    return sum(k * n + mm * k for mm, k, n in shapes), shapes


def restrict_launch_bytes(m, k, n, int8):
    """Algorithmic bytes of one k_restrict_cols(8) launch over A (m x k) and B (k x n): B once (int8 copy:
    1 byte an entry, u32: 4) and L_j's digits (16 per column) on the weight side; A (4 per entry), L_i
    (16 per row) read and f_a (16 per padded column) written on the activation side."""
    return (1 if int8 else 4) * k * n + 16 * n + 4 * m * k + 16 * m + 16 * (1 << lg(k))


def restrict_by_shape(ctx, cfg, int8):
    """The restriction's timed launches grouped by launch size, named by the model's matmul shapes that
    share it: bytes, launches, average us and fraction of HBM peak per shape."""
    names = {}
    per_layer = list(zip(["q", "k", "v", "o", "gate", "up", "down"], matmul_elems(cfg)[1]))
    for name, (m, k, n) in per_layer:
        names.setdefault(restrict_launch_bytes(m, k, n, int8), []).append(f"{name} {k}x{n}")
    out = []
    for nb, ms, nl in ctx.kernel_time_by_size(K_RESTRICT_COLS):
        us = ms / nl * 1e3
        gbs = nb / (us * 1e-6) / 1e9
        out.append({"shape": "/".join(names.get(nb, [f"{nb} bytes"])), "bytes": nb, "launches": nl,
                    "avg_us": round(us, 3), "gbps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
    return out


CALL_TIME = {"matmul_claim": 0.0, "matmul_layer": 0.0, "activation_layer": 0.0, "walk": 0.0, "serialize": 0.0}


def prove_matmul(ctx, ch, a, b, proof):
    r = ch.draw_qm31s(lg(a.rows) + lg(b.cols))
    t0 = time.perf_counter()
    v = ctx.matmul_output_claim(a, b, r)
    t1 = time.perf_counter()
    ch.mix_secure_field(v)
    res = ctx.prove_matmul_layer(r, v, a, b, ch, proof)
    CALL_TIME["matmul_claim"] += t1 - t0
    CALL_TIME["matmul_layer"] += time.perf_counter() - t1
    return res


def prove_logup(ctx, ch, x, tag, tlog, proof):
    r = ch.draw_qm31s(lg(x.rows) + lg(x.cols))
    v = ch.draw_qm31()
    t0 = time.perf_counter()
    res = ctx.prove_activation_layer(r, v, x, tag, ch, tlog, proof)
    CALL_TIME["activation_layer"] += time.perf_counter() - t0
    return res


class SerialBuffer:
    """Reused output buffer for the serialized proof (felt252 calldata)."""

    def __init__(self, stream=True):
        self.buf, self.cap, self.n = None, 0, 0
        self.stream = stream

    def serialize(self, proof) -> int:
        n = C.c_size_t()
        rc = G.lib().gkr_proof_serialize(proof.handle, self.buf, self.cap, C.byref(n))
        if rc == 5:  # buffer too small: grow once and retry
            self.cap = int(n.value * 1.25) + 1024
            self.buf = (G.GkrFelt * self.cap)()
            rc = G.lib().gkr_proof_serialize(proof.handle, self.buf, self.cap, C.byref(n))
        G._check(rc)
        self.n = n.value
        return self.n

    def attach(self, proof) -> None:
        """Once the buffer exists: the proof's layers are written into it while the walk proves
        (gkr_proof_stream_to), so serialize() then writes only the layer count and the tail."""
        if self.stream and self.buf is not None:
            G._check(G.lib().gkr_proof_stream_to(proof.handle, self.buf, self.cap))

    def fingerprint(self) -> str:
        view = (C.c_uint8 * (32 * self.n)).from_address(C.addressof(self.buf))
        return hashlib.sha256(view).hexdigest()[:16]


def prove_model(ctx, layers, cfg, seed, sbuf):
    ch = G.PoseidonChannel()
    ch.mix_u64(seed)
    proof = G.Proof()
    for L in layers:
        for name in ("q", "k", "v", "o", "gate", "up"):
            a, b = L.mats[name]
            prove_matmul(ctx, ch, a, b, proof)
        prove_logup(ctx, ch, L.silu_in, 5, 16, proof)  # SiLU, 2^16 table
        a, b = L.mats["down"]
        prove_matmul(ctx, ch, a, b, proof)
        if L.scores is not None:
            prove_logup(ctx, ch, L.scores, 4, 16, proof)  # softmax-exp, 2^16 table
    t1 = time.perf_counter()
    n = sbuf.serialize(proof)  # final proof serialization (C side)
    CALL_TIME["serialize"] += time.perf_counter() - t1
    return ch.digest(), n


def model_steps(layers):
    """The per-layer step list for gkr_prove_walk (same order and claims as prove_model)."""
    F = G.CLAIM_FRESH
    steps = []
    for L in layers:
        for name in ("q", "k", "v", "o", "gate", "up"):
            a, b = L.mats[name]
            steps.append((G.STEP_MATMUL, F, a, b, 0, 0))
        steps.append((G.STEP_ACTIVATION, F, L.silu_in, None, 5, 16))
        a, b = L.mats["down"]
        steps.append((G.STEP_MATMUL, F, a, b, 0, 0))
        if L.scores is not None:
            steps.append((G.STEP_ACTIVATION, F, L.scores, None, 4, 16))
    return G.make_steps(steps), len(steps)


def prove_model_walk(ctx, steps, seed, sbuf):
    """The same proof as prove_model, with the layer loop inside the library (gkr_prove_walk)."""
    arr, n = steps
    ch = G.PoseidonChannel()
    ch.mix_u64(seed)
    proof = G.Proof()
    sbuf.attach(proof)
    t0 = time.perf_counter()
    G.prove_walk(ctx, ch, arr, proof, n_steps=n)
    t1 = time.perf_counter()
    n = sbuf.serialize(proof)
    CALL_TIME["walk"] += t1 - t0
    CALL_TIME["serialize"] += time.perf_counter() - t1
    return ch.digest(), n


def cfg1_step(ctx, a, b, sbuf):
    ch = G.PoseidonChannel()
    r = ch.draw_qm31s(16)
    v = ctx.matmul_output_claim(a, b, r)
    ch.mix_secure_field(v)
    proof = G.Proof()
    ctx.prove_matmul_layer(r, v, a, b, ch, proof)
    proof.set_input_claim(r[:8], v)
    return ch.digest(), sbuf.serialize(proof)


def poseidon_round_us(n=500):
    """Host cost of one degree-2 round of the transcript (mix_poly_coeffs + draw_qm31)."""
    ch = G.PoseidonChannel()
    c = [(1, 2, 3, 4), (5, 6, 7, 8), (9, 10, 11, 12)]
    t0 = time.perf_counter()
    for _ in range(n):
        ch.mix_poly_coeffs(*c)
        ch.draw_qm31()
    return round((time.perf_counter() - t0) / n * 1e6, 2)


def measured_traffic(name="restrict_cols_traffic.md"):
    """HBM bytes per launch of k_restrict_cols from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE runs scaled by the copy-kernel calibration), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_baseline(config="qwen48"):
    """The oracle (the reference's CPU algorithm) on the host cores, on a bounded unit of the bench's
    own workload: for the Qwen configs one whole config-4 layer (layer 0 of the bench's model: 7
    matmul reductions with their fresh claims, the SiLU and softmax-exp LogUp reductions; config 5
    is reported as 48 times that layer, labelled as an extrapolation), for smollm the whole 30-layer
    proof, for cfg1 the 256^3 layer."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    info = host_info()
    base = {"unit": "Melem/s", "cores": info["omp_threads"], "kind": "port", "host": info}
    t0 = time.perf_counter()
    if config == "cfg1":
        A, B = O.synthetic(256, 256, 0, 0), O.synthetic(256, 256, 0, 1)
        ch = O.Channel()
        r = ch.draw_qm31s(16)
        v = O.matmul_output_claim(A, B, r)
        ch.mix_secure_field(v)
        O.prove_matmul_layer(r, v, A, B, ch)
        dt = time.perf_counter() - t0
        return dict(base, value=round(2 * 256 * 256 / dt / 1e6, 3), s_per_proof=round(dt, 4),
                    sample=f"BASELINE config 1 (256x256x256 uniform M31 layer) by the oracle: {dt:.3f} s")
    och = O.Channel()
    och.mix_u64(7)
    out = []
    if config == "smollm":
        for layer in range(30):
            oracle_layer(O, och, SMOL, layer, out)
        dt = time.perf_counter() - t0
        per_layer, _ = matmul_elems(SMOL)
        return dict(base, value=round(30 * per_layer / dt / 1e6, 3), s_per_proof=round(dt, 3),
                    proved_tokens_per_s=round(1 / dt, 3),
                    sample=f"the whole BASELINE config 3 proof (30 SmolLM2-135M layers, 1 token) by the oracle: {dt:.2f} s")
    oracle_layer(O, och, QWEN, 0, out)
    dt = time.perf_counter() - t0
    per_layer, _ = matmul_elems(QWEN)
    return dict(base, value=round(per_layer / dt / 1e6, 3),
                sample=f"one whole Qwen2.5-14B layer, 64 tokens (BASELINE config 4: 7 matmul reductions with fresh "
                       f"claims, SiLU and softmax-exp LogUp reductions) by the oracle, the reference's CPU algorithm "
                       f"(forward product for each claim, pad, QM31 MLE, restrict_mle, rounds; batch inversion, "
                       f"eq-sumcheck and multiplicity rounds): {dt:.2f} s",
                s_per_layer=round(dt, 3), proved_tokens_per_s=round(QWEN["tokens"] / dt, 3),
                config5_extrapolated_s_per_proof=round(48 * dt, 1),
                config5_note="48 x the measured layer (an extrapolation, not timed)")


def oracle_host_layer(O, cfg, layer, seed_base=0):
    """Host copies of LayerWeights(ctx, cfg, layer, seed_base): the same generator and seeds."""
    h, i, q, kv, m = cfg["hidden"], cfg["inter"], cfg["q"], cfg["kv"], cfg["tokens"]
    s = seed_base + 1000 * layer
    xq, xo, xg, xd = (O.synthetic(m, h, 1, s + 1), O.synthetic(m, q, 1, s + 5), O.synthetic(m, h, 1, s + 7),
                      O.synthetic(m, i, 1, s + 10))
    mats = {"q": (xq, O.synthetic(h, q, 1, s + 2)), "k": (xq, O.synthetic(h, kv, 1, s + 3)),
            "v": (xq, O.synthetic(h, kv, 1, s + 4)), "o": (xo, O.synthetic(q, h, 1, s + 6)),
            "gate": (xg, O.synthetic(h, i, 1, s + 8)), "up": (xg, O.synthetic(h, i, 1, s + 9)),
            "down": (xd, O.synthetic(i, h, 1, s + 11))}
    silu = O.synthetic(m, i, 0, s + 12)
    scores = O.synthetic(cfg["heads"] * m, m, 0, s + 13) if m > 1 else None
    return mats, silu, scores


def oracle_layer(O, och, cfg, layer, out, seed_base=0):
    """The per-layer sequence of model_steps on the oracle (the reference's CPU algorithm): fresh
    claims, q k v o gate up matmuls, SiLU LogUp (2^16), down, softmax-exp LogUp (2^16); the serialized
    felts are appended to out."""
    mats, silu, scores = oracle_host_layer(O, cfg, layer, seed_base)

    def matmul(A, B):
        r = och.draw_qm31s(lg(A.shape[0]) + lg(B.shape[1]))
        v = O.matmul_output_claim(A, B, r)
        och.mix_secure_field(v)
        o = O.prove_matmul_layer(r, v, A, B, och)
        O.serialize_matmul_layer(out, o["round_polys"], o["final_a_eval"], o["final_b_eval"])

    def logup(X, tag):
        r = och.draw_qm31s(lg(X.shape[0]) + lg(X.shape[1]))
        v = och.draw_qm31()
        o = O.prove_activation_layer(r, v, X, tag, och, 16)
        O.serialize_activation_layer(out, tag, o)

    for name in ("q", "k", "v", "o", "gate", "up"):
        matmul(*mats[name])
    logup(silu, 5)
    matmul(*mats["down"])
    if scores is not None:
        logup(scores, 4)


def host_info():
    """CPU model, threads and the oracle's compiler, for the CPU baseline records."""
    import platform
    import subprocess
    model = platform.processor()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        cc = subprocess.run(["gcc", "--version"], capture_output=True, text=True, timeout=10).stdout.splitlines()[0]
    except (OSError, IndexError, subprocess.SubprocessError):
        cc = None
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "cpus_usable": usable, "omp_threads": threads,
            "oracle_compiler": cc, "oracle_flags": "-O3 -march=x86-64-v3 -fopenmp (oracle/Makefile)"}


def cpu_configs():
    """The oracle (reference CPU algorithm) on whole configurations: config 1 (256^3 uniform matmul),
    config 3 (the 30-layer SmolLM2 walk, 1 token) and config 4 (one Qwen2.5-14B layer, 64 tokens: 7
    matmuls, the SiLU and softmax-exp LogUps), each the workload the GPU bench times for that config."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    res = {"host": host_info()}
    t0 = time.perf_counter()
    A, B = O.synthetic(256, 256, 0, 0), O.synthetic(256, 256, 0, 1)
    ch = O.Channel()
    r = ch.draw_qm31s(16)
    v = O.matmul_output_claim(A, B, r)
    ch.mix_secure_field(v)
    O.prove_matmul_layer(r, v, A, B, ch)
    res["cfg1"] = {"s_per_proof": round(time.perf_counter() - t0, 4)}
    log("[cpu] config 1 done")
    t0 = time.perf_counter()
    och = O.Channel()
    out = [0]
    for layer in range(30):
        oracle_layer(O, och, SMOL, layer, out)
    res["smollm"] = {"s_per_proof": round(time.perf_counter() - t0, 3), "tokens": 1}
    log("[cpu] config 3 done")
    t0 = time.perf_counter()
    och = O.Channel()
    out = [0]
    oracle_layer(O, och, QWEN, 0, out)
    dt = time.perf_counter() - t0
    res["qwen1"] = {"s_per_layer": round(dt, 3), "tokens": QWEN["tokens"],
                    "qwen48_extrapolated_s": round(48 * dt, 1)}
    log("[cpu] config 4 done")
    return res


WEIGHT_NAMES = ("q", "k", "v", "o", "gate", "up", "down")


def merkle_hashes(rows, cols):
    """Poseidon hashes the commitment of a rows x cols weight computes: the real nodes of levels >= 1
    (subtrees of grid padding come from a table)."""
    lpk, lpn = lg(rows), lg(cols)
    n = 0
    for s in range(1, max(1, lpk + lpn) + 1):
        n += cols * -(-rows // (1 << s)) if s <= lpk else -(-cols // (1 << (s - lpk)))
    return n


def merkle_valu_profile(name="merkle_commit.md"):
    """(VALU wave instructions per Poseidon hash, mix-weighted VALU issue peak in G wave-instr/s)
    of the Merkle level kernel, from the committed rocprofv3 PMC summary, or (None, None)."""
    vals = {}
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                for key in ("valu_wave_insts_per_hash", "valu_mix_peak_gwips"):
                    if line.startswith(key + ":"):
                        vals[key] = float(line.split(":")[1])
    except OSError:
        pass
    return vals.get("valu_wave_insts_per_hash"), vals.get("valu_mix_peak_gwips")


def cpu_commit_baseline(budget_rows=256, budget_cols=512):
    """The oracle's weight commitment (reference algorithm, one thread) on a bounded matrix."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    B = O.synthetic(budget_rows, budget_cols, 1, 3)
    t0 = time.perf_counter()
    O.weight_commitment(B)
    dt = time.perf_counter() - t0
    h = budget_rows * budget_cols - 1
    return {"value": round(h / dt / 1e6, 4), "unit": "Mhash/s", "cores": 1, "kind": "port",
            "sample": f"commit_mle_root_only of a {budget_rows}x{budget_cols} weight (int8-range) by the oracle "
                      f"(the reference's root_only algorithm, sequential): {h} hashes in {dt:.2f} s"}


def bench_commit(ctx, args):
    """Weight commitments of one Qwen2.5-14B layer: the 7 weights (q, k, v, o, gate, up, down;
    int8-range synthetic, resident) committed as one batch per step
    (commit_mle_root_only(matrix_to_mle_col_major_padded(W)) each).  After the timed steps, the
    layer's 7 weight openings at drawn points are timed once (prove_mle_opening_with_commitment:
    folds, all folded-layer trees, 10 queries)."""
    lw = LayerWeights(ctx, QWEN, 0, 0)
    mats = [lw.mats[k][1] for k in WEIGHT_NAMES]
    shapes = [(m.rows, m.cols) for m in mats]
    hashes = sum(merkle_hashes(r, c) for r, c in shapes)
    padded = sum((1 << lg(r)) * (1 << lg(c)) - 1 for r, c in shapes)
    ctx.synchronize()

    def fresh_roots():  # the roots kept on the matrices are dropped, so every step hashes
        for m in mats:
            m.invalidate()
        return ctx.weight_commitments(mats)

    for _ in range(args.warmup):
        roots = fresh_roots()
    ctx.set_timing(0 if args.no_timing else 1)
    ctx.reset_timing()
    t0 = time.perf_counter()
    outs = [fresh_roots() for _ in range(args.steps)]
    dt = (time.perf_counter() - t0) / args.steps
    t0 = time.perf_counter()
    assert ctx.weight_commitments(mats) == outs[0]  # the roots the last step left on the matrices
    cached_ms = (time.perf_counter() - t0) * 1e3
    assert all(o == outs[0] for o in outs), "non-deterministic commitment"
    ms, nl, nh = ctx.kernel_time(K_MERKLE)
    ctx.set_timing(0)
    # openings of the same weights at points drawn from a channel
    ch = G.PoseidonChannel()
    ch.mix_u64(5120)
    proof = G.Proof()
    t1 = time.perf_counter()
    for m in mats:
        ctx.prove_weight_opening(m, ch.draw_qm31s(lg(m.rows) + lg(m.cols)), ch, proof)
    open_s = time.perf_counter() - t1
    felts = len(proof.serialize())
    kernel = None
    roofline = None
    if nl:
        kh = nh / (ms * 1e-3)
        kernel = {"launches_per_step": nl // args.steps, "ms_per_step": round(ms / args.steps, 3),
                  "hashes_per_s_M": round(kh / 1e6, 1)}
        ipw, peak = merkle_valu_profile()
        if ipw and peak:
            ach = kh / 64 * ipw / 1e9
            roofline = {"bound": "valu", "achieved": round(ach, 1), "peak": peak,
                        "unit": "G wave-instr/s", "frac": round(ach / peak, 4), "traffic": None,
                        "kernel": "k_merkle_level", "valu_wave_insts_per_hash": ipw,
                        "source": "profiles/merkle_commit.md (rocprofv3 PMC SQ_INSTS_VALU; peak weighted by "
                                  "the hash's 64-bit/32-bit instruction mix at the published vector rates)"}
    result = {
        "metric": "Poseidon Merkle weight commitment, hashes/s (Qwen2.5-14B layer)",
        "value": round(hashes / dt / 1e6, 1), "unit": "Mhash/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "felt252 (9 x 29-bit limbs)",
        "data": "synthetic (counter-mode SplitMix64, int8-range weights)",
        "config": {"workload": "qwen2.5-14b-layer-weight-commitments", "weights": dict(zip(WEIGHT_NAMES, shapes)),
                   "hashes_per_step": hashes, "padded_tree_hashes_per_step": padded},
        "padded_tree_equivalent_Mhash_s": round(padded / dt / 1e6, 1),
        "kernel": kernel, "roofline": roofline,
        "openings": {"s_per_layer": round(open_s, 3), "felts": felts},
        "cached_roots_ms": round(cached_ms, 3),
        "roots_sha256_16": hashlib.sha256(",".join(hex(r) for r in outs[0]).encode()).hexdigest()[:16],
        "cpu_baseline": None if args.no_cpu_baseline else cpu_commit_baseline(),
    }
    print(json.dumps(result), flush=True)
    ctx.close()


def bench_forward(ctx, args):
    """Forward pass of one Qwen2.5-14B layer, 64 tokens: the 7 matmul products C = A * B mod P
    (int8-range synthetic weights and activations, resident) on the matrix cores, each into a
    preallocated output.  The weights' digit planes are built during warm-up (once per weight)."""
    lw = LayerWeights(ctx, QWEN, 0, 0)
    pairs = [(lw.mats[k][0], lw.mats[k][1]) for k in WEIGHT_NAMES]
    outs = [ctx.matmul_forward(a, b) for a, b in pairs]
    for _ in range(max(1, args.warmup)):
        for (a, b), o in zip(pairs, outs):
            ctx.matmul_forward_into(a, b, o)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for (a, b), o in zip(pairs, outs):
            ctx.matmul_forward_into(a, b, o)
    ctx.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    macs = sum(a.rows * a.cols * b.cols for a, b in pairs)
    wbytes = sum(b.rows * b.cols for _, b in pairs)  # one digit plane (1 byte per weight) streamed
    digest = hashlib.sha256(b"".join(o.download().tobytes() for o in outs)).hexdigest()[:16]
    result = {
        "metric": "forward M31 GEMM, Qwen2.5-14B layer (64 tokens) on the matrix cores",
        "value": round(macs / dt / 1e12, 3), "unit": "T M31-MAC/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8 digit planes -> i32 -> M31",
        "data": "synthetic (counter-mode SplitMix64, int8-range weights and activations)",
        "config": {"workload": "qwen2.5-14b-layer-forward-64-tokens", "weights": dict(zip(WEIGHT_NAMES,
                   [(b.rows, b.cols) for _, b in pairs])), "macs_per_step": macs},
        "roofline": {"bound": "hbm", "achieved": round(wbytes / dt / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(wbytes / dt / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_gemm_m31 (whole step incl. packing and split reduction)",
                     "note": "bytes = the weights' digit plane 0 (int8-range), 1 byte per weight"},
        "u32_weight_equivalent_gbps": round(4 * wbytes / dt / 1e9, 1),
        "outputs_sha256_16": digest, "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    ctx.close()


def bench_simd(ctx, args, blocks=8):
    """Shared-weight SIMD matmul layer (reduce_matmul_layer_simd_gpu): `blocks` activation blocks of
    64x5120 (one per transformer block of a batch) against the Qwen2.5-14B MLP gate weight 5120x13824,
    int8-range synthetic data resident in HBM; a step is one layer proof with a fresh channel."""
    m, k, n = 64, 5120, 13824
    a = [ctx.synthetic(m, k, 1, 300 + i) for i in range(blocks)]
    b = ctx.synthetic(k, n, 1, 400)
    prng = __import__("random").Random(5)
    ws = [tuple(prng.randrange(P) for _ in range(4)) for _ in range(blocks)]
    nv = lg(m) + lg(n)

    def step():
        ch = G.PoseidonChannel()
        ch.mix_u64(blocks)
        r = ch.draw_qm31s(nv)
        res = ctx.prove_matmul_layer_simd(r, (1, 2, 3, 4), a, ws, b, ch)
        return ch.digest(), res["final_a_eval"]

    for _ in range(max(1, args.warmup)):
        step()
    ctx.set_timing(0 if args.no_timing else 1)
    ctx.reset_timing()
    ctx.synchronize()
    t0 = time.perf_counter()
    outs = [step() for _ in range(args.steps)]
    ctx.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    assert all(o == outs[0] for o in outs), "non-deterministic proof"
    elems = blocks * m * k + k * n
    kernels, roofline = {}, None
    for kid, name in [(K_RESTRICT_COLS, "restrict_cols (weight side)"), (K_RESTRICT_ROWS, "restrict_rows_simd")]:
        ms, nl, nb = ctx.kernel_time(kid)
        if nl:
            kernels[name] = {"launches": nl, "avg_us": round(ms / nl * 1e3, 3),
                             "gbps": round(nb / (ms * 1e-3) / 1e9, 1), "bytes_per_launch": nb // nl}
    rc = kernels.get("restrict_cols (weight side)")
    if rc:
        roofline = {"bound": "hbm", "achieved": rc["gbps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(rc["gbps"] / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_restrict_cols",
                    "avg_launch_us": rc["avg_us"], "bytes_per_launch": rc["bytes_per_launch"]}
    ctx.set_timing(0)
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        As = [O.synthetic(m, k, 1, 300 + i) for i in range(blocks)]
        B = O.synthetic(k, n, 1, 400)
        ch = O.Channel()
        ch.mix_u64(blocks)
        r = ch.draw_qm31s(nv)
        t1 = time.perf_counter()
        O.prove_matmul_layer_simd(r, (1, 2, 3, 4), As, B, ws, ch)
        dtc = time.perf_counter() - t1
        cpu = {"value": round(elems / dtc / 1e6, 3), "unit": "Melem/s",
               "cores": int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count(), "kind": "port",
               "sample": f"the same layer by the oracle (reference CPU algorithm): {dtc:.2f} s"}
    # dual-operand SIMD layer: 64 attention heads, score_h = Q_h (64 x 128) . K_h^T (128 x 64)
    heads, hm, hk, hn = 64, 64, 128, 64
    qa = [ctx.synthetic(hm, hk, 1, 500 + i) for i in range(heads)]
    kb = [ctx.synthetic(hk, hn, 1, 600 + i) for i in range(heads)]
    hw = [tuple(prng.randrange(P) for _ in range(4)) for _ in range(heads)]

    def dual_step():
        ch = G.PoseidonChannel()
        ch.mix_u64(heads)
        r = ch.draw_qm31s(lg(hm) + lg(hn))
        ctx.prove_matmul_layer_dual_simd(r, (1, 2, 3, 4), qa, kb, hw, ch)
        return ch.digest()

    dual_step()
    ctx.synchronize()
    t2 = time.perf_counter()
    dd = [dual_step() for _ in range(args.steps)]
    ctx.synchronize()
    dual_ms = (time.perf_counter() - t2) / args.steps * 1e3
    assert all(x == dd[0] for x in dd), "non-deterministic proof"
    result = {
        "metric": "GKR SIMD matmul layer (shared weight) Melem/s + % HBM peak",
        "value": round(elems / dt / 1e6, 1), "unit": "Melem/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u32-m31", "data": "synthetic (counter-mode SplitMix64, int8-range)",
        "config": {"workload": f"qwen2.5-14b-gate-simd-{blocks}-blocks", "blocks": blocks, "block_shape": [m, k],
                   "weight_shape": [k, n]},
        "roofline": roofline, "kernels": kernels, "digest": hex(outs[0][0]), "cpu_baseline": cpu,
        "dual_simd": {"workload": f"{heads} heads, Q_h {hm}x{hk} . K_h^T {hk}x{hn}", "ms_per_layer": round(dual_ms, 3),
                      "digest": hex(dd[0])},
    }
    print(json.dumps(result), flush=True)
    ctx.close()


def bench_norm(ctx, args):
    """The two RMSNorm layers of one Qwen2.5-14B block (input and post-attention: 64 tokens x 5120,
    learned per-column scale), each with a fresh output claim on one channel through
    gkr_prove_walk (reduce_rmsnorm_layer_with_gamma, prover.rs:8407-8801); a LayerNorm layer of the
    same shape (reduce_layernorm_layer, prover.rs:7944-8395) is timed beside it.  int8-range
    synthetic activations resident in HBM."""
    import numpy as np
    m, h = QWEN["tokens"], QWEN["hidden"]
    xs = [ctx.synthetic(m, h, 1, 700 + i) for i in range(2)]
    gv = [np.random.default_rng(7 + i).integers(1, 1 << 12, size=(1, h), dtype=np.uint32) for i in range(2)]
    gam = [ctx.upload(g) for g in gv]
    steps = G.make_steps([(G.STEP_RMSNORM, G.CLAIM_FRESH, xs[i], gam[i], 0, 0, h) for i in range(2)])
    ln_steps = G.make_steps([(G.STEP_LAYERNORM, G.CLAIM_FRESH, xs[0], None, 0, 0, h)])

    def run(arr, n):
        ch = G.PoseidonChannel()
        ch.mix_u64(m)
        proof = G.Proof()
        G.prove_walk(ctx, ch, arr, proof, n_steps=n)
        return ch.digest()

    for _ in range(max(1, args.warmup)):
        run(steps, 2)
    ctx.set_timing(0 if args.no_timing else 2 if args.timing_all else 1)
    ctx.reset_timing()
    ctx.synchronize()
    t0 = time.perf_counter()
    outs = [run(steps, 2) for _ in range(args.steps)]
    ctx.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    assert all(o == outs[0] for o in outs), "non-deterministic proof"
    ms, nl, nb = ctx.kernel_time(K_NORM)
    kernels = {}
    for kid, name in [(K_NORM, "norm_rows+prepare"), (K_MM_ROUND, "product_trips"), (K_EQ3_ROUND, "eq3_trips"),
                      (K_EQ_TABLE, "eq_tables")]:
        km, kn, kb = ctx.kernel_time(kid)
        if kn:
            kernels[name] = {"launches": kn // args.steps, "avg_us": round(km / kn * 1e3, 3),
                             "ms_per_step": round(km / args.steps, 3)}
    host = {}
    for kid, name in [(K_HOST_FS, "fiat_shamir"), (K_HOST_WAIT, "device_wait"), (K_HOST_WAIT_TAIL, "device_wait_handover"),
                      (K_HOST_DRAW, "claim_draws"), (K_HOST_LAUNCH, "launch_calls"), (K_HOST_FINISH, "host_finish")]:
        hm, hn, _ = ctx.kernel_time(kid)
        if hn:
            host[name] = {"ms_per_step": round(hm / args.steps, 3), "calls": hn // args.steps}
    roofline = None
    if nl:
        gbps = nb / (ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbps / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_norm_rows + k_norm_prepare",
                    "avg_launch_us": round(ms / nl * 1e3, 3), "bytes_per_launch": nb // nl}
    ctx.set_timing(0)
    run(ln_steps, 1)
    ctx.synchronize()
    t1 = time.perf_counter()
    ln = [run(ln_steps, 1) for _ in range(args.steps)]
    ctx.synchronize()
    ln_ms = (time.perf_counter() - t1) / args.steps * 1e3
    assert all(x == ln[0] for x in ln), "non-deterministic proof"
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        X = O.synthetic(m, h, 1, 700)
        g = gv[0].reshape(-1)
        ch = O.Channel()
        r = ch.draw_qm31s(lg(m) + lg(h))
        t2 = time.perf_counter()
        O.prove_rmsnorm_layer(r, (1, 2, 3, 4), X, h, ch, g)
        dtc = time.perf_counter() - t2
        cpu = {"value": round(m * h / dtc / 1e6, 4), "unit": "Melem/s", "cores": 1, "kind": "port",
               "sample": f"one RMSNorm layer {m}x{h} by the oracle (reference CPU algorithm, one core): {dtc:.2f} s"}
    result = {
        "metric": "GKR RMSNorm layer proving, normalized Melem/s", "value": round(2 * m * h / dt / 1e6, 2),
        "unit": "Melem/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u32-m31", "data": "synthetic (counter-mode SplitMix64, int8-range activations, 12-bit scales)",
        "config": {"workload": "qwen2.5-14b-block-rmsnorms-64-tokens", "layers": 2, "shape": [m, h]},
        "roofline": roofline, "kernels": kernels, "host": host, "layernorm_ms_per_layer": round(ln_ms, 3),
        "digest": hex(outs[0]),
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    ctx.close()


def bench_binding(ctx, args):
    """The full aggregated weight binding (STWO_AGGREGATED_FULL_BINDING=1, gkr/prover.rs:1233-1330) of one
    Qwen2.5-14B layer: the layer's walk (fresh claims, bench order) records its 7 weight claims, then the
    weight phase proves the commitments and two AggregatedWeightBindingProofs (groups of 4 and 3 claims,
    aggregated_opening.rs:1647-1720).  Only the weight phase is timed; weights resident in HBM."""
    lw = LayerWeights(ctx, QWEN, 0, 0)
    steps = model_steps([lw])
    weight_elems = sum(lw.mats[k][1].rows * lw.mats[k][1].cols for k in WEIGHT_NAMES)

    def step():
        ch = G.PoseidonChannel()
        ch.mix_u64(7)
        proof = G.Proof()
        G.prove_walk(ctx, ch, steps[0], proof, n_steps=steps[1])
        ctx.synchronize()
        t0 = time.perf_counter()
        ctx.prove_weight_binding(ch, proof, G.WEIGHT_AGGREGATED_FULL)
        ctx.synchronize()
        dt = time.perf_counter() - t0
        groups = proof.binding_groups()
        return dt, ch.digest(), [len(g) for g in groups]

    for _ in range(max(1, args.warmup)):
        step()
    ctx.set_timing(0 if args.no_timing else 1)
    ctx.reset_timing()
    res = [step() for _ in range(args.steps)]
    dt = sum(r[0] for r in res) / len(res)
    assert all(r[1] == res[0][1] for r in res), "non-deterministic proof"
    ms, nl, nh = ctx.kernel_time(K_MERKLE)
    fs, fsn, _ = ctx.kernel_time(K_HOST_FS)
    ctx.set_timing(0)
    result = {
        "metric": "aggregated weight binding (full), weight elements/s (Qwen2.5-14B layer)",
        "value": round(weight_elems / dt / 1e6, 1), "unit": "Melem/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u32-m31/qm31", "data": "synthetic (counter-mode SplitMix64, int8-range)",
        "config": {"workload": "qwen2.5-14b-layer-full-weight-binding", "claims": 7, "groups": res[0][2],
                   "weight_elements": weight_elems},
        "merkle": {"ms_per_step": round(ms / args.steps, 3), "Mhash_per_s": round(nh / (ms * 1e-3) / 1e6, 1)} if nl else None,
        "host_fiat_shamir_ms_per_step": round(fs / args.steps, 3) if fsn else None,
        "digest": hex(res[0][1]), "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    ctx.close()


def bench_lookup(ctx, args, n_inst=96, log_n=16):
    """STWO LogUp-GKR batch (prove_batch, stwo-gpu/crates/stwo/src/prover/lookups/gkr_prover.rs:396-500) as
    prove_logup_gkr (engine/src/aggregation.rs:3926-4062) builds it for a Qwen2.5-14B model: one
    LogUpMultiplicities instance per activation table of the 48 layers (SiLU and softmax-exp, 2^16 entries
    each): numerators the table's multiplicities, denominators alpha - table input.  Synthetic tables and
    counts resident in HBM; a step is one batch proof on a fresh channel."""
    import numpy as np
    n = 1 << log_n
    rng = np.random.default_rng(11)
    alpha = [int(x) for x in rng.integers(0, P, size=4)]
    host = []
    for i in range(n_inst):
        mult = rng.integers(0, 8, size=n, dtype=np.uint32)
        tin = rng.integers(0, P, size=n, dtype=np.uint64)
        den = np.empty((n, 4), dtype=np.uint32)
        den[:, 0] = (alpha[0] + P - tin) % P
        den[:, 1:] = alpha[1:]
        host.append((mult, den))
    dev = [(G.LOOKUP_LOGUP_MULTIPLICITIES, log_n, ctx.upload(m.reshape(1, -1)), ctx.qvec_upload(d)) for m, d in host]

    def step():
        ch = G.PoseidonChannel()
        ch.mix_u64(n_inst)
        G.prove_lookup_batch(ctx, ch, dev)
        return ch.digest()

    for _ in range(max(1, args.warmup)):
        step()
    ctx.set_timing(0 if args.no_timing else 2 if args.timing_all else 1)
    ctx.reset_timing()
    ctx.synchronize()
    t0 = time.perf_counter()
    outs = [step() for _ in range(args.steps)]
    ctx.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    assert all(o == outs[0] for o in outs), "non-deterministic proof"
    ms, nl, nb = ctx.kernel_time(K_LOOKUP)
    hostt = {}
    for kid, name in [(K_HOST_FS, "fiat_shamir"), (K_HOST_WAIT, "device_wait"), (K_HOST_LAUNCH, "launch_calls")]:
        hm, hn, _ = ctx.kernel_time(kid)
        if hn:
            hostt[name] = {"ms_per_step": round(hm / args.steps, 3), "calls": hn // args.steps}
    roofline = None
    if nl:
        gbps = nb / (ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbps / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_lk_tree + k_lk_round",
                    "avg_launch_us": round(ms / nl * 1e3, 3), "bytes_per_launch": nb // nl,
                    "launches_per_step": nl // args.steps, "device_ms_per_step": round(ms / args.steps, 3)}
    ctx.set_timing(0)
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        k = 8
        sample = [(O.LOOKUP_LOGUP_MULTIPLICITIES, m, d) for m, d in host[:k]]
        ch = O.Channel()
        ch.mix_u64(k)
        t1 = time.perf_counter()
        O.prove_lookup_batch(ch, sample)
        dtc = time.perf_counter() - t1
        cpu = {"value": round(k * n / dtc / 1e6, 3), "unit": "Mentries/s", "cores": 1, "kind": "port",
               "sample": f"{k} of the {n_inst} instances by the oracle (reference CPU algorithm, one core): {dtc:.2f} s"}
    result = {
        "metric": "STWO LogUp-GKR batch proving, table entries/s", "value": round(n_inst * n / dt / 1e6, 2),
        "unit": "Mentries/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u32-m31/qm31", "data": "synthetic (uniform table inputs, multiplicities 0..7)",
        "config": {"workload": f"qwen2.5-14b-logup-gkr-{n_inst}-tables-2^{log_n}", "instances": n_inst,
                   "log_size": log_n},
        "roofline": roofline, "host": hostt, "digest": hex(outs[0]), "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    ctx.close()


def trip_k(n, big=1 << 16, huge=1 << 20):
    """Rounds per device trip over a vector of n entries (the library's trip_k)."""
    return 1 if n > huge else 2 if n > big else 3


def trip_plan(T, host_len=128):
    """(first round, rounds, vector length) of the device trips of a product sumcheck over 2^T entries
    (the library's plan_trips with the first trip of trip_k(2^T) rounds)."""
    if T <= 0:
        return []
    t = min(trip_k(1 << T), T)
    out = [(0, t, 1 << T)]
    while t < T and (1 << (T - t)) > host_len:
        n = 1 << (T - t)
        k = min(trip_k(n), T - t)
        out.append((t, k, n))
        t += k
    return out


def bench_c2(ctx, args):
    """Config 2: the product sumcheck alone over uniform QM31 vectors f_a, f_b of 2^L entries each
    (channel new(), mix_u64(L); eval -> mix_poly_coeffs -> draw -> fold until size 1).  Algorithmic
    bytes per sumcheck, as the trip kernels move them (trip_plan): the first trip reads both vectors
    (32 N); trip j >= 1 reads both at its predecessor's length and writes them at its own."""
    logs = [int(x) for x in args.c2_logs.split(",")]
    sizes = []
    for L in logs:
        n = 1 << L
        fa, fb = ctx.qvec_synthetic(n, 1000 + L), ctx.qvec_synthetic(n, 2000 + L)
        ctx.synchronize()

        def run():
            ch = G.PoseidonChannel()
            ch.mix_u64(L)
            res = ctx.sumcheck_product(fa, fb, ch)
            return ch.digest(), res["final_a_eval"]

        for _ in range(args.warmup):
            run()
        ctx.set_timing(0 if args.no_timing else 2)  # the roofline kernel here is the product trip
        ctx.reset_timing()
        t0 = time.perf_counter()
        outs = [run() for _ in range(args.steps)]
        ctx.synchronize()
        dt = (time.perf_counter() - t0) / args.steps
        assert all(o == outs[0] for o in outs), "non-deterministic proof"
        ms, nl, nb = ctx.kernel_time(K_MM_ROUND)
        fs_ms, fs_n, _ = ctx.kernel_time(K_HOST_FS)
        ctx.set_timing(False)
        alg = 0
        prev = None
        for _, _, tn in trip_plan(L):
            alg += 32 * (prev if prev else tn) + (32 * tn if prev else 0)
            prev = tn
        entry = {"log2_n": L, "ms_per_sumcheck": round(dt * 1e3, 3),
                 "wall_gbps": round(alg / dt / 1e9, 1), "wall_frac": round(alg / dt / 1e9 / HBM_PEAK_GBS, 4),
                 "qm31_evals_per_s_M": round(2 * (2 * n - 1) / dt / 1e6, 1), "digest": hex(outs[0][0])}
        if nl:
            entry["round_kernels"] = {"launches_per_sumcheck": nl // args.steps, "avg_us": round(ms / nl * 1e3, 3),
                                      "gbps": round(nb / (ms * 1e-3) / 1e9, 1),
                                      "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                      "ms_per_sumcheck": round(ms / args.steps, 3)}
            entry["host_fs_ms_per_sumcheck"] = round(fs_ms / args.steps, 3)
        sizes.append(entry)
        log(f"[bench c2] 2^{L}: {entry}")
        del fa, fb
    big = sizes[-1]
    rk = big.get("round_kernels")
    result = {
        "metric": METRIC, "value": big["qm31_evals_per_s_M"], "unit": "M QM31 evals/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": big["ms_per_sumcheck"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32-m31",
        "data": "synthetic (uniform QM31, SplitMix64)",
        "config": {"workload": f"config2-product-sumcheck-2^{big['log2_n']}", "log2_sizes": logs},
        "roofline": ({"bound": "hbm", "achieved": rk["gbps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": rk["frac"], "traffic": None, "kernel": "k_trip<0,K> (product trips)"} if rk else None),
        "sizes": sizes, "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    ctx.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="qwen48",
                    choices=["qwen48", "qwen1", "smollm", "cfg1", "c2", "commit", "forward", "simd", "norm", "lookup", "binding"])
    ap.add_argument("--c2-logs", default="20,24,28",
                    help="config 2: log2 sizes of the QM31 vectors f_a, f_b (product sumcheck alone)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-configs", action="store_true",
                    help="time the oracle (reference CPU algorithm) on configs 1, 3 and 4 and print one JSON line")
    ap.add_argument("--no-timing", action="store_true", help="no HIP events and no host timers")
    ap.add_argument("--timing-all", action="store_true",
                    help="HIP events on every timed kernel (default: only the roofline kernel k_restrict_cols)")
    ap.add_argument("--u32-weights", action="store_true",
                    help="u32 weight-side restriction (GKR_INT8_WEIGHTS=0) instead of the default int8 weight copy")
    ap.add_argument("--driver", default="walk", choices=["walk", "calls"],
                    help="walk: one gkr_prove_walk call per proof; calls: one library call per layer")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path is measured on one GPU's share)", file=sys.stderr)
        sys.exit(2)

    if args.cpu_configs:
        print(json.dumps({"cpu_configs": cpu_configs()}), flush=True)
        return
    if args.u32_weights:
        os.environ["GKR_INT8_WEIGHTS"] = "0"
    ctx = G.Context(0)
    if args.config == "c2":
        return bench_c2(ctx, args)
    if args.config == "commit":
        return bench_commit(ctx, args)
    if args.config == "forward":
        return bench_forward(ctx, args)
    if args.config == "simd":
        return bench_simd(ctx, args)
    if args.config == "norm":
        return bench_norm(ctx, args)
    if args.config == "lookup":
        return bench_lookup(ctx, args)
    if args.config == "binding":
        return bench_binding(ctx, args)
    sbuf = SerialBuffer()
    if args.config == "cfg1":
        cfg, n_layers = None, 1
        a, b = ctx.synthetic(256, 256, 0, 0), ctx.synthetic(256, 256, 0, 1)
        elems = 256 * 256 * 2
        step = lambda: cfg1_step(ctx, a, b, sbuf)  # noqa: E731
        tokens = 0
        workload = "config1-matmul-256x256x256-uniform-m31"
    else:
        cfg = QWEN if args.config.startswith("qwen") else SMOL
        n_layers = {"qwen48": 48, "qwen1": 1, "smollm": 30}[args.config]
        t0 = time.perf_counter()
        layers = [LayerWeights(ctx, cfg, l, 0) for l in range(n_layers)]
        ctx.synchronize()
        log(f"[bench] {n_layers} layers of synthetic weights resident ({time.perf_counter() - t0:.2f} s)")
        per_layer, shapes = matmul_elems(cfg)
        elems = per_layer * n_layers
        tokens = cfg["tokens"]
        if args.driver == "walk":
            steps = model_steps(layers)
            step = lambda: prove_model_walk(ctx, steps, 7, sbuf)  # noqa: E731
        else:
            step = lambda: prove_model(ctx, layers, cfg, 7, sbuf)  # noqa: E731
        workload = {"qwen48": "qwen2.5-14b-48-layers-64-tokens", "qwen1": "qwen2.5-14b-1-layer-64-tokens",
                    "smollm": "smollm2-135m-30-layers-1-token"}[args.config]

    for w in range(args.warmup):
        t0 = time.perf_counter()
        out = step()
        log(f"[bench] warmup {w}: {time.perf_counter() - t0:.3f} s digest={out[0]:#x}")
    ctx.set_timing(0 if args.no_timing else (2 if args.timing_all else 1))
    ctx.reset_timing()
    ctx.synchronize()
    for key in CALL_TIME:
        CALL_TIME[key] = 0.0
    t0 = time.perf_counter()
    digests = []
    for s in range(args.steps):
        digests.append(step())
        log(f"[bench] step {s} done ({time.perf_counter() - t0:.3f} s)")
    ctx.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    assert all(d == digests[0] for d in digests), "non-deterministic proof"

    kernels = {}
    # at timing level 1 the restriction's and LogUp prepare's events time every
    # 8th launch (sampled_launches: a timed dispatch waits ~4 us for its events
    # on each side); their device time per step is the sampled mean times the
    # launches per step
    per_step = {"restrict_cols": 7 * n_layers if cfg is not None else 1,
                "logup_prepare": sum(1 + (L.scores is not None) for L in layers) if cfg is not None else 0}
    for kid, name in [(K_RESTRICT_COLS, "restrict_cols"), (K_RESTRICT_ROWS, "restrict_rows"),
                      (K_MM_ROUND, "product_trip"), (K_EQ3_ROUND, "eq3_or_sum_trip"), (K_LOGUP_PREP, "logup_prepare"),
                      (K_EQ_TABLE, "eq_table")]:
        ms, nl, nb = ctx.kernel_time(kid)
        if nl:
            kernels[name] = {"launches": nl, "avg_us": round(ms / nl * 1e3, 3),
                             "gbps": round(nb / (ms * 1e-3) / 1e9, 1) if ms > 0 else None,
                             "ms_per_step": round(ms / args.steps, 3)}
    if not args.timing_all:
        for name, n in per_step.items():
            if name in kernels:
                k = kernels[name]
                k["sampled_launches"] = k.pop("launches")
                k["ms_per_step"] = round(k["avg_us"] * n / 1e3, 3)
    host = {}
    for kid, name in [(K_HOST_FS, "fiat_shamir"), (K_HOST_WAIT, "device_wait"),
                      (K_HOST_WAIT_TAIL, "device_wait_handover"), (K_HOST_DRAW, "claim_draws"),
                      (K_HOST_LAUNCH, "launch_calls"), (K_HOST_FINISH, "host_finish"),
                      (K_HOST_GRAM, "round_polys_from_trip_sums"), (K_HOST_PROOF, "proof_records"),
                      (K_HOST_WALK_MM, "walk_matmul_steps"), (K_HOST_WALK_ACT, "walk_activation_steps")]:
        ms, nl, _ = ctx.kernel_time(kid)
        if nl:
            host[name] = {"ms_per_step": round(ms / args.steps, 3), "avg_us": round(ms / nl * 1e3, 3), "calls": nl}
    # counts over the timed steps: activation layers whose first kernels were
    # launched ahead of their claim point, walk steps proved a second time
    for kid, name in [(K_ACT_AHEAD, "activations_launched_ahead"), (K_WALK_RETRY, "walk_steps_retried")]:
        _, nl, _ = ctx.kernel_time(kid)
        host[name] = nl
    rc = kernels.get("restrict_cols")
    roofline = None
    if rc:
        ms, nl, nb = ctx.kernel_time(K_RESTRICT_COLS)
        ach = nb / (ms * 1e-3) / 1e9
        prof = "restrict_cols_traffic.md" if args.u32_weights else "restrict_cols8_traffic.md"
        traffic = measured_traffic(prof) if cfg is QWEN else None
        roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                    "kernel": "k_restrict_cols" if args.u32_weights else "k_restrict_cols8",
                    "avg_launch_us": rc["avg_us"], "bytes_per_launch": nb // nl,
                    "timed_launches": "every launch" if args.timing_all else
                    "every 8th launch (HIP start/end events carried in the kernel's dispatch)",
                    "bytes_basis": "B as the int8 copy" if not args.u32_weights else "B as u32",
                    "by_shape": restrict_by_shape(ctx, cfg, not args.u32_weights) if cfg is not None else None,
                    "traffic_source": f"profiles/{prof} (rocprofv3 PMC, qwen1)" if traffic else None}

    result = {
        "metric": METRIC,
        "value": round(elems / (ms_per_step * 1e-3) / 1e6, 1),
        "unit": "Melem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32-m31",
        "data": "synthetic (counter-mode SplitMix64; int8-range weights/activations, uniform-M31 LogUp inputs)",
        "config": {"workload": workload, "layers": n_layers, "tokens": tokens,
                   "weight_restriction": "u32" if args.u32_weights else "int8",
                   "matmul_elements_per_step": elems, "logup_tables": "2^16 (SiLU, softmax-exp)"},
        "runtime_env": {"HSA_ENABLE_INTERRUPT": os.environ.get("HSA_ENABLE_INTERRUPT")},
        "proved_tokens_per_s": round(tokens / (ms_per_step * 1e-3), 3) if tokens else None,
        "roofline": roofline,
        "kernels": kernels,
        "host": host,
        "driver": args.driver,
        "calls_ms_per_step": {k: round(v / args.steps * 1e3, 3) for k, v in CALL_TIME.items() if v},
        "host_poseidon_us_per_round": poseidon_round_us(),
        "proof": {"felts": digests[0][1], "sha256_16": sbuf.fingerprint(), "final_digest": hex(digests[0][0])},
    }
    cp, rd = ctx.bench_copy(1 << 32, 5)
    result["hbm_measured"] = {"copy_gbps": round(cp, 1), "read_gbps": round(rd, 1),
                              "note": "128-bit streaming copy (read+write) / read kernels over 4 GiB"}
    if rc:
        result["roofline"]["frac_of_measured_read"] = round(rc["gbps"] / rd, 4)
    if not args.no_cpu_baseline:
        log("[bench] timing CPU baseline sample")
        cb = cpu_baseline(args.config)
        cb["gpu_over_cpu"] = round(result["value"] / cb["value"], 1)  # same unit (Melem/s), same workload unit
        result["cpu_baseline"] = cb
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
