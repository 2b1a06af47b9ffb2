"""Write the CPU oracle's whole config-5 proof fingerprint into config5_oracle.json.

Config 5 is 48 Qwen2.5-14B-shaped layers, 64 tokens. This script
runs the oracle, which restates the reference's CPU prover algorithm, over the bench's own
synthetic inputs (bench.oracle_host_layer: the same SplitMix64 generator and seeds as
bench.LayerWeights). It uses one Poseidon channel seeded with mix_u64(7) and the per-layer
sequence of bench.model_steps. For every layer it records:
  - the SHA-256 of the layer's serialized felts, as 8 little-endian u32 words per felt (the
    `gkr_proof_serialize` word layout);
  - the felt count;
  - the channel state after the layer (the reference's to_gpu_state layout, 11 words).
It also records the SHA-256 of the whole serialized proof: the layer count, the 432 layer
proofs and the tail (no input-claim point, a zero input-claim value, no weight commitments,
no openings, a zero IO commitment).

It is deterministic and needs no GPU. It takes about 45 minutes on 8 cores and reads nothing
from the reference:
    python3 tests/golden/make_config5_fixture.py
The GPU test `test_config5_qwen_48_layers` compares the GPU proof with this file, layer by
layer.
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import bench  # noqa: E402
import oracle as O  # noqa: E402

SEED = 7
N_LAYERS = 48
OUT = os.path.join(HERE, "config5_oracle.json")


def words(felts) -> bytes:
    """felt252 ints -> the serializer's little-endian 32-byte words."""
    return b"".join(int(v).to_bytes(32, "little") for v in felts)


def main() -> None:
    t_all = time.time()
    och = O.Channel()
    och.mix_u64(SEED)
    steps_per_layer = 9  # q k v o gate up SiLU down softmax
    whole = hashlib.sha256(words([N_LAYERS * steps_per_layer]))
    layers = []
    n_total = 1
    for layer in range(N_LAYERS):
        t0 = time.time()
        out = []
        bench.oracle_layer(O, och, bench.QWEN, layer, out)
        w = words(out)
        whole.update(w)
        n_total += len(out)
        layers.append({"felts": len(out), "sha256": hashlib.sha256(w).hexdigest(),
                       "state_after": O.channel_state(och)})
        print(f"layer {layer}: {len(out)} felts, {time.time() - t0:.1f} s", flush=True)
    # tail: in_point count 0, in_value (4 zero felts), 0 weight commitments, 0 openings, io_commitment 0
    tail = [0] * 8
    whole.update(words(tail))
    n_total += len(tail)
    res = {
        "what": "CPU oracle proof of BASELINE config 5 (48 Qwen2.5-14B layers, 64 tokens) on the bench's "
                "synthetic inputs, channel mix_u64(7), fresh claims, step order q k v o gate up SiLU down "
                "softmax-exp; felts as 8 LE u32 words",
        "generator": "tests/golden/make_config5_fixture.py",
        "seed": SEED,
        "n_layers": N_LAYERS,
        "n_felts": n_total,
        "proof_sha256": whole.hexdigest(),
        "final_state": O.channel_state(och),
        "layers": layers,
        "oracle_seconds": round(time.time() - t_all, 1),
    }
    with open(OUT, "w") as f:
        json.dump(res, f, indent=1)
    print("wrote", OUT, res["proof_sha256"], n_total, flush=True)


if __name__ == "__main__":
    np.seterr(all="ignore")
    main()
