"""The config-5 oracle fixture (tests/golden/config5_oracle.json) on the CPU: its layout is consistent
(48 layers of equal length, the felt count, channel states in the reference's to_gpu_state layout),
and its first layer is reproduced by the oracle now (same SHA-256 and channel state), so the file
stays the oracle's proof of the bench's inputs.  The GPU proof is compared with it in
tests/test_gpu_configs.py."""
import hashlib
import json
import os
import sys

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import bench  # noqa: E402


def load():
    with open(os.path.join(HERE, "golden", "config5_oracle.json")) as f:
        return json.load(f)


def test_fixture_layout():
    ref = load()
    assert ref["n_layers"] == 48 == len(ref["layers"])
    per = ref["layers"][0]["felts"]
    assert all(L["felts"] == per for L in ref["layers"])
    assert ref["n_felts"] == 1 + 48 * per + 8
    assert all(len(L["state_after"]) == 11 and len(L["sha256"]) == 64 for L in ref["layers"])
    assert ref["final_state"] == ref["layers"][-1]["state_after"]


def test_fixture_first_layer_reproduced():
    """Layer 0 of the fixture from the oracle (about a minute on 8 cores)."""
    ref = load()
    och = O.Channel()
    och.mix_u64(ref["seed"])
    out = []
    bench.oracle_layer(O, och, bench.QWEN, 0, out)
    words = b"".join(int(v).to_bytes(32, "little") for v in out)
    assert len(out) == ref["layers"][0]["felts"]
    assert hashlib.sha256(words).hexdigest() == ref["layers"][0]["sha256"]
    assert O.channel_state(och) == ref["layers"][0]["state_after"]
