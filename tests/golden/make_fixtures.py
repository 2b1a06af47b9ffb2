"""Extract the reference's golden vectors for this path into reference_vectors.json.

Run in the build container (where /root/reference exists):
    python3 tests/golden/make_fixtures.py
Only data is written: expected outputs and inputs that the reference's own
tests and artifacts hold.  Sources:
  - engine/tests/artifacts/sp3_matmul_only_proof.json (SP3 matmul-only GKR proof)
  - elo-cairo-verifier/tests/test_sp3_cross_language.cairo:87-115, 147-150, 205-206
    (proof data, post-walk channel digest, input-claim point)
  - stwo-gpu/crates/stwo/src/core/channel/poseidon252.rs:229-252 (mix_u64, mix_u32s KATs)
  - engine/src/crypto/poseidon_channel.rs:1619-1636 (mix_felts / starknet.js vector)
  - stwo-gpu/crates/stwo/src/core/fields/qm31.rs:150-170 (QM31 KATs)
  - elo-cairo-verifier/tests/test_field.cairo:14-142 (M31 / CM31 vectors)
  - engine/src/crypto/poseidon_constants.rs:98-191 (round constants: only a
    SHA-256 digest of the decimal list and the first/last value are kept)
  - engine/tests/artifacts/d10_verify_gkr_calldata.txt and d10_onchain_summary.json
    (MatMul -> LayerNorm -> MatMul on-chain calldata, e2e_cairo_verify.rs:312, 1479)
  - engine/scripts/deploy_policy_upgrade.mjs, engine/docs/ENV_VARS.md and
    elo-cairo-verifier/tests/test_model_gkr_contract.cairo (the policy
    presets' commitments)
"""
import hashlib
import json
import os
import re

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
P = (1 << 31) - 1


def read(rel: str) -> str:
    with open(os.path.join(REF, rel)) as f:
        return f.read()


def main() -> None:
    out = {}
    sp3 = json.loads(read("engine/tests/artifacts/sp3_matmul_only_proof.json"))
    out["sp3"] = {
        "source": "engine/tests/artifacts/sp3_matmul_only_proof.json",
        "input_data": sp3["input_data"],
        "output_data": sp3["output_data"],
        "model": sp3["model"],
        "calldata_hex": sp3["calldata_hex"],
        "weight_claims": sp3["weight_claims"],
        "weight_commitments": sp3["weight_commitments"],
        "io_commitment": sp3["io_commitment"],
        "final_channel_digest_after_openings": sp3["verification"]["final_channel_digest"],
    }
    cairo = read("elo-cairo-verifier/tests/test_sp3_cross_language.cairo")
    m = re.search(r"expected_digest: felt252 =\s*(0x[0-9a-fA-F]+);", cairo)
    out["sp3"]["post_walk_digest"] = m.group(1)
    pts = re.findall(r"let expected_p(\d) = qm31_new\((0x[0-9a-f]+), (0x[0-9a-f]+), (0x[0-9a-f]+), (0x[0-9a-f]+)\);",
                     cairo)
    out["sp3"]["input_claim_point"] = [[int(x, 16) for x in p[1:]] for p in sorted(pts)]
    out["sp3"]["cairo_source"] = "elo-cairo-verifier/tests/test_sp3_cross_language.cairo"

    p252 = read("stwo-gpu/crates/stwo/src/core/channel/poseidon252.rs")
    mu64 = re.search(r"fn test_mix_u64\(\).*?from_hex_be\(\s*\"(0x[0-9a-f]+)\"", p252, re.S).group(1)
    mu32 = re.search(r"fn test_mix_u32s\(\).*?from_hex_be\(\s*\"(0x[0-9a-f]+)\"", p252, re.S).group(1)
    chan = read("engine/src/crypto/poseidon_channel.rs")
    js = re.search(r"fn test_poseidon252_digest_matches_js_reference.*?from_hex_be\(\s*\"(0x[0-9a-f]+)\"", chan,
                   re.S).group(1)
    out["poseidon"] = {
        "mix_u64": {"value": 0x1111222233334444, "digest": mu64,
                    "source": "stwo-gpu/crates/stwo/src/core/channel/poseidon252.rs:229-240"},
        "mix_u32s": {"values": list(range(1, 10)), "digest": mu32,
                     "source": "stwo-gpu/crates/stwo/src/core/channel/poseidon252.rs:243-252"},
        "mix_felts_qm31_1234": {"value": [1, 2, 3, 4], "digest": js,
                                "packed": "0x10000000200000008000000180000004",
                                "source": "engine/src/crypto/poseidon_channel.rs:1619-1636"},
    }
    consts = re.findall(r"\"(\d{20,})\"", read("engine/src/crypto/poseidon_constants.rs"))
    out["hades_round_constants"] = {
        "count": len(consts),
        "sha256_of_decimal_list": hashlib.sha256(",".join(consts).encode()).hexdigest(),
        "first": consts[0],
        "last": consts[-1],
        "source": "engine/src/crypto/poseidon_constants.rs:98-191",
    }
    # QM31 KATs (qm31.rs:150-170) and M31/CM31 vectors (test_field.cairo)
    out["fields"] = {
        "qm31_mul": {"x": [1, 2, 3, 4], "y": [4, 5, 6, 7], "xy": [P - 71, 93, P - 16, 50],
                     "source": "stwo-gpu/crates/stwo/src/core/fields/qm31.rs:157-161"},
        "qm31_add": {"x": [1, 2, 3, 4], "y": [4, 5, 6, 7], "sum": [5, 7, 9, 11]},
        "qm31_neg": {"x": [1, 2, 3, 4], "neg": [P - 1, P - 2, P - 3, P - 4]},
        "qm31_sub": {"x": [1, 2, 3, 4], "y": [4, 5, 6, 7], "diff": [P - 3, P - 3, P - 3, P - 3]},
        "cm31_mul": {"x": [2, 3], "y": [4, 5], "xy": [P - 7, 22],
                     "source": "elo-cairo-verifier/tests/test_field.cairo"},
        "cm31_i_squared": {"x": [0, 1], "xx": [P - 1, 0]},
        "m31_inv2": {"x": 2, "inv": 0x40000000},
    }
    d10 = read("engine/tests/artifacts/d10_verify_gkr_calldata.txt").split()
    out["d10"] = {
        "source": "engine/tests/artifacts/d10_verify_gkr_calldata.txt",
        "model": "build_gkr_mlp_layernorm (engine/tests/e2e_cairo_verify.rs:312-351): 2x4 input "
                 "[[7,9,11,13],[17,19,21,23]], identity 4x4 W0, W2[i][j] = i+j+1 (4x2)",
        "verify_calldata": [int(x, 16) if x.startswith("0x") else int(x) for x in d10],
        "summary": json.loads(read("engine/tests/artifacts/d10_onchain_summary.json")),
    }
    # PolicyConfig::policy_commitment of the three presets, as the reference
    # records them in three places (the deployment script's table, the
    # environment-variable documentation, the Cairo contract tests)
    dep = read("engine/scripts/deploy_policy_upgrade.mjs")
    pol = {k: v for k, v in re.findall(r'^\s*(strict|standard|relaxed):\s*"(0x[0-9a-f]{64})"', dep, re.M)}
    doc = dict(re.findall(r"^(strict|standard|relaxed):\s+(0x[0-9a-f]{64})$", read("engine/docs/ENV_VARS.md"), re.M))
    cairo_t = read("elo-cairo-verifier/tests/test_model_gkr_contract.cairo")
    assert pol == doc and set(pol) == {"strict", "standard", "relaxed"}
    assert pol["strict"] in cairo_t and pol["standard"] in cairo_t
    out["policy"] = {
        "commitments": pol,
        "source": "engine/scripts/deploy_policy_upgrade.mjs:44-48, engine/docs/ENV_VARS.md:36-42, "
                  "elo-cairo-verifier/tests/test_model_gkr_contract.cairo:189, 249 "
                  "(PolicyConfig::policy_commitment, engine/src/policy.rs:236-254)",
    }
    with open(os.path.join(HERE, "reference_vectors.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print("wrote", os.path.join(HERE, "reference_vectors.json"))


if __name__ == "__main__":
    main()
