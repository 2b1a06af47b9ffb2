"""Shared pytest setup: markers, import paths and the built libraries."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "stwo-ml_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

PRODUCT_SO = os.path.join(ROOT, "stwo-ml_amd", "lib", "libgkr_mi355x.so")
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "liboracle.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")
    # Build what is missing (in the build container; the GPU box receives
    # the libraries prebuilt).
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)
    if not os.path.exists(PRODUCT_SO) and os.path.exists("/opt/rocm/bin/hipcc"):
        subprocess.run(["make", "-C", os.path.join(ROOT, "stwo-ml_amd")], check=True)


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(ROOT, "tests", "golden", "reference_vectors.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def gpu_ctx():
    import gkr_mi355x as G
    ctx = G.Context(0)
    yield ctx
    ctx.close()
