"""The device felt252 arithmetic (nine 29-bit limbs, R = 2^261; stwo-ml_amd/csrc/felt9.h and
poseidon9.h) compiled for the CPU and compared with the oracle's Poseidon: the same source the
Merkle kernels run, checked without a GPU.  Inputs include the field's edge values and
non-canonical representatives up to 8p (the bound the kernels rely on)."""
import ctypes as C
import os
import random
import subprocess

import numpy as np
import oracle as O
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "native", "felt9_host.cpp")
OUT = os.path.join(ROOT, "tests", "native", "_build", "libfelt9_host.so")
CLANG = "/opt/rocm/llvm/bin/clang++"
PF = (1 << 251) + 17 * (1 << 192) + 1


@pytest.fixture(scope="module")
def f9():
    deps = [SRC] + [os.path.join(ROOT, "stwo-ml_amd", "csrc", f) for f in
                    ("felt9.h", "poseidon9.h", "poseidon9_host.h", "poseidon.h", "felt252.h")]
    if not os.path.exists(OUT) or os.path.getmtime(OUT) < max(os.path.getmtime(d) for d in deps):
        if not os.path.exists(CLANG):
            pytest.skip("clang++ from ROCm not available")
        os.makedirs(os.path.dirname(OUT), exist_ok=True)
        subprocess.run([CLANG, "-O2", "-std=c++17", "-mbmi2", "-shared", "-fPIC", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include", "-o", OUT, SRC], check=True)
    lib = C.CDLL(OUT)
    P32 = C.POINTER(C.c_uint32)
    lib.f9_hash2.argtypes = [P32, P32, C.c_uint32, C.c_uint32, P32]
    lib.f9_chain.argtypes = [P32, P32, C.c_int, P32]
    lib.f9_mulmod.argtypes = [P32, P32, P32]
    return lib


def words(v):
    return np.array([(v >> (32 * i)) & 0xFFFFFFFF for i in range(8)], dtype=np.uint32)


def ptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def to_int(w):
    return sum(int(x) << (32 * i) for i, x in enumerate(w))


def hash2(lib, a, b, ka=0, kb=0):
    out = np.zeros(8, dtype=np.uint32)
    wa, wb = words(a), words(b)
    assert lib.f9_hash2(ptr(wa), ptr(wb), ka, kb, ptr(out)) == 0, "output not normalized"
    return to_int(out)


def test_hash2_matches_oracle(f9):
    rng = random.Random(3)
    edge = [0, 1, 2, PF - 1, PF - 2, (1 << 251) - 1, 1 << 124, (1 << 250) + 12345]
    cases = [(a, b) for a in edge for b in edge] + [(rng.randrange(PF), rng.randrange(PF)) for _ in range(150)]
    for a, b in cases:
        assert hash2(f9, a, b) == O.hades([a, b, 2])[0], (hex(a), hex(b))


def test_hash2_on_representatives_up_to_8p(f9):
    rng = random.Random(4)
    for t in range(64):
        a, b = rng.randrange(PF), rng.randrange(PF)
        assert hash2(f9, a, b, t % 8, t // 8) == O.hades([a, b, 2])[0]


def test_chained_hashes_stay_in_bounds(f9):
    x, y = 5, 7
    out = np.zeros(8, dtype=np.uint32)
    f9.f9_chain(ptr(words(x)), ptr(words(y)), 40, ptr(out))
    for _ in range(40):
        x, y = O.hades([x, y, 2])[0], x
    assert to_int(out) == x


def test_montgomery_product(f9):
    rng = random.Random(6)
    for _ in range(200):
        a, b = rng.randrange(PF), rng.randrange(PF)
        out = np.zeros(8, dtype=np.uint32)
        f9.f9_mulmod(ptr(words(a)), ptr(words(b)), ptr(out))
        assert to_int(out) == a * b % PF
