"""The host-side AVX2 QM31 routines (stwo-ml_amd/csrc/hostfield.h) that finish the last sumcheck
rounds on the host, against the pure-Python field (tests/qm31_py.py) on random and edge values:
products, sums and differences four at a time, the degree-2 product round, the degree-3
eq-weighted round, the halves' sums and the fold, at lengths that exercise the four-wide loop
and the scalar rest (no GPU)."""
import os
import random
import subprocess

import pytest
import qm31_py as Q

P = (1 << 31) - 1
HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "native", "hostfield_check.cpp")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("hf") / "hostfield_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-mavx2", "-mbmi2", "-o", exe, SRC], check=True)
    return exe


def run(exe, text):
    return subprocess.run([exe], input=text, capture_output=True, text=True, check=True).stdout.split("\n")


def rq(rng):
    edge = [0, 1, 2, P - 1, P - 2, 1 << 30, (1 << 31) - 3]
    return tuple(rng.choice(edge) if rng.random() < 0.2 else rng.randrange(P) for _ in range(4))


def fmt(vals):
    return " ".join(str(w) for q in vals for w in q)


def parse(line, n):
    w = [int(x) for x in line.split()]
    assert len(w) == 4 * n
    return [tuple(w[4 * i:4 * i + 4]) for i in range(n)]


def test_products_sums_differences(driver):
    rng = random.Random(1)
    n = 40
    x, y = [rq(rng) for _ in range(n)], [rq(rng) for _ in range(n)]
    out = run(driver, f"mul {n}\n{fmt(x)}\n{fmt(y)}\naddsub {n}\n{fmt(x)}\n{fmt(y)}\n")
    assert parse(out[0], n) == [Q.qmul(a, b) for a, b in zip(x, y)]
    assert parse(out[1], n) == [Q.qadd(a, b) for a, b in zip(x, y)]
    assert parse(out[2], n) == [Q.qsub(a, b) for a, b in zip(x, y)]


@pytest.mark.parametrize("half", [1, 3, 4, 7, 64, 129])
def test_rounds_and_fold(driver, half):
    rng = random.Random(half)
    a, b, c = ([rq(rng) for _ in range(2 * half)] for _ in range(3))
    r = rq(rng)
    txt = (f"product {half}\n{fmt(a)}\n{fmt(b)}\neq3 {half}\n{fmt(a)}\n{fmt(b)}\n{fmt(c)}\n"
           f"halves {half}\n{fmt(a)}\nfold {half}\n{fmt(a)}\n{fmt([r])}\n")
    out = run(driver, txt)
    lo, hi = range(half), range(half, 2 * half)

    def lin(v, i, t):  # v(i) + t (v(i + half) - v(i))
        return Q.qadd(v[i], Q.qmul((t, 0, 0, 0), Q.qsub(v[i + half], v[i])))
    want = []
    for t in range(3):
        s = (0, 0, 0, 0)
        for i in lo:
            s = Q.qadd(s, Q.qmul(lin(a, i, t), lin(b, i, t)))
        want.append(s)
    assert parse(out[0], 3) == want
    want = []
    for t in range(4):
        s = (0, 0, 0, 0)
        for i in lo:
            s = Q.qadd(s, Q.qmul(Q.qmul(lin(a, i, t), lin(b, i, t)), lin(c, i, t)))
        want.append(s)
    assert parse(out[1], 4) == want
    s0, s1 = (0, 0, 0, 0), (0, 0, 0, 0)
    for i in lo:
        s0 = Q.qadd(s0, a[i])
    for i in hi:
        s1 = Q.qadd(s1, a[i])
    assert parse(out[2], 2) == [s0, s1]
    assert parse(out[3], half) == [Q.qadd(a[i], Q.qmul(r, Q.qsub(a[i + half], a[i]))) for i in lo]
