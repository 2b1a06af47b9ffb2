"""Pure-Python M31/CM31/QM31 for brute-force checks on tiny inputs (tests only).

Written from the field definitions: CM31 = M31[i]/(i^2+1),
QM31 = CM31[u]/(u^2-(2+i)).  Values are 4-tuples (a, b, c, d).
"""
P = (1 << 31) - 1


def qadd(x, y):
    return tuple((a + b) % P for a, b in zip(x, y))


def qsub(x, y):
    return tuple((a - b) % P for a, b in zip(x, y))


def _cmul(a, b, c, d):
    return ((a * c - b * d) % P, (a * d + b * c) % P)


def qmul(x, y):
    lo = _cmul(x[0], x[1], y[0], y[1])
    hh = _cmul(x[2], x[3], y[2], y[3])
    rhh = ((2 * hh[0] - hh[1]) % P, (hh[0] + 2 * hh[1]) % P)  # (2 + i) * hh
    h1 = _cmul(x[0], x[1], y[2], y[3])
    h2 = _cmul(x[2], x[3], y[0], y[1])
    return ((lo[0] + rhh[0]) % P, (lo[1] + rhh[1]) % P, (h1[0] + h2[0]) % P, (h1[1] + h2[1]) % P)


ONE = (1, 0, 0, 0)
ZERO = (0, 0, 0, 0)


def qpow(x, e):
    r = ONE
    while e:
        if e & 1:
            r = qmul(r, x)
        x = qmul(x, x)
        e >>= 1
    return r


def qinv(x):
    # |QM31^*| = P^4 - 1
    return qpow(x, P**4 - 2)


def m31(v):
    return (v % P, 0, 0, 0)


def eq_weight(point, idx, n):
    """prod_l (bit_l(idx) ? r_l : 1 - r_l), r_0 on the most significant bit."""
    w = ONE
    for l in range(n):
        bit = (idx >> (n - 1 - l)) & 1
        w = qmul(w, point[l] if bit else qsub(ONE, point[l]))
    return w


def mle_bruteforce(evals, point):
    """sum_x evals[x] * eq(point, x) over the hypercube (direct Lagrange sum)."""
    n = len(point)
    acc = ZERO
    for x in range(1 << n):
        acc = qadd(acc, qmul(evals[x], eq_weight(point, x, n)))
    return acc
