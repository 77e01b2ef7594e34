#!/usr/bin/env python3
"""Derives the constants of the table-driven fp64 tanh in fastmath.h.

2^f for f in [-1/256, 1/256] is p(f) = 1 + f q(f), q a cubic interpolating
(2^f - 1) / f at the four Chebyshev nodes of the interval (near-minimax);
the table holds 2^(j/128), j = 0..127, correctly rounded. Everything is
computed with 60-digit decimal arithmetic and rounded to fp64 once. Prints
the C++ initialisers and the interpolant's worst relative error on a dense
grid (evaluated in exact arithmetic from the rounded coefficients).
"""
from decimal import Decimal, getcontext

getcontext().prec = 60
LN2 = Decimal(2).ln()


def exp2(x):
    return (x * LN2).exp()


def q_true(f):
    if f == 0:
        return LN2
    return (exp2(f) - 1) / f


def cheb_cubic(h):
    """Coefficients c1..c4 of q(f) = c1 + c2 f + c3 f^2 + c4 f^3 through the
    Chebyshev nodes of [-h, h] (Newton divided differences)."""
    import math
    nodes = [Decimal(math.cos((2 * k + 1) * math.pi / 8)) * h for k in range(4)]
    ys = [q_true(x) for x in nodes]
    n = 4
    coef = list(ys)
    for j in range(1, n):
        for i in range(n - 1, j - 1, -1):
            coef[i] = (coef[i] - coef[i - 1]) / (nodes[i] - nodes[i - j])
    # expand the Newton form into monomials
    poly = [Decimal(0)] * n
    basis = [Decimal(1)]
    for k in range(n):
        for d, b in enumerate(basis):
            poly[d] += coef[k] * b
        nb = [Decimal(0)] * (len(basis) + 1)
        for d, b in enumerate(basis):
            nb[d + 1] += b
            nb[d] -= nodes[k] * b
        basis = nb
    return poly


def main():
    h = Decimal(1) / 256
    c = [float(x) for x in cheb_cubic(h)]
    table = [float(exp2(Decimal(j) / 128)) for j in range(128)]
    worst = Decimal(0)
    for k in range(-4000, 4001):
        f = h * k / 4000
        p = 1 + f * (Decimal(c[0]) + f * (Decimal(c[1]) + f * (Decimal(c[2]) + f * Decimal(c[3]))))
        worst = max(worst, abs(p / exp2(f) - 1))
    print("// q(f) coefficients c1..c4:", ", ".join(repr(x) for x in c))
    print("// worst relative error of p:", f"{float(worst):.3e}")
    print("constexpr double kExp2Tab128[128] = {")
    for j in range(0, 128, 4):
        print("    " + ", ".join(repr(t) for t in table[j:j + 4]) + ",")
    print("};")


if __name__ == "__main__":
    main()
