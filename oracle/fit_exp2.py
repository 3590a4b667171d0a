"""Provenance of the degree-5 exp2 polynomial of the fused pruning
(``exp2_neg`` in csrc/gr_prune.hip, restated in oracle/prune_ref.c).  Test
infrastructure: run by hand, nothing imports it.

Method: Remez exchange for the minimax *relative* error of 2^f on
[-1/2, 1/2] with p(0) = 1 fixed.  Writing p(f) = 1 + f q(f), the relative
error is (p(f) - 2^f) / 2^f = w(f) (q(f) - g(f)) with g(f) = (2^f - 1) / f
and weight w(f) = f 2^-f, so q (degree 4, five coefficients) is the weighted
minimax approximation of g: six alternation points of sign(q - g), the
exchange moving each to the extremum of |w (q - g)| in its sign run.  The
coefficients are then rounded to float32.

The script prints the minimax coefficients, their float32 roundings, and for
both that rounding and the shipped set: the polynomial's relative error in
exact arithmetic and the error of the shipped evaluation (Horner with fma in
float32) in float32 ulps of 2^f over a dense sample.  The shipped set equals
the rounded minimax in c0, c1, c2 and c4; c3 and c5 differ by 12 and 1,170
float32 ulps (the shipped set evaluates to 2.013 ulp at most, the plain
rounding to 2.020).

    python oracle/fit_exp2.py        (needs mpmath; about a minute)
"""

from __future__ import annotations

import struct

import mpmath as mp
import numpy as np

SHIPPED = ["0x1.000000p+0", "0x1.62e42ap-1", "0x1.ebf9bcp-3", "0x1.c6b746p-5", "0x1.3cea88p-7",
           "0x1.5bbea6p-10"]
M = 5  # coefficients of q


def _f32(x) -> float:
    return struct.unpack("f", struct.pack("f", float(x)))[0]


def _g(x):
    return (mp.power(2, x) - 1) / x if x != 0 else mp.log(2)


def _w(x):
    return x * mp.power(2, -x)


def _golden_max(fn, lo, hi, it=60):
    r = (mp.sqrt(5) - 1) / 2
    x1, x2 = hi - r * (hi - lo), lo + r * (hi - lo)
    for _ in range(it):
        if fn(x1) > fn(x2):
            hi, x2 = x2, x1
            x1 = hi - r * (hi - lo)
        else:
            lo, x1 = x1, x2
            x2 = lo + r * (hi - lo)
    return (lo + hi) / 2


def remez(iters: int = 8, grid: int = 600):
    """Weighted Remez exchange; returns q's coefficients and the levelled error."""
    mp.mp.dps = 30
    a, b = mp.mpf(-0.5), mp.mpf(0.5)
    xs = [(a + b) / 2 - (b - a) / 2 * mp.cos(mp.pi * (i + mp.mpf(0.37)) / (M + 0.74)) for i in range(M + 1)]
    c, lev = None, None
    for _ in range(iters):
        A, rhs = mp.matrix(M + 1, M + 1), mp.matrix(M + 1, 1)
        for i, x in enumerate(xs):  # q(x_i) - (-1)^i E / |w(x_i)| = g(x_i)
            for k in range(M):
                A[i, k] = x ** k
            A[i, M] = -(-1) ** i / abs(_w(x))
            rhs[i] = _g(x)
        s = mp.lu_solve(A, rhs)
        c, lev = [s[k] for k in range(M)], abs(s[M])

        def dev(x, c=c):
            return sum(c[k] * x ** k for k in range(M)) - _g(x)
        pts = [a + (b - a) * i / grid for i in range(grid + 1)]
        v = [dev(x) for x in pts]
        runs, cur = [], [0]
        for i in range(1, grid + 1):
            if (v[i] >= 0) == (v[cur[0]] >= 0):
                cur.append(i)
            else:
                runs.append(cur)
                cur = [i]
        runs.append(cur)
        best = [max(r, key=lambda i: abs(_w(pts[i]) * v[i])) for r in runs]
        new = [pts[i] if i in (0, grid) else
               _golden_max(lambda x: abs(_w(x) * dev(x)), pts[i - 1], pts[i + 1]) for i in best]
        if len(new) != M + 1:
            raise RuntimeError(f"{len(new)} alternation points, expected {M + 1}")
        xs = new
    return c, lev


def poly_rel_error(coef) -> float:
    """max |p(f) / 2^f - 1| on a dense grid, exact arithmetic (float64)."""
    f = np.linspace(-0.5, 0.5, 200001)
    return float(np.abs(np.polyval(coef[::-1], f) / np.exp2(f) - 1).max())


def f32_ulp_error(coef, n: int = 2000001) -> float:
    """max error of the float32 Horner-with-fma evaluation, in ulps of 2^f."""
    f = np.linspace(-0.5, 0.5, n).astype(np.float32)
    q = np.full_like(f, np.float32(coef[5]))
    for c in coef[4::-1]:  # one rounding per fma: exact product and sum in float64
        q = (q.astype(np.float64) * f.astype(np.float64) + np.float64(np.float32(c))).astype(np.float32)
    exact = np.exp2(f.astype(np.float64))
    return float((np.abs(q.astype(np.float64) - exact) / np.spacing(exact.astype(np.float32))).max())


def main() -> None:
    c, lev = remez()
    fitted = [1.0] + [_f32(x) for x in c]
    shipped = [float.fromhex(h) for h in SHIPPED]
    print(f"levelled relative error of the minimax: {mp.nstr(lev, 6)}")
    print("k  minimax (float64)          float32 rounding     shipped")
    for k in range(6):
        mm = 1.0 if k == 0 else float(c[k - 1])
        print(f"{k}  {mm!r:26} {fitted[k].hex():20} {shipped[k].hex()}")
    for name, coef in (("float32 rounding", fitted), ("shipped", shipped)):
        print(f"{name}: relative error {poly_rel_error(coef):.3e}, float32 evaluation "
              f"{f32_ulp_error(coef):.3f} ulp")


if __name__ == "__main__":
    main()
