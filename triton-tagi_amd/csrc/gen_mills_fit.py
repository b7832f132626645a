"""Generates the polynomial constants of ``mills_differences`` in tagi_moments.h.

For x >= 2 the kernels need u1(x) = 1 - x R(x) and u2(x) = (1 + x^2) R(x) - x, where
R = Q / phi is the Mills ratio of the standard normal; both are small differences of
terms near 1 and x, so they are fitted directly instead of being formed from R. The
fitted functions are g1 = x^2 u1 and g2 = x^3 u2 / 2, which tend to 1 as x grows, as
polynomials in t = 1 / (1 + x / (2 sqrt 2)) (the variable of the erfc fit the kernels
already evaluate), t in (0, t(2)]. Method: least squares on 400 Chebyshev nodes in t of
values computed with mpmath at 90 digits, converted to the power basis in t. Prints the
constants and the worst relative error of the fit and of its float32 Horner evaluation
over x in [2, 1e5].

    python triton-tagi_amd/csrc/gen_mills_fit.py
"""

from __future__ import annotations

import mpmath as mp
import numpy as np

DEG1, DEG2 = 9, 10
mp.mp.dps = 90


def g12(x: float) -> tuple[float, float]:
    xm = mp.mpf(x)
    r = mp.erfc(xm / mp.sqrt(2)) / 2 / mp.npdf(xm)
    return float((1 - xm * r) * xm * xm), float(((1 + xm * xm) * r - xm) * xm ** 3 / 2)


def t_of(x):
    return 1.0 / (1.0 + x / (2.0 * np.sqrt(2.0)))


def x_of(t):
    return 2.0 * np.sqrt(2.0) * (1.0 / t - 1.0)


def fit():
    t0 = t_of(2.0)
    n = 400
    k = np.arange(n)
    t = np.maximum(t0 / 2 * (1 - np.cos(np.pi * (k + 0.5) / n)), 1e-5)
    g = np.array([g12(x_of(v)) for v in t])
    out = []
    for j, deg in enumerate((DEG1, DEG2)):
        c = np.polynomial.chebyshev.Chebyshev.fit(t, g[:, j], deg, domain=[0, t0])
        p = c.convert(kind=np.polynomial.Polynomial, domain=[0, t0], window=[0, t0])
        out.append(p.coef)
    return out


def horner32(coef, t):
    f = np.float32
    acc = np.full_like(t, f(coef[-1]), dtype=f)
    for c in coef[-2::-1]:
        acc = (acc.astype(np.float64) * t + f(c)).astype(f)  # fma: one rounding
    return acc


def main():
    c1, c2 = fit()
    for name, c in (("G1", c1), ("G2", c2)):
        print(f"{name} (t^0 .. t^{len(c) - 1}):")
        print(",\n".join(f"    {v:.9e}f" for v in c))
    xs = np.concatenate([np.linspace(2.0, 12.0, 3000), np.geomspace(12.0, 1e5, 300)])
    ex = np.array([g12(v) for v in xs])
    t64 = t_of(xs)
    t32 = (1.0 / (1.0 + (xs.astype(np.float32) * np.float32(1 / (2 * np.sqrt(2)))).astype(np.float32))).astype(
        np.float32)
    for j, c in enumerate((c1, c2)):
        fit_err = np.max(np.abs(np.polynomial.polynomial.polyval(t64, c) / ex[:, j] - 1))
        f32_err = np.max(np.abs(horner32(c, t32.astype(np.float64)) / ex[:, j] - 1))
        print(f"g{j + 1}: fit rel err {fit_err:.2e}, float32 Horner rel err {f32_err:.2e}")


if __name__ == "__main__":
    main()
