"""Derivation of the soft cap's tanh constants in qmm.hip (cap_tanh): the degree-5 polynomial Q
with tanh(y) ~ y + y^3 Q(y^2) for |y| < 0.625, fitted by least squares in a Chebyshev basis to
(tanh y / y - 1) / y^2 on [0, 0.625^2]; then the largest error of the whole formula (the series
below 0.625, 1 - 2 / (2^(2 log2(e) |y|) + 1) above) in a float32 simulation, in ulp of tanh.

    python3 softcap_tanh_fit.py
"""
import numpy as np
from numpy.polynomial import chebyshev

SWITCH = 0.625
DEGREE = 5


def fit():
    t = np.linspace(1e-12, SWITCH * SWITCH, 20001)
    y = np.sqrt(t)
    q = (np.tanh(y) / y - 1.0) / t
    cheb = chebyshev.Chebyshev.fit(t, q, DEGREE, domain=[0, SWITCH * SWITCH])
    return cheb.convert(kind=np.polynomial.Polynomial).coef  # c0 + c1 t + ...


def simulate(coef, y):
    """The device formula in float32 arithmetic (products rounded separately, exp2 and the
    reciprocal correctly rounded)."""
    y = y.astype(np.float32)
    c = [np.float32(v) for v in coef]
    t = (y * y).astype(np.float32)
    q = np.full_like(t, c[-1])
    for ci in reversed(c[:-1]):
        q = (q * t + ci).astype(np.float32)
    small = (y + (y * t).astype(np.float32) * q).astype(np.float32)
    a = np.abs(y)
    e = np.exp2((a * np.float32(2.885390082)).astype(np.float32).astype(np.float64)).astype(np.float32)
    big = (np.float32(1) - np.float32(2) * (np.float32(1) / (e + np.float32(1))).astype(np.float32)).astype(np.float32)
    return np.where(a < SWITCH, small, np.copysign(big, y))


if __name__ == "__main__":
    coef = fit()
    print("Q coefficients, c0 .. c5:", ", ".join("%.9e" % np.float32(c) for c in coef))
    y = np.concatenate([np.linspace(0, SWITCH, 200001), np.linspace(SWITCH, 12, 200001)]).astype(np.float32)
    want = np.tanh(y.astype(np.float64))
    ulp = np.maximum(np.spacing(np.abs(want).astype(np.float32)).astype(np.float64), 1e-45)
    print("largest error in float32 simulation: %.2f ulp" % np.max(np.abs(simulate(coef, y) - want) / ulp))
