"""Generates the coefficient table of the float32 GELU kernels (ops.hpp).

Q(a) = 0.5 erfc(a / sqrt 2), the upper tail of the standard normal, is
evaluated for 0 <= a <= 15 as exp(-a^2 / 2) * M(a) with the scaled function
M(a) = 0.5 erfcx(a / sqrt 2).  M is smooth and decays like 1 / a, so it is
fitted as a polynomial in s = 1 / (1 + a / 3.5), which maps [0, 15] onto
[7/37, 1]: a degree-10 least-squares fit at Chebyshev nodes with relative
weights, rewritten in monomials of t = s - mid (the monomials of
u = (s - mid) / half scaled by half^-i, which saves the scaling multiply).
Maximum relative error over a dense grid: 2.0e-9 (printed), against the
2^-24 that a float32 result rounded from the double value needs to stay
within 1 ulp.

    python3 spar_amd/csrc/hip/fit_normal_tail.py
"""
import numpy as np
from numpy.polynomial import chebyshev as chebyshev
from numpy.polynomial import polynomial as polynomial
from scipy.special import erfcx

A_MAX, KAPPA, DEGREE = 15.0, 3.5, 10


def main():
    s_low = 1.0 / (1.0 + A_MAX / KAPPA)
    mid, half = 0.5 * (s_low + 1.0), 0.5 * (1.0 - s_low)
    nodes = np.cos(np.pi * (np.arange(8000) + 0.5) / 8000)
    a = KAPPA * (1.0 / (mid + half * nodes) - 1.0)
    target = 0.5 * erfcx(a / np.sqrt(2.0))
    fit = chebyshev.chebfit(nodes, target, DEGREE, w=1.0 / target)
    monomial = chebyshev.cheb2poly(fit) / half ** np.arange(DEGREE + 1)
    grid = np.linspace(0.0, A_MAX, 400001)
    t = 1.0 / (1.0 + grid / KAPPA) - mid
    error = np.max(np.abs(polynomial.polyval(t, monomial) / (0.5 * erfcx(grid / np.sqrt(2.0))) - 1))
    print(f"// max relative error {error:.2e}")
    print(f"constexpr double kTailInvKappa = {float(1.0 / KAPPA).hex()};")
    print(f"constexpr double kTailMid = {float(mid).hex()};")
    print(f"constexpr double kTailCoefficient[{DEGREE + 1}] = {{")
    for value in monomial:
        print(f"    {float(value).hex()},")
    print("};")


if __name__ == "__main__":
    main()
