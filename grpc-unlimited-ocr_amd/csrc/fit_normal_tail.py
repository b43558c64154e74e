"""Derives the polynomial the GELU kernel uses for the standard normal tail.

GELU(x) = x * Phi(x) with Phi the standard normal CDF. The kernel writes
Phi(x) = 1 - Q(|x|) for x >= 0 and Q(|x|) for x < 0, where
Q(t) = Phi(-t) = erfc(t / sqrt 2) / 2 is the upper tail, and evaluates
    Q(t) = 2^P(t),   P(t) ~ log2 Q(t)   for t in [0, T],
with P a degree-10 polynomial in Horner form and 2^y from the hardware's
v_exp_f32. P is the Chebyshev interpolant of log2 Q on [0, T] at 4000
Chebyshev nodes (a least-squares Chebyshev fit), converted to a power series
in t. For x < -T the kernel returns x * 0: the reference's
0.5 x (1 + erff(x / sqrt 2)) is exactly x * 0 there, because erff rounds to
-1 in fp32 once x < -5.44.

Error: P's fit error is below 1e-7 in log2 units; the fp32 evaluation of P
adds about |P| * 2^-24, so Q has relative error below 3e-6 and absolute
error below 3e-8 on [0, T]. Run this file to print the coefficients
(float32, ascending powers of t) and the resulting error of x * Phi(x) on a
dense grid.
"""

import numpy as np
import numpy.polynomial.chebyshev as C
from scipy.special import log_ndtr, ndtr

T = 5.5
DEGREE = 10


def coefficients(T=T, degree=DEGREE):
    k = np.arange(4000)
    xs = np.cos(np.pi * (k + 0.5) / 4000)
    ts = (xs + 1) * T / 2
    cheb = C.chebfit(xs, log_ndtr(-ts) / np.log(2.0), degree)
    in_x = np.polynomial.Polynomial(C.cheb2poly(cheb))
    in_t = in_x(np.polynomial.Polynomial([-1.0, 2.0 / T]))  # x = 2t/T - 1
    return in_t.coef.astype(np.float32)


def gelu_fp32(x, coef, T=T):
    """The kernel's arithmetic in float32 (each FMA rounded once)."""
    x = np.asarray(x, np.float32)
    t = np.minimum(np.abs(x), np.float32(T))
    acc = np.full_like(t, coef[-1])
    for c in coef[-2::-1]:
        acc = (acc.astype(np.float64) * t + np.float64(c)).astype(np.float32)
    q = np.exp2(acc.astype(np.float64)).astype(np.float32)
    phi = np.where(x >= 0, np.float32(1) - q, q).astype(np.float32)
    phi = np.where(x < -T, np.float32(0), phi)
    return (x * phi).astype(np.float32)


if __name__ == "__main__":
    coef = coefficients()
    for i, c in enumerate(coef):
        print(f"  c{i:<2d} = {float(c):.9e}f  ({np.float32(c).view(np.uint32):#010x})")
    x = np.linspace(-8, 8, 2_000_001).astype(np.float32)
    got = gelu_fp32(x, coef).astype(np.float64)
    want = x.astype(np.float64) * ndtr(x.astype(np.float64))
    err = np.abs(got - want)
    print(f"max |gelu err| = {err.max():.3e}, max err / max(1, |x|) = {(err / np.maximum(1, np.abs(x))).max():.3e}")
