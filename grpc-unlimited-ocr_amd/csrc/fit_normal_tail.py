"""Derives the polynomials the GELU kernel uses for the standard normal tail.

GELU(x) = x * Phi(x) with Phi the standard normal CDF. The kernel writes
Phi(x) = 1 - Q(|x|) for x >= 0 and Q(|x|) for x < 0, where
Q(t) = Phi(-t) = erfc(t / sqrt 2) / 2 is the upper tail, and evaluates
    Q(t) = 2^P(t),   P(t) ~ log2 Q(t)   for t in [0, T],
with P a polynomial in Horner form and 2^y from the hardware's v_exp_f32:
degree 10 for fp32 activations, degree 6 for bf16 activations. P is the
Chebyshev interpolant of log2 Q on [0, T] at 4000 Chebyshev nodes (a
least-squares Chebyshev fit), converted to a power series in t and rounded
to float32. For x < -T the kernel returns x * 0: the reference's
0.5 x (1 + erff(x / sqrt 2)) is exactly x * 0 once fp32 erff rounds to -1
(x < -5.5426) and fp32 noise below 2e-7 in magnitude between there and -T.

Run this file to print both coefficient sets (float32, ascending powers of
t) and their errors, measured with the kernel's fp32 arithmetic on a dense
grid: the fit error of P in log2 units, the relative error of Q, the
absolute error of Phi and the error of x * Phi(x). Measured:
    degree 10: P 6.7e-7, Q 2.6e-6 relative, Phi 1.4e-7, x Phi 9.9e-8 max(1, |x|)
    degree  6: P 3.8e-5, Q 2.7e-5 relative, Phi 1.0e-5, x Phi 3.9e-6 max(1, |x|)
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


def errors(coef, T=T):
    """(fit error of P in log2 units, max relative error of Q, max absolute
    error of Phi, max error of x Phi(x) / max(1, |x|)), in fp32 arithmetic."""
    from scipy.special import ndtr

    t = np.linspace(0, T, 200_001)
    acc = np.full_like(t, coef[-1], dtype=np.float64)
    for c in coef[-2::-1]:
        acc = acc * t + np.float64(c)
    fit = float(np.max(np.abs(acc - log_ndtr(-t) / np.log(2.0))))
    x = np.linspace(-T, T, 4_000_001).astype(np.float32)
    tt = np.minimum(np.abs(x), np.float32(T))
    p = np.full_like(tt, coef[-1])
    for c in coef[-2::-1]:
        p = (p.astype(np.float64) * tt + np.float64(c)).astype(np.float32)
    q32 = np.exp2(p.astype(np.float64)).astype(np.float32)
    q = q32.astype(np.float64)
    q_want = ndtr(-tt.astype(np.float64))
    phi = np.where(x >= 0, np.float32(1) - q32, q32).astype(np.float64)  # 1 - q rounded to fp32
    x8 = np.linspace(-8, 8, 2_000_001).astype(np.float32)
    g = gelu_fp32(x8, coef, T).astype(np.float64) - x8.astype(np.float64) * ndtr(x8.astype(np.float64))
    return (fit, float(np.max(np.abs(q - q_want) / q_want)), float(np.max(np.abs(phi - ndtr(x.astype(np.float64))))),
            float(np.max(np.abs(g) / np.maximum(1.0, np.abs(x8)))))


if __name__ == "__main__":
    for degree in (10, 6):
        coef = coefficients(T, degree)
        print(f"degree {degree}:")
        for i, c in enumerate(coef):
            print(f"  c{i:<2d} = {float(c):.9e}f  ({np.float32(c).view(np.uint32):#010x})")
        fit, q, phi, g = errors(coef)
        print(f"  P {fit:.1e} log2, Q {q:.1e} relative, Phi {phi:.1e}, x Phi {g:.1e} max(1, |x|)")
