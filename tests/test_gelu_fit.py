"""The GELU kernel's tail polynomials against their derivation
(grpc-unlimited-ocr_amd/csrc/fit_normal_tail.py), on the CPU: the float32
coefficients written in act_math.hpp are the ones the fit produces, for both
degrees, and the errors the kernel's comments state hold for the kernel's
fp32 arithmetic."""

import importlib.util
import os
import re

import numpy as np

from conftest import PKG_DIR

CSRC = os.path.join(PKG_DIR, "csrc")


def _fit():
    spec = importlib.util.spec_from_file_location("fit_normal_tail", os.path.join(CSRC, "fit_normal_tail.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _kernel_coefficients():
    """{degree: float32 coefficients in ascending powers} from gelu_f in act_math.hpp."""
    src = open(os.path.join(CSRC, "act_math.hpp")).read()
    body = src[src.index("float gelu_f(float x)"):src.index("float gelu_of(float x)")]
    top = body[body.index("if constexpr (kDegree == 10) {"):]
    rest = top[top.index("} else {") + len("} else {"):]
    branches = {10: top[:top.index("} else {")], 6: rest[:rest.index("}")]}
    out = {}
    for degree, branch in branches.items():
        lits = re.findall(r"(-?\d\.\d+e[+-]\d+)f", branch)
        out[degree] = np.array([np.float32(v) for v in reversed(lits)], np.float32)  # Horner lists the top first
    return out


def test_kernel_coefficients_are_the_fit():
    fit = _fit()
    kern = _kernel_coefficients()
    for degree in (10, 6):
        want = fit.coefficients(fit.T, degree)
        assert len(kern[degree]) == degree + 1
        assert np.array_equal(kern[degree].view(np.uint32), want.view(np.uint32)), degree


def test_stated_error_bounds_hold():
    fit = _fit()
    bounds = {10: (1e-6, 3e-6, 1.4e-7, 1e-7), 6: (4e-5, 3e-5, 1.1e-5, 4e-6)}
    for degree, (p_b, q_b, phi_b, g_b) in bounds.items():
        p, q, phi, g = fit.errors(fit.coefficients(fit.T, degree))
        assert p < p_b and q < q_b and phi < phi_b and g < g_b, (degree, p, q, phi, g)
