"""Constants baked into the HIP kernels, checked on the CPU against what defines them.

The erf-GELU of the fused post-attention kernels is Abramowitz & Stegun 7.1.26 rewritten in
y = |x| sqrt(log2(e)/2) (fewer operations).  The rescaled constants are read from the kernel source and
re-derived here from the published A&S coefficients; the kernel's formula, evaluated in float64 with those
constants, must then match the exact erf-GELU to A&S's error bound.  A mistyped digit, a dropped term or
a wrong rescaling fails one of the two checks.
"""

from __future__ import annotations

import math
import re
from pathlib import Path

import numpy as np
from scipy.special import erf

SRC = Path(__file__).resolve().parents[1] / "turbo-roformer_amd" / "csrc" / "trf_kernels.hip"

# Abramowitz & Stegun 7.1.26: erfc(z) = t (a1 + a2 t + ... + a5 t^4) e^(-z^2), t = 1/(1 + p z)
AS_P = 0.3275911
AS_A = (0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429)


def kernel_constants() -> dict[str, float]:
    text = SRC.read_text()
    found = dict(re.findall(r"constexpr float (kGelu\w+) = (-?[0-9.]+)f;", text))
    assert set(found) == {"kGeluC", "kGeluP", "kGeluA1", "kGeluA2", "kGeluA3", "kGeluA4", "kGeluA5"}, found
    return {k: float(v) for k, v in found.items()}


def test_gelu_constants_derive_from_abramowitz_stegun():
    c = kernel_constants()
    log2e = 1.0 / math.log(2.0)
    kc = math.sqrt(0.5 * log2e)
    k = 0.5 / kc
    assert math.isclose(c["kGeluC"], kc, rel_tol=1e-15)
    assert math.isclose(c["kGeluP"], AS_P / math.sqrt(log2e), rel_tol=1e-15)
    for i, a in enumerate(AS_A, start=1):
        assert math.isclose(c[f"kGeluA{i}"], k * a, rel_tol=1e-15), i


def test_gelu_formula_matches_exact_gelu():
    c = kernel_constants()
    x = np.concatenate([np.linspace(-12.0, 12.0, 400001), [0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0]])
    y = np.abs(x) * c["kGeluC"]
    t = 1.0 / (1.0 + c["kGeluP"] * y)
    p = c["kGeluA5"]
    for a in (c["kGeluA4"], c["kGeluA3"], c["kGeluA2"], c["kGeluA1"]):
        p = p * t + a
    got = np.maximum(x, 0.0) - y * t * p * np.exp2(-y * y)
    exact = 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))
    err = np.abs(got - exact)
    # A&S bound |erf error| <= 1.5e-7 becomes |GELU error| <= 0.5 |x| 1.5e-7; the GELU is never off by more
    # than 2.2e-7 in absolute terms, and large |x| gives x or (to far below float32 range) 0
    assert (err <= 0.5 * np.abs(x) * 1.5e-7 + 1e-12).all()
    assert err.max() <= 2.2e-7
    assert got[-2] == 30.0 and abs(got[-1]) < 1e-150
