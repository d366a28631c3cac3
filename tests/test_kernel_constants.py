"""Constants baked into the HIP kernels, checked on the CPU against what defines them.

The erf-GELU of the split-bf16 post-attention kernel is Abramowitz & Stegun 7.1.26 rewritten in
y = |x| sqrt(log2(e)/2) (fewer operations).  The rescaled constants are read from the kernel source and
re-derived here from the published A&S coefficients; the kernel's formula, evaluated in float64 with those
constants, must then match the exact erf-GELU to A&S's error bound.  A mistyped digit, a dropped term or
a wrong rescaling fails one of the two checks.

The fp16 / bf16 post-attention kernel's GELU is x sigmoid(x P(min(x^2, 30))) with a cubic P: a minimax fit
of logit Phi, re-derived here as a linear program (minimise the largest weighted residual), whose
solution the kernel's constants must equal; the formula, evaluated with float32 rounding at every step,
must stay within 1.25e-5 of the exact GELU and saturate to x and -0 for large |x|.
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
    found = dict(re.findall(r"constexpr float (kGelu\w+) = (-?[0-9.]+(?:e[-+]?[0-9]+)?)f;", text))
    assert set(found) == {"kGeluC", "kGeluP", "kGeluA1", "kGeluA2", "kGeluA3", "kGeluA4", "kGeluA5",
                          "kGeluClamp", "kGeluL0", "kGeluL1", "kGeluL2", "kGeluL3"}, found
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


def _logistic_gelu_f32(x: np.ndarray, c: dict[str, float]) -> np.ndarray:
    """The kernel's gelu_logistic with float32 rounding after every operation (exp2 and the reciprocal
    rounded from float64, as the hardware's are within an ulp)."""
    f = np.float32
    x = x.astype(np.float32)
    x2 = np.minimum(x * x, f(c["kGeluClamp"]))
    p = f(c["kGeluL3"]) * x2 + f(c["kGeluL2"])
    p = p * x2 + f(c["kGeluL1"])
    p = p * x2 + f(c["kGeluL0"])
    with np.errstate(over="ignore"):  # 2^(large) = inf, as on the device
        e = np.exp2(-(x * p).astype(np.float64)).astype(np.float32)
    r = (1.0 / (f(1.0) + e).astype(np.float64)).astype(np.float32)
    return x * r


def test_logistic_gelu_constants_are_the_minimax_fit():
    from scipy.optimize import linprog
    from scipy.special import log_ndtr, ndtr

    c = kernel_constants()
    clamp = c["kGeluClamp"]
    assert clamp == 30.0
    # minimise t subject to |w(x) (x P(min(x^2, 30)) - logit Phi(x))| <= t on x in (0, 10], with
    # w = x Phi (1 - Phi), the GELU's sensitivity to z; P(x^2) = sum_k a_k x^2k (natural-log units)
    x = np.linspace(1e-4, 10.0, 6000)
    phi = ndtr(x)
    w = x * phi * (1.0 - phi)
    x2 = np.minimum(x * x, clamp)
    A = np.stack([w * x * x2**k for k in range(4)], 1)
    b = w * (log_ndtr(x) - log_ndtr(-x))
    ones = np.ones((len(x), 1))
    res = linprog(np.r_[np.zeros(4), 1.0], A_ub=np.vstack([np.hstack([A, -ones]), np.hstack([-A, -ones])]),
                  b_ub=np.concatenate([b, -b]), bounds=[(None, None)] * 4 + [(0, None)], method="highs")
    assert res.success
    log2e = 1.0 / math.log(2.0)
    for k in range(4):
        assert math.isclose(c[f"kGeluL{k}"], res.x[k] * log2e, rel_tol=1e-5, abs_tol=1e-9), k


def test_logistic_gelu_error_bound_and_saturation():
    c = kernel_constants()
    x = np.concatenate([np.linspace(-14.0, 14.0, 1400001), [0.0, 30.0, -30.0, 1e4, -1e4]])
    got = _logistic_gelu_f32(x, c).astype(np.float64)
    exact = 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))
    err = np.abs(got - exact)
    assert err.max() <= 1.25e-5
    # the error equioscillates (a minimax fit): near its largest value at several x of alternating sign
    grid = np.linspace(0.05, 8.0, 80001)
    e = _logistic_gelu_f32(grid, c).astype(np.float64) - 0.5 * grid * (1.0 + erf(grid / math.sqrt(2.0)))
    big = np.flatnonzero(np.abs(e) >= 0.9 * np.abs(e).max())
    assert len(set(np.sign(e[big]))) == 2
    assert got[-5] == 0.0 and got[-4] == 30.0 and got[-2] == 1e4
    assert abs(got[-3]) < 1e-30 and got[-1] == 0.0  # saturated below (-0 once 2^-z overflows)
