"""The erf-GELU of the fp16 epilogues (gelu_erf_fast in zk_common.hpp), on
the CPU: its coefficients are the ones fit_gelu_poly.py derives, and the
fp32-evaluated form meets the accuracy its comment states against the exact
GELU x Phi(x) (scipy's erf), including the large-|x| behaviour that needs no
clamp. The kernels' own outputs are checked on the GPU against the oracle."""
import importlib.util
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "zenith_amd", "csrc")


def _fit_module():
    spec = importlib.util.spec_from_file_location("fit_gelu_poly", os.path.join(CSRC, "fit_gelu_poly.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _header_coefficients():
    src = open(os.path.join(CSRC, "zk_common.hpp")).read()
    body = src[src.index("float gelu_erf_fast(float x)"):]
    body = body[:body.index("\n}\n")]
    lits = re.findall(r"(-?\d\.\d+e[+-]\d+)f|(-1\.0)f\)", body)
    return np.array([float(a or b) for a, b in lits], dtype=np.float32)


def test_coefficients_are_the_fit():
    """The header holds the fit's coefficients. A different scipy / HiGHS
    release may land a coefficient one fp32 ulp away from the one in the
    header, which the comparison allows; the accuracy the kernels rely on is
    checked on the header's own coefficients below."""
    fit = _fit_module()
    coef, bound = fit.fit()
    hdr = _header_coefficients()
    assert hdr.shape == coef.shape == (fit.DEG + 1,)
    coef = np.asarray(coef, np.float32)
    assert np.all(np.abs(hdr - coef) <= np.spacing(np.maximum(np.abs(hdr), np.abs(coef)))), (hdr, coef)
    assert hdr[-1] == -1.0          # Phi(0) = 1/2 exactly
    assert bound < 5e-7


def test_accuracy_against_exact_gelu():
    fit = _fit_module()
    coef = _header_coefficients()
    x = np.linspace(-12, 12, 1_200_001, dtype=np.float32)
    out, _ = fit.gelu_fp32(coef, x)
    ex = fit.exact_gelu(x)
    assert np.abs(out - ex).max() <= 7.2e-7
    # relative accuracy near zero, where GELU(x) ~ x / 2
    s = np.concatenate([np.logspace(-30, 0, 200_001), -np.logspace(-30, 0, 200_001)]).astype(np.float32)
    outs, _ = fit.gelu_fp32(coef, s)
    exs = fit.exact_gelu(s)
    assert (np.abs(outs - exs) / np.abs(exs)).max() <= 6e-6
    assert fit.gelu_fp32(coef, np.float32(0.0))[0] == 0.0


def test_large_inputs_need_no_clamp():
    """p falls monotonically beyond the fitted range and 2^p underflows, so
    GELU(x) is max(x, 0) to far below fp32 resolution, for every finite x."""
    fit = _fit_module()
    coef = _header_coefficients().astype(np.float64)
    a = np.concatenate([np.linspace(8.0, 100.0, 100_001), np.logspace(2, 38.5, 100_001)])
    dp = np.polyval(np.polyder(coef), a)
    assert (dp < 0).all()
    x = np.concatenate([a, -a]).astype(np.float32)
    x = x[np.isfinite(x)]
    out, p = fit.gelu_fp32(_header_coefficients(), x)
    assert not np.isnan(out).any()
    assert p.max() < -52
    assert np.array_equal(out[x > 0], x[x > 0])
    assert (np.abs(out[x < 0]) <= 1e-14 * np.abs(x[x < 0])).all()
