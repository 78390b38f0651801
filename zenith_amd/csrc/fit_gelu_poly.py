"""Coefficients of gelu_erf_fast (zk_common.hpp): the fp16 epilogues' erf-GELU.

GELU(x) = x Phi(x) = max(x, 0) - |x| Phi(-|x|), and the kernels evaluate
Phi(-a) = 2^p(a) with one v_exp_f32. p is a polynomial of degree DEG with
p(0) = -1 (Phi(0) = 1/2 exactly), fitted to log2 Phi(-a) on [0, A] by
weighted minimax, the discrete Chebyshev approximation solved as a linear
program: minimise t subject to |w(a_i) (p(a_i) - log2 Phi(-a_i))| <= t on
N Chebyshev points, with w(a) = a Phi(-a) ln 2, the first-order change of
|x| Phi(-|x|) per unit error in p, so that t bounds the absolute error of
the GELU value.

Run `python fit_gelu_poly.py` to print the coefficients (highest degree
first, as fp32 literals) and the fp32-evaluated error against the exact
GELU. Needs numpy and scipy; nothing in the library imports this file.
"""
import numpy as np
from scipy.optimize import linprog
from scipy.special import erf, log_ndtr

DEG, A, N = 5, 8.0, 4000


def fit(deg=DEG, upper=A, n=N):
    ln2 = np.log(2.0)
    a = np.sort(np.cos(np.linspace(0.0, np.pi, n)) * upper / 2 + upper / 2)
    f = log_ndtr(-a) / ln2                       # log2 Phi(-a)
    w = a * np.exp2(f) * ln2
    # p(a) = -1 + sum_k c_k a^k, k = deg .. 1; unknowns c and t
    V = np.vander(a, deg + 1)[:, :-1] * w[:, None]
    g = (f + 1.0) * w
    ones = np.ones((n, 1))
    A_ub = np.vstack([np.hstack([V, -ones]), np.hstack([-V, -ones])])
    b_ub = np.concatenate([g, -g])
    cost = np.zeros(deg + 1)
    cost[-1] = 1.0
    res = linprog(cost, A_ub=A_ub, b_ub=b_ub, bounds=[(None, None)] * (deg + 1), method="highs")
    assert res.success, res.message
    return np.append(res.x[:-1], -1.0).astype(np.float32), float(res.x[-1])


def gelu_fp32(coef, x):
    """gelu_erf_fast evaluated in fp32 (fma rounded once per step)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x)
    p = np.full_like(a, coef[0])
    with np.errstate(over="ignore", invalid="ignore"):
        for c in coef[1:]:
            p = (p.astype(np.float64) * a + np.float64(c)).astype(np.float32)
        e = np.exp2(p.astype(np.float64)).astype(np.float32)
        out = (-a.astype(np.float64) * e + np.maximum(x, 0)).astype(np.float32)
    return out, p


def exact_gelu(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


if __name__ == "__main__":
    coef, t = fit()
    print("p(a), highest degree first:")
    print(",\n".join("  %.9ef" % c for c in coef))
    x = np.linspace(-12, 12, 2_000_001, dtype=np.float32)
    out, _ = gelu_fp32(coef, x)
    print("minimax bound %.2e; fp32 max abs error on [-12, 12] %.2e" %
          (t, np.abs(out - exact_gelu(x)).max()))
