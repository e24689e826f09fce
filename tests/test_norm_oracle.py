"""CPU checks that pin orc_norm_rows, the float64 restatement of the
reference's q8-producing norm kernels (bruce.cu:541-641, 1110-1228).

Each check uses a property that a plausible slip breaks. Such slips include a
dropped eps, a norm taken before the op instead of after, swapped inputs, and a
sigmoid with the wrong sign:
- the output has the closed-form length |v|^2 = ss / (ss + eps);
- the output is parallel to the op result;
- scaling the inputs does not move the output;
- resid reduces to norm(x) at alpha = 0 and to norm(upd) at alpha = 1;
- gate reduces to norm(aout/2) at sg = 0, since sigmoid(0) = 1/2;
- the gate and silu products are restated with scipy.special.expit.
"""
import numpy as np
import pytest
from scipy.special import expit

EPS = float(np.float32(1e-6))


def rnd(oracle, seed, rows, n, mean=0.0, std=1.0):
    return oracle.gaussian(seed, rows * n, mean, std).reshape(rows, n)


def unit(t):
    """t / sqrt(sum t^2 + eps): what l2_scale(ss, n) = (1/sqrt(ss/n + eps/n)) / sqrt(n) applies."""
    t = np.asarray(t, np.float64)
    return t / np.sqrt((t * t).sum(-1, keepdims=True) + EPS)


@pytest.mark.parametrize("n", [32, 3072, 9216])
def test_norm_unit_length_and_direction(oracle, n):
    x = rnd(oracle, 1, 3, n)
    v = oracle.norm_rows("norm", x)
    ss = (x.astype(np.float64) ** 2).sum(-1)
    assert np.allclose((v * v).sum(-1), ss / (ss + EPS), rtol=1e-12)
    cos = (v * x).sum(-1) / np.sqrt((v * v).sum(-1) * (x.astype(np.float64) ** 2).sum(-1))
    assert np.allclose(cos, 1.0, rtol=1e-12)
    # eps matters only for tiny rows: a row of 1e-4 values has ss ~ n*1e-8
    tiny = np.full((1, n), 1e-4, np.float32)
    vt = oracle.norm_rows("norm", tiny)
    assert np.allclose(vt, unit(tiny), rtol=1e-12)
    s1 = n * float(np.float32(1e-4)) ** 2
    assert abs((vt * vt).sum() - s1 / (s1 + EPS)) < 1e-12


def test_norm_scale_invariance(oracle):
    x = rnd(oracle, 2, 2, 2560)
    a = oracle.norm_rows("norm", x)
    b = oracle.norm_rows("norm", x * np.float32(8.0))   # exact power-of-two scaling
    assert np.allclose(a, b, rtol=1e-9, atol=1e-12)


def test_add_is_norm_of_sum(oracle):
    x, h = rnd(oracle, 3, 2, 3072), rnd(oracle, 4, 2, 3072)
    v = oracle.norm_rows("add", x, h)
    assert np.allclose(v, unit(x.astype(np.float64) + h), rtol=1e-12, atol=1e-15)


def test_resid_special_cases(oracle):
    n = 3072
    x, u = rnd(oracle, 5, 2, n), rnd(oracle, 6, 2, n, 0.0, 3.0)
    zeros, ones = np.zeros(n, np.float32), np.ones(n, np.float32)
    assert np.allclose(oracle.norm_rows("resid", x, u, zeros), unit(unit(x)), rtol=1e-12, atol=1e-15)
    assert np.allclose(oracle.norm_rows("resid", x, u, ones), unit(unit(u)), rtol=1e-12, atol=1e-15)
    half = np.full(n, 0.5, np.float32)
    assert np.allclose(oracle.norm_rows("resid", x, u, half), unit(0.5 * (unit(x) + unit(u))), rtol=1e-12, atol=1e-15)


def test_gate_special_cases_and_expit(oracle):
    n = 4096
    a, g = rnd(oracle, 7, 2, n), rnd(oracle, 8, 2, n, 0.0, 2.0)
    sg = oracle.gaussian(9, n, 1.0, 0.3)
    assert np.allclose(oracle.norm_rows("gate", a, g, np.zeros(n, np.float32)), unit(0.5 * a.astype(np.float64)),
                       rtol=1e-12, atol=1e-15)
    ref = unit(a.astype(np.float64) * expit(g.astype(np.float64) * sg))
    assert np.allclose(oracle.norm_rows("gate", a, g, sg), ref, rtol=1e-10, atol=1e-14)


def test_silu_mul_expit(oracle):
    n = 9216
    g, u = rnd(oracle, 10, 2, n, 0.0, 2.0), rnd(oracle, 11, 2, n)
    sg, su = oracle.gaussian(12, n, 1.0, 0.3), oracle.gaussian(13, n, 1.0, 0.3)
    gv = g.astype(np.float64) * sg
    ref = unit(gv * expit(gv) * u * su)
    assert np.allclose(oracle.norm_rows("silu", g, u, sg, su), ref, rtol=1e-10, atol=1e-14)
    # silu(0) = 0: a zero gate row gives the zero row (eps keeps the scale finite)
    z = oracle.norm_rows("silu", np.zeros((1, n), np.float32), u[:1], sg, su)
    assert np.all(z == 0)
