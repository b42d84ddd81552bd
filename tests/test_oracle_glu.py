"""Pins the GLU oracle (oracle/glu.py) without a GPU: closed forms, symmetries and the
relations between the activations, none of them the oracle's own formula retyped."""
import math

import numpy as np
import pytest

from oracle import glu as G

X = np.linspace(-12.0, 12.0, 2401)


def test_swiglu_is_x_times_the_logistic():
    # silu(x) = x sigma(x); sigma(x) + sigma(-x) = 1, so silu(x) - silu(-x) = x
    s = G.act(G.SWIGLU, X)
    np.testing.assert_allclose(s - G.act(G.SWIGLU, -X), X, atol=1e-12)
    assert G.act(G.SWIGLU, np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(G.act(G.SWIGLU, np.array([math.log(3.0)])), [math.log(3.0) * 0.75], rtol=1e-15)


def test_gelu_forms():
    # erf GELU: x Phi(x), Phi the normal CDF; gelu(x) - gelu(-x) = x
    e = G.act(G.GEGLU_ERF, X)
    np.testing.assert_allclose(e - G.act(G.GEGLU_ERF, -X), X, atol=1e-12)
    phi1 = 0.8413447460685429                         # Phi(1), from the normal table
    np.testing.assert_allclose(G.act(G.GEGLU_ERF, np.array([1.0])), [phi1], rtol=1e-12)
    # the tanh form approximates it to < 1e-3 absolute everywhere (Hendrycks & Gimpel)
    assert np.abs(G.act(G.GEGLU, X) - e).max() < 1e-3
    np.testing.assert_allclose(G.act(G.GEGLU, X) - G.act(G.GEGLU, -X), X, atol=1e-12)
    # the quick form is x sigma(1.702 x): silu(1.702 x) / 1.702
    np.testing.assert_allclose(G.act(G.GEGLU_QUICK, X), G.act(G.SWIGLU, 1.702 * X) / 1.702, rtol=1e-12, atol=1e-300)


def test_tanh_gelu_against_torch():
    """the tanh form against torch's gelu(approximate='tanh') in float64: a wrong cubic
    coefficient or constant moves it by far more than 1e-12"""
    torch = pytest.importorskip("torch")
    ref = torch.nn.functional.gelu(torch.from_numpy(X), approximate="tanh").numpy()
    np.testing.assert_allclose(G.act(G.GEGLU, X), ref, rtol=1e-12, atol=1e-15)
    e = torch.nn.functional.gelu(torch.from_numpy(X)).numpy()
    np.testing.assert_allclose(G.act(G.GEGLU_ERF, X), e, rtol=1e-12, atol=1e-15)


def test_reglu_and_the_product():
    assert list(G.act(G.REGLU, np.array([-2.0, 0.0, 3.5]))) == [0.0, 0.0, 3.5]
    g = np.random.default_rng(1).standard_normal(50)
    u = np.random.default_rng(2).standard_normal(50)
    for op in (G.REGLU, G.GEGLU, G.SWIGLU, G.GEGLU_ERF, G.GEGLU_QUICK):
        np.testing.assert_allclose(G.glu(op, g, u), G.act(op, g) * u, rtol=0, atol=0)
        # large positive x: every activation is x to within e^-x terms
        np.testing.assert_allclose(G.act(op, np.array([30.0])), [30.0], rtol=1e-9)


def test_unknown_op():
    with pytest.raises(ValueError):
        G.act(3, X)                                   # SWIGLU_OAI is not taken
