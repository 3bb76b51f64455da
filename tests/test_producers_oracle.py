"""Pins of the producer-side q8 oracle (oracle/producers.py), CPU only: the seeded Newton square
root against the correctly rounded sqrt and the reference's 24-step fallback, the ordered sum of
squares against an exact sum, the reference's exp against the library exp within its stated
accuracy (1e-9 relative on [-20, 20]) and at its clamps, and the RMSNorm closed form."""

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import formats, producers


def test_seeded_newton_sqrt():
    rng = np.random.default_rng(0)
    v = np.exp(rng.uniform(math.log(1e-9), math.log(1e9), 20000))
    for x in v:
        got = producers._sqrt_ref(x)
        y = x
        for _ in range(24):
            y = 0.5 * (y + x / y)
        assert got == y  # the reference's claim for [1e-9, 1e9]: same fixed point as 24 steps
        assert abs(got - math.sqrt(x)) <= 2 * math.ulp(math.sqrt(x))
    assert producers._sqrt_ref(0.0) == 0.0
    # outside the seeded range: 24 steps from y = v, which have not converged from that far
    # (sqrt(4e12) comes out 2000000.2069...): the reference's value, kept as is
    y = 4e12
    for _ in range(24):
        y = 0.5 * (y + 4e12 / y)
    assert producers._sqrt_ref(4e12) == y and abs(y - 2e6) > 0.2


def test_ordered_sum_of_squares():
    rng = np.random.default_rng(1)
    x = rng.integers(-1000, 1000, 5120).astype(np.float64)  # every partial sum exact
    assert producers.rms_scale(x) == float(np.sum(x * x))
    x = rng.standard_normal(3000)
    exact = float(sum(Fraction(v) * Fraction(v) for v in x))
    assert abs(producers.rms_scale(x) - exact) <= 1e-13 * exact


def test_vexp_accuracy_and_clamps():
    x = np.linspace(-20, 20, 40001)
    got = producers.vexp(x)
    want = np.exp(x)
    assert np.max(np.abs(got - want) / want) < 1e-9
    assert producers.vexp(np.array([0.0]))[0] == 1.0
    assert producers.vexp(np.array([25.0]))[0] == producers.vexp(np.array([20.0]))[0]
    assert producers.vexp(np.array([-40.0]))[0] == producers.vexp(np.array([-20.0]))[0]


def test_rms_norm_closed_form_and_q8():
    # x = c * ones: sum x^2 / N = c^2, so y = w * c / sqrt(c^2 + eps)
    N, c, eps = 512, 0.5, 0.0
    w = np.linspace(-1, 1, N)
    y, y32, q, d = producers.rms_norm(np.full(N, c), w, eps)
    np.testing.assert_allclose(y, w, rtol=1e-15)
    q2, d2 = formats.quant_q8_act(y32)
    np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(d, d2)


def test_silu_mul_against_library_sigmoid():
    rng = np.random.default_rng(2)
    g = rng.uniform(-15, 15, 4096)
    u = rng.standard_normal(4096)
    h, h32, q, d = producers.silu_mul(g, u)
    want = g / (1.0 + np.exp(-g)) * u
    assert np.max(np.abs(h - want) / np.maximum(np.abs(want), 1e-300)) < 1e-8
    assert h32.dtype == np.float32 and q.dtype == np.int8 and d.size == 128
