"""The oracle's gated activations and argmax: the reference's own known answers and properties
(each names the reference test it follows, file:line), plus float64 closed forms.
"""
import math

import numpy as np
import pytest

import oracle as O

TINY = np.float32(np.finfo(np.float32).tiny)  # f32::MIN_POSITIVE


def swiglu_inputs(n):
    """tests/wave1_rope_swiglu_fidelity.rs:248-270: gate cycles -100, 100, 0, MIN_POSITIVE,
    -MIN_POSITIVE and (i % 41 - 20) * 0.45; up = 1.25 - (i % 5) * 0.5."""
    i = np.arange(n)
    g = ((i % 41).astype(np.float32) - np.float32(20.0)) * np.float32(0.45)
    g = np.where(i % 7 == 0, np.float32(-100.0), g)
    g = np.where(i % 7 == 1, np.float32(100.0), g)
    g = np.where(i % 7 == 2, np.float32(0.0), g)
    g = np.where(i % 7 == 3, TINY, g)
    g = np.where(i % 7 == 4, -TINY, g).astype(np.float32)
    u = (np.float32(1.25) - (i % 5).astype(np.float32) * np.float32(0.5)).astype(np.float32)
    return g, u


@pytest.mark.parametrize("n", [1, 7, 31, 137, 4864, 14336])
def test_swiglu_extreme_logits_against_float64(n):
    # tests/wave1_rope_swiglu_fidelity.rs:248-300 with the float64 SiLU as the reference and the
    # reference's tolerance max(1e-6, 1e-5 |y|)
    g, u = swiglu_inputs(n)
    out = O.swiglu_f32(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    silu = np.where(g64 < -20, 0.0, np.where(g64 > 20, g64, g64 / (1.0 + np.exp(-g64))))
    ref = silu * u64
    assert np.all(np.isfinite(out))
    assert np.all(np.abs(out - ref) <= np.maximum(1e-6, 1e-5 * np.abs(ref)))
    # the branches are exact: -100 -> 0 * up, 100 -> 100 * up
    i = np.arange(n)
    assert np.all(out[i % 7 == 1] == np.float32(100.0) * u[i % 7 == 1])
    assert np.all(out[i % 7 == 0] == 0.0)


def test_swiglu_random_against_float64():
    rng = np.random.default_rng(0)
    g = (rng.standard_normal(100000) * 6).astype(np.float32)
    u = rng.standard_normal(100000).astype(np.float32)
    out = O.swiglu_f32(g, u)
    g64 = g.astype(np.float64)
    ref = np.where(g64 < -20, 0.0, np.where(g64 > 20, g64, g64 / (1.0 + np.exp(-g64)))) * u.astype(np.float64)
    # each of the f32 steps rounds once: a few units in the last place of the result
    assert np.all(np.abs(out - ref) <= 4 * np.finfo(np.float32).eps * np.abs(ref) + 1e-30)


def test_relu_squared_kats():
    # tests/empirical_challenge_m3_bitnet.rs:299-378
    assert np.all(O.relu_squared_gate_f32(np.float32([-1000, -10, -1, -0.001, -1e-12, -1e-25]),
                                          np.float32([10, -5, 2, 0.5, 100, -100])) == 0.0)
    assert np.all(O.relu_squared_gate_f32(np.float32([0, -0.0, 0, -0.0]), np.float32([100, -50, 1e10, -1e10])) == 0.0)
    cases = [(0.5, 4.0, 1.0), (2.0, 3.0, 12.0), (3.0, -2.0, -18.0), (10.0, 0.05, 5.0), (100.0, 0.0001, 1.0),
             (1e4, 1e-8, 1.0)]
    out = O.relu_squared_gate_f32(np.float32([c[0] for c in cases]), np.float32([c[1] for c in cases]))
    assert np.all(np.abs(out - np.float32([c[2] for c in cases])) < 1e-5)
    # closed form: (relu * relu) * up, each product rounded to f32
    rng = np.random.default_rng(1)
    g, u = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    r = np.maximum(g, np.float32(0))
    assert np.array_equal(O.relu_squared_gate_f32(g, u).view(np.uint32), ((r * r) * u).astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("v", [32000, 128256, 151936, 152064, 262144])
def test_argmax_large_vocab(v):
    # tests/wave4_quant_gemv_and_argmax.rs:545-564
    x = np.full(v, -12.5, np.float32)
    x[0] = x[v // 2] = np.nan
    x[v // 3 + 7] = x[v - 19] = 99.75
    assert O.argmax_f32(x) == v // 3 + 7


def test_argmax_edge_cases():
    # lib.rs:555-568: None (-1) for empty / all-NaN, ties keep the first, +-0 compare equal,
    # -inf is a value
    assert O.argmax_f32(np.zeros(0, np.float32)) == -1
    assert O.argmax_f32(np.full(5, np.nan, np.float32)) == -1
    assert O.argmax_f32(np.float32([np.nan, -np.inf, np.nan])) == 1
    assert O.argmax_f32(np.float32([-0.0, 0.0, -1.0])) == 0
    assert O.argmax_f32(np.float32([-1.0, 0.0, -0.0])) == 1
    assert O.argmax_f32(np.float32([1.0, np.inf, 5.0, np.inf])) == 1
    rng = np.random.default_rng(2)
    for _ in range(20):
        x = rng.standard_normal(1000).astype(np.float32)
        x[rng.random(1000) < 0.05] = np.nan
        m = np.nanmax(x)
        assert O.argmax_f32(x) == int(np.flatnonzero(x == m)[0])


def test_epilogue_validation():
    assert O.status_of(O.swiglu_f32, np.zeros(0, np.float32), np.zeros(0, np.float32)) == 1
    assert O.status_of(O.relu_squared_gate_f32, np.zeros(0, np.float32), np.zeros(0, np.float32)) == 1
    assert math.isfinite(float(O.swiglu_f32(np.float32([20.0]), np.float32([1.0]))[0]))
