"""Pins the oracle's restatement of internal/simd/simd.go and
internal/device/utils.go: the reference's own test values, then properties
that a plausible slip (a wrong coefficient, a dropped `k--`, rounding instead
of truncating) would break."""
import json
import math
import pathlib

import numpy as np
import pytest

KNOWN = json.loads((pathlib.Path(__file__).parent / "golden" /
                    "reference_known_answers.json").read_text())


def test_fast_math_reference_points(orc):
    # simd_test.go:72-103: within 5% relative (or 1e-3 absolute) at 11 points.
    case = KNOWN["fast_math"]
    for x in case["x"]:
        for fn, ref in ((orc.exp_fast, math.exp), (orc.tanh_fast, math.tanh)):
            got, want = fn(x), ref(x)
            diff = abs(got - want)
            rel = diff / (abs(want) or 1.0)
            assert diff <= case["abs_floor"] or rel <= case["rel_tol"], (fn, x, got, want)


def test_exp_fast_floor_semantics(orc):
    # k = floor(t) (truncate, then k-- for t < 0): the mantissa factor
    # ExpFast(x) / 2^floor(x*log2e) lies in [1, p(1)) with p(1) = 1.9888778.
    # Truncating without the decrement gives factors below 1 for x < 0.
    xs = np.linspace(-80, 80, 20001).astype(np.float32)
    got = orc.exp_fast_vec(xs).astype(np.float64)
    t = (xs * np.float32(1.442695)).astype(np.float32)
    k = np.floor(t.astype(np.float64))
    # exact negative integers take the k-- branch too: factor p(1)
    k = np.where((t < 0) & (t == np.floor(t)), k - 1, k)
    factor = got / np.exp2(k)
    assert factor.min() >= 1.0 - 1e-6 and factor.max() <= 1.9888779 + 1e-6


def test_exp_fast_error_bound(orc):
    # Max relative error of the cubic 2^f model is 0.56% (at f -> 1).
    xs = np.linspace(-60, 60, 40001).astype(np.float32)
    got = orc.exp_fast_vec(xs).astype(np.float64)
    rel = np.abs(got - np.exp(xs.astype(np.float64))) / np.exp(xs.astype(np.float64))
    assert 4.0e-3 < rel.max() <= 5.6e-3


def test_exp_fast_special_values(orc):
    assert orc.exp_fast(0.0) == 1.0
    assert orc.exp_fast(88.5) == np.float32(1e38)
    assert orc.exp_fast(-88.5) == 0.0
    # t = -1 exactly takes k = -2, f = 1: 0.25 * p(1)
    x = np.float32(-1.0) / np.float32(1.442695)
    if np.float32(x * np.float32(1.442695)) == np.float32(-1.0):
        assert abs(orc.exp_fast(float(x)) - 0.25 * 1.9888778) < 1e-6


def test_tanh_fast_properties(orc):
    xs = np.linspace(-6, 6, 12001).astype(np.float32)
    got = orc.tanh_fast_vec(xs).astype(np.float64)
    np.testing.assert_array_equal(got, -orc.tanh_fast_vec(-xs))      # odd
    assert np.all(got[xs > 4] == 1.0) and np.all(got[xs < -4] == -1.0)  # clamps
    inner = np.abs(xs) <= 4
    err = np.abs(got[inner] - np.tanh(xs[inner].astype(np.float64)))
    assert 1.5e-2 < err.max() <= 2.4e-2                                 # [3/2] Pade error
    # slope at 0 of x(27+x^2)/(27+9x^2) is 1
    assert abs(orc.tanh_fast(1e-4) / 1e-4 - 1.0) < 1e-6


def test_gelu_fast_properties(orc):
    xs = np.linspace(-8, 8, 4001).astype(np.float32)
    g = orc.gelu_fast(xs).astype(np.float64)
    gm = orc.gelu_fast(-xs).astype(np.float64)
    # odd tanh => gelu(x) - gelu(-x) = x
    np.testing.assert_allclose(g - gm, xs, atol=2e-6)
    exact = 0.5 * xs * (1 + np.tanh(math.sqrt(2 / math.pi) * (xs + 0.044715 * xs.astype(np.float64) ** 3)))
    assert np.all(np.abs(g - exact) <= 0.5 * np.abs(xs) * 2.4e-2 + 1e-6)


def test_softmax_fast_properties(orc):
    rng = np.random.default_rng(5)
    for n in (1, 7, 128, 1000):
        row = (rng.standard_normal(n) * 3).astype(np.float32)
        p = orc.softmax_fast(row)
        assert abs(float(p.sum(dtype=np.float64)) - 1.0) < 1e-5
        assert int(np.argmax(p)) == int(np.argmax(row))
        e = np.exp(row.astype(np.float64) - row.max())
        exact = e / e.sum()
        assert np.max(np.abs(p - exact) / exact) < 1.2e-2


def test_dot_and_matvec(orc):
    assert orc.dot(KNOWN["dot"]["a"], KNOWN["dot"]["b"]) == KNOWN["dot"]["want"]
    mat = np.array(KNOWN["matvec"]["mat"], np.float32)
    got = [orc.dot(r, KNOWN["matvec"]["vec"]) for r in mat]
    assert got == KNOWN["matvec"]["want"]


def test_vec_add(orc):
    c = KNOWN["vec_add"]
    assert orc.add(c["dst"], c["src"]).tolist() == c["want"]


def test_f16_known_and_truncation(orc):
    c = KNOWN["cast_f16"]
    assert [orc.f32_to_f16_bits(x) for x in c["x"]] == c["want_bits"]
    # truncation (not round-to-nearest): 1 + 3*2^-12 -> 0x3C00, RNE would give 0x3C01
    assert orc.f32_to_f16_bits(1.0 + 3 * 2 ** -12) == 0x3C00
    assert orc.f32_to_f16_bits(1.0 + 2 ** -10) == 0x3C01
    assert orc.f32_to_f16_bits(7e4) == 0x7BFF and orc.f32_to_f16_bits(-7e4) == 0xFBFF
    assert orc.f32_to_f16_bits(5e-5) == 0x0000 and orc.f32_to_f16_bits(-5e-5) == 0x8000
    assert orc.f32_to_f16_bits(float("nan")) == 0x7E00
    assert orc.f32_to_f16_bits(float("inf")) == 0x7C00
    rng = np.random.default_rng(3)
    for x in (rng.standard_normal(2000) * 100).astype(np.float32):
        h = orc.f32_to_f16_bits(float(x))
        back = orc.f16_bits_to_f32(h)
        # truncation moves toward zero by less than one half-precision ulp
        assert abs(back) <= abs(x) and abs(x) - abs(back) < abs(x) * 2 ** -10 + 1e-30
        assert np.float16(back).astype(np.float32) == np.float32(back)


@pytest.mark.parametrize("h", [0x0001, 0x03FF, 0x3C00, 0xC000, 0x7BFF, 0x7C00])
def test_f16_to_f32(orc, h):
    want = 0.0 if (h & 0x7C00) == 0 else float(np.array([h], np.uint16).view(np.float16)[0])
    assert orc.f16_bits_to_f32(h) == want
