"""Pins the oracle's restatement of internal/device/cpu_backend.go: the
reference's known answers, library routines (BLAS vs numpy float64) and
mathematical invariants of each op."""
import json
import math
import pathlib
import zlib

import numpy as np
import pytest

KNOWN = json.loads((pathlib.Path(__file__).parent / "golden" /
                    "reference_known_answers.json").read_text())
RNG = np.random.default_rng(11)


@pytest.fixture(autouse=True)
def _inputs_per_test(request):
    """Each test draws its random inputs from a seed of its own (derived from
    its name), so they do not depend on which tests ran before it."""
    global RNG
    RNG = np.random.default_rng([11, zlib.crc32(request.node.name.encode())])


def rand(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def test_device_test_known_answers(orc):
    c = KNOWN["add"]
    assert np.allclose(orc.add(c["a"], c["b"]).ravel(), c["want"], atol=c["tol"])
    c = KNOWN["mul"]
    assert np.allclose(orc.mul(c["a"], c["b"]).ravel(), c["want"], atol=c["tol"])
    c = KNOWN["scale"]
    assert np.allclose(orc.scale(c["a"], c["v"]).ravel(), c["want"], atol=c["tol"])
    c = KNOWN["layernorm"]
    got = orc.layernorm(c["x"], np.ones(4), np.zeros(4), c["eps"])
    assert np.allclose(got.ravel(), c["want"], atol=c["tol"])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_mul_is_matmul(orc, ta, tb):
    a, b = rand(37, 53), rand(53, 29)
    A = a.T.copy() if ta else a
    B = b.T.copy() if tb else b
    got = orc.mul(A, B, bool(ta), bool(tb))
    np.testing.assert_allclose(got, a.astype(np.float64) @ b, rtol=1e-5, atol=1e-5)


def test_linear_and_activations(orc):
    x, w, b = rand(20, 64), rand(64, 96, scale=0.3), rand(96)
    lin = x.astype(np.float64) @ w + b
    np.testing.assert_allclose(orc.linear(x, w, b), lin, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(orc.linear_activation(x, w, b, 2), np.tanh(lin), atol=2.5e-2)
    sm = orc.linear_activation(x, w, b, 3)
    np.testing.assert_allclose(sm.sum(1), 1.0, atol=1e-5)


def test_swiglu_identity_trick(orc):
    # swiglu_test.go:68-77,118-140: X = I, W = data -> silu(first half) * second half
    c = KNOWN["swiglu"]
    n, inter = c["n"], c["inter"]
    data = (np.arange(n * 2 * inter) % 100 / 10.0).astype(np.float32).reshape(n, 2 * inter)
    got = orc.linear_activation(np.eye(n, dtype=np.float32), data, np.zeros(2 * inter), 4)
    g, u = data[:, :inter].astype(np.float64), data[:, inter:].astype(np.float64)
    np.testing.assert_allclose(got, g / (1 + np.exp(-g)) * u, rtol=1e-6, atol=1e-5)


def test_layernorm_invariants(orc):
    x = rand(50, 768, scale=4.0) + 3.0
    y = orc.layernorm(x, np.ones(768), np.zeros(768), 1e-7).astype(np.float64)
    np.testing.assert_allclose(y.mean(1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y.var(1), 1.0, atol=1e-4)
    r = rand(50, 768)
    np.testing.assert_array_equal(orc.add_layernorm(x, r, np.ones(768), np.zeros(768), 1e-7),
                                  orc.layernorm(orc.add(x, r), np.ones(768), np.zeros(768), 1e-7))


def _naive_attention(q, k, v, b, s, heads, scale):
    hd = q.shape[1] // heads
    out = np.zeros(q.shape)
    for bi in range(b):
        for h in range(heads):
            rs, cs = slice(bi * s, (bi + 1) * s), slice(h * hd, (h + 1) * hd)
            sc = q[rs, cs].astype(np.float64) @ k[rs, cs].astype(np.float64).T * scale
            p = np.exp(sc - sc.max(1, keepdims=True))
            out[rs, cs] = (p / p.sum(1, keepdims=True)) @ v[rs, cs]
    return out


def test_attention_reference_case(orc):
    # attention_test.go:70-125 inputs, MSE <= 1e-3 against exact attention
    c = KNOWN["attention"]
    n = c["seq"] * c["heads"] * c["head_dim"]
    q = (np.arange(n) * 0.1).astype(np.float32).reshape(c["seq"], -1)
    k = ((n - np.arange(n)) * 0.1).astype(np.float32).reshape(c["seq"], -1)
    v = ((np.arange(n) % 3) * 0.5).astype(np.float32).reshape(c["seq"], -1)
    sc = 1 / math.sqrt(c["head_dim"])
    got = orc.attention(q, k, v, 1, c["seq"], c["heads"], sc)
    want = _naive_attention(q, k, v, 1, c["seq"], c["heads"], sc)
    assert np.mean((got - want) ** 2) <= c["mse_tol"]


def test_attention_vs_exact_and_invariants(orc):
    b, s, heads = 3, 50, 2
    q, k, v = (rand(b * s, heads * 64) for _ in range(3))
    got = orc.attention(q, k, v, b, s, heads, 0.125)
    want = _naive_attention(q, k, v, b, s, heads, 0.125)
    # only ExpFast's 0.56% weight error separates them
    assert np.abs(got - want).max() < 1.2e-2 * np.abs(v).max()
    # identical keys -> every score equal -> output = mean of V, exactly in weights
    kk = np.tile(k[:1], (b * s, 1))
    got = orc.attention(q, kk, v, b, s, heads, 0.125)
    means = np.concatenate([np.tile(v[i * s:(i + 1) * s].mean(0, dtype=np.float64), (s, 1))
                            for i in range(b)])
    np.testing.assert_allclose(got, means, atol=1e-5)


def test_attention_varlen_is_per_sequence(orc):
    lengths = np.array([5, 31, 64], np.int64)
    q, k, v = (rand(int(lengths.sum()), 128) for _ in range(3))
    got = orc.attention_varlen(q, k, v, lengths, 2, 0.125)
    off = 0
    for L in lengths:
        sl = slice(off, off + L)
        np.testing.assert_allclose(got[sl], orc.attention(q[sl], k[sl], v[sl], 1, L, 2, 0.125),
                                   atol=2e-6)
        off += L


def test_rope_invariants(orc):
    # rope_test.go:11-75 shape; properties of a rotation by pos*theta_i
    c = KNOWN["rope"]
    b, s, heads, hd = c["batch"], c["seq"], c["heads"], c["head_dim"]
    x = rand(b * s, heads * hd)
    y = orc.rope(x, b, s, heads, hd, c["base"])
    half = hd // 2
    xr, yr = x.reshape(b * s, heads, hd), y.reshape(b * s, heads, hd)
    # position 0 of every sequence is unrotated
    np.testing.assert_array_equal(yr[0::s], xr[0::s])
    # each (i, i + d/2) pair keeps its norm
    n0 = xr[..., :half] ** 2 + xr[..., half:] ** 2
    n1 = yr[..., :half].astype(np.float64) ** 2 + yr[..., half:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=2e-5, atol=1e-6)
    # relative position: <R_p u, R_r w> depends only on p - r
    u, w = rand(1, hd), rand(1, hd)
    uu = np.tile(u, (s, 1))
    ww = np.tile(w, (s, 1))
    ru = orc.rope(uu, 1, s, 1, hd, c["base"]).astype(np.float64)
    rw = orc.rope(ww, 1, s, 1, hd, c["base"]).astype(np.float64)
    dots = ru @ rw.T
    for delta in (0, 1, 7, 40):
        diag = np.diagonal(dots, offset=-delta)
        np.testing.assert_allclose(diag, diag[0], atol=2e-4)
    # the base is a real parameter: base 1000 and 10000 differ beyond pos 0
    assert not np.allclose(orc.rope(x, b, s, heads, hd, 1000.0), y)


def test_gather(orc):
    table = rand(30, 7)
    idx = np.array([0, 29, 3, 3], np.int64)
    np.testing.assert_array_equal(orc.gather(table, idx), table[idx])
