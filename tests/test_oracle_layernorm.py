"""Pins the oracle's restatement of the reference LayerNorm forward
(dnn/layers/layer_norm_layer.cu:26-63) on the CPU: closed forms, numpy
binary64 evaluation, the normalisation invariants and the affine relation.
A planted mistake (variance over C-1, eps outside the root, gamma and beta
swapped, a missing mean subtraction) fails one of these."""
import numpy as np
import pytest

from oracle import pyoracle as orc


def ln64(x, g=None, b=None, eps=1e-5):
    x = x.astype(np.float64)
    m = x.mean(axis=1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=1, keepdims=True)
    y = (x - m) / np.sqrt(v + eps)
    if g is not None:
        y = y * g.astype(np.float64) + b.astype(np.float64)
    return y


def test_closed_forms():
    # equal values: mean exact, deviations 0, y = beta
    x = np.full((1, 4), 0.5, np.float32)
    g = np.array([2.0, 3.0, 4.0, 5.0], np.float32)
    b = np.array([0.25, -1.0, 0.0, 7.0], np.float32)
    assert orc.layernorm(x, g, b).tolist() == [b.tolist()]
    # [1, 2, 3, 4]: mean 2.5, var 1.25
    y = orc.layernorm(np.array([[1, 2, 3, 4]], np.float32), eps=0.0)
    r = 1 / np.sqrt(1.25)
    np.testing.assert_allclose(y[0], [-1.5 * r, -0.5 * r, 0.5 * r, 1.5 * r], rtol=2e-7)
    # eps inside the root: var 1.25, eps 0.75 -> rstd = 1/sqrt(2)
    y = orc.layernorm(np.array([[1, 2, 3, 4]], np.float32), eps=0.75)
    np.testing.assert_allclose(y[0], np.array([-1.5, -0.5, 0.5, 1.5]) / np.sqrt(2.0), rtol=2e-7)


@pytest.mark.parametrize("C", [7, 64, 768, 1600])
def test_against_binary64(C):
    rng = np.random.default_rng(C)
    x = (rng.standard_normal((33, C)) * 3 + 1.5).astype(np.float32)
    g = rng.uniform(0.5, 1.5, C).astype(np.float32)
    b = rng.uniform(-1, 1, C).astype(np.float32)
    np.testing.assert_allclose(orc.layernorm(x), ln64(x), atol=2e-5)
    np.testing.assert_allclose(orc.layernorm(x, g, b), ln64(x, g, b), atol=4e-5)
    # normalisation invariants without the affine map
    y = orc.layernorm(x).astype(np.float64)
    np.testing.assert_allclose(y.mean(axis=1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y.var(axis=1), 1.0 - 1e-5 / (x.astype(np.float64).var(axis=1) + 1e-5), rtol=1e-4)


def test_affine_relation_and_bf16_rounding():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8, 100)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 100).astype(np.float32)
    b = rng.uniform(-1, 1, 100).astype(np.float32)
    plain = orc.layernorm(x)
    aff = orc.layernorm(x, g, b)
    # fma(y, g, b): one rounding of the exact y*g + b
    exact = plain.astype(np.float64) * g + b
    assert np.abs(aff - exact).max() <= np.abs(exact).max() * 2 ** -24 * 1.01
    yb = orc.layernorm(x, g, b, round_bf16=True)
    assert np.array_equal(yb, orc.bf16_to_f32(orc.f32_to_bf16(aff)).reshape(aff.shape))
