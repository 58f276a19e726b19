"""Pins the oracle's restatement of the reference FC loops (CPU only).

dnn/layers/fully_connected_layer.cu:14-106 (kernel order: sequential fp32
sums, bias last, dW/db overwritten) and the GTest host oracle
tests/layers/fully_connected_layer_test.cu:29-81 (bias first).
Checked against the reference's own known-answer case, closed forms and a
float64 numpy product; a planted mistake in the oracle (transposed W, bias
dropped, dW not overwritten) fails one of these.
"""
import json
import os

import numpy as np

from oracle import pyoracle as orc

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "fp8_golden.json")))


def test_reference_known_answer():
    """NonzeroInputGivesNonzeroOutput (fully_connected_layer_test.cu:258-284)."""
    kat = GOLDEN["fc_kat"]
    X = np.array(kat["x"], np.float32)
    W = np.array(kat["W"], np.float32)
    b = np.array(kat["b"], np.float32)
    y = orc.fc_forward(X, W, b)
    assert y.tolist() == kat["y_fp32"]
    assert orc.fc_forward(X, W, b, bias_first=True).tolist() == kat["y_fp32"]


def test_forward_pass_shapes_like_reference():
    """ForwardPass / DifferentDimensions: in=4/out=3 and in=5/out=2, input i/in."""
    rng = np.random.default_rng(0)
    for fin, fout in ((4, 3), (5, 2)):
        x = (np.arange(fin, dtype=np.float32) / fin).reshape(1, fin)
        W = rng.uniform(-1, 1, (fout, fin)).astype(np.float32)
        b = rng.uniform(-1, 1, fout).astype(np.float32)
        y = orc.fc_forward(x, W, b)
        ref = (x.astype(np.float64) @ W.T.astype(np.float64)) + b
        np.testing.assert_allclose(y, ref, atol=1e-5)  # the reference test's tolerance
        np.testing.assert_allclose(orc.fc_forward(x, W, b, bias_first=True), ref, atol=1e-5)


def test_backward_pass_like_reference():
    """BackwardPass: grad j/out; dX = dY.W; for N=1, dW = outer(dY, x), db = dY."""
    rng = np.random.default_rng(1)
    fin, fout = 4, 3
    x = (np.arange(fin, dtype=np.float32) / fin).reshape(1, fin)
    W = rng.uniform(-1, 1, (fout, fin)).astype(np.float32)
    dy = (np.arange(fout, dtype=np.float32) / fout).reshape(1, fout)
    dx = orc.fc_backward_input(dy, W)
    np.testing.assert_allclose(dx, dy.astype(np.float64) @ W.astype(np.float64), atol=1e-5)
    dw = orc.fc_backward_weights(dy, x)
    assert np.array_equal(dw, np.outer(dy[0], x[0]).astype(np.float32))
    assert np.array_equal(orc.fc_backward_bias(dy), dy[0])


def test_against_float64_products():
    rng = np.random.default_rng(2)
    N, K, O = 37, 53, 29
    X = rng.standard_normal((N, K)).astype(np.float32)
    W = rng.standard_normal((O, K)).astype(np.float32)
    b = rng.standard_normal(O).astype(np.float32)
    dY = rng.standard_normal((N, O)).astype(np.float32)
    X64, W64, dY64 = (a.astype(np.float64) for a in (X, W, dY))
    np.testing.assert_allclose(orc.fc_forward(X, W, b), X64 @ W64.T + b, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(orc.fc_backward_input(dY, W), dY64 @ W64, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(orc.fc_backward_weights(dY, X), dY64.T @ X64, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(orc.fc_backward_bias(dY), dY64.sum(0), rtol=1e-5, atol=1e-4)


def test_sequential_order_and_bias_last():
    """The kernel order sums in k order then adds the bias (:29-35); the
    GTest oracle starts from the bias (:38-42).  Chosen values make the two
    orders differ in binary32, so swapping them is caught."""
    X = np.array([[1.0, 1e-8, -1.0]], np.float32)
    W = np.array([[1.0, 1.0, 1.0]], np.float32)
    b = np.array([1e8], np.float32)
    last = orc.fc_forward(X, W, b)[0, 0]
    first = orc.fc_forward(X, W, b, bias_first=True)[0, 0]
    s = np.float32(0)
    for v in (np.float32(1.0), np.float32(1e-8), np.float32(-1.0)):
        s = np.float32(s + v)
    assert last == np.float32(s + np.float32(1e8))
    a = np.float32(1e8)
    for v in (np.float32(1.0), np.float32(1e-8), np.float32(-1.0)):
        a = np.float32(a + v)
    assert first == a


def test_threaded_equals_single_thread():
    rng = np.random.default_rng(3)
    X = rng.standard_normal((64, 96)).astype(np.float32)
    W = rng.standard_normal((80, 96)).astype(np.float32)
    dY = rng.standard_normal((64, 80)).astype(np.float32)
    assert np.array_equal(orc.fc_forward(X, W, None, threads=1), orc.fc_forward(X, W, None, threads=7))
    assert np.array_equal(orc.fc_backward_input(dY, W, threads=1), orc.fc_backward_input(dY, W, threads=5))
    assert np.array_equal(orc.fc_backward_weights(dY, X, threads=1), orc.fc_backward_weights(dY, X, threads=3))
