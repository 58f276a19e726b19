"""Pins the oracle's restatement of the consumer side of dW (CPU only).

Gradient-norm clipping follows dnn/utils/clip_grad_norm.cu:13-67 and the Adam
update the float path of dnn/optimizers/adam_optimizer.cu:11-30,83-109.
Checked against the reference's own GTest expectations
(tests/optimizers/adam_optimizer_test.cu), closed forms of the recurrences,
numpy binary64 sums and exact special cases.  A planted mistake in the oracle
(beta1 and beta2 swapped, a missing bias correction, decoupled instead of
coupled weight decay, a clip applied at norm == max_norm, a binary32 norm
accumulator) fails one of these.
"""
import math

import numpy as np
import pytest

from oracle import pyoracle as orc

B1, B2, EPS = 0.9, 0.999, 1e-8


def f32(*a):
    return [np.array(x, np.float32) for x in a]


def adam(p, g, steps=1, lr=1e-3, wd=0.0, t0=1, clip_factor=1.0):
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for k in range(steps):
        orc.adam_step(p, g, m, v, t0 + k, lr=lr, beta1=B1, beta2=B2, eps=EPS, wd=wd, clip_factor=clip_factor)
    return p, m, v


# ---- the reference's GTest cases (adam_optimizer_test.cu) ----
def test_basic_update_moves_against_gradient():
    """BasicUpdate (:21-54): both tensors decrease; the first step of Adam
    moves each element by lr * g / (|g| + eps)."""
    p1, p2 = np.full(4, 1.0, np.float32), np.full(4, 2.0, np.float32)
    adam(p1, np.full(4, 0.1, np.float32))
    adam(p2, np.full(4, 0.2, np.float32))
    assert (p1 < 1.0).all() and (p2 < 2.0).all()
    assert p1[0] == pytest.approx(1.0 - 1e-3 * 0.1 / (0.1 + EPS), abs=1.2e-7)
    assert p2[0] == pytest.approx(2.0 - 1e-3 * 0.2 / (0.2 + EPS), abs=2.4e-7)


def test_momentum_and_rms_second_step_differs():
    """MomentumAndRMS (:56-84): a second step with the same gradient moves the
    parameter again."""
    p = np.full(4, 1.0, np.float32)
    g = np.full(4, 0.1, np.float32)
    m, v = np.zeros(4, np.float32), np.zeros(4, np.float32)
    orc.adam_step(p, g, m, v, 1)
    first = p.copy()
    orc.adam_step(p, g, m, v, 2)
    assert p[0] != first[0]


def test_learning_rate_change_scales_the_step():
    """LearningRateChange (:138-170): doubling lr doubles the (constant
    gradient) step."""
    p = np.full(4, 1.0, np.float32)
    g = np.full(4, 0.1, np.float32)
    m, v = np.zeros(4, np.float32), np.zeros(4, np.float32)
    orc.adam_step(p, g, m, v, 1, lr=1e-3)
    first = p.copy()
    orc.adam_step(p, g, m, v, 2, lr=2e-3)
    assert abs(p[0] - first[0]) > abs(first[0] - 1.0)
    assert (first[0] - p[0]) == pytest.approx(2 * (1.0 - first[0]), rel=1e-3)


def test_parameter_update_only_touches_listed_tensors():
    """ParameterUpdate (:172-214): a step over one tensor leaves another
    unchanged."""
    p1, p3 = np.full(4, 1.0, np.float32), np.full(4, 3.0, np.float32)
    adam(p1, np.full(4, 0.1, np.float32))
    before = p1.copy()
    adam(p3, np.full(4, 0.3, np.float32))
    assert np.array_equal(p1, before) and p3[0] != 3.0


# ---- closed forms ----
def test_weight_decay_is_coupled_l2():
    """WeightDecay (:86-112) plus the form of the decay: the reference adds
    wd*p to the gradient before the moments (L2, not decoupled AdamW).  With
    g = 0 the first step is lr * wd*p / (|wd*p| + eps) ~ lr, where AdamW
    would move lr*wd*p = 1e-4."""
    p, _, _ = adam(np.full(4, 1.0, np.float32), np.zeros(4, np.float32), wd=0.1)
    assert 1.0 - p[0] == pytest.approx(1e-3, abs=1.2e-7)  # ulp(1) bounds the rounding of p
    p, _, _ = adam(np.full(4, 1.0, np.float32), np.full(4, 0.1, np.float32), wd=0.1)
    assert 1.0 - p[0] > 0.0


def test_two_step_closed_form():
    """After gradients g1, g2 (m = v = 0 at the start):
    m_hat_2 = (b1 g1 + g2) / (1 + b1), v_hat_2 = (b2 g1^2 + g2^2) / (1 + b2)."""
    rng = np.random.default_rng(1)
    g1 = rng.standard_normal(4096).astype(np.float32)
    g2 = rng.standard_normal(4096).astype(np.float32)
    p = np.zeros(4096, np.float32)
    m, v = np.zeros_like(p), np.zeros_like(p)
    lr = 1e-3
    orc.adam_step(p, g1, m, v, 1, lr=lr)
    orc.adam_step(p, g2, m, v, 2, lr=lr)
    G1, G2 = g1.astype(np.float64), g2.astype(np.float64)
    b1, b2 = float(np.float32(B1)), float(np.float32(B2))  # the binary32 betas the step uses
    mh = (b1 * G1 + G2) / (1 + b1)
    vh = (b2 * G1 ** 2 + G2 ** 2) / (1 + b2)
    expect = -lr * G1 / (np.abs(G1) + EPS) - lr * mh / (np.sqrt(vh) + EPS)
    np.testing.assert_allclose(p, expect, rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(m, (1 - b1) * (b1 * G1 + G2), rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(v, (1 - b2) * (b2 * G1 ** 2 + G2 ** 2), rtol=1e-5, atol=1e-12)
    # beta1 and beta2 swapped in the recurrence moves p far beyond the tolerance
    swapped = -lr * G1 / (np.abs(G1) + EPS) - lr * ((b2 * G1 + G2) / (1 + b2)) / (
        np.sqrt((b1 * G1 ** 2 + G2 ** 2) / (1 + b1)) + EPS)
    assert np.abs(swapped - expect).max() > 1e-5  # vs a tolerance of ~3e-8 above


def test_constant_gradient_fixed_point():
    """With a constant gradient m_hat = g and v_hat = g^2 at every step, so
    each step moves lr * g / (|g| + eps)."""
    g = np.array([0.5, -0.25, 3.0, -7.0], np.float32)
    p, _, _ = adam(np.zeros(4, np.float32), g, steps=10)
    np.testing.assert_allclose(p, -10 * 1e-3 * np.sign(g), rtol=1e-5)


def test_bias_correction_exact_cases():
    for t in range(1, 25):
        assert orc.bias_correction(0.5, t) == 1.0 - 2.0 ** -t  # exact in binary32 up to t = 24
    assert orc.bias_correction(0.5, 25) == 1.0  # 1 - 2^-25: the tie rounds to even
    b = np.float32(0.9)
    assert orc.bias_correction(0.9, 1) == np.float32(1.0) - b  # Sterbenz: exact
    for t in (1, 7, 100, 1000, 10000):
        # RN32(b^t) is within half an ulp of b^t < 1 (3e-8); the subtraction is exact
        assert orc.bias_correction(0.999, t) == pytest.approx(1 - float(np.float32(0.999)) ** t, abs=3e-8)


def test_clip_factor_is_applied_to_the_gradient():
    """clip_factor f gives the same step as the gradient f*g."""
    g = np.array([0.5, -0.25, 3.0, -7.0], np.float32)
    f = np.float32(0.37)
    pa, ma, va = adam(np.ones(4, np.float32), g, steps=3, wd=0.01, clip_factor=float(f))
    pb, mb, vb = adam(np.ones(4, np.float32), (g * f).astype(np.float32), steps=3, wd=0.01)
    assert np.array_equal(pa, pb) and np.array_equal(ma, mb) and np.array_equal(va, vb)


# ---- norm and clip ----
def test_norm_closed_forms():
    assert orc.grad_norm(f32([3.0, 4.0])) == 5.0
    assert orc.grad_norm(f32([3.0], [4.0])) == 5.0
    assert orc.grad_norm([np.ones(1_000_000, np.float32)]) == 1000.0
    assert orc.grad_norm([np.zeros(0, np.float32)]) == 0.0
    assert orc.grad_norm_ref_f32(f32([3.0], [4.0])) == 5.0


def test_norm_matches_exact_sum():
    """binary32 squares summed exactly (math.fsum) then rounded once."""
    rng = np.random.default_rng(2)
    arrays = [rng.standard_normal(n).astype(np.float32) * s
              for n, s in ((1, 1.0), (1000, 1e-3), (8193, 10.0), (100_000, 1.0))]
    exact = math.sqrt(math.fsum(float(x) for a in arrays for x in (a * a).astype(np.float32)))
    assert orc.grad_norm(arrays) == np.float32(exact)


def test_reference_binary32_norm_and_its_error():
    """The reference's host loop sums in binary32 (clip_grad_norm.cu:40-48):
    exact on small integer data, within n*2^-24 relative otherwise, and
    stuck at 2^24 for 2^25 ones (a binary32 running sum stops growing), the
    case the binary64 accumulation of the product avoids."""
    assert orc.grad_norm_ref_f32([np.ones(4096, np.float32)]) == 64.0
    rng = np.random.default_rng(3)
    a = rng.standard_normal(20000).astype(np.float32)
    ours, ref = orc.grad_norm([a]), orc.grad_norm_ref_f32([a])
    assert abs(ours - ref) <= ours * 20000 * 2.0 ** -24
    big = np.ones(1 << 25, np.float32)
    assert orc.grad_norm_ref_f32([big]) == 4096.0
    assert orc.grad_norm([big]) == np.float32(math.sqrt(1 << 25))


def test_clip_scale_rules():
    g = np.array([3.0, 4.0], np.float32)
    assert orc.clip_scale(g, 5.0, 1.0)
    assert np.array_equal(g, np.array([3.0, 4.0], np.float32) * np.float32(np.float32(1.0) / np.float32(5.0)))
    assert orc.grad_norm([g]) == pytest.approx(1.0, rel=1e-6)
    h = np.array([3.0, 4.0], np.float32)
    assert not orc.clip_scale(h, 5.0, 5.0)  # norm == max_norm: unchanged
    assert not orc.clip_scale(h, 4.0, 5.0)
    assert not orc.clip_scale(h, float("nan"), 1.0)  # a NaN norm compares false
    assert np.array_equal(h, np.array([3.0, 4.0], np.float32))


# ---- delayed scaling: amax history (oracle dfo_history_push) ----
def test_history_push_closed_forms():
    """Newest first, oldest drops out; the next scale is FMAX-normalised
    max(history) under the D1/D2 rule (zero history -> scale 1)."""
    h = np.zeros(2, np.float32)
    assert orc.history_push(h, 0.0, 0) == 1.0
    assert orc.history_push(h, 1.0, 0) == np.float32(1.0) / np.float32(448.0)
    assert orc.history_push(h, 5.0, 0) == np.float32(5.0) / np.float32(448.0)
    assert h.tolist() == [5.0, 1.0]
    assert orc.history_push(h, 2.0, 0) == np.float32(5.0) / np.float32(448.0)  # 5 still inside
    assert h.tolist() == [2.0, 5.0]
    assert orc.history_push(h, 3.0, 1) == np.float32(3.0) / np.float32(57344.0)  # 5 dropped out
    one = np.zeros(1, np.float32)
    for a in (7.0, 0.5, 300.0):  # length 1 = most recent amax
        assert orc.history_push(one, a, 0) == np.float32(a) / np.float32(448.0)
