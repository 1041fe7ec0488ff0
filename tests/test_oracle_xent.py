"""Pins of the oracle's LM-head cross entropy (oracle/llattn_oracle.py:cross_entropy_rows) on the CPU:
closed forms, a library log-sum-exp, finite differences and torch's argmax tie rule."""
import numpy as np
import pytest
from scipy.special import logsumexp

from oracle.llattn_oracle import cross_entropy_rows


def test_uniform_logits_give_log_v():
    V = 1000
    x = np.full((3, V), 2.5)
    t = np.array([0, 17, V - 1])
    loss, pred, grad = cross_entropy_rows(x, t)
    np.testing.assert_allclose(loss, np.log(V), rtol=0, atol=1e-12)
    assert (pred == 0).all()  # ties: the first index
    want = np.full((3, V), 1.0 / V)
    want[np.arange(3), t] -= 1.0
    np.testing.assert_allclose(grad, want, atol=1e-15)


def test_two_classes_softplus():
    d = np.array([-30.0, -1.5, 0.0, 2.0, 40.0])
    x = np.stack([np.zeros_like(d), d], axis=1)  # target 0: loss = log(1 + e^d)
    loss, pred, grad = cross_entropy_rows(x, np.zeros(5, dtype=np.int64))
    np.testing.assert_allclose(loss, np.logaddexp(0.0, d), rtol=1e-12, atol=1e-15)  # log(1 + 1e-13) in float64
    np.testing.assert_allclose(grad[:, 1], 1.0 / (1.0 + np.exp(-d)), rtol=1e-12)
    np.testing.assert_allclose(grad.sum(axis=1), 0.0, atol=1e-12)
    assert list(pred) == [0, 0, 0, 1, 1]


def test_random_rows_against_logsumexp_and_finite_differences():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(6, 37)) * 4.0
    t = rng.integers(0, 37, size=6)
    t[2] = -100  # ignored
    loss, pred, grad = cross_entropy_rows(x, t)
    want = logsumexp(x, axis=1) - x[np.arange(6), np.where(t < 0, 0, t)]
    want[2] = 0.0
    np.testing.assert_allclose(loss, want, rtol=1e-12, atol=1e-12)
    assert (pred == x.argmax(axis=1)).all()
    assert (grad[2] == 0).all()
    eps = 1e-6
    for r, j in ((0, 3), (4, int(t[4])), (5, 36)):
        xp, xm = x.copy(), x.copy()
        xp[r, j] += eps
        xm[r, j] -= eps
        fd = (cross_entropy_rows(xp, t)[0][r] - cross_entropy_rows(xm, t)[0][r]) / (2 * eps)
        assert fd == pytest.approx(grad[r, j], abs=1e-7)
