"""Pins of the oracle's binary loss path by the mathematics, not by the
engine: the gradient and hessian it feeds the tree builder (est:2861,
2873-2874), the training log-loss it records (est:2320-2325) and the
predict_proba sigmoid (est:3335).

* Known answers at F = 0 (p = 1/2, g = w(1/2 - y), h = w/4, loss ln 2) and
  at the clips (F beyond +-500; p clipped to [1e-15, 1 - 1e-15]).
* Inside a fit: every round's g and h equal the first and second
  finite-difference derivatives of the weighted per-row log-loss
  w (log(1 + e^F) - y F) at the F rebuilt by an independent traversal of the
  fitted trees; the recorded loss equals the unweighted mean of
  log(1 + e^F) - y F there (np.logaddexp, no clip in range).
* predict_proba equals scipy's expit of the traversed score.
"""
import math

import numpy as np
import pytest
from scipy.special import expit

from conftest import make_data
from oracle import model as om


def _traverse(X_bin, tree):
    """Leaf value of every row, by a vectorised walk from the root."""
    tf, tt, tv, tl, tr, nc, _ = tree
    n = X_bin.shape[0]
    node = np.zeros(n, np.int64)
    rows = np.arange(n)
    for _ in range(nc):
        f = tf[node]
        inner = f >= 0
        if not inner.any():
            break
        code = X_bin[rows, np.where(inner, f, 0)].astype(np.int64)
        nxt = np.where(code <= tt[node], tl[node], tr[node])
        node = np.where(inner, nxt, node)
    return tv[node]


def _scores_before_each_round(model):
    """F before round m (m = 0 .. T) from base_score and the trees."""
    F = np.full(model.X_bin_.shape[0], model.base_score_)
    out = [F.copy()]
    for tree in model.trees:
        F = F + model.learning_rate * _traverse(model.X_bin_, tree)
        out.append(F.copy())
    return out


def _row_loss(F, y, w):
    return w * (np.logaddexp(0.0, F) - y * F)


def test_known_answers_at_zero():
    y = np.array([0.0, 1.0, 0.0, 1.0])
    w = np.array([0.7, 2.5, 1.0, 1.0])
    F = np.zeros(4)
    g, h = np.empty(4), np.empty(4)
    om.binary_grad_hess(F, y, w, g, h)
    np.testing.assert_array_equal(g, w * np.array([0.5, -0.5, 0.5, -0.5]))
    np.testing.assert_array_equal(h, w * 0.25)
    assert om.binary_logloss(y, F) == pytest.approx(math.log(2.0), rel=1e-15)
    np.testing.assert_array_equal(om.binary_proba(F), 0.5)


def test_known_answers_at_the_clips():
    F = np.array([600.0, 600.0, -600.0, -600.0, 40.0])
    y = np.array([1.0, 0.0, 1.0, 0.0, 0.0])
    p = om.binary_proba(F)
    # F is clipped to +-500 before the exponential.
    np.testing.assert_array_equal(p[:4], expit(np.array([500.0, 500.0, -500.0, -500.0])))
    top = 1.0 - 1e-15   # the upper probability clip, as a double
    per_row = [-math.log(top),            # y=1, p rounds to 1 -> clipped to top
               -math.log1p(-top),         # y=0, p -> top
               -math.log(1e-15),          # y=1, p ~ 7e-218 -> clipped to 1e-15
               -math.log1p(-1e-15),       # y=0, p -> 1e-15
               -math.log1p(-top)]         # y=0, p = expit(40) rounds above top
    for k in range(5):
        got = om.binary_logloss(y[k:k + 1], F[k:k + 1])
        assert got == pytest.approx(per_row[k], rel=1e-14), k
    assert om.binary_logloss(y, F) == pytest.approx(np.mean(per_row), rel=1e-14)
    g, h = np.empty(5), np.empty(5)
    om.binary_grad_hess(F, y, np.ones(5), g, h)
    np.testing.assert_array_equal(g, p - y)
    assert np.all(h >= 0) and np.all(h[:4] < 1e-200)


def test_fit_round0_closed_form():
    """Balanced labels, no class weight: base score 0, so round 0 has
    g = 1/2 - y and h = 1/4 exactly."""
    X, _ = make_data(4000, 6, seed=21)
    y = np.zeros(4000, np.int64)
    y[np.random.default_rng(3).permutation(4000)[:2000]] = 1
    seen = []
    m = om.OracleGBM(n_estimators=2, max_depth=3, learning_rate=0.3, n_bins=63,
                     class_weight=None, random_state=0)
    m.fit(X, y, round_callback=lambda r, g, h, si, fi, t: seen.append((g.copy(), h.copy())))
    assert m.base_score_ == 0.0
    np.testing.assert_array_equal(seen[0][0], 0.5 - y)
    np.testing.assert_array_equal(seen[0][1], np.full(4000, 0.25))


@pytest.mark.parametrize("class_weight", [None, "balanced_sqrt", "balanced"])
def test_fit_grad_hess_are_loss_derivatives(class_weight):
    X, _ = make_data(3000, 8, seed=22, nan_frac=0.05)
    rng = np.random.default_rng(4)
    y = (rng.random(3000) < 0.12 + 0.3 * (np.nan_to_num(X[:, 0]) > 1)).astype(np.int64)
    seen = []
    m = om.OracleGBM(n_estimators=5, max_depth=4, learning_rate=0.4, n_bins=255,
                     class_weight=class_weight, random_state=1)
    m.fit(X, y, round_callback=lambda r, g, h, si, fi, t: seen.append((g.copy(), h.copy())))
    n1 = int(y.sum())
    if class_weight is None:
        w = np.ones(3000)
    else:
        power = 0.35 if class_weight == "balanced_sqrt" else 1.0
        w = np.where(y == 1, (3000 / (2 * n1)) ** power, (3000 / (2 * (3000 - n1))) ** power)
    Fs = _scores_before_each_round(m)
    eps1, eps2 = 1e-5, 1e-3
    for r, (g, h) in enumerate(seen):
        F = Fs[r]
        g_fd = (_row_loss(F + eps1, y, w) - _row_loss(F - eps1, y, w)) / (2 * eps1)
        h_fd = (_row_loss(F + eps2, y, w) - 2 * _row_loss(F, y, w)
                + _row_loss(F - eps2, y, w)) / eps2 ** 2
        np.testing.assert_allclose(g, g_fd, rtol=0, atol=1e-8 * w.max(), err_msg=f"g round {r}")
        np.testing.assert_allclose(h, h_fd, rtol=0, atol=1e-6 * w.max(), err_msg=f"h round {r}")
    # The recorded loss is unweighted (est:2320-2325), after each round.
    for r, loss in enumerate(m.train_loss_history_):
        F = Fs[r + 1]
        assert np.max(np.abs(F)) < 30  # the probability clip does not apply
        want = np.mean(np.logaddexp(0.0, F) - y * F)
        assert loss == pytest.approx(want, rel=1e-12), r


def test_predict_proba_is_sigmoid_of_traversed_score():
    X, y = make_data(2500, 7, seed=23, nan_frac=0.1)
    m = om.OracleGBM(n_estimators=6, max_depth=4, learning_rate=0.5, n_bins=100,
                     random_state=2).fit(X, y)
    F = _scores_before_each_round(m)[-1]
    p = m.predict_proba(X)
    np.testing.assert_allclose(p[:, 1], expit(F), rtol=0, atol=1e-14)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, rtol=0, atol=1e-15)
    np.testing.assert_array_equal(m.predict(X), (p[:, 1] > 0.5).astype(np.int64))
