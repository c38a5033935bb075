"""Multiclass softmax boosting (est:2949-3065; predict est:3293-3315).

CPU tests pin the oracle's multiclass loop by checks that do not restate
it: the recorded training loss equals the loss recomputed from the fitted
trees by the independent traversal; the K trees of a round share one
bagging draw, which equals a fresh RandomState's shuffle stream; softmax
gradients sum to zero over the classes of a row; the K-dependent parameter
rules give hand-derived values.  GPU tests rebuild every oracle tree on the
engine from the same inputs and compare the estimator's own trees, losses
and predict_proba with the oracle's, following certified gain ties
(tests/fitcmp.py).
"""
import numpy as np
import pytest

import fitcmp
from oracle import model as om


def _mc_data(n, F, K, seed, nan_frac=0.0):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, F)).astype(np.float32)
    W = rng.standard_normal((F, K))
    logits = X.astype(np.float64) @ W + 0.5 * rng.standard_normal((n, K))
    y = np.argmax(logits, axis=1)
    if nan_frac:
        X[rng.random((n, F)) < nan_frac] = np.nan
    labels = np.array([3, 7, 11, 20, 21, 40, 41, 50, 60, 70, 80, 90])[:K]
    return X, labels[y]


def _softmax(F):
    e = np.exp(F - F.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def test_oracle_multiclass_loss_matches_traversal():
    X, y = _mc_data(2500, 6, 3, seed=1)
    ref = om.OracleGBM(n_estimators=6, max_depth=4, n_bins=64, random_state=3).fit(X, y)
    K = 3
    assert ref._is_multiclass and len(ref.mc_trees) == K
    yi = np.searchsorted(ref.classes_, y)
    F = np.zeros((len(y), K))
    for k in range(K):
        packed = om.pack_trees(ref.mc_trees[k])
        F[:, k] = om.predict_all_trees(ref.X_bin_, packed, len(ref.mc_trees[k]), ref.learning_rate)
    p = np.clip(_softmax(F), 1e-15, 1 - 1e-15)
    loss = -np.mean(np.log(p[np.arange(len(y)), yi]))
    assert abs(loss - ref.train_loss_history_[-1]) <= 1e-12 * max(1.0, loss)
    assert ref.train_loss_history_[-1] < ref.train_loss_history_[0] < np.log(K)
    proba = ref.predict_proba(X)
    assert np.allclose(proba.sum(axis=1), 1.0)
    assert np.mean(ref.predict(X) == y) > 0.6


def test_oracle_multiclass_rounds_share_one_bagging_draw():
    X, y = _mc_data(3000, 8, 4, seed=2)
    seen = []
    om.OracleGBM(n_estimators=3, max_depth=3, n_bins=32, random_state=11).fit(
        X, y, round_callback=lambda m, k, g, h, si, fi, t: seen.append((m, k, g, h, si, fi)))
    assert [(m, k) for m, k, *_ in seen] == [(m, k) for m in range(3) for k in range(4)]
    rng = np.random.RandomState(11)
    rows = np.arange(3000, dtype=np.int64)
    feats = np.arange(8, dtype=np.int32)
    n_sub, f_sub = int(3000 * 0.8), int(8 * 0.8)
    for m in range(3):
        rng.shuffle(rows)
        rng.shuffle(feats)
        for k in range(4):
            _, _, g, h, si, fi = seen[4 * m + k]
            np.testing.assert_array_equal(si, rows[:n_sub])
            np.testing.assert_array_equal(fi, np.sort(feats[:f_sub]))
        gsum = sum(seen[4 * m + k][2] for k in range(4))
        assert np.max(np.abs(gsum)) <= 1e-12
        assert min(seen[4 * m + k][3].min() for k in range(4)) >= 1e-8


def test_oracle_multiclass_adaptive_parameters():
    """est:1925-2029 for K = 7 and K = 12 on 2000 rows (hand-derived)."""
    for K, depth, lr, n_est in [(7, 6, 0.20 * 0.85, 250), (12, 7, 0.20 * 0.75, 250)]:
        X, y = _mc_data(2000, 5, K, seed=K)
        m = om.OracleGBM(random_state=0)
        m.classes_ = np.unique(y)
        m.n_classes_ = K
        m._adaptive(X.astype(np.float64) * 0.1)
        assert (m.max_depth, m.n_estimators, m.max_leaves) == (depth, n_est, 31)
        assert m.learning_rate == lr


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("K,n,nan", [(3, 6000, 0.0), (7, 12000, 0.1)])
def test_multiclass_lockstep_and_end_to_end(engine, K, n, nan):
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    print(f"[case] multiclass K={K} n={n} nan={nan}", flush=True)
    X, y = _mc_data(n, 9, K, seed=K, nan_frac=nan)
    params = dict(n_estimators=4, max_depth=5, n_bins=255, random_state=5)
    est = HybridHistGBMNumbaV1_0_1(verbose=False, **params).fit(X, y)
    np.testing.assert_array_equal(est.classes_, np.unique(y))
    assert est._is_multiclass and len(est.mc_trees) == K
    ref, rep = fitcmp.follow_fit(engine, est, X, y, params)
    print(rep.line(f"multiclass K={K}"), flush=True)
    assert rep.rounds == params["n_estimators"]
    assert len(rep.end_to_end_ties) == K * params["n_estimators"]
    Xp, _ = _mc_data(3000, 9, K, seed=100 + K, nan_frac=nan)
    fitcmp.assert_fit_equal(ref, est, Xp)
    np.testing.assert_array_equal(est.predict(Xp), ref.predict(Xp))


@pytest.mark.gpu
def test_multiclass_host_path_matches_oracle(engine, monkeypatch):
    """More classes than the device rounds take keep the (n, K) arithmetic
    on the host (est:2949-3065 in NumPy, each tree through the builder seam);
    forced here for K = 3, that path too follows the oracle."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1, _native
    print("[case] multiclass host path K=3", flush=True)
    monkeypatch.setattr(_native, "MC_DEVICE_MAX_CLASSES", 0)
    X, y = _mc_data(6000, 9, 3, seed=3)
    params = dict(n_estimators=4, max_depth=5, n_bins=255, random_state=5)
    est = HybridHistGBMNumbaV1_0_1(verbose=False, **params).fit(X, y)
    ref, rep = fitcmp.follow_fit(engine, est, X, y, params)
    print(rep.line("multiclass host path K=3"), flush=True)
    assert rep.rounds == params["n_estimators"]
    Xp, _ = _mc_data(3000, 9, 3, seed=103)
    fitcmp.assert_fit_equal(ref, est, Xp)
