"""JSON model format: save_model / load_model (est:4035-4205).

The CPU tests fill an estimator with a model fitted by the oracle and check
the written layout against the reference's (keys, value types), the
round trip, and the reference's reading rules: thresholds come back as
float64, a missing split_gains list becomes zeros, and the NaN-bin map is
reset to 'no NaN' (est:4200-4202).  The GPU test scores reloaded models.
"""
import json

import numpy as np
import pytest

from conftest import make_data
from oracle import model as om

from bsscl_gbm import HybridHistGBMNumbaV1_0_1

# Top-level keys the reference writes for a binary model (est:4044-4109).
REFERENCE_KEYS = {
    'version', 'params', 'n_classes_', 'classes_', 'n_features_in_', 'objective',
    '_is_multiclass', 'init_score_', 'base_score_', 'n_trees_fitted_',
    'best_iteration_', 'train_loss_history_', 'val_loss_history_', '_max_bins',
    'bin_edges', 'feature_bin_counts', 'trees', 'feature_importances_',
    'feature_split_counts_', '_categorical_set', '_is_categorical',
}
TREE_KEYS = {'features', 'thresholds', 'values', 'left', 'right', 'node_count', 'split_gains'}
PARAM_KEYS = {
    'n_estimators', 'max_depth', 'learning_rate', 'n_bins', 'reg_lambda',
    'min_samples_leaf', 'min_child_weight', 'gamma', 'subsample', 'colsample_bytree',
    'class_weight', 'monotone_constraints', 'categorical_features',
    'early_stopping_rounds', 'verbose', 'random_state',
}


def _fitted_from_oracle(X, y, **params):
    """An estimator carrying the fitted state of the oracle's model."""
    ref = om.OracleGBM(**params).fit(X, y)
    est = HybridHistGBMNumbaV1_0_1(verbose=False, **params)
    est.classes_ = ref.classes_
    est.n_classes_ = 2
    est.n_features_in_ = X.shape[1]
    est.base_score_ = float(ref.base_score_)
    est.trees = list(ref.trees)
    est.n_trees_fitted_ = len(ref.trees)
    est.train_loss_history_ = [float(v) for v in ref.train_loss_history_]
    est.bin_edges = ref.bin_edges
    est.feature_bin_counts = ref.feature_bin_counts
    est._max_bins = int(ref._max_bins)
    est._nan_bin_id = ref._nan_bin_id
    est.learning_rate = ref.learning_rate
    est._is_categorical = np.zeros(X.shape[1], dtype=bool)
    est._pack_trees()
    est._compute_feature_importances()
    return est, ref


def test_json_layout_and_round_trip(tmp_path):
    X, y = make_data(3000, 5, seed=4, nan_frac=0.1, nan_cols=[2])
    est, ref = _fitted_from_oracle(X, y, n_estimators=4, max_depth=4, n_bins=255,
                                   random_state=0)
    path = tmp_path / "model.json"
    est.save_model(str(path))
    data = json.loads(path.read_text())
    assert set(data) == REFERENCE_KEYS
    assert set(data['params']) == PARAM_KEYS
    assert data['version'] == '1.2.2'
    assert all(set(t) == TREE_KEYS for t in data['trees'])
    assert all(isinstance(v, int) for t in data['trees'] for v in t['thresholds'])

    m = HybridHistGBMNumbaV1_0_1.load_model(str(path))
    assert m.get_params() == est.get_params()
    np.testing.assert_array_equal(m.classes_, est.classes_)
    assert m.base_score_ == est.base_score_
    np.testing.assert_array_equal(m.bin_edges, est.bin_edges)
    np.testing.assert_array_equal(m.feature_bin_counts, est.feature_bin_counts)
    assert m._max_bins == est._max_bins
    assert m.train_loss_history_ == est.train_loss_history_
    for a, b in zip(m.trees, est.trees):
        assert a[1].dtype == np.float64          # the reference reads thresholds as float64
        for k in (0, 1, 2, 3, 4, 6):
            np.testing.assert_array_equal(a[k], b[k])
        assert a[5] == b[5]
    np.testing.assert_array_equal(m._packed_thresholds, est._packed_thresholds)
    assert m._packed_thresholds.dtype == np.int64
    np.testing.assert_array_equal(m._packed_values, est._packed_values)
    np.testing.assert_array_equal(m.feature_importances_, est.feature_importances_)
    # est:4200-4202: the NaN-bin map is not saved.
    assert np.all(m._nan_bin_id == -1) and np.any(est._nan_bin_id == 0)
    assert m.binning_strategy == 'standard'


def test_load_without_split_gains(tmp_path):
    X, y = make_data(2000, 4, seed=5)
    est, _ = _fitted_from_oracle(X, y, n_estimators=2, max_depth=3, n_bins=64, random_state=1)
    path = tmp_path / "m.json"
    est.save_model(str(path))
    data = json.loads(path.read_text())
    for t in data['trees']:
        del t['split_gains']
    path.write_text(json.dumps(data))
    m = HybridHistGBMNumbaV1_0_1.load_model(str(path))
    for t in m.trees:
        np.testing.assert_array_equal(t[6], np.zeros(t[5]))


def test_reload_reads_learning_rate_as_the_reference(tmp_path):
    """est:4133: the model is rebuilt from get_params(), where an 'auto'
    learning rate is still 'auto': the reloaded model scores with the
    constructor's 0.1, not the rate resolved during fit."""
    X, y = make_data(2000, 4, seed=7)
    est, _ = _fitted_from_oracle(X, y, n_estimators=2, max_depth=3, n_bins=64, random_state=1)
    assert est.learning_rate != 0.1
    path = tmp_path / "m.json"
    est.save_model(str(path))
    assert HybridHistGBMNumbaV1_0_1.load_model(str(path)).learning_rate == 0.1


def _reference_reload_scores(m, X):
    """What the reference's reloaded model computes (est:3274-3336 with the
    loaded state): bins with the NaN-bin map of est:4200-4202 (no NaN
    features) and scores with the loaded learning rate."""
    codes = om.bin_features(X, m.bin_edges, m.feature_bin_counts, m._nan_bin_id, "standard")
    F = om.predict_all_trees(codes, om.pack_trees(m.trees), len(m.trees),
                             m.learning_rate) + m.base_score_
    p = 1.0 / (1.0 + np.exp(-np.clip(F, -500, 500)))
    return np.column_stack([1 - p, p])


@pytest.mark.gpu
def test_reloaded_model_scores_like_the_reference(engine, tmp_path):
    """A model fitted without NaN and with a given learning rate scores the
    same after a reload.  One fitted on NaN features with learning_rate
    'auto' scores as the reference's reloaded model does (codes unshifted,
    rate 0.1), which differs from the fitted model."""
    print("[case] json reload scoring", flush=True)
    X, y = make_data(20000, 6, seed=6)
    est = HybridHistGBMNumbaV1_0_1(n_estimators=5, max_depth=4, learning_rate=0.15, n_bins=255,
                                   random_state=0, verbose=False).fit(X, y)
    path = tmp_path / "a.json"
    est.save_model(str(path))
    m = HybridHistGBMNumbaV1_0_1.load_model(str(path))
    np.testing.assert_array_equal(m.predict_proba(X[:5000]), est.predict_proba(X[:5000]))

    Xn, yn = make_data(20000, 6, seed=7, nan_frac=0.1, nan_cols=[1, 4])
    est = HybridHistGBMNumbaV1_0_1(n_estimators=5, max_depth=4, n_bins=255, random_state=0,
                                   verbose=False).fit(Xn, yn)
    path = tmp_path / "b.json"
    est.save_model(str(path))
    m = HybridHistGBMNumbaV1_0_1.load_model(str(path))
    got = m.predict_proba(Xn[:5000])
    assert np.max(np.abs(got - _reference_reload_scores(m, Xn[:5000]))) <= 1e-6
    assert not np.allclose(got, est.predict_proba(Xn[:5000]))
