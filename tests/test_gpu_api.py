"""The reference's own behaviour tests that apply to the binary path
(tests/test_bsscl_gbm_v101.py, test_reproducibility.py, test_regression.py,
test_properties.py, test_serialization.py, test_fuzz.py, test_precision.py
of the reference), run against the drop-in estimator on the GPU."""
import pickle

import numpy as np
import pytest
from sklearn.datasets import make_classification
from sklearn.metrics import accuracy_score

from bsscl_gbm import HybridHistGBMNumbaV1_0_1
from conftest import make_data

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bin_data():
    return make_classification(n_samples=500, n_features=10, n_classes=2, random_state=42)


def test_binary_classification(engine, bin_data):
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=10, max_depth=3, random_state=42, verbose=False)
    m.fit(X, y)
    assert accuracy_score(y, m.predict(X)) > 0.8


def test_imbalanced_balanced_sqrt(engine):
    X, y = make_classification(n_samples=500, n_features=10, n_classes=2,
                               weights=[0.99, 0.01], random_state=42)
    m = HybridHistGBMNumbaV1_0_1(n_estimators=50, max_depth=3, class_weight="balanced_sqrt",
                                 random_state=42, verbose=False).fit(X, y)
    assert len(m.predict(X)) == len(y)


def test_nan_handling(engine, bin_data):
    X, y = bin_data
    Xn = X.copy()
    Xn[0, 0] = np.nan
    Xn[10, 5] = np.nan
    m = HybridHistGBMNumbaV1_0_1(n_estimators=10, max_depth=3, verbose=False).fit(Xn, y)
    assert len(m.predict(Xn)) == len(y)
    assert (m._nan_bin_id[[0, 5]] == 0).all()


def test_early_stopping(engine, bin_data):
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=100, max_depth=3, early_stopping_rounds=5,
                                 verbose=False)
    m.fit(X, y, eval_set=[(X, y)])
    assert m.best_iteration_ > 0
    assert len(m.val_loss_history_) >= m.best_iteration_ + 1


def test_scale_pos_weight(engine, bin_data):
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=10, max_depth=3, objective="binary",
                                 scale_pos_weight=3.0, verbose=False).fit(X, y)
    assert len(m.predict(X)) == len(y)


def test_reproducibility_and_checksum(engine):
    """tests/test_reproducibility.py and tests/test_regression.py."""
    X = np.random.RandomState(42).randn(100, 5)
    y = np.random.RandomState(42).randint(0, 2, size=100)
    ref = None
    for _ in range(20):
        m = HybridHistGBMNumbaV1_0_1(n_estimators=5, max_depth=2, random_state=42, verbose=False)
        m.fit(X, y)
        p = m.predict_proba(X)
        if ref is None:
            ref = p
        np.testing.assert_array_equal(p, ref)
    np.testing.assert_allclose(np.sum(ref), 100.0, atol=1e-5)


def test_properties(engine, bin_data):
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=10, max_depth=3, verbose=False).fit(X, y)
    p = m.predict_proba(X)
    assert p.shape == (len(X), 2) and np.all(np.isfinite(p))
    assert np.all((p >= 0) & (p <= 1))
    np.testing.assert_allclose(p.sum(1), 1.0)
    assert set(np.unique(m.predict(X))) <= set(np.unique(y))
    # Single-row prediction (tests/test_coverage.py:72-86 of the reference).
    assert m.predict_proba(X[:1]).shape == (1, 2)


def test_serialization_roundtrip(engine, bin_data):
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=10, max_depth=3, verbose=False).fit(X, y)
    m2 = pickle.loads(pickle.dumps(m))
    np.testing.assert_array_equal(m.predict_proba(X), m2.predict_proba(X))
    import joblib, io
    buf = io.BytesIO()
    joblib.dump(m, buf)
    buf.seek(0)
    np.testing.assert_array_equal(m.predict(X), joblib.load(buf).predict(X))


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.int64, np.float64])
def test_input_dtypes(engine, dtype, bin_data):
    X, y = bin_data
    Xc = (X * 10).astype(dtype)
    m = HybridHistGBMNumbaV1_0_1(n_estimators=5, max_depth=3, verbose=False).fit(Xc, y)
    assert m.predict_proba(Xc).shape == (len(y), 2)


def test_extreme_values(engine):
    rng = np.random.RandomState(0)
    X = rng.randn(300, 4)
    X[0, 0], X[1, 1], X[2, 2] = 1e308, -1e308, np.inf
    y = rng.randint(0, 2, 300)
    m = HybridHistGBMNumbaV1_0_1(n_estimators=5, max_depth=3, verbose=False).fit(X, y)
    assert np.all(np.isfinite(m.predict_proba(X)))


def test_feature_importances(engine, bin_data):
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=10, max_depth=3, verbose=False).fit(X, y)
    assert m.feature_importances_.shape == (10,)
    np.testing.assert_allclose(m.feature_importances_.sum(), 1.0)
    assert m.feature_split_counts_.sum() == sum(int((t[0][:t[5]] >= 0).sum()) for t in m.trees)


def test_threads_fit_and_predict_concurrently():
    """Estimators share the device's engine; fits and predictions from two
    threads at once give what they give one after the other."""
    import threading
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    data = [make_data(20000, 10, seed=s, nan_frac=0.05) for s in (41, 42)]
    params = [dict(n_estimators=15, max_depth=5, random_state=0, verbose=False),
              dict(n_estimators=12, max_depth=4, n_bins=100, random_state=3, verbose=False)]
    seq = [HybridHistGBMNumbaV1_0_1(**p).fit(X, y) for p, (X, y) in zip(params, data)]
    want = [m.predict_proba(X) for m, (X, _) in zip(seq, data)]
    for rep in range(3):
        out, errors = [None, None], []

        def work(i):
            try:
                X, y = data[i]
                m = HybridHistGBMNumbaV1_0_1(**params[i]).fit(X, y)
                out[i] = (m, m.predict_proba(X), seq[1 - i].predict_proba(data[1 - i][0]))
            except Exception as e:  # noqa: BLE001 - reported below
                errors.append(e)

        threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert not errors, errors
        for i in range(2):
            m, p, p_other = out[i]
            assert m.train_loss_history_ == seq[i].train_loss_history_, (rep, i)
            for a, b in zip(m.trees, seq[i].trees):
                nc = a[5]
                assert nc == b[5]
                np.testing.assert_array_equal(a[0][:nc], b[0][:nc])
                np.testing.assert_array_equal(a[1][:nc], b[1][:nc])
            np.testing.assert_array_equal(p, want[i])
            np.testing.assert_array_equal(p_other, want[1 - i])


def test_score_and_batch_parallel_predictions(engine, bin_data, monkeypatch):
    """score is the mean accuracy (est:3577-3578); the batch-parallel
    predictions (est:3842-3916) equal predict and predict_proba, one batch
    or many, also when the device passes are cut into several slices."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=20, max_depth=4, random_state=0,
                                 verbose=False).fit(X, y)
    pred, proba = m.predict(X), m.predict_proba(X)
    assert m.score(X, y) == np.mean(pred == y)
    for bs in (len(X), 100, 77):
        np.testing.assert_array_equal(m.predict_batch_parallel(X, n_workers=2, batch_size=bs), pred)
        np.testing.assert_array_equal(m.predict_proba_batch_parallel(X, batch_size=bs), proba)
    monkeypatch.setattr(est_mod, "_BATCH_ROWS", 150)  # slices of 140 rows
    np.testing.assert_array_equal(m.predict_batch_parallel(X, batch_size=70), pred)
    np.testing.assert_array_equal(m.predict_proba_batch_parallel(X, batch_size=70), proba)


def test_predict_proba_device_equals_numpy_expression(engine, bin_data):
    """A binary model's predict_proba, computed on the device from F
    (bsscl_predict_proba), against NumPy's expression on the same F
    (est:3335-3336): within 2 ulp of 1, and mostly bit-identical (the
    device's exp and NumPy's may round a last bit differently).  Scores far
    past the clip (|F| > 500) saturate as NumPy's do."""
    from bsscl_gbm import estimator as est_mod
    X, y = bin_data
    m = HybridHistGBMNumbaV1_0_1(n_estimators=30, max_depth=4, random_state=0,
                                 verbose=False).fit(X, y)
    rng = np.random.default_rng(1)
    Xp = np.vstack([X, rng.standard_normal((20000, X.shape[1])) * 3.0])
    F = m._raw_score(Xp)
    p = 1.0 / (1.0 + np.exp(-np.clip(F, -500, 500)))
    want = np.column_stack([1 - p, p])
    got = m.predict_proba(Xp)
    worst = float(np.max(np.abs(got - want))) / np.finfo(np.float64).eps
    same = float(np.mean(got == want))
    print(f"[result] predict_proba on the device: {100 * same:.3f}% bit-identical, "
          f"max |diff| {worst:.2f} ulp(1)", flush=True)
    assert worst <= 2.0 and same >= 0.9
    np.testing.assert_array_equal(m.predict(Xp), m.classes_[(want[:, 1] > 0.5).astype(int)])
    # One-leaf trees worth +-1000: F past the clip on either side (p then
    # exactly 1, or exp(500)'s last bit apart), and exactly 0 (p = 0.5).
    eng = est_mod._engine(0)
    packed = {"features": np.array([-1, -1], np.int16), "thresholds": np.zeros(2, np.int64),
              "values": np.array([1000.0, -1000.0]), "left": np.full(2, -1, np.int32),
              "right": np.full(2, -1, np.int32), "offsets": np.array([0, 1, 2], np.int32)}
    for n_trees, base in ((1, 0.0), (2, 0.0), (1, 1e4), (1, -2000.0)):
        got = eng.predict_proba(1, len(Xp), packed, n_trees, 1.0, base)
        F2 = eng.predict(1, len(Xp), packed, n_trees, 1.0) + base
        p2 = 1.0 / (1.0 + np.exp(-np.clip(F2, -500, 500)))
        np.testing.assert_allclose(got, np.column_stack([1 - p2, p2]), rtol=4.5e-16, atol=0)


@pytest.mark.parametrize("case", ["chunks_f32_nan", "chunks_f64", "one_short_chunk",
                                  "bins_300", "no_trees"])
def test_predict_proba_rows_equals_binning_then_predict(engine, monkeypatch, case):
    """bsscl_predict_proba_rows (binning, walk and probabilities of host rows
    in overlapped row chunks) equals bsscl_bin_features followed by
    bsscl_predict_proba bit for bit, over ragged last chunks, float64 rows,
    fewer rows than one walk block, codes in two tiers and an empty model;
    matrix slot 1 keeps the codes binned before it."""
    from bsscl_gbm import estimator as est_mod
    print(f"[case] predict_proba_rows {case}", flush=True)
    rng = np.random.default_rng(7)
    X, y = make_data(6000, 12, seed=5, nan_frac=0.1, nan_cols=[0, 3])
    n_bins = 300 if case == "bins_300" else 255
    n_est = 0 if case == "no_trees" else 25
    m = HybridHistGBMNumbaV1_0_1(n_estimators=max(n_est, 1), max_depth=5, n_bins=n_bins,
                                 random_state=3, verbose=False).fit(X, y)
    if n_est == 0:
        m.trees = []
        m._pack_trees()
    n = {"one_short_chunk": 300, "chunks_f64": 40_001}.get(case, 50_003)
    Xp = rng.standard_normal((n, 12)) * 1.5
    Xp[rng.random(Xp.shape) < 0.05] = np.nan
    Xp = Xp if case == "chunks_f64" else Xp.astype(np.float32)
    if case != "one_short_chunk":
        monkeypatch.setenv("BSSCL_TEST_PREDICT_CHUNK_ROWS", "4096")
    eng = est_mod._engine(0)
    packed = {"features": m._packed_features, "thresholds": m._packed_thresholds,
              "values": m._packed_values, "left": m._packed_left, "right": m._packed_right,
              "offsets": m._tree_offsets}
    eng.bin_features(1, Xp, m.bin_edges, m.feature_bin_counts, m._nan_bin_id)
    want = eng.predict_proba(1, n, packed, len(m.trees), m.learning_rate, m.base_score_)
    codes_before = eng.get_codes(1, n, 12)
    got = eng.predict_proba_rows(Xp, m.bin_edges, m.feature_bin_counts, m._nan_bin_id, packed,
                                 len(m.trees), m.learning_rate, m.base_score_)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(m.predict_proba(Xp), want)
    np.testing.assert_array_equal(eng.get_codes(1, n, 12), codes_before)
