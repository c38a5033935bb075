"""Host-side behaviour of the drop-in estimator and the C ABI library that
needs no GPU: argument errors (tests/test_fault_injection.py of the
reference), the parameter surface, the bagging stream, and the library's
exported symbols."""
import ctypes
import os
import pickle
import re

import numpy as np
import pytest

from bsscl_gbm import HybridHistGBMNumbaV1_0_1
from bsscl_gbm import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol():
    header = open(os.path.join(ROOT, "include", "bsscl_hip.h")).read()
    names = set(re.findall(r"\b(bsscl_[A-Za-z0-9_]+)\s*\(", header))
    assert len(names) >= 20
    lib = ctypes.CDLL(_native.library_path())
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # The Python binding declares every exported entry point.
    assert names == set(_native._SIGS), names ^ set(_native._SIGS)


def test_invalid_hyperparameters_raise_value_error():
    X = np.random.randn(100, 5)
    y = np.random.randint(0, 2, 100)
    with pytest.raises(ValueError):
        HybridHistGBMNumbaV1_0_1(max_depth=-5, verbose=False).fit(X, y)
    with pytest.raises(ValueError):
        HybridHistGBMNumbaV1_0_1(learning_rate=-0.1, verbose=False).fit(X, y)
    with pytest.raises(ValueError):
        HybridHistGBMNumbaV1_0_1(n_estimators=0, verbose=False).fit(X, y)


def test_mismatched_rows_raise_value_error():
    with pytest.raises(ValueError):
        HybridHistGBMNumbaV1_0_1(verbose=False).fit(np.random.randn(100, 5),
                                                    np.random.randint(0, 2, 99))


def test_unfitted_predict_raises_value_error():
    with pytest.raises(ValueError):
        HybridHistGBMNumbaV1_0_1().predict(np.random.randn(10, 5))


@pytest.mark.parametrize("kw", [dict(objective="regression"), dict(grow_policy="level"),
                                dict(sampling_method="goss"), dict(boosting_type="dart"),
                                dict(categorical_features=[0]),
                                dict(monotone_constraints=[1, 0, 0, 0, 0])])
def test_modes_outside_the_engine_raise(kw):
    X = np.random.randn(200, 5)
    y = np.random.randint(0, 2, 200)
    with pytest.raises(NotImplementedError):
        HybridHistGBMNumbaV1_0_1(verbose=False, **kw).fit(X, y)


def test_single_class_raises():
    X = np.random.randn(300, 5)
    y = np.zeros(300, dtype=np.int64)
    with pytest.raises(NotImplementedError):
        HybridHistGBMNumbaV1_0_1(verbose=False).fit(X, y)


def test_params_surface_and_pickle():
    m = HybridHistGBMNumbaV1_0_1(n_estimators=7, max_depth=3, random_state=1)
    p = m.get_params()
    assert p["n_estimators"] == 7 and p["max_depth"] == 3 and p["random_state"] == 1
    assert m.set_params(reg_lambda=2.0) is m and m.reg_lambda == 2.0
    assert "n_estimators=7" in repr(m)
    m2 = pickle.loads(pickle.dumps(m))
    assert m2.get_params() == m.get_params()


@pytest.mark.parametrize("dtype", [np.int64, np.int32])
@pytest.mark.parametrize("n", [0, 1, 2, 5, 1000, 65537])
def test_native_shuffle_matches_randomstate(dtype, n):
    for seed in (0, 42, 2**32 - 1):
        rng = np.random.RandomState(seed)
        rng.randint(0, 10, size=3)
        a = np.arange(n, dtype=dtype)
        b = a.copy()
        key, pos = _native.rs_shuffle(rng.get_state(), b)
        rng.shuffle(a)
        st = rng.get_state()
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(st[1], key)
        assert st[2] == pos


@pytest.mark.parametrize("sub,col", [(0.75, 0.8), (1.0, 0.7), (0.5, 1.0), (1.0, 1.0)])
def test_sampler_stream_matches_reference_calls(sub, col):
    """The reference's est:2502-2517 call sequence on one RandomState."""
    n, F, rounds = 20011, 28, 6
    n_sub, f_sub = max(1, int(n * sub)), max(1, int(F * col))
    rng = np.random.RandomState(9)
    s = _native.Sampler(rng.get_state(), n, n_sub if sub < 1 else n, sub < 1, F,
                        f_sub if col < 1 else F, col < 1, rounds)
    all_rows = np.arange(n, dtype=np.int64)
    all_feats = np.arange(F, dtype=np.int32)
    for _ in range(rounds):
        if sub < 1:
            rng.shuffle(all_rows)
            si = all_rows[:n_sub].copy()
        else:
            si = all_rows.copy()
        if col < 1:
            rng.shuffle(all_feats)
            fi = np.sort(all_feats[:f_sub])
        else:
            fi = all_feats.copy()
        r, f = s.next()
        np.testing.assert_array_equal(r, si)
        np.testing.assert_array_equal(f, fi)
    key, pos = s.state()
    st = rng.get_state()
    np.testing.assert_array_equal(key, st[1])
    assert pos == st[2]
    s.close()


def test_sampler_rejects_bad_arguments():
    st = np.random.RandomState(0).get_state()
    with pytest.raises(ValueError):
        _native.Sampler(st, 10, 11, True, 3, 2, True, 1)
    with pytest.raises(ValueError):
        _native.Sampler(st, 10, 5, False, 3, 2, True, 1)


def test_label_encoding_equals_unique_and_searchsorted(monkeypatch):
    """The estimator's label encoding (a counting path for integer labels
    0 .. K-1) equals np.unique + np.searchsorted (est:3124-3129), dtype
    included, and the base score's weighted mean built by lookup equals
    np.average with the reference's np.where weights bit for bit."""
    from bsscl_gbm import estimator as em
    monkeypatch.setattr(em, "_PASS_THREAD_ROWS", 1 << 19)  # the large cases in row blocks
    rng = np.random.default_rng(5)
    cases = [rng.integers(0, 2, 1000), rng.integers(0, 5, 1000).astype(np.int32),
             np.array([3, 7, 3, 9]), rng.random(100) < 0.3, np.array(["b", "a", "b"]),
             np.array([2, 2, 5]), np.array([-1, 1, -1]), rng.integers(0, 2, 10).astype(np.uint8),
             np.array([0.0, 1.0, 1.0]), np.zeros(5, np.int64), np.ones(6, np.int64),
             np.ones(4, bool), np.array([1, 0, 1], np.uint8), rng.integers(0, 2, 700_001),
             np.ones(600_000, np.int64), rng.integers(0, 3, 600_000).astype(np.int16)]
    for y in cases:
        c, e = em._encode_labels(y)
        c2 = np.unique(y)
        np.testing.assert_array_equal(c, c2)
        assert c.dtype == c2.dtype and e.dtype == np.int64
        np.testing.assert_array_equal(e, np.searchsorted(c2, y))
    for n in (1, 7, 1000, 100_003, 700_001):
        y = (rng.random(n) < 0.3).astype(np.int64)
        assert em._count_nonzero(y) == np.count_nonzero(y)
        for w0, w1 in ((1.0, 1.0), (0.785, 7.31), (1.0, 6.0)):
            want = np.average(y, weights=np.where(y == 1, w1, w0))
            got = em._take(np.array([0.0, w1]), y).sum() / em._take(np.array([w0, w1]), y).sum()
            assert got == want


def test_feature_importances_equal_node_loop():
    """feature_importances_ (est:2343-2363) equals the node-by-node loop of
    the reference bit for bit, over random trees with leaves (-1) mixed in."""
    rng = np.random.default_rng(7)
    trees = []
    for _ in range(60):
        nc = int(rng.integers(1, 64))
        tf = rng.integers(-1, 12, 130).astype(np.int32)
        sg = rng.standard_normal(130) * 10.0 ** rng.integers(-6, 3)
        trees.append((tf, None, None, None, None, nc, sg))
    est = HybridHistGBMNumbaV1_0_1(verbose=False)
    est.n_features_in_, est._is_multiclass, est.trees = 12, False, trees
    est._compute_feature_importances()
    gain, cnt = np.zeros(12), np.zeros(12, np.int64)
    for tf, _, _, _, _, nc, sg in trees:
        for i in range(nc):
            if tf[i] >= 0:
                gain[tf[i]] += sg[i]
                cnt[tf[i]] += 1
    np.testing.assert_array_equal(est.feature_importances_, gain / gain.sum())
    np.testing.assert_array_equal(est.feature_split_counts_, cnt)
