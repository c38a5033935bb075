"""Parity at the benchmark workloads' full sizes (bench.py:make_workload).

* dense_1m (1,000,000 x 28, 5% NaN, depth 6): the workload's complete
  100-round fit.
* imbalanced (284,807 x 30, 0.17% positives, balanced_sqrt) and sparse_hd
  (100,000 x 100, 90% zeros, balanced_sqrt): the complete fits, 200 and 300
  trees.
* stress_10m (10,000,000 x 50, 10 columns 70% NaN, depth 8): bin edges and
  codes of all 10M rows against the oracle's; the first ten rounds of the
  workload's fit; one depth-8 tree from 5M rows x 35 features; rounds 250
  and 499 of the workload's 500-tree fit, tree by tree, each from the
  engine's own scores before the round; and the 500-tree fit scored on a
  fresh 10M-row batch, checked on all 10M rows (codes bit-exact, raw scores
  within 1e-12, predict_proba within 1e-6).

Every fit compares each round in lockstep and end to end with the oracle,
following certified gain ties (tests/fitcmp.py), then every round's loss
and predict_proba.
"""
import numpy as np
import pytest

import bench
import fitcmp
import treecmp
from oracle import model as om
from test_gpu_parity import _grad_hess

pytestmark = pytest.mark.gpu

_CACHE = {}


def _workload(name, predict=False):
    key = (name, predict)
    if key not in _CACHE:
        if name == "stress_10m":
            _CACHE.clear()  # keep at most one 10M matrix in memory
        _CACHE[key] = bench.make_workload(name, predict=predict)
    return _CACHE[key]


def _fit_and_follow(engine, name, n_estimators=None, eval_rows=200_000):
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    X, y, params = _workload(name)
    if n_estimators is not None:
        params = dict(params, n_estimators=n_estimators)
    print(f"[case] {name} full size, {params['n_estimators']} rounds", flush=True)
    est = HybridHistGBMNumbaV1_0_1(**params).fit(X, y)
    ref, rep = fitcmp.follow_fit(engine, est, X, y, params)
    print(rep.line(name), flush=True)
    assert rep.rounds == params["n_estimators"]
    fitcmp.assert_fit_equal(ref, est, X[:eval_rows])
    return est, ref


def test_dense_1m_full_fit(engine):
    _fit_and_follow(engine, "dense_1m")


@pytest.mark.parametrize("name", ["imbalanced", "sparse_hd"])
def test_workload_full_fit(engine, name):
    est, ref = _fit_and_follow(engine, name)
    if name == "imbalanced":
        w0, w1 = est._class_weight_pair(_workload(name)[1])
        print(f"[result] imbalanced class weights w0={w0:.6f} w1={w1:.6f}", flush=True)
        assert abs(w1 - 7.31) < 0.01 and abs(w0 - 0.785) < 0.01
    Xp, _, _ = bench.make_workload(name, predict=True)
    np.testing.assert_allclose(est.predict_proba(Xp), ref.predict_proba(Xp), rtol=0, atol=1e-6)


def test_stress_10m_binning(engine):
    """Edges and codes of the whole 10M x 50 matrix equal the oracle's."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    print("[case] stress_10m binning, 10M x 50", flush=True)
    X, y, params = _workload("stress_10m")
    est = HybridHistGBMNumbaV1_0_1(**dict(params, n_estimators=1)).fit(X, y)
    e, bc, nid = om.build_bin_edges(X, 255, threads=16)
    np.testing.assert_array_equal(est.bin_edges, e)
    np.testing.assert_array_equal(est.feature_bin_counts, bc)
    np.testing.assert_array_equal(est._nan_bin_id, nid)
    want = om.bin_features(X, e, bc, nid, "hybrid")
    got = est_mod._engine(0).get_codes(0, *X.shape)
    np.testing.assert_array_equal(got, want)
    print(f"[result] stress_10m binning: edges and {got.size} codes identical", flush=True)


def test_stress_10m_rounds(engine):
    _fit_and_follow(engine, "stress_10m", n_estimators=10, eval_rows=500_000)


def test_stress_10m_tree(engine):
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    print("[case] stress_10m full size, one tree from 5M rows x 35 features", flush=True)
    X, y, params = _workload("stress_10m")
    n, F = X.shape
    est = HybridHistGBMNumbaV1_0_1(**dict(params, n_estimators=1)).fit(X, y)
    eng = est_mod._engine(0)  # the estimator's engine holds the codes in slot 0
    codes = eng.get_codes(0, n, F)
    bc = np.asarray(est.feature_bin_counts)
    g, h = _grad_hess(y, 17, (0.8, 1.3))
    rng = np.random.default_rng(18)
    rows = np.sort(rng.permutation(n)[: n // 2]).astype(np.int64)
    feats = np.sort(rng.permutation(F)[:35]).astype(np.int32)
    args = (rows, feats, est.max_leaves, est.max_depth, est.min_samples_leaf,
            est.min_child_weight, bc, int(bc.max()), est.reg_lambda, 0.0)
    got = eng.build_tree(g, h, *args)
    out = treecmp.follow(got, codes, g, h, *args)
    print(f"[result] stress_10m tree: {got[5]} nodes, ties {out.ties}", flush=True)
    assert got[5] > 100


def test_stress_10m_late_rounds(engine, monkeypatch):
    """Rounds 250 and 499 of the workload's 500-tree fit, tree by tree.  The
    engine's scores before each round come back from the device
    (boost_get_F, rounds not pipelined); the oracle's expressions give the
    round's gradients (est:2861, 2873-2874) and its builder the tree, from
    that round's rows and features as a host-rows sampler started from the
    fit's RandomState state draws them (the sampler equals rng.shuffle:
    tests/test_sampler.py).  The estimator's tree must equal the oracle's,
    following certified ties, and the loss it recorded after the previous
    round must equal the loss of those scores."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1, _native
    X, y, params = _workload("stress_10m")
    picks = (250, 499)
    print(f"[case] stress_10m rounds {picks} of the {params['n_estimators']}-tree fit",
          flush=True)
    made = []
    init = _native.Sampler.__init__

    def record(self, *args, **kw):
        made.append((args, kw))
        init(self, *args, **kw)

    monkeypatch.setattr(_native.Sampler, "__init__", record)
    F_at = {}
    est = HybridHistGBMNumbaV1_0_1(**params)
    est._pipeline_rounds = False
    est._round_hook = lambda m, eng: (F_at.__setitem__(m, eng.boost_get_F(len(y)))
                                      if m in picks else None)
    est.fit(X, y)
    monkeypatch.setattr(_native.Sampler, "__init__", init)
    assert len(est.trees) == params["n_estimators"] and sorted(F_at) == list(picks)
    assert len(made) == 1
    args, kw = made[0]
    sampler = _native.Sampler(*args, **dict(kw, device_rows=False))
    draws = {}
    for m in range(max(picks) + 1):
        rows, feats = sampler.next()
        if m in picks:
            draws[m] = (rows.astype(np.int64), feats.copy())
    sampler.close()
    X_bin = om.bin_features(X, est.bin_edges, est.feature_bin_counts, est._nan_bin_id, "hybrid")
    ref = om.OracleGBM(**{k: v for k, v in params.items() if k != "verbose"})
    ref.n_classes_ = 2
    w = ref._class_weights(y)
    g = np.empty(len(y))
    h = np.empty(len(y))
    for m in picks:
        F = F_at[m]
        loss = om.binary_logloss(y, F)
        assert abs(est.train_loss_history_[m - 1] - loss) <= 1e-9 * abs(loss), m
        om.binary_grad_hess(F, y, w, g, h)
        rows, feats = draws[m]
        out = treecmp.follow(est.trees[m], X_bin, g, h, rows, feats, est.max_leaves,
                             est.max_depth, est.min_samples_leaf, est.min_child_weight,
                             np.asarray(est.feature_bin_counts), est._max_bins, est.reg_lambda,
                             est.gamma)
        print(f"[result] stress_10m round {m}: {est.trees[m][5]} nodes from {len(rows)} rows x "
              f"{len(feats)} features, ties {out.n_ties}; loss before it {loss:.9f}", flush=True)


def test_stress_10m_inference(engine):
    """The workload's 500-tree fit, then predict_proba of a fresh 10M-row
    batch (default_rng(5)), checked on every row."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    X, y, params = _workload("stress_10m")
    print(f"[case] stress_10m inference: {params['n_estimators']}-tree fit", flush=True)
    est = HybridHistGBMNumbaV1_0_1(**params).fit(X, y)
    assert len(est.trees) == 500
    Xp, _, _ = _workload("stress_10m", predict=True)
    n, F = Xp.shape
    p = est.predict_proba(Xp)
    assert p.shape == (n, 2) and np.all(np.isfinite(p))
    eng = est_mod._engine(0)
    k = n
    # (predict_proba bins and walks the rows in chunks of its own; the codes
    # and F are checked through the matrix the same binning fills.)
    eng.bin_features(1, Xp, est.bin_edges, est.feature_bin_counts, est._nan_bin_id)
    codes = eng.get_codes(1, n, F)
    want = om.bin_features(Xp, est.bin_edges, est.feature_bin_counts, est._nan_bin_id,
                           "hybrid")
    # A NaN feature's value above its training maximum gets the reference
    # code bin_counts = 256 (uint16 codes, est:2163-2166); every threshold
    # there is <= 254, so the engine stores it as 255.
    assert want.max() <= 256
    np.testing.assert_array_equal(codes, np.minimum(want, 255))
    packed = {"features": est._packed_features, "thresholds": est._packed_thresholds,
              "values": est._packed_values, "left": est._packed_left,
              "right": est._packed_right, "offsets": est._tree_offsets}
    F_dev = eng.predict(1, n, packed, len(est.trees), est.learning_rate)
    F_ref = om.predict_all_trees(want, packed, len(est.trees), est.learning_rate)
    np.testing.assert_allclose(F_dev[:k], F_ref, rtol=0, atol=1e-12)
    p_ref = 1.0 / (1.0 + np.exp(-np.clip(F_ref + est.base_score_, -500, 500)))
    np.testing.assert_allclose(p[:k, 1], p_ref, rtol=0, atol=1e-6)
    print(f"[result] stress_10m inference: 500 trees over {n} rows; all {k} rows: codes "
          f"identical, max |dF| {np.max(np.abs(F_dev[:k] - F_ref)):.3g}", flush=True)
