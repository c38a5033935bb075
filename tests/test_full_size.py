"""Parity at the benchmark workloads' full sizes (bench.py:make_workload):
1,000,000 x 28 (depth 6, 255 bins) and 10,000,000 x 50 (depth 8, 10
columns 70% NaN), where the oracle still finishes a tree in seconds.

* 1M x 28: the oracle's first rounds of the workload's fit, every tree
  rebuilt by the engine from the oracle's gradients, rows and features
  (identical, or a certified gain tie: tests/treecmp.py); the estimator's
  own fit of the same rounds, which must give the oracle's losses (rtol
  1e-9) and trees, and predict_proba within 1e-6.
* 10M x 50: the estimator bins the matrix on the device (its codes are the
  oracle's codes: test_gpu_parity.py::test_binning_bit_exact pins the
  binning); one tree of the workload's shape from 5,000,000 rows and 35
  features, engine against the oracle's tree builder on those codes.
"""
import numpy as np
import pytest

import bench
import treecmp
from oracle import model as om
from test_gpu_parity import _grad_hess

pytestmark = pytest.mark.gpu


def test_dense_1m_rounds_lockstep_and_fit(engine):
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    print("[case] dense_1m full size, 3 rounds", flush=True)
    X, y, params = bench.make_workload("dense_1m")
    params = dict(params, n_estimators=3)
    rounds = []
    ref = om.OracleGBM(**{k: v for k, v in params.items() if k != "verbose"})
    ref.fit(X, y, round_callback=lambda m, g, h, si, fi, t: rounds.append((g.copy(), h.copy(), si, fi, t)))
    Xb, bc = ref.X_bin_, ref.feature_bin_counts
    engine.load_codes(0, Xb)
    ties = 0
    for g, h, si, fi, tree in rounds:
        got = engine.build_tree(g, h, si, fi, ref.max_leaves, ref.max_depth,
                                ref.min_samples_leaf, ref.min_child_weight, bc,
                                ref._max_bins, ref.reg_lambda, ref.gamma)
        ties += treecmp.compare(tree, got, Xb, g, h, si, bc, ref.reg_lambda) == "tie"
    est = HybridHistGBMNumbaV1_0_1(**params).fit(X, y)
    np.testing.assert_array_equal(est.bin_edges, ref.bin_edges)
    diverged = None
    for k in range(len(rounds)):
        g, h, si, _, _ = rounds[k]
        if treecmp.compare(ref.trees[k], est.trees[k], Xb, g, h, si, bc, ref.reg_lambda) == "tie":
            diverged = k
            break
        np.testing.assert_allclose(est.train_loss_history_[k], ref.train_loss_history_[k],
                                   rtol=1e-9)
    print(f"[result] dense_1m: lockstep ties {ties}/{len(rounds)}, end-to-end "
          f"{'identical' if diverged is None else f'tie at tree {diverged}'}", flush=True)
    if diverged is None:
        np.testing.assert_allclose(est.predict_proba(X[:200_000]), ref.predict_proba(X[:200_000]),
                                   rtol=0, atol=1e-6)


def test_stress_10m_tree(engine):
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    print("[case] stress_10m full size, one tree from 5M rows x 35 features", flush=True)
    X, y, params = bench.make_workload("stress_10m")
    n, F = X.shape
    est = HybridHistGBMNumbaV1_0_1(**dict(params, n_estimators=1)).fit(X, y)
    del X
    eng = est_mod._engine(0)  # the estimator's engine holds the codes in slot 0
    codes = eng.get_codes(0, n, F)
    bc = np.asarray(est.feature_bin_counts)
    g, h = _grad_hess(y, 17, (0.8, 1.3))
    rng = np.random.default_rng(18)
    rows = np.sort(rng.permutation(n)[: n // 2]).astype(np.int64)
    feats = np.sort(rng.permutation(F)[:35]).astype(np.int32)
    args = (rows, feats, est.max_leaves, est.max_depth, est.min_samples_leaf,
            est.min_child_weight, bc, int(bc.max()), est.reg_lambda, 0.0)
    ref = om.build_tree(codes, g, h, *args)
    got = eng.build_tree(g, h, *args)
    verdict = treecmp.compare(ref, got, codes, g, h, rows, bc, est.reg_lambda)
    print(f"[result] stress_10m tree: {verdict}, {got[5]} nodes", flush=True)
    assert got[5] > 100
