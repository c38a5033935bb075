"""Multiclass softmax boosting (est:2949-3065; predict est:3293-3315).

CPU tests pin the oracle's multiclass loop by checks that do not restate
it: every round's gradients and hessians equal central finite differences
of the weighted softmax cross-entropy sum_i w_i (logsumexp(F_i) - F_i[y_i])
(scipy's logsumexp) in each class's score, at the scores rebuilt by the
independent traversal, under balanced_sqrt weights, and the hessian floor
of 1e-8 holds exactly where w p (1 - p) falls below it; the recorded
training loss equals the loss recomputed from the fitted trees; the K trees
of a round share one bagging draw, which equals a fresh RandomState's
shuffle stream; the K-dependent parameter rules give hand-derived values;
NumPy's row sum over the classes adds in the pairwise order the device
kernels restate.  GPU tests rebuild every oracle tree on the engine from the
same inputs and compare the estimator's own trees, losses and predict_proba
with the oracle's, following certified gain ties (tests/fitcmp.py), up to
16 classes, and compare the device's gradients and hessians with NumPy's on
the device's own scores.
"""
import numpy as np
import pytest
from scipy.special import logsumexp

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
    labels = np.array([3, 7, 11, 20, 21, 40, 41, 50, 60, 70, 80, 90, 91, 95, 99, 120])[:K]
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


def _weighted_ce(F, yi, w):
    """Per-row weighted softmax cross-entropy w_i (logsumexp(F_i) - F_i[y_i])."""
    return w * (logsumexp(F, axis=1) - F[np.arange(len(yi)), yi])


def _fd_grad_hess(F, yi, w, eps1=1e-5, eps2=1e-3):
    """Central differences of the per-row loss in each class's score."""
    n, K = F.shape
    G, H = np.empty((n, K)), np.empty((n, K))
    base = _weighted_ce(F, yi, w)
    for k in range(K):
        d1, d2 = np.zeros(K), np.zeros(K)
        d1[k], d2[k] = eps1, eps2
        G[:, k] = (_weighted_ce(F + d1, yi, w) - _weighted_ce(F - d1, yi, w)) / (2 * eps1)
        H[:, k] = (_weighted_ce(F + d2, yi, w) - 2 * base + _weighted_ce(F - d2, yi, w)) / eps2 ** 2
    return G, H


def _balanced_sqrt(yi, K):
    n = len(yi)
    counts = np.bincount(yi, minlength=K)
    return (n / (K * np.maximum(counts, 1)))[yi] ** 0.35


@pytest.mark.parametrize("K", [3, 5])
def test_oracle_multiclass_grad_hess_are_loss_derivatives(K):
    """Every round's (g, h) of every class, as handed to the tree builder,
    against finite differences of the weighted softmax loss at the scores
    rebuilt from the fitted trees (balanced_sqrt weights on unequal classes,
    so a missing weight on either fails)."""
    X, y = _mc_data(2400, 6, K, seed=30 + K)
    seen = {}
    m = om.OracleGBM(n_estimators=4, max_depth=4, learning_rate=0.6, n_bins=64,
                     class_weight="balanced_sqrt", random_state=4)
    m.fit(X, y, round_callback=lambda r, k, g, h, si, fi, t: seen.__setitem__((r, k),
                                                                             (g.copy(), h.copy())))
    yi = np.searchsorted(m.classes_, y)
    w = _balanced_sqrt(yi, K)
    assert np.ptp(w) > 0.05  # the weights differ between classes
    F = np.zeros((len(y), K))
    for r in range(4):
        G, H = _fd_grad_hess(F, yi, w)
        for k in range(K):
            g, h = seen[(r, k)]
            np.testing.assert_allclose(g, G[:, k], rtol=0, atol=1e-8 * w.max(),
                                       err_msg=f"g round {r} class {k}")
            np.testing.assert_allclose(h, np.maximum(H[:, k], 1e-8), rtol=0,
                                       atol=1e-6 * w.max(), err_msg=f"h round {r} class {k}")
        for k in range(K):  # the scores after round r, by the independent walk
            packed = om.pack_trees([m.mc_trees[k][r]])
            F[:, k] += om.predict_all_trees(m.X_bin_, packed, 1, m.learning_rate)


def test_oracle_multiclass_hessian_floor():
    """Confident rows: w p (1 - p) below 1e-8 is floored to exactly 1e-8
    (est:3019), elsewhere the hessian is the loss's second derivative."""
    rng = np.random.default_rng(7)
    n, K = 4000, 4
    yi = rng.integers(0, K, n)
    w = _balanced_sqrt(yi, K)
    F = rng.standard_normal((n, K))
    F[: n // 2] *= 25.0  # margins of tens: p of the losing classes ~ e^-50
    e = np.exp(F - F.max(axis=1, keepdims=True))
    proba = e / e.sum(axis=1, keepdims=True)
    G, H = om.multiclass_grad_hess(proba, np.eye(K)[yi], w)
    raw = w[:, None] * proba * (1.0 - proba)
    floored = raw < 1e-8
    assert floored.sum() > n // 4 and (~floored).sum() > n
    assert np.all(H[floored] == 1e-8)
    Gfd, Hfd = _fd_grad_hess(F, yi, w)
    np.testing.assert_allclose(G, Gfd, rtol=0, atol=1e-7 * w.max())
    np.testing.assert_allclose(H[~floored], Hfd[~floored], rtol=0, atol=1e-5 * w.max())


def _numpy_row_sum_order(e):
    """The order the device kernels add a row's K <= 16 class terms in:
    one running sum below 8 terms; else eight partial sums over whole blocks
    of eight, combined pairwise, then the remaining terms in order."""
    K = len(e)
    if K < 8:
        s = e[0]
        for j in range(1, K):
            s = s + e[j]
        return s
    r = [e[j] + e[j + 8] if K == 16 else e[j] for j in range(8)]
    s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))
    for j in range(8, K if K < 16 else 8):
        s = s + e[j]
    return s


def test_numpy_row_sum_is_pairwise_from_eight_classes():
    rng = np.random.default_rng(8)
    for K in range(2, 17):
        F = 3.0 * rng.standard_normal((3000, K))
        e = np.exp(F - F.max(axis=1, keepdims=True))
        want = e.sum(axis=1, keepdims=True)[:, 0]
        got = np.array([_numpy_row_sum_order(row) for row in e])
        np.testing.assert_array_equal(got, want, err_msg=f"K={K}")
        if K >= 8:  # the class-order sum differs somewhere
            seq = np.zeros(len(e))
            for k in range(K):
                seq = seq + e[:, k]
            assert np.any(seq != want), K


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
@pytest.mark.parametrize("K,n,nan", [(3, 6000, 0.0), (7, 12000, 0.1), (12, 16000, 0.05),
                                     (16, 20000, 0.0)])
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


@pytest.mark.gpu
@pytest.mark.parametrize("K", [3, 8, 12, 16])
def test_multiclass_device_grad_hess_equal_numpy(engine, K):
    """The device's softmax gradients and hessians against the reference's
    NumPy expressions (est:2327-2332, 3013-3014, 3019) on the device's own
    scores after two rounds.  NumPy's exp and the device's may round a term
    differently by an ulp, which moves p by a few ulp of 1; g = w (p - y)
    and h = w p (1 - p) cancel near p = 1, so the bar is absolute: within
    8 ulp of 1, times the row's weight.  The share of bit-identical values
    is printed and must stay high; from 8 classes on it must also be well
    above the share the same expressions reach with the row's terms summed
    in class order (which changes p in a third to a half of the rows)."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    print(f"[case] multiclass device grad/hess K={K}", flush=True)
    X, y = _mc_data(20000, 9, K, seed=40 + K)
    params = dict(n_estimators=2, max_depth=5, n_bins=255, random_state=5,
                  class_weight="balanced_sqrt", learning_rate=0.7)
    est = HybridHistGBMNumbaV1_0_1(verbose=False, **params).fit(X, y)
    eng = est_mod._engine(0)
    yi = np.searchsorted(est.classes_, y)
    n = len(y)
    w = _balanced_sqrt(yi, K)
    eng.mc_round(np.arange(n, dtype=np.int64))  # gradients at the fitted scores
    g_dev, h_dev = eng.mc_grad_hess()
    F = eng.mc_scores()
    assert np.ptp(F) > 0.5
    F_shifted = F - F.max(axis=1, keepdims=True)
    exp_F = np.exp(F_shifted)
    proba = exp_F / exp_F.sum(axis=1, keepdims=True)
    g_np, h_np = om.multiclass_grad_hess(proba, np.eye(K)[yi], w)
    seq = np.zeros(n)
    for k in range(K):
        seq = seq + exp_F[:, k]
    g_seq, h_seq = om.multiclass_grad_hess(exp_F / seq[:, None], np.eye(K)[yi], w)
    bars = []
    for name, a, b in (("grad", g_dev, g_np), ("hess", h_dev, h_np)):
        worst = float(np.max(np.abs(a - b) / (np.finfo(np.float64).eps * w[:, None])))
        same = float(np.mean(a == b))
        print(f"[result] multiclass K={K} {name}: {100 * same:.3f}% bit-identical, "
              f"max |diff| {worst:.2f} ulp(1) x w", flush=True)
        bars.append((name, worst, same))
    for (name, worst, same), alt in zip(bars, (g_seq, h_seq)):
        dev = g_dev if name == "grad" else h_dev
        same_seq = float(np.mean(dev == alt))
        print(f"[result] multiclass K={K} {name}: {100 * same_seq:.3f}% bit-identical to the "
              f"class-order sum", flush=True)
        assert worst <= 8.0, (name, worst)
        assert same >= 0.75, (name, same)
        if K >= 8:
            assert same >= same_seq + 0.05, (name, same, same_seq)


@pytest.mark.gpu
@pytest.mark.parametrize("K,subsample", [(3, None), (9, None), (4, 1.0)])
def test_multiclass_round_paths_agree(engine, monkeypatch, K, subsample):
    """A round in one call (mc_round_trees: the K trees with device replay
    and one readback, the next round's rows made meanwhile on the rows
    stream) against the same round in separate calls without the look-ahead
    (mc_round_sampled, mc_build_trees, mc_loss), against the K trees one
    class at a time (mc_build_tree: host replay per tree), against the rows
    in the reference's order from a host-rows sampler instead of the
    device-permuted, sorted ones, and against the one-call round on its
    fallbacks: the host replay (forced), a node table too small for the
    first round's trees (every class rebuilt on the host-driven path, then
    grown) and the replay reading the node table from HBM.  Trees, split
    gains, losses and scores must be identical.  (subsample=1.0: every row
    in every round, without draws.)"""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1, _native
    X, y = _mc_data(9000, 9, K, seed=60 + K, nan_frac=0.05)
    params = dict(n_estimators=3, max_depth=5, n_bins=255, random_state=7,
                  class_weight="balanced_sqrt")
    if subsample is not None:
        params["subsample"] = subsample
    hooks = ("BSSCL_TEST_HOST_REPLAY", "BSSCL_TEST_NODE_CAP", "BSSCL_TEST_REPLAY_GLOBAL")

    def separate(per_class):
        def round_trees(self, sampler, max_leaves, *args):
            feats = self.mc_round_sampled(sampler)
            if per_class:
                trees = [self.mc_build_tree(k, feats, max_leaves, *args)
                         for k in range(self._mc[1])]
            else:
                trees = self.mc_build_trees(feats, max_leaves, *args)
            return feats, trees, self.mc_loss()
        return round_trees

    sampler_init = _native.Sampler.__init__

    def host_rows_sampler(self, *args, **kw):
        sampler_init(self, *args, **dict(kw, device_rows=False))

    fits = {}
    for mode, env in [("one_call", {}), ("separate", {}), ("per_class", {}), ("host_rows", {}),
                      ("host", {"BSSCL_TEST_HOST_REPLAY": "1"}),
                      ("regrow", {"BSSCL_TEST_NODE_CAP": "9"}),
                      ("global", {"BSSCL_TEST_REPLAY_GLOBAL": "1"})]:
        print(f"[case] multiclass round path {mode} K={K} subsample={subsample}", flush=True)
        for k in hooks:
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        with monkeypatch.context() as mp:
            if mode in ("separate", "per_class"):
                mp.setattr(_native.Engine, "mc_round_trees", separate(mode == "per_class"))
            if mode == "host_rows":
                mp.setattr(_native.Sampler, "__init__", host_rows_sampler)
            est = HybridHistGBMNumbaV1_0_1(verbose=False, **params).fit(X, y)
        fits[mode] = (est, est.predict_proba(X))
    for k in hooks:
        monkeypatch.delenv(k, raising=False)
    ref, ref_p = fits["one_call"]
    for mode in ("separate", "per_class", "host_rows", "host", "regrow", "global"):
        got, got_p = fits[mode]
        assert got.train_loss_history_ == ref.train_loss_history_, mode
        for k in range(K):
            assert len(got.mc_trees[k]) == len(ref.mc_trees[k]) == params["n_estimators"]
            for a, b in zip(ref.mc_trees[k], got.mc_trees[k]):
                nc = a[5]
                assert nc == b[5], (mode, k)
                for i in (0, 1, 2, 3, 4, 6):
                    np.testing.assert_array_equal(a[i][:nc], b[i][:nc], err_msg=f"{mode} {k}")
        np.testing.assert_array_equal(got_p, ref_p, err_msg=mode)


@pytest.mark.gpu
def test_multiclass_round_ahead_handed_back(engine):
    """An early-stopped multiclass fit leaves a round taken ahead by the
    engine; the fit hands it back before closing its sampler, and the next
    fits on the same engine (multiclass, then binary) equal fresh ones."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    X, y = _mc_data(8000, 9, 4, seed=71)
    Xv, yv = _mc_data(2000, 9, 4, seed=72)
    yv = np.random.default_rng(73).permutation(yv)  # labels unrelated to X: stops early
    est = HybridHistGBMNumbaV1_0_1(verbose=False, n_estimators=40, max_depth=4, n_bins=64,
                                   learning_rate=1.0, early_stopping_rounds=1, random_state=3)
    est.fit(X, y, eval_set=[(Xv, yv)])
    assert len(est.mc_trees[0]) < 40  # stopped early, with rounds left in the sampler
    params = dict(verbose=False, n_estimators=3, max_depth=4, n_bins=64, random_state=5)
    a = HybridHistGBMNumbaV1_0_1(**params).fit(X, y)
    b = HybridHistGBMNumbaV1_0_1(**params).fit(X, y)
    assert a.train_loss_history_ == b.train_loss_history_
    np.testing.assert_array_equal(a.predict_proba(X), b.predict_proba(X))
    yb = (y == y[0]).astype(np.int64)
    c = HybridHistGBMNumbaV1_0_1(**params).fit(X, yb)
    d = HybridHistGBMNumbaV1_0_1(**params).fit(X, yb)
    assert c.train_loss_history_ == d.train_loss_history_


@pytest.mark.gpu
def test_multiclass_trees_from_int64_rows(engine):
    """A round whose rows come as int64 sample indices (bsscl_mc_round, in
    the reference's order) has no int32 row list: mc_build_trees then
    gathers each class's root itself.  Its trees and scores equal the
    per-class path's (mc_build_tree) on a second engine from the same
    state."""
    from bsscl_gbm import _native
    rng = np.random.default_rng(81)
    n, F, K = 20000, 12, 4
    codes = rng.integers(0, 40, (n, F)).astype(np.uint8)
    y = rng.integers(0, K, n).astype(np.int64)
    w = rng.uniform(0.5, 2.0, n)
    bc = np.full(F, 40, np.int32)
    rows = rng.permutation(n)[: int(0.8 * n)].astype(np.int64)
    feats = np.sort(rng.permutation(F)[:9]).astype(np.int32)
    args = (31, 5, 5, 3.0, bc, 40, 1.0, 0.0, 0.3)
    other = _native.Engine(0)
    try:
        got = {}
        for name, eng in (("batched", engine), ("per_class", other)):
            eng.load_codes(0, codes)
            eng.mc_begin(y, K, w)
            eng.mc_round(rows)
            if name == "batched":
                trees = eng.mc_build_trees(feats, *args)
            else:
                trees = [eng.mc_build_tree(k, feats, *args) for k in range(K)]
            got[name] = (trees, eng.mc_scores())
        (ta, fa), (tb, fb) = got["batched"], got["per_class"]
        for k in range(K):
            nc = ta[k][5]
            assert nc == tb[k][5] and nc > 1, k
            for i in (0, 1, 2, 3, 4, 6):
                np.testing.assert_array_equal(ta[k][i][:nc], tb[k][i][:nc], err_msg=str(k))
        np.testing.assert_array_equal(fa, fb)
    finally:
        other.close()


@pytest.mark.gpu
@pytest.mark.parametrize("K", [3, 9, 16])
def test_multiclass_predict_proba_device_equals_numpy_softmax(engine, K):
    """A multiclass model's predict_proba with the softmax on the device
    (bsscl_predict_proba_mc) against the reference's NumPy softmax
    (est:2327-2332 at est:3315) of the same per-class scores: within 4 ulp
    of 1 and mostly bit-identical (the device's exp may round a last bit
    differently, more often with more classes per row: the same bar as the
    gradients above).  A class without trees scores 0.0, as the reference's
    zero-initialised column does."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    print(f"[case] multiclass predict_proba on the device K={K}", flush=True)
    X, y = _mc_data(8000, 9, K, seed=60 + K)
    m = HybridHistGBMNumbaV1_0_1(n_estimators=6, max_depth=4, random_state=2,
                                 verbose=False).fit(X, y)
    Xp, _ = _mc_data(30000, 9, K, seed=70 + K, nan_frac=0.05)
    for case in ("fitted", "empty_class"):
        if case == "empty_class":
            m.mc_trees[1] = []
            m._pack_trees()
        F = m._raw_score(Xp)
        want = m._softmax(F)
        got = m.predict_proba(Xp)
        worst = float(np.max(np.abs(got - want))) / np.finfo(np.float64).eps
        same = float(np.mean(got == want))
        print(f"[result] multiclass K={K} {case} predict_proba on the device: "
              f"{100 * same:.3f}% bit-identical, max |diff| {worst:.2f} ulp(1)", flush=True)
        assert got.shape == (len(Xp), K)
        assert worst <= 4.0 and same >= 0.75, (case, worst, same)
        np.testing.assert_array_equal(m.predict(Xp), m.classes_[np.argmax(got, axis=1)])
