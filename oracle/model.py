"""CPU restatement of the reference's binary histogram-GBM path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of bench.py, always as the checker or the
timed baseline.  The product package never imports it.

Host logic follows ``src/bsscl_gbm/estimator_v1_0_1.py`` ("est:" below) with
the same NumPy calls in the same order; the hot loops call ``oracle.c``
through ctypes.  ``OracleGBM`` reproduces ``HybridHistGBMNumbaV1_0_1`` for
``objective='auto'`` with two classes, ``grow_policy='leaf'``,
``sampling_method='uniform'``, ``boosting_type='gbdt'``, numeric features.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build():
    """Compile oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i32, i64, f64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_double
        L.oracle_bin_features.argtypes = [P, ctypes.c_int, i64, i32, P, i32, P,
                                          ctypes.c_int, P]
        L.oracle_build_tree_leafwise.argtypes = [
            P, ctypes.c_int, i64, i32, P, P, P, i64, P, i32, i32, i32, i32,
            f64, P, i32, f64, f64, P, P, P, P, P, P, P, P, P, P, P, P]
        L.oracle_predict_tree.argtypes = [P, ctypes.c_int, i64, i32, P, P, P, P,
                                          P, P]
        L.oracle_predict_all_trees.argtypes = [P, ctypes.c_int, i64, i32, P, P,
                                               P, P, P, P, i32, f64, P]
        L.oracle_post_prune.argtypes = [P, P, P, P, f64, i32]
        L.oracle_hist_stats.argtypes = [P, P, ctypes.c_int]
        L.oracle_hist_stats.restype = None
        for name in ("oracle_bin_features", "oracle_build_tree_leafwise",
                     "oracle_predict_tree", "oracle_predict_all_trees"):
            getattr(L, name).restype = ctypes.c_int
        L.oracle_post_prune.restype = None
        _lib = L
    return _lib


def hist_stats(reset=False):
    """(seconds, row x feature updates) the builder's histogram phase took
    since the last reset (the CPU baseline's histogram rate)."""
    sec = ctypes.c_double()
    rf = ctypes.c_int64()
    lib().oracle_hist_stats(ctypes.byref(sec), ctypes.byref(rf), int(bool(reset)))
    return sec.value, rf.value


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------------
# Binning (est:2073-2189)
# --------------------------------------------------------------------------

def weighted_quantiles(values, weights, q):
    """est:2114-2124: the quantiles q of ``values`` under ``weights``.  Each
    sorted value sits at the midpoint of its weight's share of the total,
    (cumsum(w) - w/2) / sum(w), and q is interpolated linearly between those
    positions (clamped to the end values outside them)."""
    sorter = np.argsort(values)
    v = values[sorter]
    w = weights[sorter]
    pos = (np.cumsum(w) - 0.5 * w) / np.sum(w)
    return np.interp(q, pos, v)


def _column_edges(col, n_bins, weights=None):
    """One feature of ``_build_bin_edges`` (est:2092-2133): (edges, count,
    has_nan).  ``weights`` (the rows' sample weights) selects the weighted
    quantiles of est:2114-2124 for the edges of a column with more distinct
    values than bins."""
    has_nan = np.any(np.isnan(col))
    if has_nan:
        col_clean = col[~np.isnan(col)]
        if len(col_clean) == 0:
            return np.array([0.0, 1.0]), 1, True
    else:
        col_clean = col
    n_unique = len(np.unique(col_clean))
    max_numeric = n_bins - (1 if has_nan else 0)
    if n_unique <= max_numeric:
        e = np.sort(np.unique(col_clean))
    else:
        q = np.linspace(0, 1, min(max_numeric + 1, n_unique))
        if weights is not None:
            w_clean = weights[~np.isnan(col)] if has_nan else weights
            e = np.unique(weighted_quantiles(col_clean, w_clean, q))
        else:
            e = np.unique(np.percentile(col_clean, q * 100))
    e = np.append(e, e[-1] + 1e-8)
    return e, len(e) - 1 + (1 if has_nan else 0), has_nan


def build_bin_edges(X, n_bins, threads=1, sample_weight=None):
    """``_build_bin_edges`` without the categorical branch (est:2073-2141).
    Returns (edges_2d, bin_counts, nan_bin_id).  ``sample_weight`` selects
    the weighted-quantile branch (est:2114-2124, scale_pos_weight).  With
    ``threads`` > 1 the columns are processed concurrently (each column's
    NumPy calls are unchanged, so the result is the same)."""
    F = X.shape[1]
    bin_counts = np.zeros(F, dtype=np.int32)
    nan_bin_id = np.full(F, -1, dtype=np.int32)
    if threads > 1:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(threads) as pool:
            per = list(pool.map(lambda j: _column_edges(X[:, j], n_bins, sample_weight), range(F)))
    else:
        per = [_column_edges(X[:, j], n_bins, sample_weight) for j in range(F)]
    edges = []
    for j, (e, count, has_nan) in enumerate(per):
        edges.append(e)
        bin_counts[j] = count
        if has_nan:
            nan_bin_id[j] = 0
    max_b = int(np.max(bin_counts)) + 1
    edges_2d = np.zeros((F, max_b), dtype=np.float64)
    for j, e in enumerate(edges):
        edges_2d[j, :len(e)] = e
        edges_2d[j, len(e):] = e[-1]
    return edges_2d, bin_counts, nan_bin_id


def bin_features(X, edges_2d, bin_counts, nan_bin_id, strategy):
    """``_bin_features`` (est:2144-2189): NaN placeholder 0.0, kernel codes,
    +1 shift of NaN-feature codes in the code dtype, NaN -> 0."""
    max_bins = int(np.max(bin_counts))
    dtype = np.uint8 if max_bins <= 255 else np.uint16
    has_any_nan = nan_bin_id is not None and np.any(nan_bin_id >= 0)
    Xs = X
    nan_mask = None
    if has_any_nan:
        nan_mask = np.isnan(X)
        Xs = X.copy()
        Xs[nan_mask] = 0.0
    Xs = np.ascontiguousarray(Xs)
    if Xs.dtype not in (np.float32, np.float64):
        Xs = Xs.astype(np.float64)
    n, F = Xs.shape
    out16 = np.empty((n, F), dtype=np.uint16)
    e = np.ascontiguousarray(edges_2d, dtype=np.float64)
    bc = np.ascontiguousarray(bin_counts, dtype=np.int32)
    lib().oracle_bin_features(_p(Xs), int(Xs.dtype == np.float64), n, F, _p(e),
                              e.shape[1], _p(bc), int(strategy == "hybrid"),
                              _p(out16))
    codes = out16.astype(dtype)
    if has_any_nan:
        for j in range(F):
            if nan_bin_id[j] >= 0:
                codes[:, j] += dtype(1)
                codes[nan_mask[:, j], j] = 0
    return codes


# --------------------------------------------------------------------------
# Tree builder / prediction wrappers
# --------------------------------------------------------------------------

def build_tree(X_bin, grad, hess, sample_indices, feature_indices, max_leaves,
               max_depth, min_samples_leaf, min_child_weight, bin_counts,
               max_bins, reg_lambda, gamma, trace=False, forced=None,
               forced_pops=None):
    """``_build_tree_leafwise`` (est:517-823); returns the reference 7-tuple,
    plus (partition counts per split, number of pops) when ``trace``.

    ``forced`` ({node id: (feature, bin)}) replaces the argmax of those
    nodes' split searches by the given candidate (with the gain this builder
    computes for it); a tie-following comparison uses it to adopt the other
    builder's choice at a certified gain tie.  ``forced_pops`` ({split
    index s: node id}) makes the pop that would make split s take that node
    instead of the max-gain candidate (the other builder's order where two
    nodes' gains tie).  ValueError when a forced split or pop is not a
    candidate."""
    X_bin = np.ascontiguousarray(X_bin)
    u16 = int(X_bin.dtype == np.uint16)
    assert X_bin.dtype in (np.uint8, np.uint16)
    n, F = X_bin.shape
    grad = np.ascontiguousarray(grad, dtype=np.float64)
    hess = np.ascontiguousarray(hess, dtype=np.float64)
    si = np.ascontiguousarray(sample_indices, dtype=np.int64)
    fi = np.ascontiguousarray(feature_indices, dtype=np.int32)
    bc = np.ascontiguousarray(bin_counts, dtype=np.int32)
    M = 2 * max_leaves + 2
    tf = np.empty(M, np.int32)
    tt = np.empty(M, np.int64)
    tv = np.empty(M, np.float64)
    tl = np.empty(M, np.int32)
    tr = np.empty(M, np.int32)
    sg = np.empty(M, np.float64)
    nc = np.zeros(1, np.int32)
    tc = np.zeros(2 * max_leaves + 2, np.int64)
    tp = np.zeros(1, np.int32)
    ff = fb = None
    if forced:
        ff = np.full(M, -1, np.int32)
        fb = np.zeros(M, np.int32)
        for node, (f, b) in forced.items():
            ff[int(node)] = int(f)
            fb[int(node)] = int(b)
    fp = None
    if forced_pops:
        fp = np.full(max(1, max_leaves), -1, np.int32)
        for k, node in forced_pops.items():
            fp[int(k)] = int(node)
    rc = lib().oracle_build_tree_leafwise(
        _p(X_bin), u16, n, F, _p(grad), _p(hess), _p(si), len(si), _p(fi),
        len(fi), int(max_leaves), int(max_depth), int(min_samples_leaf),
        float(min_child_weight), _p(bc), int(max_bins), float(reg_lambda),
        float(gamma), _p(tf), _p(tt), _p(tv), _p(tl), _p(tr), _p(nc), _p(sg),
        _p(tc), _p(tp), None if ff is None else _p(ff), None if fb is None else _p(fb),
        None if fp is None else _p(fp))
    if rc == 2:
        raise ValueError(f"forced split or pop is not a candidate: {forced} {forced_pops}")
    if rc != 0:
        raise MemoryError("oracle tree builder allocation failed")
    lib().oracle_post_prune(_p(tf), _p(tl), _p(tr), _p(sg), float(gamma),
                            int(nc[0]))
    tree = (tf, tt, tv, tl, tr, int(nc[0]), sg)
    if trace:
        n_split = int(np.sum(tf[:nc[0]] >= 0))
        return tree, tc[:2 * n_split].reshape(-1, 2), int(tp[0])
    return tree


def predict_tree(X_bin, tree):
    X_bin = np.ascontiguousarray(X_bin)
    tf, tt, tv, tl, tr, nc, _ = tree
    n, F = X_bin.shape
    out = np.empty(n, np.float64)
    a = [np.ascontiguousarray(x[:nc]) for x in (tf, tt, tv, tl, tr)]
    lib().oracle_predict_tree(_p(X_bin), int(X_bin.dtype == np.uint16), n, F,
                              *[_p(x) for x in a], _p(out))
    return out


def pack_trees(trees):
    """``_pack_tree_list`` (est:2192-2216)."""
    total = sum(t[5] for t in trees)
    features = np.empty(total, np.int16)
    thresholds = np.empty(total, np.int64)
    values = np.empty(total, np.float64)
    left = np.empty(total, np.int32)
    right = np.empty(total, np.int32)
    offsets = np.empty(len(trees) + 1, np.int32)
    off = 0
    for t, (tf, tt, tv, tl, tr, nc, _) in enumerate(trees):
        offsets[t] = off
        features[off:off + nc] = tf[:nc]
        thresholds[off:off + nc] = tt[:nc]
        values[off:off + nc] = tv[:nc]
        left[off:off + nc] = tl[:nc]
        right[off:off + nc] = tr[:nc]
        off += nc
    offsets[len(trees)] = off
    return dict(features=features, thresholds=thresholds, values=values,
                left=left, right=right, offsets=offsets)


def predict_all_trees(X_bin, packed, n_trees, lr):
    X_bin = np.ascontiguousarray(X_bin)
    n, F = X_bin.shape
    out = np.empty(n, np.float64)
    lib().oracle_predict_all_trees(
        _p(X_bin), int(X_bin.dtype == np.uint16), n, F,
        _p(packed["features"]), _p(packed["thresholds"]),
        _p(packed["values"]), _p(packed["left"]), _p(packed["right"]),
        _p(packed["offsets"]), int(n_trees), float(lr), _p(out))
    return out


# --------------------------------------------------------------------------
# Binary logistic loss (est:2861, 2873-2874, 2320-2325, 3335)
# --------------------------------------------------------------------------

def binary_proba(F):
    """p = 1 / (1 + exp(-clip(F, -500, 500))) (est:2861, est:3335)."""
    return 1.0 / (1.0 + np.exp(-np.clip(F, -500, 500)))


def binary_grad_hess(F, y, w, grad, hess):
    """grad = w (p - y), hess = w p (1 - p) into the given buffers
    (est:2861, 2873-2874)."""
    p = binary_proba(F)
    grad[:] = w * (p - y)
    hess[:] = w * p * (1.0 - p)


def multiclass_grad_hess(proba, y_onehot, sample_weight):
    """Softmax gradients and hessians of every class, (n, K) each:
    est:3013-3014, and the hessian floor of est:3019 applied to every class."""
    grad_all = sample_weight[:, None] * (proba - y_onehot)
    hess_all = sample_weight[:, None] * proba * (1.0 - proba)
    return grad_all, np.maximum(hess_all, 1e-8)


def binary_logloss(y, F):
    """``_compute_logloss`` (est:2320-2325): unweighted mean of the log-loss
    of p clipped to [1e-15, 1 - 1e-15]."""
    pc = np.clip(binary_proba(F), 1e-15, 1 - 1e-15)
    return -np.mean(y * np.log(pc) + (1 - y) * np.log(1 - pc))


# --------------------------------------------------------------------------
# Estimator restatement
# --------------------------------------------------------------------------

class OracleGBM:
    """Binary-classification restatement of ``HybridHistGBMNumbaV1_0_1``
    (est:1820-1923 constructor defaults, est:3070-3271 fit,
    est:3274-3336 predict_proba)."""

    def __init__(self, n_estimators="auto", max_depth="auto",
                 learning_rate="auto", n_bins="auto", reg_lambda=1.0,
                 min_samples_leaf=5, min_child_weight="auto", gamma="auto",
                 subsample="auto", colsample_bytree="auto",
                 class_weight="balanced_sqrt", max_leaves=31,
                 binning_strategy="auto", random_state=None, edge_threads=1,
                 scale_pos_weight=None, objective="auto"):
        self.binning_strategy_init = binning_strategy
        self.n_estimators_init = n_estimators
        self.max_depth_init = max_depth
        self.learning_rate_init = learning_rate
        self.n_bins_init = n_bins
        self.reg_lambda = reg_lambda
        self.min_samples_leaf = min_samples_leaf
        self.min_child_weight_init = min_child_weight
        self.gamma_init = gamma
        self.subsample_init = subsample
        self.colsample_init = colsample_bytree
        self.class_weight = class_weight
        self.scale_pos_weight = scale_pos_weight
        self.objective = objective  # 'auto' or 'binary' (the reference never resolves 'auto')
        self.max_leaves = max_leaves
        self.random_state = random_state
        self.edge_threads = edge_threads  # columns of the edge pass run concurrently
        self.n_estimators = 100 if n_estimators == "auto" else n_estimators
        self.max_depth = 5 if max_depth == "auto" else max_depth
        self.learning_rate = 0.1 if learning_rate == "auto" else learning_rate
        self.n_bins = 256 if n_bins == "auto" else n_bins
        self.min_child_weight = 1.0 if min_child_weight == "auto" else min_child_weight
        self.gamma = 0.0 if gamma == "auto" else gamma
        self.subsample = 0.8 if subsample == "auto" else subsample
        self.colsample_bytree = 0.8 if colsample_bytree == "auto" else colsample_bytree
        self.trees = []
        self.train_loss_history_ = []

    def _adaptive(self, X):
        """est:1925-2029 (K = number of classes)."""
        n, p = X.shape
        K = getattr(self, "n_classes_", 2)
        if self.binning_strategy_init == "auto":
            self.binning_strategy = "hybrid" if (n > 20000 or p > 40) else "standard"
        else:
            self.binning_strategy = self.binning_strategy_init
        if self.max_depth_init == "auto":
            if K > 10:
                self.max_depth = min(8, max(4, int(np.log2(max(n // 8, 8)))))
            else:
                self.max_depth = min(6, max(3, int(np.log2(max(n // 10, 8)))))
        if self.learning_rate_init == "auto":
            # The reference computes np.std(X) unconditionally; its value is
            # only read when n <= 20000.
            data_std = np.std(X) if n <= 20000 else 0.0
            if n > 20000:
                self.learning_rate = 0.08
            elif data_std > 2.0:
                self.learning_rate = 0.10
            elif data_std > 1.5:
                self.learning_rate = 0.12
            elif data_std > 1.0:
                self.learning_rate = 0.15
            elif data_std > 0.5:
                self.learning_rate = 0.18
            else:
                self.learning_rate = 0.20
            if K > 10:
                self.learning_rate *= 0.75
            elif K > 6:
                self.learning_rate *= 0.85
        if self.n_bins_init == "auto":
            self.n_bins = min(256, p * 8 + 32)
        if self.n_estimators_init == "auto":
            if K <= 2:
                self.n_estimators = 150
            elif K <= 6:
                self.n_estimators = max(150, min(300, n // 10))
            elif K <= 15:
                self.n_estimators = max(200, min(400, n // 8))
            else:
                self.n_estimators = max(250, min(500, n // 6))
        if self.gamma_init == "auto":
            self.gamma = 0.0
        if self.min_child_weight_init == "auto":
            self.min_child_weight = 3.0 if n > 20000 else (2.0 if n > 5000 else 1.0)
        if self.subsample_init == "auto":
            self.subsample = 0.5 if n > 1000000 else (0.75 if n > 20000 else 0.8)
        if n > 1000000:
            self.reg_lambda = max(self.reg_lambda, 5.0)
        if self.colsample_init == "auto":
            self.colsample_bytree = 0.7 if p > 40 else 0.8
        self.max_leaves = 63 if n > 10000 else (15 if n < 2000 else 31)

    def _class_weights(self, y):
        """est:2570-2603: scale_pos_weight with objective='binary' replaces
        the class weights by 1 for class 0 and scale_pos_weight for class 1
        (with the default objective 'auto' the reference ignores it)."""
        n = len(y)
        K = getattr(self, "n_classes_", 2)
        if self.scale_pos_weight is not None and self.objective == "binary":
            w = np.ones(n, dtype=np.float64)
            w[y == 1] = self.scale_pos_weight
            return w
        if self.class_weight not in ("balanced", "balanced_sqrt"):
            return np.ones(n, dtype=np.float64)
        w = np.ones(n, dtype=np.float64)
        for k in range(K):
            n_k = np.sum(y == k)
            w_k = n / (K * max(n_k, 1))
            if self.class_weight == "balanced_sqrt":
                w_k = w_k ** 0.35
            w[y == k] = w_k
        return w

    def fit(self, X, y, max_rounds=None, round_callback=None, tree_hook=None):
        """est:3070-3271 then est:2825-2944.  ``max_rounds`` stops the
        boosting loop early (used to time a bounded CPU sample);
        ``round_callback(m, grad, hess, sample_idx, feat_idx, tree)`` sees
        each round's tree-builder inputs and output.  ``tree_hook`` (same
        arguments; with the class index after ``m`` for multiclass) returns
        the tree the round keeps: a
        tie-following comparison returns this builder's tree rebuilt with
        the other builder's choices at certified gain ties, so the two fits
        stay on one trajectory."""
        self.classes_ = np.unique(y)
        self.n_classes_ = len(self.classes_)
        assert self.n_classes_ >= 2, "oracle covers classification with 2+ classes"
        self._is_multiclass = self.n_classes_ > 2
        label_map = {c: i for i, c in enumerate(self.classes_)}
        y = np.array([label_map[v] for v in y], dtype=np.int64)
        self.trees = []
        self.train_loss_history_ = []
        self.n_features_in_ = X.shape[1]
        rng = np.random.RandomState(self.random_state)
        if not np.issubdtype(X.dtype, np.floating) or X.dtype == np.float16:
            X = X.astype(np.float64)
        self._adaptive(X)
        edge_w = None  # est:3211-3215: scale_pos_weight weights the edges' quantiles
        if self.scale_pos_weight is not None and self.objective == "binary":
            edge_w = np.ones(len(y), dtype=np.float64)
            edge_w[y == 1] = self.scale_pos_weight
        self.bin_edges, self.feature_bin_counts, self._nan_bin_id = \
            build_bin_edges(X, self.n_bins, threads=self.edge_threads, sample_weight=edge_w)
        self._max_bins = int(np.max(self.feature_bin_counts))
        X_bin = bin_features(X, self.bin_edges, self.feature_bin_counts,
                             self._nan_bin_id, self.binning_strategy)
        self.X_bin_ = X_bin

        if self._is_multiclass:
            return self._fit_multiclass(X_bin, y, rng, max_rounds, round_callback, tree_hook)
        n = len(y)
        F_cnt = X_bin.shape[1]
        w_init = self._class_weights(y)
        p0 = np.clip(np.average(y, weights=w_init), 1e-7, 1.0 - 1e-7)
        self.base_score_ = np.log(p0 / (1.0 - p0))
        F = np.full(n, self.base_score_)
        n_sub = max(1, int(n * self.subsample))
        f_sub = max(1, int(F_cnt * self.colsample_bytree))
        w = self._class_weights(y)
        all_rows = np.arange(n, dtype=np.int64)
        all_feats = np.arange(F_cnt, dtype=np.int32)
        grad = np.zeros(n, dtype=np.float64)
        hess = np.zeros(n, dtype=np.float64)
        rounds = self.n_estimators if max_rounds is None else min(max_rounds, self.n_estimators)
        import time as _time
        self.round_times_ = [_time.perf_counter()]
        for m in range(rounds):
            binary_grad_hess(F, y, w, grad, hess)
            # est:2502-2517
            if self.subsample < 1.0:
                rng.shuffle(all_rows)
                sample_idx = all_rows[:n_sub].copy()
            else:
                sample_idx = all_rows.copy()
            if self.colsample_bytree < 1.0:
                rng.shuffle(all_feats)
                feat_idx = np.sort(all_feats[:f_sub]).copy()
            else:
                feat_idx = all_feats.copy()
            tree = build_tree(X_bin, grad, hess, sample_idx, feat_idx,
                              self.max_leaves, self.max_depth,
                              self.min_samples_leaf, self.min_child_weight,
                              self.feature_bin_counts, self._max_bins,
                              self.reg_lambda, self.gamma)
            if tree_hook is not None:
                tree = tree_hook(m, grad, hess, sample_idx, feat_idx, tree)
            if round_callback is not None:
                round_callback(m, grad, hess, sample_idx, feat_idx, tree)
            self.trees.append(tree)
            F += self.learning_rate * predict_tree(X_bin, tree)
            self.train_loss_history_.append(binary_logloss(y, F))
            self.round_times_.append(_time.perf_counter())
        self.F_train_ = F
        self._packed = pack_trees(self.trees)
        return self

    @staticmethod
    def _softmax(F):
        """est:2327-2332."""
        F_shifted = F - F.max(axis=1, keepdims=True)
        exp_F = np.exp(F_shifted)
        return exp_F / exp_F.sum(axis=1, keepdims=True)

    @staticmethod
    def _multiclass_logloss(y_onehot, F):
        """est:2334-2341."""
        F_shifted = F - F.max(axis=1, keepdims=True)
        exp_F = np.exp(F_shifted)
        proba = exp_F / exp_F.sum(axis=1, keepdims=True)
        proba = np.clip(proba, 1e-15, 1 - 1e-15)
        return -np.mean(np.sum(y_onehot * np.log(proba), axis=1))

    def _fit_multiclass(self, X_bin, y, rng, max_rounds, round_callback, tree_hook=None):
        """est:2949-3065 (gbdt, uniform sampling, no eval set): K trees per
        round from softmax gradients, one bagging draw shared by the K trees.
        ``round_callback(m, k, grad, hess, sample_idx, feat_idx, tree)``;
        ``tree_hook`` (same arguments) returns the tree the round keeps."""
        n = len(y)
        F_cnt = X_bin.shape[1]
        K = self.n_classes_
        y_onehot = np.eye(K, dtype=np.float64)[y]
        F_train = np.zeros((n, K), dtype=np.float64)
        n_sub = max(1, int(n * self.subsample))
        f_sub = max(1, int(F_cnt * self.colsample_bytree))
        sample_weight = self._class_weights(y)
        self.mc_trees = [[] for _ in range(K)]
        all_rows = np.arange(n, dtype=np.int64)
        all_feats = np.arange(F_cnt, dtype=np.int32)
        rounds = self.n_estimators if max_rounds is None else min(max_rounds, self.n_estimators)
        import time as _time
        self.round_times_ = [_time.perf_counter()]
        for m in range(rounds):
            proba = self._softmax(F_train)
            if self.subsample < 1.0:
                rng.shuffle(all_rows)
                sample_idx = all_rows[:n_sub].copy()
            else:
                sample_idx = all_rows.copy()
            if self.colsample_bytree < 1.0:
                rng.shuffle(all_feats)
                feat_idx = np.sort(all_feats[:f_sub]).copy()
            else:
                feat_idx = all_feats.copy()
            grad_all, hess_all = multiclass_grad_hess(proba, y_onehot, sample_weight)
            for k in range(K):
                grad_k = np.ascontiguousarray(grad_all[:, k])
                hess_k = np.ascontiguousarray(hess_all[:, k])
                tree = build_tree(X_bin, grad_k, hess_k, sample_idx, feat_idx,
                                  self.max_leaves, self.max_depth,
                                  self.min_samples_leaf, self.min_child_weight,
                                  self.feature_bin_counts, self._max_bins,
                                  self.reg_lambda, self.gamma)
                if tree_hook is not None:
                    tree = tree_hook(m, k, grad_k, hess_k, sample_idx, feat_idx, tree)
                if round_callback is not None:
                    round_callback(m, k, grad_k, hess_k, sample_idx, feat_idx, tree)
                self.mc_trees[k].append(tree)
                F_train[:, k] += self.learning_rate * predict_tree(X_bin, tree)
            self.train_loss_history_.append(self._multiclass_logloss(y_onehot, F_train))
            self.round_times_.append(_time.perf_counter())
        self.F_train_ = F_train
        self._mc_packed = [pack_trees(t) for t in self.mc_trees]
        return self

    def predict_proba(self, X):
        """est:3274-3336."""
        if not np.issubdtype(X.dtype, np.floating) or X.dtype == np.float16:
            X = X.astype(np.float64)
        X_bin = bin_features(X, self.bin_edges, self.feature_bin_counts,
                             self._nan_bin_id, self.binning_strategy)
        if self._is_multiclass:
            F = np.zeros((len(X), self.n_classes_), dtype=np.float64)
            for k in range(self.n_classes_):
                F[:, k] = predict_all_trees(X_bin, self._mc_packed[k], len(self.mc_trees[k]),
                                            self.learning_rate)
            return self._softmax(F)
        F = predict_all_trees(X_bin, self._packed, len(self.trees),
                              self.learning_rate) + self.base_score_
        proba = binary_proba(F)
        return np.column_stack([1 - proba, proba])

    def predict(self, X):
        """est:3345-3368."""
        proba = self.predict_proba(X)
        if self._is_multiclass:
            return self.classes_[np.argmax(proba, axis=1)]
        return self.classes_[(proba[:, 1] > 0.5).astype(int)]
