"""Drop-in ``HybridHistGBMNumbaV1_0_1`` whose fit/predict run on the MI355X
engine.

The public surface -- constructor parameters and their 'auto' resolution,
``fit``/``predict``/``predict_proba``, ``get_params``/``set_params``, the
fitted attributes (``trees``, ``bin_edges``, ``feature_bin_counts``,
``base_score_``, ``train_loss_history_``, ``feature_importances_``, the packed
tree arrays, ``times``) -- follows the reference class
``HybridHistGBMNumbaV1_0_1`` in src/bsscl_gbm/estimator_v1_0_1.py ("est:"
below, class at est:1776).  Host logic that decides results (parameter
resolution, bin edges, class weights, base score, the random stream) is the
reference's NumPy code path; every per-row loop (binning, gradients, trees,
F updates, prediction) runs in libbsscl_hip.so.

Covered: binary and multiclass (softmax, K trees per round) classification
(objective 'auto' or 'binary'), grow_policy='leaf', sampling_method='uniform',
boosting_type='gbdt', numeric features with NaN, class_weight
None/'balanced'/'balanced_sqrt', scale_pos_weight, eval_set with early
stopping, JSON save_model/load_model.  Other modes of the
reference raise NotImplementedError instead of computing something else.
"""
from __future__ import annotations

import os
import threading
import time

import numpy as np

from . import _native

__all__ = ["HybridHistGBMNumbaV1_0_1"]

_ENGINES: dict = {}
_ENGINES_LOCK = threading.Lock()
# Rows per device pass of the batch-parallel predictions (their codes and
# scores on the device: about 1 GB at 50 features).
_BATCH_ROWS = 1 << 24


def _engine(device: int) -> _native.Engine:
    """Per-process engine cache; a forked child creates its own.  Every
    estimator of the process shares the device's engine, whose matrices and
    boosting state one operation at a time may use: callers hold
    ``eng.lock`` (re-entrant) for a whole fit or prediction, so estimators
    may be fitted and used from several threads."""
    key = (os.getpid(), int(device))
    with _ENGINES_LOCK:
        eng = _ENGINES.get(key)
        if eng is None:
            for k in [k for k in _ENGINES if k[0] != os.getpid()]:
                _ENGINES.pop(k)._h = None  # the parent's handle is not ours to free
            eng = _native.Engine(device)
            eng.lock = threading.RLock()
            _ENGINES[key] = eng
    return eng


def _encode_labels(y):
    """np.unique(y) and the labels as 0 .. K-1 (est:3124-3129), as
    np.searchsorted(classes, y).  Integer labels that are already 0 .. K-1
    (the usual case) skip the sort and the search: counting gives the
    classes, and the labels are their own codes."""
    y = np.asarray(y)
    if y.ndim == 1 and y.size and (y.dtype.kind in "iu" or y.dtype == np.bool_):
        ext = _row_blocks(len(y), lambda a, b: (int(y[a:b].min()), int(y[a:b].max())))
        lo, hi = min(e[0] for e in ext), max(e[1] for e in ext)
        if lo >= 0 and hi <= 1:  # 0/1 labels: which occur follows from one count
            n1 = _count_nonzero(y)
            classes = np.array([v for v, c in ((0, len(y) - n1), (1, n1)) if c], dtype=y.dtype)
            codes = y.astype(np.int64, copy=False)
            return classes, (codes if len(classes) == 2 or n1 == 0 else np.zeros(len(y), np.int64))
        if lo >= 0 and hi < (1 << 16):
            present = np.bincount(y.astype(np.int64, copy=False), minlength=hi + 1) > 0
            classes = np.nonzero(present)[0].astype(y.dtype)
            if len(classes) == hi + 1:  # every value 0 .. hi occurs: codes = labels
                return classes, y.astype(np.int64, copy=False)
            return classes, np.searchsorted(classes, y).astype(np.int64)
    classes = np.unique(y)
    return classes, np.searchsorted(classes, y).astype(np.int64)


def _to_dense(X):
    try:
        import scipy.sparse
        if scipy.sparse.issparse(X):
            return X.toarray()
    except ImportError:
        pass
    return X


def _as_float(X):
    """est:3197-3201: non-float and float16 inputs become float64; float32
    and float64 are kept."""
    X = np.asarray(X)
    if not np.issubdtype(X.dtype, np.floating) or X.dtype == np.float16:
        X = X.astype(np.float64)
    return X


def _sigmoid(F):
    return 1.0 / (1.0 + np.exp(-np.clip(F, -500, 500)))


# Rows from which the estimator's label, count and lookup passes (one
# memory pass each) run in row blocks on a few threads: NumPy's loops
# release the GIL, and each element, or each block's count, is NumPy's own.
# The threads' dispatch cost more than they saved at 1M rows; at 10M they
# gain.
_PASS_THREAD_ROWS = 1 << 22


_POOL = None  # (pid, ThreadPoolExecutor, workers): one per process, made on first use
_POOL_LOCK = threading.Lock()


def _host_pool():
    """The process's thread pool for _row_blocks and its thread count, or
    None with fewer than two CPUs (a child made by fork() makes its own)."""
    global _POOL
    with _POOL_LOCK:
        if _POOL is None or _POOL[0] != os.getpid():
            workers = min(8, os.cpu_count() or 1)
            if workers < 2:
                return None
            from concurrent.futures import ThreadPoolExecutor
            _POOL = (os.getpid(), ThreadPoolExecutor(max_workers=workers,
                                                     thread_name_prefix="bsscl-host"), workers)
        return _POOL[1:]


def _row_blocks(n, fn):
    """[fn(a, b) for the row blocks [a, b) of [0, n)], on the process's
    host threads from _PASS_THREAD_ROWS rows on; one block otherwise."""
    hp = _host_pool() if n >= _PASS_THREAD_ROWS else None
    if hp is None:
        return [fn(0, n)]
    pool, workers = hp
    step = -(-n // (4 * workers))
    futures = [pool.submit(fn, a, min(a + step, n)) for a in range(0, n, step)]
    return [f.result() for f in futures]


def _take(table, idx):
    """table[idx] for a small float64 table and integer indices already in
    range (encoded labels): the same values, gathered in row blocks.  (With
    an output array, np.take's default mode buffers the whole gather to
    check the indices; 'clip' writes in place, 2.6x faster at 1M rows.)"""
    out = np.empty(len(idx), dtype=np.float64)
    _row_blocks(len(idx), lambda a, b: np.take(table, idx[a:b], out=out[a:b], mode='clip'))
    return out


def _count_nonzero(y):
    return sum(_row_blocks(len(y), lambda a, b: int(np.count_nonzero(y[a:b]))))


class _HostPrep:
    """A fit's host work that needs only the labels, on a thread of its own
    while the caller stages and bins X: the bagging stream's sampler
    (est:2502-2517) and, for a binary fit, its class weights and base score
    (est:2570-2603, 2829-2834).  NumPy's loops and the native calls release
    the GIL, so both threads run at once (1M x 28: the 2.6 ms of these
    passes overlap the binning instead of preceding the first round)."""

    def __init__(self, est, eng, rng, y):
        self._sampler = None
        self._binary = None
        self._error = None
        self._thread = threading.Thread(target=self._run, args=(est, eng, rng, y),
                                        name="bsscl-fit-prep", daemon=True)
        self._thread.start()

    def _run(self, est, eng, rng, y):
        # (The label passes first: the sampler's start contends less with
        # the staging copy after it, and its first round still has the
        # binning's remaining time to draw.)
        try:
            if not est._is_multiclass:
                self._binary = est._binary_start(y)
            self._sampler = est._make_sampler(eng, rng, len(y))
        except BaseException as e:  # handed to the fitting thread
            self._error = e

    def result(self):
        """(sampler, (w0, w1, base score) or None); raises what the thread
        raised."""
        self._thread.join()
        if self._error is not None:
            raise self._error
        return self._sampler, self._binary

    def close(self):
        self._thread.join()
        if self._sampler is not None:
            self._sampler.close()
            self._sampler = None


def _percentile_ranks(m, q100, dtype):
    """Ranks np.percentile(col, q100) reads from a NaN-free column of m
    values of `dtype`, and its interpolation weights (NumPy 2.x 'linear'
    method: q = q100 / dtype(100), virtual index (m - 1) * q, neighbours
    floor and floor + 1, both clamped to the last value at or beyond it).
    m may be a column vector of lengths: then row i is column i's."""
    q = np.true_divide(q100, dtype.type(100))
    vi = (m - 1) * q
    prev = np.floor(vi)
    nxt = prev + 1
    above = vi >= m - 1
    prev[above] = -1
    nxt[above] = -1
    below = vi < 0
    prev[below] = 0
    nxt[below] = 0
    prev = prev.astype(np.intp)
    nxt = nxt.astype(np.intp)
    gamma = np.asanyarray(vi - prev, dtype=vi.dtype)
    return np.where(prev < 0, m - 1, prev), np.where(nxt < 0, m - 1, nxt), gamma


def _percentile_lerp(a, b, t):
    """The interpolation np.percentile applies to the neighbours a, b (arrays
    of the column's dtype) with weights t: NumPy's own sequence of ufuncs,
    so the result carries the same roundings."""
    diff_b_a = np.subtract(b, a)
    out = np.asanyarray(np.add(a, diff_b_a * t))
    np.subtract(b, diff_b_a * (1 - t), out=out, where=t >= 0.5,
                casting='unsafe', dtype=type(out.dtype))
    return out


class HybridHistGBMNumbaV1_0_1:
    """Histogram GBM with the reference's parameters (est:1820-1923)."""

    def __init__(self, n_estimators='auto', max_depth='auto', learning_rate='auto',
                 n_bins='auto', reg_lambda=1.0, min_samples_leaf=5,
                 min_child_weight='auto', gamma='auto',
                 subsample='auto', colsample_bytree='auto',
                 class_weight='balanced_sqrt',
                 grow_policy='leaf', max_leaves=31, binning_strategy='auto',
                 monotone_constraints=None, categorical_features=None,
                 early_stopping_rounds=None, verbose=True, random_state=None,
                 objective='auto', focal_gamma=2.0, loss='mse', device='cpu',
                 sampling_method='uniform', top_rate=0.2, other_rate=0.1,
                 scale_pos_weight=None,
                 custom_objective=None,
                 boosting_type='gbdt',
                 dart_rate=0.1,
                 interaction_constraints=None):
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
        # The reference's 'cpu'/'cuda' selects a Numba path; here every
        # device string runs the HIP engine.  An integer selects the GPU.
        self.device = device
        self.sampling_method = sampling_method
        self.top_rate = top_rate
        self.other_rate = other_rate
        self.scale_pos_weight = scale_pos_weight
        self.class_weight = class_weight
        self.grow_policy = grow_policy
        self.custom_objective = custom_objective
        self.boosting_type = boosting_type
        self.dart_rate = dart_rate
        self.interaction_constraints = interaction_constraints
        self.max_leaves = max_leaves
        self.monotone_constraints = monotone_constraints
        self.categorical_features = categorical_features
        self.early_stopping_rounds = early_stopping_rounds
        self.verbose = verbose
        self.random_state = random_state

        self.n_estimators = 100 if n_estimators == 'auto' else n_estimators
        self.max_depth = 5 if max_depth == 'auto' else max_depth
        self.learning_rate = 0.1 if learning_rate == 'auto' else learning_rate
        self.n_bins = 256 if n_bins == 'auto' else n_bins
        self.min_child_weight = 1.0 if min_child_weight == 'auto' else min_child_weight
        self.gamma = 0.0 if gamma == 'auto' else gamma
        self.subsample = 0.8 if subsample == 'auto' else subsample
        self.colsample_bytree = 0.8 if colsample_bytree == 'auto' else colsample_bytree
        self.objective = objective
        self.focal_gamma = focal_gamma
        self.loss = loss
        self.init_score_ = 0.0

        self.trees = []
        self.bin_edges = None
        self.feature_bin_counts = None
        self._max_bins = 0
        self.n_features_in_ = None
        self.n_classes_ = 2
        self.classes_ = None
        self._is_multiclass = False
        self.mc_trees = None
        self.feature_importances_ = None
        self.feature_split_counts_ = None
        self.train_loss_history_ = []
        self.val_loss_history_ = []
        self.n_trees_fitted_ = 0
        self.best_iteration_ = 0
        self.times = {'binning': 0.0, 'training': 0.0, 'inference': 0.0}
        self._packed_features = None
        self._packed_thresholds = None
        self._packed_values = None
        self._packed_left = None
        self._packed_right = None
        self._tree_offsets = None
        self._mc_packed = None
        self._auto_no_weights = False
        self._auto_full_weights = False
        self._categorical_set = set()
        self._is_categorical = None
        self._nan_bin_id = None

    # ------------------------------------------------------------------
    # Pickling: no device handle is ever stored on the instance.
    # ------------------------------------------------------------------
    def _device_index(self):
        return self.device if isinstance(self.device, (int, np.integer)) else 0

    def _check_supported(self):
        unsupported = []
        if self.objective not in ('auto', 'binary'):
            unsupported.append(f"objective={self.objective!r}")
        if self.grow_policy != 'leaf':
            unsupported.append(f"grow_policy={self.grow_policy!r}")
        if self.sampling_method != 'uniform':
            unsupported.append(f"sampling_method={self.sampling_method!r}")
        if getattr(self, 'boosting_type', 'gbdt') != 'gbdt':
            unsupported.append(f"boosting_type={self.boosting_type!r}")
        if self.categorical_features is not None:
            unsupported.append("categorical_features")
        if self.monotone_constraints is not None:
            unsupported.append("monotone_constraints")
        if getattr(self, 'custom_objective', None) is not None:
            unsupported.append("custom_objective")
        if unsupported:
            raise NotImplementedError(
                "the MI355X engine covers the leaf-wise histogram path for classification; "
                "not supported: " + ", ".join(unsupported))

    # ------------------------------------------------------------------
    # est:1925-2029
    # ------------------------------------------------------------------
    def _compute_adaptive_hyperparameters(self, X, y):
        n, p = X.shape
        K = self.n_classes_
        if self.binning_strategy_init == 'auto':
            self.binning_strategy = 'hybrid' if (n > 20000 or p > 40) else 'standard'
        else:
            self.binning_strategy = self.binning_strategy_init
        if self.max_depth_init == 'auto':
            if K > 10:
                self.max_depth = min(8, max(4, int(np.log2(max(n // 8, 8)))))
            else:
                self.max_depth = min(6, max(3, int(np.log2(max(n // 10, 8)))))
        if self.learning_rate_init == 'auto':
            if n > 20000:
                # The reference also computes np.std(X) here; the value only
                # matters for n <= 20000, so it is not computed.
                self.learning_rate = 0.08
            else:
                data_std = np.std(X)
                if data_std > 2.0:
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
        if self.n_bins_init == 'auto':
            self.n_bins = min(256, p * 8 + 32)
        if self.n_estimators_init == 'auto':
            if K <= 2:
                self.n_estimators = 150
            elif K <= 6:
                self.n_estimators = max(150, min(300, n // 10))
            elif K <= 15:
                self.n_estimators = max(200, min(400, n // 8))
            else:
                self.n_estimators = max(250, min(500, n // 6))
        if self.gamma_init == 'auto':
            self.gamma = 0.0
        if self.min_child_weight_init == 'auto':
            if n > 20000:
                self.min_child_weight = 3.0
            elif n > 5000:
                self.min_child_weight = 2.0
            else:
                self.min_child_weight = 1.0
        if self.subsample_init == 'auto':
            if n > 1000000:
                self.subsample = 0.5
            elif n > 20000:
                self.subsample = 0.75
            else:
                self.subsample = 0.8
        if n > 1000000:
            self.reg_lambda = max(self.reg_lambda, 5.0)
        if self.colsample_init == 'auto':
            self.colsample_bytree = 0.7 if p > 40 else 0.8
        if n > 10000:
            self.max_leaves = 63
        elif n < 2000:
            self.max_leaves = 15
        else:
            self.max_leaves = 31
        if self.verbose:
            print("  🔧 Adaptive Hyperparameters:")
            print(f"     n_estimators:  {self.n_estimators}")
            print(f"     max_depth:     {self.max_depth} (from {n} samples)")
            print(f"     learning_rate: {self.learning_rate:.4f}")
            print(f"     n_bins:        {self.n_bins} (from {p} features)")
            print(f"     gamma:         {self.gamma:.2f}")
            print(f"     min_child_w:   {self.min_child_weight:.1f}")
            print(f"     subsample:     {self.subsample}")
            print(f"     colsample:     {self.colsample_bytree}")

    # ------------------------------------------------------------------
    # est:2073-2141 (numeric features)
    # ------------------------------------------------------------------
    def _build_bin_edges(self, X, sample_weight=None, eng=None):
        """Edges of est:2073-2141.  With `eng` (X staged on its device) the
        data passes run there: NaN counts, distinct counts, distinct values
        and the order statistics np.percentile interpolates between; the
        arithmetic between them is the reference's, on the host."""
        if eng is None:
            return self._build_bin_edges_host(X, sample_weight)
        n, n_features = X.shape
        nan_count, n_unique = eng.sort_columns(n_features)
        dtype = X.dtype
        edges = [None] * n_features
        bin_counts = np.zeros(n_features, dtype=np.int32)
        self._nan_bin_id = np.full(n_features, -1, dtype=np.int32)
        lerp_cols = []  # (feature, m, number of quantiles)
        for j in range(n_features):
            has_nan = bool(nan_count[j] > 0)
            m = n - int(nan_count[j])
            if has_nan:
                self._nan_bin_id[j] = 0
                if m == 0:
                    edges[j] = np.array([0.0, 1.0])
                    bin_counts[j] = 1
                    continue
            max_numeric_bins = self.n_bins - (1 if has_nan else 0)
            if n_unique[j] <= max_numeric_bins:
                e = eng.sorted_uniques(j, int(n_unique[j])).astype(dtype)
                edges[j] = e
            else:
                lerp_cols.append((j, m, min(max_numeric_bins + 1, int(n_unique[j]))))
        # One gather for every rank the percentiles read.  Columns with the
        # same number of quantiles share each NumPy call, one row per column
        # (the arithmetic is elementwise, so every value is the one the
        # column's own call gives).
        by_k = {}
        for j, m, k in lerp_cols:
            by_k.setdefault(k, []).append((j, m))
        plans, cols, pos, off = [], [], [], 0
        for k, members in by_k.items():
            js = np.array([j for j, _ in members], dtype=np.int32)
            ms = np.array([m for _, m in members], dtype=np.int64)[:, None]
            q = np.linspace(0, 1, k)
            lo, hi, gamma = _percentile_ranks(ms, q * 100, dtype)
            plans.append((js, off, k, gamma))
            cols.append(np.repeat(js, 2 * k))
            pos.append(np.concatenate([lo, hi], axis=1).ravel())
            off += 2 * k * len(js)
        if plans:
            vals = eng.sorted_gather(np.concatenate(cols), np.concatenate(pos)).astype(dtype)
            for js, off, k, gamma in plans:
                v = vals[off:off + 2 * k * len(js)].reshape(len(js), 2 * k)
                lerp = _percentile_lerp(v[:, :k], v[:, k:], gamma)
                for i, j in enumerate(js):
                    edges[j] = np.unique(lerp[i])
        for j in range(n_features):
            if bin_counts[j] == 1 and self._nan_bin_id[j] == 0 and nan_count[j] == n:
                continue
            e = np.append(edges[j], edges[j][-1] + 1e-8)
            edges[j] = e
            bin_counts[j] = len(e) - 1 + (1 if self._nan_bin_id[j] == 0 else 0)
        return self._edges_2d(edges, bin_counts)

    def _build_bin_edges_host(self, X, sample_weight=None):
        """est:2073-2141 with the reference's NumPy calls on the host: the
        weighted-quantile branch (scale_pos_weight with objective='binary')."""
        edges = []
        n_features = X.shape[1]
        bin_counts = np.zeros(n_features, dtype=np.int32)
        self._nan_bin_id = np.full(n_features, -1, dtype=np.int32)
        for j in range(n_features):
            col = X[:, j]
            nan_mask = np.isnan(col)
            has_nan = bool(np.any(nan_mask))
            if has_nan:
                self._nan_bin_id[j] = 0
                col_clean = col[~nan_mask]
                if len(col_clean) == 0:
                    edges.append(np.array([0.0, 1.0]))
                    bin_counts[j] = 1
                    continue
            else:
                col_clean = col
            uniq = np.unique(col_clean)
            n_unique = len(uniq)
            max_numeric_bins = self.n_bins - (1 if has_nan else 0)
            if n_unique <= max_numeric_bins:
                e = np.sort(uniq)
            else:
                q = np.linspace(0, 1, min(max_numeric_bins + 1, n_unique))
                if sample_weight is not None:
                    sw_clean = sample_weight[~nan_mask] if has_nan else sample_weight
                    sorter = np.argsort(col_clean)
                    c_sorted = col_clean[sorter]
                    sw_sorted = sw_clean[sorter]
                    cw = np.cumsum(sw_sorted) - 0.5 * sw_sorted
                    cw /= np.sum(sw_sorted)
                    e = np.unique(np.interp(q, cw, c_sorted))
                else:
                    e = np.unique(np.percentile(col_clean, q * 100))
            e = np.append(e, e[-1] + 1e-8)
            edges.append(e)
            bin_counts[j] = len(e) - 1 + (1 if has_nan else 0)
        return self._edges_2d(edges, bin_counts)

    @staticmethod
    def _edges_2d(edges, bin_counts):
        n_features = len(edges)
        max_b = int(np.max(bin_counts)) + 1
        edges_2d = np.zeros((n_features, max_b), dtype=np.float64)
        for j, e in enumerate(edges):
            edges_2d[j, :len(e)] = e
            edges_2d[j, len(e):] = e[-1]
        return edges_2d, bin_counts

    # ------------------------------------------------------------------
    # est:2570-2603
    # ------------------------------------------------------------------
    def _class_weight_pair(self, y):
        """(w0, w1): the per-class values of the reference's sample_weight."""
        if self.scale_pos_weight is not None and self.objective == 'binary':
            return 1.0, float(self.scale_pos_weight)
        if self.class_weight not in ('balanced', 'balanced_sqrt'):
            return 1.0, 1.0
        n = len(y)
        n1 = _count_nonzero(y)  # y holds 0 and 1
        w = []
        for k in range(2):
            n_k = n1 if k == 1 else n - n1
            w_k = n / (2 * max(n_k, 1))
            if self.class_weight == 'balanced_sqrt':
                w_k = w_k ** 0.35
            w.append(float(w_k))
        if self.verbose:
            mode = "sqrt-dampened" if self.class_weight == 'balanced_sqrt' else "full"
            print(f"  ⚖️  Class weights ({mode}): class_0={w[0]:.3f}, class_1={w[1]:.3f}")
        return w[0], w[1]

    # ------------------------------------------------------------------
    # est:3070-3271 and est:2825-2944
    # ------------------------------------------------------------------
    def fit(self, X, y, group=None, X_val=None, y_val=None, group_val=None,
            eval_set=None):
        self._group = group
        self._group_val = group_val
        X = _to_dense(X)
        if X_val is not None:
            X_val = _to_dense(X_val)
        if self.max_depth <= 0 and self.max_depth != 'auto':
            raise ValueError(f"max_depth must be > 0, got {self.max_depth}")
        if self.learning_rate <= 0:
            raise ValueError(f"learning_rate must be > 0, got {self.learning_rate}")
        if self.n_estimators <= 0:
            raise ValueError(f"n_estimators must be > 0, got {self.n_estimators}")
        if eval_set is not None and len(eval_set) > 0:
            X_val, y_val = eval_set[0]
            X_val = _to_dense(X_val)
        X = np.asarray(X)
        y = np.asarray(y)
        if X.ndim != 2:
            raise ValueError("X must be a 2-D array")
        if len(y) != X.shape[0]:
            raise ValueError(f"X has {X.shape[0]} rows but y has {len(y)} labels")
        self._check_supported()

        self.classes_, y = _encode_labels(y)
        self.n_classes_ = len(self.classes_)
        self._is_multiclass = self.n_classes_ > 2
        if self.n_classes_ < 2:
            raise NotImplementedError(
                "the MI355X engine needs at least two classes; got "
                f"{self.n_classes_}")
        if y_val is not None:
            y_val = np.asarray(y_val)
            label_map = {c: i for i, c in enumerate(self.classes_)}
            y_val = np.array([label_map[v] for v in y_val], dtype=np.int64)
        if self.verbose:
            print("\n" + "=" * 70)
            print("  Training Hybrid GBM v3.0 — Binary")
            print("=" * 70)

        self.trees = []
        self.mc_trees = None
        self.train_loss_history_ = []
        self.val_loss_history_ = []
        self.n_features_in_ = X.shape[1]
        rng = np.random.RandomState(self.random_state)
        self._mono_arr = None
        self._categorical_set = set()
        self._is_categorical = np.zeros(X.shape[1], dtype=bool)
        X = _as_float(X)
        if X_val is not None:
            X_val = _as_float(X_val)

        self._compute_adaptive_hyperparameters(X, y)
        sample_weight = None
        if self.scale_pos_weight is not None and self.objective in ('binary', 'binary_focal'):
            sample_weight = np.ones(len(y), dtype=np.float64)
            sample_weight[y == 1] = self.scale_pos_weight
        eng = _engine(self._device_index())
        with eng.lock:
            # The bagging stream (est:2502-2517) starts drawing now, so that its
            # first rounds are ready when the boosting loop begins: the draws
            # run on host threads while the device bins X.  The sampler is made,
            # and a binary fit's class weights and base score are computed, on
            # a thread of their own meanwhile: they need only the labels.
            prep = _HostPrep(self, eng, rng, y)
            try:
                self._fit_locked(eng, X, y, X_val, y_val, sample_weight, prep)
            finally:
                prep.close()
        self._pack_trees()
        self._compute_feature_importances()
        if self.verbose:
            print(f"\n  ✓ Training complete! ({self.n_trees_fitted_} trees)")
            print(f"    Binning:  {self.times['binning']:.2f} ms")
            print(f"    Training: {self.times['training']:.2f} ms")
            print(f"    Total:    {self.times['binning'] + self.times['training']:.2f} ms")
        return self

    def _make_sampler(self, eng, rng, n_samples):
        """The native RandomState.shuffle stream for this fit's rounds: rows
        and features per round (est:2502-2517), from rng's current state.
        Binary fits, and multiclass fits whose scores stay on the device,
        hand the draws to the device (the engine applies the swaps); other
        multiclass fits take the rows back on the host."""
        n_features = self.n_features_in_
        n_sub = max(1, int(n_samples * self.subsample))
        f_sub = max(1, int(n_features * self.colsample_bytree))
        do_rows = self.subsample < 1.0
        do_feats = self.colsample_bytree < 1.0
        return _native.Sampler(rng.get_state(), n_samples,
                               n_sub if do_rows else n_samples, do_rows,
                               n_features, f_sub if do_feats else n_features,
                               do_feats, int(self.n_estimators),
                               device_rows=(not self._is_multiclass
                                            or self.n_classes_ <= _native.MC_DEVICE_MAX_CLASSES),
                               device=eng.device)

    def _fit_locked(self, eng, X, y, X_val, y_val, sample_weight, prep):
        """Binning and the boosting loop, with the engine's lock held."""
        t0 = time.perf_counter()
        # Unweighted edges come from the device (X is staged once and binned
        # from there); the weighted-quantile branch stays on the host.
        X = np.ascontiguousarray(X)
        staged = sample_weight is None
        if staged:
            eng.stage_features(X)
        try:
            self.bin_edges, self.feature_bin_counts = self._build_bin_edges(
                X, sample_weight=sample_weight, eng=eng if staged else None)
            self._max_bins = int(np.max(self.feature_bin_counts))
            if self._max_bins > 65536:
                # The reference's codes are uint16 above 255 bins (est:2163-2166).
                raise ValueError(
                    f"n_bins={self.n_bins} gives {self._max_bins} bins for some feature; "
                    "codes are uint16, so at most 65536 bins per feature")
            if staged:
                eng.bin_staged(0, X.shape[0], X.shape[1], X.dtype == np.float64, self.bin_edges,
                               self.feature_bin_counts, self._nan_bin_id)
            else:
                eng.bin_features(0, X, self.bin_edges, self.feature_bin_counts, self._nan_bin_id)
        finally:
            if staged:
                eng.release_staged()
        self.times['binning'] = (time.perf_counter() - t0) * 1000
        n_val = 0
        if X_val is not None and y_val is not None:
            eng.bin_features(1, X_val, self.bin_edges, self.feature_bin_counts, self._nan_bin_id)
            n_val = X_val.shape[0]

        t0_train = time.perf_counter()
        sampler, binary_start = prep.result()
        if self._is_multiclass:
            self._fit_multiclass(eng, y, n_val, y_val, sampler)
        else:
            self._fit_binary(eng, y, n_val, y_val, sampler, binary_start)
        self.times['training'] = (time.perf_counter() - t0_train) * 1000

    def _binary_start(self, y):
        """A binary fit's class weights (w0, w1) and base score, from the
        labels alone."""
        w0, w1 = self._class_weight_pair(y)
        # np.average(y, weights=np.where(y == 1, w1, w0)) of the reference
        # (est:2829-2834): sum(y * w) / sum(w) over the same float64 arrays,
        # built by lookup (y holds 0 and 1), so the sums are NumPy's own.
        sw = _take(np.array([w0, w1]), y)
        weighted_mean = _take(np.array([0.0, w1]), y).sum() / sw.sum()
        p0 = np.clip(weighted_mean, 1e-7, 1.0 - 1e-7)
        return w0, w1, np.log(p0 / (1.0 - p0))

    def _fit_binary(self, eng, y, n_val, y_val, sampler, binary_start):
        w0, w1, self.base_score_ = binary_start
        F_val = np.full(n_val, self.base_score_) if n_val else None
        eng.boost_begin(y, w0, w1, self.base_score_)
        best_val_loss = np.inf
        rounds_no_improve = 0
        hook = getattr(self, '_round_hook', None)
        self._live_sampler = sampler  # read by profiling hooks during the fit
        # Without an eval set every round runs: the engine may enqueue the
        # next round while this one is returned.
        eng.set_pipeline(not n_val and getattr(self, '_pipeline_rounds', True))
        try:
            for m in range(self.n_estimators):
                if hook is not None:
                    hook(m, eng)
                tree, train_loss = eng.boost_round(
                    sampler, self.max_leaves, self.max_depth,
                    self.min_samples_leaf, self.min_child_weight,
                    self.feature_bin_counts, self._max_bins, self.reg_lambda,
                    self.gamma, self.learning_rate)
                self.trees.append(tree)
                self.train_loss_history_.append(train_loss)
                val_loss = None
                if n_val:
                    F_val += self.learning_rate * eng.predict_tree(1, n_val, tree)
                    pv = np.clip(_sigmoid(F_val), 1e-15, 1 - 1e-15)
                    val_loss = -np.mean(y_val * np.log(pv) + (1 - y_val) * np.log(1 - pv))
                    self.val_loss_history_.append(val_loss)
                if self.verbose and ((m + 1) % 20 == 0 or m == 0):
                    msg = f"  ✓ Tree {m+1:>3}/{self.n_estimators}  |  train-loss: {train_loss:.6f}"
                    if val_loss is not None:
                        msg += f"  |  val-loss: {val_loss:.6f}"
                    print(msg)
                if self.early_stopping_rounds is not None and val_loss is not None:
                    if val_loss < best_val_loss:
                        best_val_loss = val_loss
                        self.best_iteration_ = m
                        rounds_no_improve = 0
                    else:
                        rounds_no_improve += 1
                        if rounds_no_improve >= self.early_stopping_rounds:
                            if self.verbose:
                                print(f"\n  ⏹ Early stopping at tree {m+1} (best: {self.best_iteration_+1})")
                            self.trees = self.trees[:self.best_iteration_ + 1]
                            break
        finally:
            eng.set_pipeline(False)
            self._live_sampler = None
        if hook is not None:
            hook(self.n_estimators, eng)
        self.n_trees_fitted_ = len(self.trees)

    # ------------------------------------------------------------------
    # est:2949-3065 (multiclass softmax) and its helpers est:2327-2341
    # ------------------------------------------------------------------
    @staticmethod
    def _softmax(F):
        F_shifted = F - F.max(axis=1, keepdims=True)
        exp_F = np.exp(F_shifted)
        return exp_F / exp_F.sum(axis=1, keepdims=True)

    @staticmethod
    def _compute_multiclass_logloss(y_onehot, F):
        F_shifted = F - F.max(axis=1, keepdims=True)
        exp_F = np.exp(F_shifted)
        proba = exp_F / exp_F.sum(axis=1, keepdims=True)
        proba = np.clip(proba, 1e-15, 1 - 1e-15)
        return -np.mean(np.sum(y_onehot * np.log(proba), axis=1))

    def _class_weight_vector(self, y):
        """sample_weight of est:2570-2603 for K classes."""
        n = len(y)
        if self.scale_pos_weight is not None and self.objective == 'binary':
            w = np.ones(n, dtype=np.float64)
            w[y == 1] = self.scale_pos_weight
            return w
        w = np.ones(n, dtype=np.float64)
        if self.class_weight not in ('balanced', 'balanced_sqrt'):
            return w
        K = self.n_classes_
        for k in range(K):
            n_k = np.sum(y == k)
            w_k = n / (K * max(n_k, 1))
            if self.class_weight == 'balanced_sqrt':
                w_k = w_k ** 0.35
            w[y == k] = w_k
        return w

    def _fit_multiclass(self, eng, y, n_val, y_val, sampler):
        """K trees per round from softmax gradients (est:2949-3065).  The
        host keeps the reference's NumPy arithmetic on the (n, K) scores;
        every tree is built and applied to all rows on the device."""
        n_samples = len(y)
        n_features = self.n_features_in_
        K = self.n_classes_
        on_device = K <= _native.MC_DEVICE_MAX_CLASSES
        y_onehot = None if on_device else np.eye(K, dtype=np.float64)[y]
        F_train = None if on_device else np.zeros((n_samples, K), dtype=np.float64)
        F_val = None
        y_val_onehot = None
        if n_val:
            F_val = np.zeros((n_val, K), dtype=np.float64)
            y_val_onehot = np.eye(K, dtype=np.float64)[y_val]
        sample_weight = self._class_weight_vector(y)
        self.mc_trees = [[] for _ in range(K)]
        # The reference's rng.shuffle stream (est:2502-2517), one draw per
        # round shared by the K trees (the sampler made by fit).
        # Up to MC_DEVICE_MAX_CLASSES classes the scores, gradients, score
        # updates and loss stay on the device (the engine's multiclass
        # rounds); more classes keep the (n, K) arithmetic on the host.
        if on_device:
            eng.mc_begin(y, K, sample_weight)
        try:
            self._mc_rounds(eng, y, K, on_device, sampler, sample_weight, y_onehot, F_train,
                            F_val, y_val_onehot, n_val)
        finally:
            # A round the engine took ahead goes back before the sampler is closed.
            eng.set_pipeline(False)
        self.n_trees_fitted_ = sum(len(t) for t in self.mc_trees)

    def _mc_rounds(self, eng, y, K, on_device, sampler, sample_weight, y_onehot, F_train,
                   F_val, y_val_onehot, n_val):
        n_samples = len(y)
        best_val_loss = np.inf
        rounds_no_improve = 0
        for m in range(self.n_estimators):
            if on_device:
                # One engine call per round: the round's bagging draw, every
                # class's gradients and hessians (est:2996-3019), the K trees
                # and score updates (est:3016-3029) and the loss (est:3035);
                # the next round's rows are permuted meanwhile.
                feat_idx, trees, train_loss = eng.mc_round_trees(
                    sampler, self.max_leaves, self.max_depth, self.min_samples_leaf,
                    self.min_child_weight, self.feature_bin_counts, self._max_bins,
                    self.reg_lambda, self.gamma, self.learning_rate)
                for k, tree in enumerate(trees):
                    self.mc_trees[k].append(tree)
                    if F_val is not None:
                        F_val[:, k] += self.learning_rate * eng.predict_tree(1, n_val, tree)
            else:
                proba = self._softmax(F_train)
                sample_idx, feat_idx = sampler.next()
                grad_all = sample_weight[:, None] * (proba - y_onehot)
                hess_all = sample_weight[:, None] * proba * (1.0 - proba)
                for k in range(K):
                    grad_k = np.ascontiguousarray(grad_all[:, k])
                    hess_k = np.maximum(np.ascontiguousarray(hess_all[:, k]), 1e-8)
                    tree = eng.build_tree(grad_k, hess_k, sample_idx, feat_idx,
                                          self.max_leaves, self.max_depth,
                                          self.min_samples_leaf, self.min_child_weight,
                                          self.feature_bin_counts, self._max_bins,
                                          self.reg_lambda, self.gamma)
                    self.mc_trees[k].append(tree)
                    F_train[:, k] += self.learning_rate * eng.predict_tree(0, n_samples, tree)
                    if F_val is not None:
                        F_val[:, k] += self.learning_rate * eng.predict_tree(1, n_val, tree)
                train_loss = self._compute_multiclass_logloss(y_onehot, F_train)
            self.train_loss_history_.append(train_loss)
            val_loss = None
            if F_val is not None:
                val_loss = self._compute_multiclass_logloss(y_val_onehot, F_val)
                self.val_loss_history_.append(val_loss)
            if self.verbose and ((m + 1) % 20 == 0 or m == 0):
                msg = (f"  ✓ Round {m+1:>3}/{self.n_estimators}  |  {K} trees  |  "
                       f"train-loss: {train_loss:.6f}")
                if val_loss is not None:
                    msg += f"  |  val-loss: {val_loss:.6f}"
                print(msg)
            if self.early_stopping_rounds is not None and val_loss is not None:
                if val_loss < best_val_loss:
                    best_val_loss = val_loss
                    self.best_iteration_ = m
                    rounds_no_improve = 0
                else:
                    rounds_no_improve += 1
                    if rounds_no_improve >= self.early_stopping_rounds:
                        if self.verbose:
                            print(f"\n  ⏹ Early stopping at round {m+1} (best: {self.best_iteration_+1})")
                        for k in range(K):
                            self.mc_trees[k] = self.mc_trees[k][:self.best_iteration_ + 1]
                        break

    # ------------------------------------------------------------------
    # est:2192-2236, est:2343-2363
    # ------------------------------------------------------------------
    def _pack_tree_list(self, tree_list):
        total_nodes = sum(t[5] for t in tree_list)
        features = np.empty(total_nodes, dtype=np.int16)
        thresholds = np.empty(total_nodes, dtype=np.int64)
        values = np.empty(total_nodes, dtype=np.float64)
        left = np.empty(total_nodes, dtype=np.int32)
        right = np.empty(total_nodes, dtype=np.int32)
        offsets = np.empty(len(tree_list) + 1, dtype=np.int32)
        offset = 0
        for t_idx, (tf, tt, tv, tl, tr, nc, _) in enumerate(tree_list):
            offsets[t_idx] = offset
            features[offset:offset + nc] = tf[:nc]
            thresholds[offset:offset + nc] = tt[:nc]
            values[offset:offset + nc] = tv[:nc]
            left[offset:offset + nc] = tl[:nc]
            right[offset:offset + nc] = tr[:nc]
            offset += nc
        offsets[len(tree_list)] = offset
        return {'features': features, 'thresholds': thresholds,
                'values': values, 'left': left, 'right': right,
                'offsets': offsets}

    def _pack_trees(self):
        if self._is_multiclass:
            self._mc_packed = [self._pack_tree_list(t) if len(t) > 0 else None
                               for t in self.mc_trees]
            return
        packed = self._pack_tree_list(self.trees)
        self._packed_features = packed['features']
        self._packed_thresholds = packed['thresholds']
        self._packed_values = packed['values']
        self._packed_left = packed['left']
        self._packed_right = packed['right']
        self._tree_offsets = packed['offsets']

    def _compute_feature_importances(self):
        """est:2343-2363: every split's gain added to its feature, tree by
        tree and node by node.  np.add.at adds in that same order (it is
        unbuffered), so the float64 sums are the reference's."""
        gain_imp = np.zeros(self.n_features_in_, dtype=np.float64)
        split_cnt = np.zeros(self.n_features_in_, dtype=np.int64)
        tree_lists = self.mc_trees if self._is_multiclass else [self.trees]
        feats = [np.asarray(tf[:nc]) for trees in tree_lists for tf, tt, tv, tl, tr, nc, sg in trees]
        gains = [np.asarray(sg[:nc]) for trees in tree_lists for tf, tt, tv, tl, tr, nc, sg in trees]
        if feats:
            f = np.concatenate(feats).astype(np.int64)
            g = np.concatenate(gains).astype(np.float64)
            split = f >= 0
            np.add.at(gain_imp, f[split], g[split])
            np.add.at(split_cnt, f[split], 1)
        total = gain_imp.sum()
        self.feature_importances_ = gain_imp / total if total > 0 else np.zeros(self.n_features_in_)
        self.feature_split_counts_ = split_cnt

    # ------------------------------------------------------------------
    # est:3274-3368
    # ------------------------------------------------------------------
    def _raw_score(self, X, proba=False):
        """F = sum_t lr * value_t + base_score_ (est:3318-3324); with `proba`,
        the model's predict_proba instead (binary est:3335-3336, multiclass
        the softmax of est:3315 with at most 16 classes), computed on the
        device from that F."""
        X = _to_dense(X)
        if getattr(self, 'n_features_in_', None) is None:
            raise ValueError("This HybridHistGBMNumbaV1_0_1 instance is not fitted yet.")
        X = _as_float(X)
        if X.ndim != 2 or X.shape[1] != self.n_features_in_:
            raise ValueError(f"X must have {self.n_features_in_} features")
        eng = _engine(self._device_index())
        if proba and not self._is_multiclass:
            # Binning, walk and probabilities in one call, its row chunks'
            # uploads overlapping the device's work on the chunk before.
            packed = {'features': self._packed_features, 'thresholds': self._packed_thresholds,
                      'values': self._packed_values, 'left': self._packed_left,
                      'right': self._packed_right, 'offsets': self._tree_offsets}
            with eng.lock:
                t0 = time.perf_counter()
                out = eng.predict_proba_rows(X, self.bin_edges, self.feature_bin_counts,
                                             self._nan_bin_id, packed, len(self.trees),
                                             self.learning_rate,
                                             getattr(self, 'base_score_', 0.0))
                self.times['inference'] = (time.perf_counter() - t0) * 1000
            return out
        with eng.lock:  # matrix slot 1 holds this call's codes until it returns
            eng.bin_features(1, X, self.bin_edges, self.feature_bin_counts, self._nan_bin_id)
            t0 = time.perf_counter()
            if self._is_multiclass and proba:
                # est:3293-3315 and the softmax (est:2327-2332) on the
                # device, read back once.
                out = eng.predict_proba_mc(1, X.shape[0], self._mc_packed,
                                           [len(t) for t in self.mc_trees], self.learning_rate)
                self.times['inference'] = (time.perf_counter() - t0) * 1000
                return out
            if self._is_multiclass:
                # est:3293-3315: per class, sum its trees from 0.0.
                F = np.zeros((X.shape[0], self.n_classes_), dtype=np.float64)
                for k in range(self.n_classes_):
                    if self._mc_packed[k] is not None:
                        F[:, k] = eng.predict(1, X.shape[0], self._mc_packed[k],
                                              len(self.mc_trees[k]), self.learning_rate)
                self.times['inference'] = (time.perf_counter() - t0) * 1000
                return F
            packed = {'features': self._packed_features, 'thresholds': self._packed_thresholds,
                      'values': self._packed_values, 'left': self._packed_left,
                      'right': self._packed_right, 'offsets': self._tree_offsets}
            out = eng.predict(1, X.shape[0], packed, len(self.trees),
                              self.learning_rate) + getattr(self, 'base_score_', 0.0)
            self.times['inference'] = (time.perf_counter() - t0) * 1000
        return out

    def predict_proba(self, X):
        if self._is_multiclass:
            if self.n_classes_ <= _native.MC_DEVICE_MAX_CLASSES:
                return self._raw_score(X, proba=True)
            return self._softmax(self._raw_score(X))
        return self._raw_score(X, proba=True)

    def predict(self, X):
        proba = self.predict_proba(X)
        if self._is_multiclass:
            return self.classes_[np.argmax(proba, axis=1)]
        return self.classes_[(proba[:, 1] > 0.5).astype(int)]

    def score(self, X, y):
        """Mean accuracy (est:3577-3578)."""
        return np.mean(self.predict(X) == y)

    # ------------------------------------------------------------------
    # est:3842-3916.  The reference maps batches of batch_size rows over a
    # process pool.  Here every batch goes through the device in this
    # process: a row's prediction does not depend on its batch, so the
    # result is the one the pool would return, and worker processes would
    # each have to start their own HIP runtime.  n_workers is accepted for
    # the same signature.
    # ------------------------------------------------------------------
    def predict_batch_parallel(self, X, n_workers=4, batch_size=10000):
        return self._batched(self.predict, X, batch_size, np.concatenate)

    def predict_proba_batch_parallel(self, X, n_workers=4, batch_size=10000):
        return self._batched(self.predict_proba, X, batch_size, np.vstack)

    @staticmethod
    def _batched(fn, X, batch_size, join):
        n = len(X)
        if n <= batch_size:
            return fn(X)
        # The whole input in one device pass where it fits comfortably;
        # otherwise slices of many batches each, joined as the reference
        # joins its batches.
        step = max(int(batch_size), _BATCH_ROWS // max(int(batch_size), 1) * int(batch_size))
        return join([fn(X[i:i + step]) for i in range(0, n, step)])

    # ------------------------------------------------------------------
    # est:3773-3801
    # ------------------------------------------------------------------
    def get_params(self, deep=True):
        return {
            'n_estimators': self.n_estimators,
            'max_depth': self.max_depth_init,
            'learning_rate': self.learning_rate_init,
            'n_bins': self.n_bins_init,
            'reg_lambda': self.reg_lambda,
            'min_samples_leaf': self.min_samples_leaf,
            'min_child_weight': self.min_child_weight,
            'gamma': self.gamma,
            'subsample': self.subsample,
            'colsample_bytree': self.colsample_bytree,
            'class_weight': self.class_weight,
            'monotone_constraints': self.monotone_constraints,
            'categorical_features': self.categorical_features,
            'early_stopping_rounds': self.early_stopping_rounds,
            'verbose': self.verbose,
            'random_state': self.random_state,
        }

    def set_params(self, **params):
        for key, val in params.items():
            setattr(self, key, val)
        return self

    def __repr__(self):
        return (f"HybridHistGBMNumbaV1_0_1(n_estimators={self.n_estimators}, "
                f"max_depth='{self.max_depth_init}', subsample={self.subsample}, "
                f"colsample_bytree={self.colsample_bytree})")

    # ------------------------------------------------------------------
    # est:4035-4205: JSON model format
    # ------------------------------------------------------------------
    @staticmethod
    def _tree_to_json(tree):
        return {
            'features': np.asarray(tree[0]).tolist(),
            'thresholds': np.asarray(tree[1]).tolist(),
            'values': np.asarray(tree[2]).tolist(),
            'left': np.asarray(tree[3]).tolist(),
            'right': np.asarray(tree[4]).tolist(),
            'node_count': int(tree[5]),
            'split_gains': np.asarray(tree[6]).tolist() if len(tree) > 6 else [],
        }

    @staticmethod
    def _tree_from_json(td):
        # As the reference reads it: thresholds come back as float64 (the
        # packed arrays convert them to int64 again), and a missing
        # split_gains list becomes zeros.
        sg = np.array(td.get('split_gains', [0.0] * td['node_count']), dtype=np.float64)
        return (np.array(td['features'], dtype=np.int32),
                np.array(td['thresholds'], dtype=np.float64),
                np.array(td['values'], dtype=np.float64),
                np.array(td['left'], dtype=np.int32),
                np.array(td['right'], dtype=np.int32),
                td['node_count'],
                sg)

    def save_model(self, filepath):
        """Writes the model as JSON in the reference's layout (est:4035-4115)."""
        import json
        model_data = {
            'version': '1.2.2',
            'params': {},
            'n_classes_': int(self.n_classes_),
            'classes_': self.classes_.tolist() if self.classes_ is not None else None,
            'n_features_in_': int(self.n_features_in_) if self.n_features_in_ is not None else None,
            'objective': self.objective,
            '_is_multiclass': self._is_multiclass,
            'init_score_': float(self.init_score_),
            'base_score_': float(getattr(self, 'base_score_', 0.0)),
            'n_trees_fitted_': int(self.n_trees_fitted_),
            'best_iteration_': int(self.best_iteration_),
            'train_loss_history_': [float(x) for x in self.train_loss_history_],
            'val_loss_history_': [float(x) for x in self.val_loss_history_],
            '_max_bins': int(self._max_bins),
        }
        for k, v in self.get_params().items():
            if callable(v):
                continue
            model_data['params'][k] = v
        if self.bin_edges is not None:
            model_data['bin_edges'] = self.bin_edges.tolist()
        if self.feature_bin_counts is not None:
            model_data['feature_bin_counts'] = self.feature_bin_counts.tolist()
        if not self._is_multiclass:
            model_data['trees'] = [self._tree_to_json(t) for t in self.trees]
        else:
            model_data['mc_trees'] = [[self._tree_to_json(t) for t in k_trees]
                                      for k_trees in self.mc_trees]
        if self.feature_importances_ is not None:
            model_data['feature_importances_'] = self.feature_importances_.tolist()
        if self.feature_split_counts_ is not None:
            model_data['feature_split_counts_'] = self.feature_split_counts_.tolist()
        model_data['_categorical_set'] = list(self._categorical_set)
        if self._is_categorical is not None:
            model_data['_is_categorical'] = self._is_categorical.tolist()
        with open(filepath, 'w') as f:
            json.dump(model_data, f)

    @classmethod
    def load_model(cls, filepath):
        """Reads a model written by save_model (est:4117-4205).

        As in the reference, the NaN-bin map is not stored: every feature is
        treated as having had no NaN in training (est:4200-4202), so a model
        trained on NaN features scores NaN inputs differently after a reload.
        """
        import json
        with open(filepath, 'r') as f:
            data = json.load(f)
        model = cls(**data['params'])
        model.n_classes_ = data['n_classes_']
        model.classes_ = np.array(data['classes_']) if data['classes_'] is not None else None
        model.n_features_in_ = data['n_features_in_']
        model.objective = data['objective']
        model._is_multiclass = data['_is_multiclass']
        model.init_score_ = data['init_score_']
        model.base_score_ = data.get('base_score_', 0.0)
        model.n_trees_fitted_ = data['n_trees_fitted_']
        model.best_iteration_ = data['best_iteration_']
        model.train_loss_history_ = data['train_loss_history_']
        model.val_loss_history_ = data['val_loss_history_']
        model._max_bins = data['_max_bins']
        if 'bin_edges' in data:
            model.bin_edges = np.array(data['bin_edges'], dtype=np.float64)
        if 'feature_bin_counts' in data:
            model.feature_bin_counts = np.array(data['feature_bin_counts'], dtype=np.int32)
        if 'trees' in data:
            model.trees = [cls._tree_from_json(td) for td in data['trees']]
        if 'mc_trees' in data:
            model.mc_trees = [[cls._tree_from_json(td) for td in class_trees]
                              for class_trees in data['mc_trees']]
        if 'feature_importances_' in data:
            model.feature_importances_ = np.array(data['feature_importances_'])
        if 'feature_split_counts_' in data:
            model.feature_split_counts_ = np.array(data['feature_split_counts_'])
        model._categorical_set = set(data.get('_categorical_set', []))
        if '_is_categorical' in data and data['_is_categorical'] is not None:
            model._is_categorical = np.array(data['_is_categorical'], dtype=np.bool_)
        model.binning_strategy = (model.binning_strategy_init
                                  if model.binning_strategy_init != 'auto' else 'standard')
        if model.n_features_in_ is not None:
            model._nan_bin_id = np.full(model.n_features_in_, -1, dtype=np.int32)
        model._pack_trees()
        return model

    def warmup(self, n_features=None):
        """The reference compiles its Numba kernels here (est:3807); the HIP
        kernels are compiled ahead of time, so this only opens the device."""
        _engine(self._device_index())
        return self
