"""ctypes binding of libbsscl_hip.so (the C ABI in include/bsscl_hip.h).

There is no CPU fallback: if the library is missing or no GPU is visible the
calls raise, so a run can never silently compute on another path.
"""
from __future__ import annotations

import ctypes
import os
import threading

import numpy as np

from ._build import LIB_PATH

BSSCL_OK, BSSCL_EINVAL, BSSCL_ENOMEM, BSSCL_EDEVICE, BSSCL_EINTERNAL = range(5)

_P = ctypes.c_void_p
_i32, _i64, _f64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_double

# name -> argtypes (restype int unless listed in _VOID)
_SIGS = {
    "bsscl_last_error": [],
    "bsscl_device_count": [_P],
    "bsscl_engine_create": [_i32, _P],
    "bsscl_engine_destroy": [_P],
    "bsscl_bin_features": [_P, _i32, _P, _i32, _i64, _i32, _P, _i32, _P, _P, _P],
    "bsscl_load_codes": [_P, _i32, _P, _i32, _i64, _i32],
    "bsscl_get_codes": [_P, _i32, _P],
    "bsscl_get_codes_u16": [_P, _i32, _P],
    "bsscl_stage_features": [_P, _P, _i32, _i64, _i32],
    "bsscl_sort_columns": [_P, _P, _P],
    "bsscl_sorted_gather": [_P, _i64, _P, _P, _P],
    "bsscl_sorted_uniques": [_P, _i32, _i32, _P, _P],
    "bsscl_release_staged": [_P],
    "bsscl_build_tree": [_P, _P, _P, _P, _i64, _P, _i32, _i32, _i32, _i32, _f64,
                         _P, _i32, _f64, _f64, _P, _P, _P, _P, _P, _P, _P],
    "bsscl_boost_begin": [_P, _P, _i64, _f64, _f64, _f64],
    "bsscl_boost_round": [_P, _P, _i32, _i32, _i32, _f64, _P, _i32, _f64, _f64,
                          _f64, _P, _P, _P, _P, _P, _P, _P, _P],
    "bsscl_boost_get_F": [_P, _P],
    "bsscl_boost_grad_hess": [_P, _P, _P],
    "bsscl_boost_grad_hess_max": [_P, _P],
    "bsscl_mc_begin": [_P, _P, _i64, _i32, _P],
    "bsscl_mc_round": [_P, _P, _i64],
    "bsscl_mc_round_sampled": [_P, _P, _P],
    "bsscl_mc_build_tree": [_P, _i32, _P, _i32, _i32, _i32, _i32, _f64, _P, _i32, _f64,
                            _f64, _f64, _P, _P, _P, _P, _P, _P, _P],
    "bsscl_mc_build_trees": [_P, _P, _i32, _i32, _i32, _i32, _f64, _P, _i32, _f64, _f64, _f64,
                             _P, _P, _P, _P, _P, _P, _P],
    "bsscl_mc_round_trees": [_P, _P, _P, _i32, _i32, _i32, _f64, _P, _i32, _f64, _f64, _f64,
                             _P, _P, _P, _P, _P, _P, _P, _P],
    "bsscl_mc_loss": [_P, _P],
    "bsscl_mc_get_scores": [_P, _P],
    "bsscl_mc_get_grad_hess": [_P, _P, _P],
    "bsscl_predict": [_P, _i32, _P, _P, _P, _P, _P, _P, _i32, _f64, _P],
    "bsscl_predict_proba": [_P, _i32, _P, _P, _P, _P, _P, _P, _i32, _f64, _f64, _P],
    "bsscl_predict_proba_rows": [_P, _P, _i32, _i64, _i32, _P, _i32, _P, _P, _P, _P, _P, _P,
                                 _P, _P, _i32, _f64, _f64, _P],
    "bsscl_predict_proba_mc": [_P, _i32, _i32, _P, _P, _P, _P, _P, _P, _P, _f64, _P],
    "bsscl_predict_tree": [_P, _i32, _P, _P, _P, _P, _P, _i32, _P],
    "bsscl_predict_noalloc": [_P, _i32, _P, _P, _P, _P, _P, _P, _i32, _f64, _P],
    "bsscl_node_split": [_P, _P, _P, _P, _i64, _P, _i32, _P, _f64, _f64, _P, _P,
                         _P, _P, _P],
    "bsscl_partition": [_P, _P, _i64, _i32, _i32, _P, _P],
    "bsscl_rs_shuffle_i64": [_P, _P, _P, _i64],
    "bsscl_rs_shuffle_i32": [_P, _P, _P, _i64],
    "bsscl_rs_draws": [_P, _P, _P, _i64],
    "bsscl_fisher_yates_apply": [_P, _P, _i64, _P],
    "bsscl_sampler_create": [_P, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                             _i32, _i32, _i32, _P],
    "bsscl_sampler_next": [_P, _P, _P],
    "bsscl_sampler_state": [_P, _P, _P],
    "bsscl_sampler_stats": [_P, _P, _i32, _P],
    "bsscl_sampler_destroy": [_P],
    "bsscl_engine_set_profiling": [_P, _i32],
    "bsscl_boost_set_pipeline": [_P, _i32],
    "bsscl_engine_stats": [_P, _P, _i32, _P],
}
_VOID = {"bsscl_engine_destroy", "bsscl_sampler_destroy"}

_lib = None
_lock = threading.Lock()


DEVICE_ROWS = 1  # BSSCL_SAMPLER_DEVICE_ROWS
MC_DEVICE_MAX_CLASSES = 16  # bsscl_mc_begin's limit


class EngineError(RuntimeError):
    """A HIP engine call failed (device, allocation or internal error)."""


def library_path() -> str:
    return LIB_PATH


def lib():
    """Loads the engine library; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise EngineError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -m bsscl_gbm._build` (hipcc, gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            for name, args in _SIGS.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = None if name in _VOID else ctypes.c_int
            L.bsscl_last_error.restype = ctypes.c_char_p
            _lib = L
    return _lib


def check(rc: int) -> None:
    if rc == BSSCL_OK:
        return
    msg = lib().bsscl_last_error().decode(errors="replace")
    if rc == BSSCL_EINVAL:
        raise ValueError(msg)
    if rc == BSSCL_ENOMEM:
        raise MemoryError(msg)
    raise EngineError(msg)


def ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def device_count() -> int:
    out = np.zeros(1, np.int32)
    check(lib().bsscl_device_count(ptr(out)))
    return int(out[0])


class Engine:
    """One device context: matrices, boosting state and tree workspace."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().bsscl_engine_create(int(device), ctypes.byref(h)))
        self._h = h
        self.device = device

    @property
    def handle(self):
        if self._h is None:
            raise EngineError("engine is closed")
        return self._h

    def close(self):
        if getattr(self, "_h", None) is not None:
            lib().bsscl_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- matrices ---------------------------------------------------------
    def bin_features(self, slot, X, edges_2d, bin_counts, nan_bin_id,
                     return_codes=False):
        X = np.ascontiguousarray(X)
        if X.dtype not in (np.float32, np.float64):
            X = X.astype(np.float64)
        n, F = X.shape
        e = np.ascontiguousarray(edges_2d, dtype=np.float64)
        bc = np.ascontiguousarray(bin_counts, dtype=np.int32)
        ni = np.ascontiguousarray(nan_bin_id, dtype=np.int32)
        out = np.empty((n, F), np.uint8) if return_codes else None
        check(lib().bsscl_bin_features(
            self.handle, int(slot), ptr(X), int(X.dtype == np.float64), n, F,
            ptr(e), e.shape[1], ptr(bc), ptr(ni),
            ptr(out) if out is not None else None))
        return out

    def bin_staged(self, slot, n, F, is_f64, edges_2d, bin_counts, nan_bin_id):
        """bin_features of the matrix staged by stage_features."""
        e = np.ascontiguousarray(edges_2d, dtype=np.float64)
        bc = np.ascontiguousarray(bin_counts, dtype=np.int32)
        ni = np.ascontiguousarray(nan_bin_id, dtype=np.int32)
        check(lib().bsscl_bin_features(
            self.handle, int(slot), None, int(bool(is_f64)), int(n), int(F),
            ptr(e), e.shape[1], ptr(bc), ptr(ni), None))

    # -- bin edges ------------------------------------------------------------
    def stage_features(self, X):
        """Copies X (float32 or float64, n x F) to the device."""
        X = np.ascontiguousarray(X)
        if X.dtype not in (np.float32, np.float64):
            raise ValueError("stage_features needs float32 or float64 X")
        n, F = X.shape
        check(lib().bsscl_stage_features(self.handle, ptr(X), int(X.dtype == np.float64), n, F))

    def sort_columns(self, F):
        """Sorts the staged columns; returns (nan_count, n_unique), int64[F] each."""
        nan = np.empty(F, np.int64)
        uniq = np.empty(F, np.int64)
        check(lib().bsscl_sort_columns(self.handle, ptr(nan), ptr(uniq)))
        return nan, uniq

    def sorted_gather(self, cols, pos):
        """Values (float64) at ranks pos of sorted columns cols."""
        c = np.ascontiguousarray(cols, dtype=np.int32)
        p = np.ascontiguousarray(pos, dtype=np.int64)
        out = np.empty(len(p), np.float64)
        check(lib().bsscl_sorted_gather(self.handle, len(p), ptr(c), ptr(p), ptr(out)))
        return out

    def sorted_uniques(self, col, max_out):
        out = np.empty(max(int(max_out), 1), np.float64)
        cnt = np.zeros(1, np.int32)
        check(lib().bsscl_sorted_uniques(self.handle, int(col), int(max_out), ptr(out),
                                         ptr(cnt)))
        return out[:int(cnt[0])].copy()

    def release_staged(self):
        check(lib().bsscl_release_staged(self.handle))

    def load_codes(self, slot, codes):
        codes = np.ascontiguousarray(codes)
        if codes.dtype not in (np.uint8, np.uint16):
            raise ValueError("codes must be uint8 or uint16")
        n, F = codes.shape
        check(lib().bsscl_load_codes(self.handle, int(slot), ptr(codes),
                                     int(codes.dtype == np.uint16), n, F))

    def get_codes(self, slot, n, F, u16=False):
        """Row-major codes of matrix `slot`: uint8 min(code, 255), or with
        u16 the reference's uint16 codes (est:2163-2166)."""
        out = np.empty((n, F), np.uint16 if u16 else np.uint8)
        fn = lib().bsscl_get_codes_u16 if u16 else lib().bsscl_get_codes
        check(fn(self.handle, int(slot), ptr(out)))
        return out

    # -- trees --------------------------------------------------------------
    @staticmethod
    def _tree_out(max_leaves):
        M = 2 * int(max_leaves) + 2
        return (np.empty(M, np.int32), np.empty(M, np.int64),
                np.empty(M, np.float64), np.empty(M, np.int32),
                np.empty(M, np.int32), np.zeros(1, np.int32),
                np.empty(M, np.float64))

    def build_tree(self, grad, hess, sample_indices, feature_indices,
                   max_leaves, max_depth, min_samples_leaf, min_child_weight,
                   bin_counts, max_bins, reg_lambda, gamma):
        g = np.ascontiguousarray(grad, np.float64)
        h = np.ascontiguousarray(hess, np.float64)
        si = np.ascontiguousarray(sample_indices, np.int64)
        fi = np.ascontiguousarray(feature_indices, np.int32)
        bc = np.ascontiguousarray(bin_counts, np.int32)
        tf, tt, tv, tl, tr, nc, sg = self._tree_out(max_leaves)
        check(lib().bsscl_build_tree(
            self.handle, ptr(g), ptr(h), ptr(si), len(si), ptr(fi), len(fi),
            int(max_leaves), int(max_depth), int(min_samples_leaf),
            float(min_child_weight), ptr(bc), int(max_bins), float(reg_lambda),
            float(gamma), ptr(tf), ptr(tt), ptr(tv), ptr(tl), ptr(tr), ptr(nc),
            ptr(sg)))
        return (tf, tt, tv, tl, tr, int(nc[0]), sg)

    # Multiclass rounds with the scores on the device (include/bsscl_hip.h).
    def mc_begin(self, y, n_classes, sample_weight):
        y = np.ascontiguousarray(y, np.int64)
        w = np.ascontiguousarray(sample_weight, np.float64)
        check(lib().bsscl_mc_begin(self.handle, ptr(y), len(y), int(n_classes), ptr(w)))
        self._mc = (len(y), int(n_classes))

    def mc_round(self, sample_indices):
        si = np.ascontiguousarray(sample_indices, np.int64)
        check(lib().bsscl_mc_round(self.handle, ptr(si), len(si)))

    def mc_round_sampled(self, sampler):
        """mc_round with the sampler's next round; returns its feature subset."""
        feats = np.empty(sampler.f_sub, np.int32)
        check(lib().bsscl_mc_round_sampled(self.handle, sampler.handle, ptr(feats)))
        return feats

    def mc_build_tree(self, k, feature_indices, max_leaves, max_depth, min_samples_leaf,
                      min_child_weight, bin_counts, max_bins, reg_lambda, gamma,
                      learning_rate):
        fi = np.ascontiguousarray(feature_indices, np.int32)
        bc = np.ascontiguousarray(bin_counts, np.int32)
        tf, tt, tv, tl, tr, nc, sg = self._tree_out(max_leaves)
        check(lib().bsscl_mc_build_tree(
            self.handle, int(k), ptr(fi), len(fi), int(max_leaves), int(max_depth),
            int(min_samples_leaf), float(min_child_weight), ptr(bc), int(max_bins),
            float(reg_lambda), float(gamma), float(learning_rate), ptr(tf), ptr(tt),
            ptr(tv), ptr(tl), ptr(tr), ptr(nc), ptr(sg)))
        return (tf, tt, tv, tl, tr, int(nc[0]), sg)

    def mc_build_trees(self, feature_indices, max_leaves, max_depth, min_samples_leaf,
                       min_child_weight, bin_counts, max_bins, reg_lambda, gamma,
                       learning_rate):
        """The round's K trees (classes 0..K-1) in one call; a list of K
        7-tuples as mc_build_tree returns them."""
        K = self._mc[1]
        M = 2 * int(max_leaves) + 2
        fi = np.ascontiguousarray(feature_indices, np.int32)
        bc = np.ascontiguousarray(bin_counts, np.int32)
        tf = np.full((K, M), -1, np.int32)
        tt = np.zeros((K, M), np.int64)
        tv = np.zeros((K, M), np.float64)
        tl = np.full((K, M), -1, np.int32)
        tr = np.full((K, M), -1, np.int32)
        nc = np.zeros(K, np.int32)
        sg = np.zeros((K, M), np.float64)
        check(lib().bsscl_mc_build_trees(
            self.handle, ptr(fi), len(fi), int(max_leaves), int(max_depth),
            int(min_samples_leaf), float(min_child_weight), ptr(bc), int(max_bins),
            float(reg_lambda), float(gamma), float(learning_rate), ptr(tf), ptr(tt),
            ptr(tv), ptr(tl), ptr(tr), ptr(nc), ptr(sg)))
        return [(tf[k], tt[k], tv[k], tl[k], tr[k], int(nc[k]), sg[k]) for k in range(K)]

    def mc_round_trees(self, sampler, max_leaves, max_depth, min_samples_leaf,
                       min_child_weight, bin_counts, max_bins, reg_lambda, gamma,
                       learning_rate):
        """One multiclass round (the sampler's next round, the K trees, the
        loss), with the following round's rows made meanwhile; returns
        (feature subset, list of K 7-tuples, training loss)."""
        K = self._mc[1]
        M = 2 * int(max_leaves) + 2
        feats = np.empty(sampler.f_sub, np.int32)
        bc = np.ascontiguousarray(bin_counts, np.int32)
        tf = np.full((K, M), -1, np.int32)
        tt = np.zeros((K, M), np.int64)
        tv = np.zeros((K, M), np.float64)
        tl = np.full((K, M), -1, np.int32)
        tr = np.full((K, M), -1, np.int32)
        nc = np.zeros(K, np.int32)
        sg = np.zeros((K, M), np.float64)
        loss = np.zeros(1, np.float64)
        check(lib().bsscl_mc_round_trees(
            self.handle, sampler.handle, ptr(feats), int(max_leaves), int(max_depth),
            int(min_samples_leaf), float(min_child_weight), ptr(bc), int(max_bins),
            float(reg_lambda), float(gamma), float(learning_rate), ptr(tf), ptr(tt),
            ptr(tv), ptr(tl), ptr(tr), ptr(nc), ptr(sg), ptr(loss)))
        trees = [(tf[k], tt[k], tv[k], tl[k], tr[k], int(nc[k]), sg[k]) for k in range(K)]
        return feats, trees, float(loss[0])

    def mc_loss(self):
        out = np.zeros(1, np.float64)
        check(lib().bsscl_mc_loss(self.handle, ptr(out)))
        return float(out[0])

    def mc_scores(self):
        n, K = self._mc
        out = np.empty((K, n), np.float64)
        check(lib().bsscl_mc_get_scores(self.handle, ptr(out)))
        return out.T.copy()

    def mc_grad_hess(self):
        """The last mc_round's gradients and hessians, each (n, K)."""
        n, K = self._mc
        g = np.empty((K, n), np.float64)
        h = np.empty((K, n), np.float64)
        check(lib().bsscl_mc_get_grad_hess(self.handle, ptr(g), ptr(h)))
        return g.T.copy(), h.T.copy()

    def boost_begin(self, y, w0, w1, base_score):
        y = np.ascontiguousarray(y, np.int64)
        check(lib().bsscl_boost_begin(self.handle, ptr(y), len(y), float(w0),
                                      float(w1), float(base_score)))

    def boost_round(self, sampler, max_leaves, max_depth, min_samples_leaf,
                    min_child_weight, bin_counts, max_bins, reg_lambda, gamma,
                    learning_rate):
        bc = np.ascontiguousarray(bin_counts, np.int32)
        tf, tt, tv, tl, tr, nc, sg = self._tree_out(max_leaves)
        loss = np.zeros(1, np.float64)
        check(lib().bsscl_boost_round(
            self.handle, sampler.handle, int(max_leaves), int(max_depth),
            int(min_samples_leaf), float(min_child_weight), ptr(bc),
            int(max_bins), float(reg_lambda), float(gamma), float(learning_rate),
            ptr(tf), ptr(tt), ptr(tv), ptr(tl), ptr(tr), ptr(nc), ptr(sg),
            ptr(loss)))
        return (tf, tt, tv, tl, tr, int(nc[0]), sg), float(loss[0])

    def boost_get_F(self, n):
        out = np.empty(n, np.float64)
        check(lib().bsscl_boost_get_F(self.handle, ptr(out)))
        return out

    def boost_grad_hess(self, n):
        g = np.empty(n, np.float64)
        h = np.empty(n, np.float64)
        check(lib().bsscl_boost_grad_hess(self.handle, ptr(g), ptr(h)))
        return g, h

    def boost_grad_hess_max(self):
        """(max |g|, max h) of the current F as the device holds them for the
        next round's fixed-point scale."""
        out = np.empty(2, np.float64)
        check(lib().bsscl_boost_grad_hess_max(self.handle, ptr(out)))
        return float(out[0]), float(out[1])

    def predict(self, slot, n, packed, n_trees, learning_rate):
        out = np.empty(n, np.float64)
        f = np.ascontiguousarray(packed["features"], np.int16)
        t = np.ascontiguousarray(packed["thresholds"], np.int64)
        v = np.ascontiguousarray(packed["values"], np.float64)
        l = np.ascontiguousarray(packed["left"], np.int32)
        r = np.ascontiguousarray(packed["right"], np.int32)
        o = np.ascontiguousarray(packed["offsets"], np.int32)
        check(lib().bsscl_predict(self.handle, int(slot), ptr(f), ptr(t), ptr(v),
                                  ptr(l), ptr(r), ptr(o), int(n_trees),
                                  float(learning_rate), ptr(out)))
        return out

    def predict_proba(self, slot, n, packed, n_trees, learning_rate, base_score):
        """bsscl_predict_proba: a binary model's (1 - p, p), shape (n, 2)."""
        out = np.empty((n, 2), np.float64)
        f = np.ascontiguousarray(packed["features"], np.int16)
        t = np.ascontiguousarray(packed["thresholds"], np.int64)
        v = np.ascontiguousarray(packed["values"], np.float64)
        l = np.ascontiguousarray(packed["left"], np.int32)
        r = np.ascontiguousarray(packed["right"], np.int32)
        o = np.ascontiguousarray(packed["offsets"], np.int32)
        check(lib().bsscl_predict_proba(self.handle, int(slot), ptr(f), ptr(t), ptr(v),
                                        ptr(l), ptr(r), ptr(o), int(n_trees),
                                        float(learning_rate), float(base_score), ptr(out)))
        return out

    def predict_proba_rows(self, X, edges_2d, bin_counts, nan_bin_id, packed, n_trees,
                           learning_rate, base_score):
        """bsscl_predict_proba_rows: a binary model's (1 - p, p) of host rows
        X, shape (n, 2), binned and walked on the device in overlapped row
        chunks; matrix slots are left as they were."""
        X = np.ascontiguousarray(X)
        if X.dtype not in (np.float32, np.float64):
            X = X.astype(np.float64)
        n, F = X.shape
        e = np.ascontiguousarray(edges_2d, dtype=np.float64)
        bc = np.ascontiguousarray(bin_counts, dtype=np.int32)
        ni = np.ascontiguousarray(nan_bin_id, dtype=np.int32)
        f = np.ascontiguousarray(packed["features"], np.int16)
        t = np.ascontiguousarray(packed["thresholds"], np.int64)
        v = np.ascontiguousarray(packed["values"], np.float64)
        l = np.ascontiguousarray(packed["left"], np.int32)
        r = np.ascontiguousarray(packed["right"], np.int32)
        o = np.ascontiguousarray(packed["offsets"], np.int32)
        out = np.empty((n, 2), np.float64)
        check(lib().bsscl_predict_proba_rows(
            self.handle, ptr(X), int(X.dtype == np.float64), n, F, ptr(e), e.shape[1], ptr(bc),
            ptr(ni), ptr(f), ptr(t), ptr(v), ptr(l), ptr(r), ptr(o), int(n_trees),
            float(learning_rate), float(base_score), ptr(out)))
        return out

    def predict_proba_mc(self, slot, n, packs, n_trees, learning_rate):
        """bsscl_predict_proba_mc: a multiclass model's softmax probabilities
        of matrix `slot`, shape (n, K); packs[k] is class k's packed trees
        (None for a class without trees)."""
        K = len(packs)
        names = ("features", "thresholds", "values", "left", "right", "offsets")
        dtypes = (np.int16, np.int64, np.float64, np.int32, np.int32, np.int32)
        keep = []
        tables = []
        for name, dt in zip(names, dtypes):
            arrs = [np.ascontiguousarray(p[name], dt) if p is not None else None for p in packs]
            keep.append(arrs)
            tables.append((ctypes.c_void_p * K)(*[a.ctypes.data if a is not None else None
                                                 for a in arrs]))
        nt = np.ascontiguousarray([int(t) if p is not None else 0
                                   for p, t in zip(packs, n_trees)], np.int32)
        out = np.empty((n, K), np.float64)
        check(lib().bsscl_predict_proba_mc(self.handle, int(slot), K,
                                           *[ctypes.cast(t, ctypes.c_void_p) for t in tables],
                                           ptr(nt), float(learning_rate), ptr(out)))
        del keep
        return out

    def predict_noalloc(self, slot, packed, n_trees, learning_rate, out_dev_ptr):
        """bsscl_predict_noalloc: F of matrix `slot` into the device buffer at
        address out_dev_ptr (float64, one value per row)."""
        f = np.ascontiguousarray(packed["features"], np.int16)
        t = np.ascontiguousarray(packed["thresholds"], np.int64)
        v = np.ascontiguousarray(packed["values"], np.float64)
        l = np.ascontiguousarray(packed["left"], np.int32)
        r = np.ascontiguousarray(packed["right"], np.int32)
        o = np.ascontiguousarray(packed["offsets"], np.int32)
        check(lib().bsscl_predict_noalloc(self.handle, int(slot), ptr(f), ptr(t), ptr(v),
                                          ptr(l), ptr(r), ptr(o), int(n_trees),
                                          float(learning_rate), ctypes.c_void_p(int(out_dev_ptr))))

    def predict_tree(self, slot, n, tree):
        tf, tt, tv, tl, tr, nc, _ = tree
        a = [np.ascontiguousarray(x[:nc]) for x in (tf, tt, tv, tl, tr)]
        a[0] = a[0].astype(np.int32)
        a[1] = a[1].astype(np.int64)
        a[2] = a[2].astype(np.float64)
        a[3] = a[3].astype(np.int32)
        a[4] = a[4].astype(np.int32)
        out = np.empty(n, np.float64)
        check(lib().bsscl_predict_tree(self.handle, int(slot), *[ptr(x) for x in a],
                                       int(nc), ptr(out)))
        return out

    def node_split(self, grad, hess, rows, feature_indices, bin_counts,
                   min_child_weight, reg_lambda):
        g = np.ascontiguousarray(grad, np.float64)
        h = np.ascontiguousarray(hess, np.float64)
        r = np.ascontiguousarray(rows, np.int64)
        fi = np.ascontiguousarray(feature_indices, np.int32)
        bc = np.ascontiguousarray(bin_counts, np.int32)
        G = np.empty((len(fi), 256), np.float64)
        H = np.empty((len(fi), 256), np.float64)
        gain = np.zeros(1, np.float64)
        feat = np.zeros(1, np.int32)
        b = np.zeros(1, np.int32)
        check(lib().bsscl_node_split(self.handle, ptr(g), ptr(h), ptr(r), len(r),
                                     ptr(fi), len(fi), ptr(bc),
                                     float(min_child_weight), float(reg_lambda),
                                     ptr(G), ptr(H), ptr(gain), ptr(feat), ptr(b)))
        return G, H, float(gain[0]), int(feat[0]), int(b[0])

    def partition(self, rows, feature, bin_):
        r = np.ascontiguousarray(rows, np.int64)
        out = np.empty(len(r), np.int64)
        nl = np.zeros(1, np.int64)
        check(lib().bsscl_partition(self.handle, ptr(r), len(r), int(feature),
                                    int(bin_), ptr(out), ptr(nl)))
        return out, int(nl[0])

    def fisher_yates_apply(self, draws, data):
        """data (int32) permuted by the Fisher-Yates steps i = n-1 .. 1 with
        draws[n-1-i] = j(i), on the GPU; returns the new array."""
        a = np.ascontiguousarray(data, dtype=np.int32).copy()
        d = np.ascontiguousarray(draws, dtype=np.uint32)
        if len(a) > 1 and len(d) != len(a) - 1:
            raise ValueError("draws must have len(data) - 1 entries")
        check(lib().bsscl_fisher_yates_apply(self.handle, ptr(d), len(a), ptr(a)))
        return a

    # -- profiling ------------------------------------------------------------
    def set_pipeline(self, on):
        """Enqueue each boosting round's successor before returning it."""
        check(lib().bsscl_boost_set_pipeline(self.handle, int(bool(on))))

    def set_profiling(self, level):
        """0 off; 1 times the histogram kernel; 2 every kernel group."""
        check(lib().bsscl_engine_set_profiling(self.handle, int(level)))

    def stats(self):
        out = np.zeros(21, np.float64)
        n = np.zeros(1, np.int32)
        check(lib().bsscl_engine_stats(self.handle, ptr(out), 21, ptr(n)))
        keys = ["hist_launches", "hist_ms", "hist_row_features", "hist_bytes",
                "part_launches", "part_ms", "split_launches", "split_ms",
                "trees", "nodes_expanded", "sampler_wait_ms", "round_ms",
                "reduce_launches", "reduce_ms", "enqueue_ms", "finish_ms",
                "predict_launches", "predict_ms", "rows_graph_rounds", "tree_graph_rounds",
                "graph_captures"]
        return dict(zip(keys, out[:int(n[0])].tolist()))


class Sampler:
    """Row/column bagging stream identical to RandomState.shuffle calls."""

    def __init__(self, rng_state, n, n_sub, do_rows, n_features, f_sub,
                 do_feats, n_rounds, lookahead=3, device_rows=False, device=0):
        name, key, pos = rng_state[0], rng_state[1], rng_state[2]
        if name != "MT19937":
            raise ValueError("RandomState must use MT19937")
        key = np.ascontiguousarray(key, dtype=np.uint32)
        h = ctypes.c_void_p()
        check(lib().bsscl_sampler_create(ptr(key), int(pos), int(n), int(n_sub),
                                         int(bool(do_rows)), int(n_features),
                                         int(f_sub), int(bool(do_feats)),
                                         int(n_rounds), int(lookahead),
                                         DEVICE_ROWS if device_rows else 0,
                                         int(device),
                                         ctypes.byref(h)))
        self._h = h
        self.n_sub, self.f_sub = int(n_sub), int(f_sub)

    @property
    def handle(self):
        if self._h is None:
            raise EngineError("sampler is closed")
        return self._h

    def next(self):
        rows = np.empty(self.n_sub, np.int32)
        feats = np.empty(self.f_sub, np.int32)
        check(lib().bsscl_sampler_next(self.handle, ptr(rows), ptr(feats)))
        return rows, feats

    def state(self):
        key = np.empty(624, np.uint32)
        pos = np.zeros(1, np.int32)
        check(lib().bsscl_sampler_state(self.handle, ptr(key), ptr(pos)))
        return key, int(pos[0])

    def stats(self):
        out = np.zeros(6, np.float64)
        n = np.zeros(1, np.int32)
        check(lib().bsscl_sampler_stats(self.handle, ptr(out), 6, ptr(n)))
        return dict(rounds=out[0], draw_ms=out[1], swap_ms=out[2], gen_ms=out[3],
                    spec_chunks=out[4], seq_chunks=out[5])

    def close(self):
        if getattr(self, "_h", None) is not None:
            lib().bsscl_sampler_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rs_draws(rng_state, n):
    """The bounded draws of RandomState.shuffle of n items: d[n-1-i] = j(i)
    for i = n-1 .. 1; returns (d, key, pos) with the advanced state."""
    key = np.ascontiguousarray(rng_state[1], dtype=np.uint32).copy()
    pos = np.array([rng_state[2]], np.int32)
    d = np.empty(max(int(n) - 1, 0) + 1, np.uint32)
    check(lib().bsscl_rs_draws(ptr(key), ptr(pos), ptr(d), int(n)))
    return d[:max(int(n) - 1, 0)], key, int(pos[0])


def rs_shuffle(rng_state, arr):
    """In-place RandomState.shuffle of a 1-D int64/int32 array; returns the
    new (key, pos)."""
    key = np.ascontiguousarray(rng_state[1], dtype=np.uint32).copy()
    pos = np.array([rng_state[2]], np.int32)
    if arr.dtype == np.int64:
        check(lib().bsscl_rs_shuffle_i64(ptr(key), ptr(pos), ptr(arr), len(arr)))
    elif arr.dtype == np.int32:
        check(lib().bsscl_rs_shuffle_i32(ptr(key), ptr(pos), ptr(arr), len(arr)))
    else:
        raise ValueError("rs_shuffle supports int64 and int32 arrays")
    return key, int(pos[0])
