"""bsscl_predict_noalloc (the entry point that allocates nothing) against
bsscl_predict through the C ABI: two calls in a row, the second with fewer
rows and trees, each equal to bsscl_predict's F; sizes beyond the fixed
scratch and a host output buffer are refused.

The caller's output buffer is allocated here with hipMalloc of the HIP
runtime the engine library links (torch bundles a runtime of its own, which
cannot share the GPU with it in one process)."""
import ctypes

import numpy as np
import pytest

from conftest import make_data
from oracle import model as om

pytestmark = pytest.mark.gpu


class DeviceBuffer:
    """float64[n] in device memory of GPU 0, through the engine's runtime."""

    def __init__(self, n):
        from bsscl_gbm import _native
        _native.lib()  # the engine library (and its libamdhip64) is loaded first
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.n = n
        self.p = ctypes.c_void_p()
        assert self.hip.hipSetDevice(0) == 0
        assert self.hip.hipMalloc(ctypes.byref(self.p), ctypes.c_size_t(8 * n)) == 0
        nan = np.full(n, np.nan)
        self._copy(self.p, nan.ctypes.data_as(ctypes.c_void_p), 1)  # host -> device

    def _copy(self, dst, src, kind):
        assert self.hip.hipMemcpy(dst, src, ctypes.c_size_t(8 * self.n), kind) == 0

    def read(self):
        out = np.empty(self.n)
        self._copy(out.ctypes.data_as(ctypes.c_void_p), self.p, 2)  # device -> host
        return out

    def close(self):
        if self.p:
            self.hip.hipFree(self.p)
            self.p = ctypes.c_void_p()


def _subset(packed, k):
    o = packed["offsets"]
    end = int(o[k])
    out = {key: np.ascontiguousarray(packed[key][:end])
           for key in ("features", "thresholds", "values", "left", "right")}
    out["offsets"] = np.ascontiguousarray(o[:k + 1])
    return out


def test_predict_noalloc_equals_predict(engine):
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    print("[case] predict_noalloc: 30000 x 12, 40 trees then 7001 rows, 15 trees", flush=True)
    X, y = make_data(30000, 12, seed=31, nan_frac=0.05)
    est = HybridHistGBMNumbaV1_0_1(n_estimators=40, max_depth=6, n_bins=255, random_state=4,
                                   verbose=False).fit(X, y)
    packed = {"features": est._packed_features, "thresholds": est._packed_thresholds,
              "values": est._packed_values, "left": est._packed_left,
              "right": est._packed_right, "offsets": est._tree_offsets}
    lr = est.learning_rate
    for rows, k in ((30000, 40), (7001, 15)):
        Xs = X[:rows]
        engine.bin_features(1, Xs, est.bin_edges, est.feature_bin_counts, est._nan_bin_id)
        sub = _subset(packed, k)
        want = engine.predict(1, rows, sub, k, lr)
        out = DeviceBuffer(rows)
        try:
            engine.predict_noalloc(1, sub, k, lr, out.p.value)
            got = out.read()
        finally:
            out.close()
        np.testing.assert_array_equal(got, want)
        ref = om.predict_all_trees(om.bin_features(Xs, est.bin_edges, est.feature_bin_counts,
                                                   est._nan_bin_id, "hybrid"), sub, k, lr)
        np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)
        print(f"[result] predict_noalloc rows={rows} trees={k}: equal to bsscl_predict", flush=True)


def test_predict_noalloc_refuses(engine):
    codes = np.zeros((64, 3), np.uint8)
    engine.load_codes(1, codes)
    many = 16385
    packed = {"features": np.full(many, -1, np.int16), "thresholds": np.zeros(many, np.int64),
              "values": np.zeros(many), "left": np.zeros(many, np.int32),
              "right": np.zeros(many, np.int32), "offsets": np.arange(many + 1, dtype=np.int32)}
    out = DeviceBuffer(64)
    try:
        with pytest.raises(ValueError, match="exceed the fixed scratch"):
            engine.predict_noalloc(1, packed, many, 0.1, out.p.value)
    finally:
        out.close()
    host = np.zeros(64)
    with pytest.raises(ValueError, match="not device memory"):
        engine.predict_noalloc(1, _subset(packed, 2), 2, 0.1, host.ctypes.data)
