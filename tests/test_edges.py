"""Bin edges (est:2073-2141) computed from device-sorted columns.

CPU tests pin the host arithmetic: the percentile ranks and interpolation
restated in the estimator must reproduce np.percentile bit for bit, given
the order statistics of the column.  GPU tests check the device half: the
sorted columns, NaN and distinct counts, distinct values and the finished
edges against the reference's NumPy expressions (oracle.build_bin_edges).
Edges must be bit-exact; the one freedom is the sign of a zero edge, which
the device returns as +0.0 (np.unique may keep either zero of a column that
holds both).
"""
import numpy as np
import pytest

from conftest import make_data
from oracle import model as om

from bsscl_gbm import estimator as est_mod


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _same_values(a, b):
    """Equal NaN pattern, equal values, and equal bits for every non-zero
    value (a zero may carry either sign)."""
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    ok = ~na
    if not np.array_equal(a[ok], b[ok]):
        return False
    nz = ok & (a != 0)
    bits = np.uint64 if a.dtype.itemsize == 8 else np.uint32
    return np.array_equal(a[nz].view(bits), b[nz].view(bits))


def _columns():
    rng = np.random.default_rng(5)
    cols = {
        "normal_f32": rng.standard_normal(100_003).astype(np.float32),
        "normal_f64": rng.standard_normal(7_777),
        "ties_f32": np.round(rng.standard_normal(50_000) * 3).astype(np.float32),
        "tiny_1": np.array([2.5], np.float32),
        "tiny_2": np.array([-1.0, 3.0], np.float32),
        "tiny_3": np.array([0.1, 0.2, 0.3]),
        "exp_f32": rng.exponential(1.0, 20_000).astype(np.float32),
        "wide_range_f32": (rng.standard_normal(5000) * 1e30).astype(np.float32),
        "with_inf_f32": np.concatenate([rng.standard_normal(999), [np.inf, -np.inf]]).astype(np.float32),
    }
    return cols


@pytest.mark.parametrize("name", list(_columns()))
@pytest.mark.parametrize("k", [2, 3, 17, 256])
def test_percentile_restatement_is_bit_exact(name, k):
    """_percentile_ranks + _percentile_lerp on the sorted column equal
    np.percentile(col, q * 100) for q = linspace(0, 1, k) (est:2113, 2126)."""
    col = _columns()[name]
    q = np.linspace(0, 1, k)
    want = np.percentile(col, q * 100)
    s = np.sort(col)
    lo, hi, gamma = est_mod._percentile_ranks(len(col), q * 100, col.dtype)
    got = est_mod._percentile_lerp(s[lo], s[hi], gamma)
    assert _same_values(got, want)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("k", [3, 256])
def test_percentile_restatement_batched_over_columns(dtype, k):
    """The estimator's batched form (one row per column, column lengths as a
    column vector) gives every column np.percentile(col, q * 100) bit for
    bit, as the single-column form does."""
    rng = np.random.default_rng(11)
    cols = [rng.standard_normal(m).astype(dtype) for m in (1, 2, 5, 999, 1000, 65_537)]
    cols.append(np.round(rng.standard_normal(4000) * 2).astype(dtype))
    q = np.linspace(0, 1, k)
    ms = np.array([len(c) for c in cols], dtype=np.int64)[:, None]
    lo, hi, gamma = est_mod._percentile_ranks(ms, q * 100, np.dtype(dtype))
    assert lo.shape == hi.shape == gamma.shape == (len(cols), k)
    s = [np.sort(c) for c in cols]
    a = np.stack([s[i][lo[i]] for i in range(len(cols))])
    b = np.stack([s[i][hi[i]] for i in range(len(cols))])
    got = est_mod._percentile_lerp(a, b, gamma)
    for i, c in enumerate(cols):
        assert _same_values(got[i], np.percentile(c, q * 100)), i


def test_percentile_restatement_detects_a_shifted_rank():
    """A plausible slip (rank from n instead of n - 1) changes the result:
    the bit-exact comparison above would catch it."""
    col = np.random.default_rng(1).standard_normal(1001).astype(np.float32)
    q = np.linspace(0, 1, 33)
    s = np.sort(col)
    lo, hi, gamma = est_mod._percentile_ranks(len(col) + 1, q * 100, col.dtype)
    lo, hi = np.minimum(lo, len(col) - 1), np.minimum(hi, len(col) - 1)
    assert not np.array_equal(est_mod._percentile_lerp(s[lo], s[hi], gamma),
                              np.percentile(col, q * 100))


def test_host_edges_equal_reference_expressions():
    X, _ = make_data(3000, 6, seed=8, nan_frac=0.2, nan_cols=[1, 4])
    X[:, 2] = np.round(X[:, 2])
    X[:, 5] = np.nan
    est = est_mod.HybridHistGBMNumbaV1_0_1(n_bins=255, verbose=False)
    e, bc = est._build_bin_edges_host(X)
    we, wbc, wnid = om.build_bin_edges(X, 255)
    np.testing.assert_array_equal(e, we)
    np.testing.assert_array_equal(bc, wbc)
    np.testing.assert_array_equal(est._nan_bin_id, wnid)


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
def _canon(a):
    """Values as the device sorts them: NaN dropped, -0.0 as +0.0."""
    a = a[~np.isnan(a)]
    return np.where(a == 0, np.zeros((), a.dtype), a)


@pytest.mark.gpu
@pytest.mark.parametrize("n,F,dtype", [(1, 1, np.float32), (5, 3, np.float64),
                                       (4096, 2, np.float32), (4097, 2, np.float32),
                                       (2048, 1, np.float64), (2049, 2, np.float64),
                                       (1_200_001, 2, np.float32), (300_001, 1, np.float64)])
def test_sort_columns_match_numpy(engine, n, F, dtype):
    _announce(f"sort_columns n={n} F={F} {np.dtype(dtype).name}")
    rng = np.random.default_rng(n + F)
    X = rng.standard_normal((n, F)).astype(dtype)
    if F > 1:
        X[rng.random(n) < 0.3, 1] = np.nan
        X[: min(n, 6), 1] = [np.inf, -np.inf, -0.0, 0.0, np.nan, 1.0][: min(n, 6)]
    if F > 2:
        X[:, 2] = np.nan
    engine.stage_features(X)
    nan, uniq = engine.sort_columns(F)
    for j in range(F):
        col = X[:, j]
        clean = _canon(col)
        assert nan[j] == np.isnan(col).sum()
        assert uniq[j] == len(np.unique(clean))
        m = len(clean)
        if m:
            got = engine.sorted_gather(np.full(m, j), np.arange(m))
            want = np.sort(clean).astype(np.float64)
            assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), j
    engine.release_staged()


@pytest.mark.gpu
def test_sorted_uniques_and_bounds(engine):
    _announce("sorted_uniques")
    rng = np.random.default_rng(3)
    X = np.round(rng.standard_normal((50_000, 2)) * 4).astype(np.float32)
    X[rng.random(50_000) < 0.5, 1] = np.nan
    X[:3, 0] = [-0.0, 0.0, -0.0]
    engine.stage_features(X)
    nan, uniq = engine.sort_columns(2)
    for j in range(2):
        want = np.unique(_canon(X[:, j]))
        got = engine.sorted_uniques(j, int(uniq[j]))
        assert np.array_equal(got, want.astype(np.float64))
        with pytest.raises(ValueError):
            engine.sorted_uniques(j, int(uniq[j]) - 1)
    with pytest.raises(ValueError):
        engine.sorted_gather([0], [50_000])
    engine.release_staged()


def _edge_cases():
    rng = np.random.default_rng(21)
    out = {}
    X, _ = make_data(20000, 7, seed=1)
    out["plain"] = (X, 255)
    X, _ = make_data(20000, 9, seed=2, nan_frac=0.3, nan_cols=[0, 3, 8])
    X[:, 5] = np.nan
    out["nan_allnan"] = (X, 255)
    X, _ = make_data(5000, 5, seed=3, dtype=np.float64, nan_frac=0.05)
    out["f64"] = (X, 255)
    X, _ = make_data(4000, 6, seed=5)
    X[:, 1] = np.round(X[:, 1])
    X[:, 2] = 3.0
    X[:4, 3] = [np.inf, -np.inf, 1e38, -1e38]
    X[:, 4] = rng.exponential(1.0, 4000) * (rng.random(4000) < 0.1)
    out["special"] = (X, 255)
    X, _ = make_data(30000, 4, seed=6, nan_frac=0.1, nan_cols=[1])
    X[:, 2] = np.round(X[:, 2] * 40)
    out["nbins64"] = (X, 64)
    X, _ = make_data(1000, 3, seed=7)
    out["nbins2"] = (X, 2)
    X = np.where(rng.random((100_000, 6)) < 0.9, 0.0, rng.exponential(1.0, (100_000, 6))).astype(np.float32)
    out["sparse_zeros"] = (X, 255)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(_edge_cases()))
def test_device_edges_equal_reference(engine, case):
    """The estimator's device edges equal the reference's NumPy expressions
    (est:2073-2141) bit for bit."""
    _announce(f"edges {case}")
    X, n_bins = _edge_cases()[case]
    est = est_mod.HybridHistGBMNumbaV1_0_1(n_bins=n_bins, verbose=False)
    engine.stage_features(X)
    try:
        e, bc = est._build_bin_edges(X, eng=engine)
    finally:
        engine.release_staged()
    we, wbc, wnid = om.build_bin_edges(X, n_bins)
    np.testing.assert_array_equal(bc, wbc)
    np.testing.assert_array_equal(est._nan_bin_id, wnid)
    assert _same_values(e, we)


@pytest.mark.gpu
def test_fit_codes_equal_reference_binning(engine):
    """fit() bins the staged matrix with the device edges: the codes equal
    the oracle's binning with the reference's edges."""
    _announce("fit codes")
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm.estimator import _engine
    X, y = make_data(30000, 6, seed=9, nan_frac=0.1, nan_cols=[0, 2])
    est = HybridHistGBMNumbaV1_0_1(n_estimators=1, max_depth=3, n_bins=255,
                                   random_state=0, verbose=False).fit(X, y)
    we, wbc, wnid = om.build_bin_edges(X, 255)
    assert _same_values(est.bin_edges, we)
    want = om.bin_features(X, we, wbc, wnid, "hybrid")
    got = _engine(0).get_codes(0, *X.shape)
    np.testing.assert_array_equal(got, np.minimum(want.astype(np.int64), 255).astype(np.uint8))


@pytest.mark.gpu
def test_staging_and_sorts_keep_device_memory_flat(engine):
    """Staging, column sorts, gathers and releases, four times over, leave
    the device's free memory where the first pass left it: the sort's work
    buffers and the gathers' are kept for the next staging or freed, never
    dropped (this shape's sort needs 256 MB of them)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")

    def free_bytes():
        free, total = ctypes.c_size_t(), ctypes.c_size_t()
        assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
        return free.value

    _announce("staging memory over repeated sorts (2M x 16 float32)")
    rng = np.random.default_rng(3)
    X = rng.standard_normal((2_000_000, 16)).astype(np.float32)
    X[:, 1] = rng.integers(0, 5, len(X))
    frees = []
    for _ in range(4):
        engine.stage_features(X)
        nan, uniq = engine.sort_columns(16)
        assert nan.sum() == 0 and uniq[1] == 5
        vals = engine.sorted_gather(np.arange(16), np.zeros(16, np.int64))
        assert np.array_equal(vals, X.min(axis=0).astype(np.float64))
        assert np.array_equal(engine.sorted_uniques(1, 8), np.arange(5.0))
        engine.release_staged()
        frees.append(free_bytes())
    print(f"[result] free device memory after each pass (MiB): "
          f"{[f >> 20 for f in frees]}", flush=True)
    assert min(frees[1:]) >= frees[0] - (16 << 20), frees
