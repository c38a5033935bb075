"""Parity of the HIP engine with the oracle, through the C ABI.

Bars: bin codes and partitions bit-exact; histogram sums within
|d| <= 1e-5 * max(|ref|, sum_bin |g|); splits identical except gain ties
within 1e-7 relative, which are followed to the end of the tree
(tests/treecmp.py); every training loss within 1e-9 relative and
predict_proba within 1e-6 (tests/fitcmp.py).
"""
import numpy as np
import pytest

import fitcmp
import treecmp
from conftest import make_data
from oracle import model as om

pytestmark = pytest.mark.gpu

HIST_RTOL = 1e-5


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _binned(X, n_bins, strategy="standard"):
    e, bc, nid = om.build_bin_edges(X, n_bins)
    codes = om.bin_features(X, e, bc, nid, strategy)
    return e, bc, nid, codes


def _tier_cap(bc):
    """Largest code a matrix binned with bin counts bc reads back exactly:
    255 per code tier, one tier per 255 thresholds past the first 255."""
    nb = int(np.max(bc))
    return 255 * (1 if nb <= 256 else (nb - 2) // 255 + 1)


@pytest.mark.parametrize("case", ["plain", "nan", "f64", "wide", "special", "nbins256",
                                  "nbins300", "nbins1000"])
def test_binning_bit_exact(engine, case):
    _announce(f"binning {case}")
    rng = np.random.default_rng(11)
    n_bins = 255
    if case == "plain":
        X, _ = make_data(20000, 7, seed=1)
    elif case == "nan":
        X, _ = make_data(20000, 9, seed=2, nan_frac=0.3, nan_cols=[0, 3, 8])
        X[:, 5] = np.nan
    elif case == "f64":
        X, _ = make_data(5000, 5, seed=3, dtype=np.float64, nan_frac=0.05)
    elif case == "wide":
        X, _ = make_data(3000, 130, seed=4, nan_frac=0.02)
    elif case == "special":
        X, _ = make_data(4000, 6, seed=5)
        X[:, 1] = np.round(X[:, 1])
        X[:, 2] = 3.0
        X[:4, 3] = [np.inf, -np.inf, 1e38, -1e38]
        X[:, 4] = rng.exponential(1.0, 4000) * (rng.random(4000) < 0.1)
    elif case == "nbins256":
        X, _ = make_data(6000, 4, seed=6, nan_frac=0.1, nan_cols=[1])
        X[:, 2] = np.round(X[:, 2] * 40)
        n_bins = 256
    else:
        # More than 256 bins: codes in two and in four 8-bit tiers.
        X, _ = make_data(12000, 5, seed=7, nan_frac=0.1, nan_cols=[0, 3])
        X[:, 2] = np.round(X[:, 2] * 40)
        n_bins = 300 if case == "nbins300" else 1000
    e, bc, nid, want = _binned(X, n_bins)
    if case == "nbins256":
        # n_bins = 256: continuous columns get 257 bins and uint16 codes.
        assert bc.max() == 257 and want.dtype == np.uint16 and want.max() == 256
    if case in ("nbins300", "nbins1000"):
        assert want.dtype == np.uint16 and want.max() == n_bins
    got = engine.bin_features(0, X, e, bc, nid, return_codes=True)
    np.testing.assert_array_equal(got, np.minimum(want.astype(np.int64), 255).astype(np.uint8))
    if want.dtype == np.uint16:
        np.testing.assert_array_equal(engine.get_codes(0, *X.shape, u16=True), want)
    # Scoring matrix: values outside the training range and NaN in columns
    # that had none.
    Xp = X.copy()
    Xp[:100, 0] = np.nan
    Xp[100:200, -1] = 1e30
    want_p = om.bin_features(Xp, e, bc, nid, "hybrid")
    got_p = engine.bin_features(1, Xp, e, bc, nid, return_codes=True)
    np.testing.assert_array_equal(got_p, np.minimum(want_p.astype(np.int64), 255).astype(np.uint8))
    if want_p.dtype == np.uint16:
        # A code above every bin of its feature (a value above the training
        # range of a NaN feature) reads back capped at the tiers' range; no
        # split tells the two apart.
        np.testing.assert_array_equal(engine.get_codes(1, *Xp.shape, u16=True),
                                      np.minimum(want_p, _tier_cap(bc)))


@pytest.mark.parametrize("m,bin_", [(50_001, 255), (50_001, 254), (3000, 256)])
def test_partition_top_bin(engine, m, bin_):
    """257-bin codes (uint16): the split at bin 255 sends code 256 right."""
    _announce(f"partition 257 bins m={m} bin={bin_}")
    rng = np.random.default_rng(m + bin_)
    n = 2 * m
    codes = rng.integers(0, 257, (n, 3)).astype(np.uint16)
    codes[rng.random(n) < 0.2, 1] = 256
    engine.load_codes(0, codes)
    np.testing.assert_array_equal(engine.get_codes(0, n, 3, u16=True), codes)
    rows = rng.permutation(n)[:m].astype(np.int64)
    out, nl = engine.partition(rows, 1, bin_)
    left = codes[rows, 1] <= bin_
    assert nl == int(left.sum())
    np.testing.assert_array_equal(out[:nl], rows[left])
    np.testing.assert_array_equal(out[nl:], rows[~left])


@pytest.mark.parametrize("bin_", [254, 255, 300, 509, 510, 764, 765, 999])
def test_partition_code_tiers(engine, bin_):
    """Codes up to 1000 (uint16, four tiers): the split at any bin sends
    exactly the rows with code <= bin left, in order."""
    _announce(f"partition code tiers bin={bin_}")
    rng = np.random.default_rng(bin_)
    m = 70_001
    n = 2 * m
    codes = rng.integers(0, 1001, (n, 3)).astype(np.uint16)
    codes[rng.random(n) < 0.1, 1] = 1000
    engine.load_codes(0, codes)
    np.testing.assert_array_equal(engine.get_codes(0, n, 3, u16=True), codes)
    rows = rng.permutation(n)[:m].astype(np.int64)
    out, nl = engine.partition(rows, 1, bin_)
    left = codes[rows, 1] <= bin_
    assert nl == int(left.sum())
    np.testing.assert_array_equal(out[:nl], rows[left])
    np.testing.assert_array_equal(out[nl:], rows[~left])


def test_load_codes_roundtrip(engine):
    _announce("load_codes")
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 256, (3001, 11)).astype(np.uint8)
    engine.load_codes(0, codes)
    np.testing.assert_array_equal(engine.get_codes(0, 3001, 11), codes)
    c16 = rng.integers(0, 300, (777, 3)).astype(np.uint16)
    engine.load_codes(1, c16)
    np.testing.assert_array_equal(engine.get_codes(1, 777, 3), np.minimum(c16, 255).astype(np.uint8))


def _grad_hess(y, seed, w=(1.0, 1.0)):
    rng = np.random.default_rng(seed)
    p = 1 / (1 + np.exp(-rng.standard_normal(len(y))))
    wt = np.where(y == 1, w[1], w[0])
    return wt * (p - y), wt * p * (1 - p)


@pytest.mark.parametrize("n,F,nan,weights", [
    (50000, 12, 0.0, (1.0, 1.0)),
    (200001, 30, 0.05, (0.785, 7.31)),
    (7000, 70, 0.7, (1.0, 1.0)),
])
def test_histogram_and_split(engine, n, F, nan, weights):
    _announce(f"histogram n={n} F={F} nan={nan}")
    X, y = make_data(n, F, seed=n % 97, nan_frac=nan, nan_cols=list(range(0, F, 3)))
    e, bc, nid, codes = _binned(X, 255)
    engine.load_codes(0, codes)
    g, h = _grad_hess(y, 1, weights)
    rng = np.random.default_rng(2)
    rows = rng.permutation(n)[: int(0.75 * n)].astype(np.int64)
    feats = np.sort(rng.permutation(F)[: max(1, int(0.8 * F))]).astype(np.int32)
    G, H, gain, feat, b = engine.node_split(g, h, rows, feats, bc, 3.0, 1.0)
    absG = np.zeros_like(G)
    for i, j in enumerate(feats):
        nb = int(bc[j])
        c = np.minimum(codes[rows, j].astype(np.int64), nb - 1)
        Gr = np.bincount(c, weights=g[rows], minlength=256)
        Hr = np.bincount(c, weights=h[rows], minlength=256)
        absG[i] = np.bincount(c, weights=np.abs(g[rows]), minlength=256)
        tolG = HIST_RTOL * np.maximum(np.abs(Gr), absG[i]) + 1e-12
        tolH = HIST_RTOL * np.abs(Hr) + 1e-12
        assert np.all(np.abs(G[i] - Gr) <= tolG), f"G feature {j}"
        assert np.all(np.abs(H[i] - Hr) <= tolH), f"H feature {j}"
        # Every feature's histogram sums to the node total.
        assert abs(G[i].sum() - g[rows].sum()) <= 1e-6 * np.abs(g[rows]).sum()
    # Best split equals the oracle's root split unless the gains tie.
    tree = om.build_tree(codes, g, h, rows, feats, 2, 1, 0, 3.0, bc, int(bc.max()), 1.0, -1e300)
    rf, rt = int(tree[0][0]), int(tree[1][0])
    if (rf, rt) != (feat, b):
        ga = treecmp.split_gain(codes, g, h, rows, rf, rt, int(bc[rf]), 1.0)
        gb = treecmp.split_gain(codes, g, h, rows, feat, b, int(bc[feat]), 1.0)
        assert abs(ga - gb) <= treecmp.GAIN_TIE_RTOL * abs(ga), (rf, rt, feat, b, ga, gb)
    else:
        np.testing.assert_allclose(gain, tree[6][0], rtol=1e-7)


@pytest.mark.parametrize("m,bin_", [(1, 5), (4097, 100), (123457, 30), (60000, 0), (60000, 254),
                                    (1_200_001, 77), (2_097_151, 200)])
def test_partition_stable_and_exact(engine, m, bin_):
    """Sizes from 1 row to 2,097,151 cover the 1024-, 2048- and 4096-row
    partition tiles (chosen by the in-bag row count)."""
    _announce(f"partition m={m} bin={bin_}")
    rng = np.random.default_rng(m)
    n, F = max(m * 2, 10), 3
    codes = rng.integers(0, 256, (n, F)).astype(np.uint8)
    engine.load_codes(0, codes)
    rows = rng.permutation(n)[:m].astype(np.int64)
    out, nl = engine.partition(rows, 1, bin_)
    left = codes[rows, 1] <= bin_
    assert nl == int(left.sum())
    np.testing.assert_array_equal(out[:nl], rows[left])
    np.testing.assert_array_equal(out[nl:], rows[~left])


def _lockstep_case(engine, n, F, seed, n_bins, max_leaves, max_depth, msl, mcw,
                   lam, nan=0.0, weights=(1.0, 1.0), sub=0.8, col=0.8):
    X, y = make_data(n, F, seed=seed, nan_frac=nan)
    e, bc, nid, codes = _binned(X, n_bins, "hybrid")
    engine.load_codes(0, codes)
    g, h = _grad_hess(y, seed + 1, weights)
    rng = np.random.default_rng(seed + 2)
    rows = rng.permutation(n)[: max(1, int(sub * n))].astype(np.int64)
    feats = np.sort(rng.permutation(F)[: max(1, int(col * F))]).astype(np.int32)
    args = (rows, feats, max_leaves, max_depth, msl, mcw, bc, int(bc.max()), lam, 0.0)
    got = engine.build_tree(g, h, *args)
    out = treecmp.follow(got, codes, g, h, *args)
    print(f"[result] lockstep n={n} F={F} seed={seed}: {got[5]} nodes, ties {out.ties}", flush=True)
    return out


@pytest.mark.parametrize("n", [1, 2, 3, 5, 64, 1000, 4099, 70_001])
@pytest.mark.parametrize("form", ["lists", "sorted"])
def test_fisher_yates_device_adversarial(engine, n, form, monkeypatch):
    """GPU swaps (per-position lists, or the sorted (position, step) form)
    against the sequential loop for draws no RNG would give: one position
    chosen by every step, no swaps, a chain through all steps.  70,001 rows
    sort their keys over 35 tiles in three passes."""
    from test_sampler import _adversarial_draws
    import fy_model
    monkeypatch.setenv("BSSCL_FY_SORTED", "1" if form == "sorted" else "0")
    a0 = np.random.default_rng(n).permutation(n).astype(np.int32)
    draws = _adversarial_draws(n) if n > 1 else {"empty": np.zeros(0, np.uint32)}
    for name, d in draws.items():
        _announce(f"fisher-yates n={n} {form} {name}")
        np.testing.assert_array_equal(engine.fisher_yates_apply(d, a0),
                                      fy_model.fisher_yates_sequential(a0, d), err_msg=name)


@pytest.mark.parametrize("n", [7, 65_537, 1_000_003])
@pytest.mark.parametrize("form", ["lists", "sorted"])
def test_fisher_yates_device_equals_numpy_shuffle(engine, n, form, monkeypatch):
    """The two halves (host draws, GPU swaps) equal RandomState.shuffle."""
    from bsscl_gbm import _native
    monkeypatch.setenv("BSSCL_FY_SORTED", "1" if form == "sorted" else "0")
    _announce(f"fisher-yates mt n={n} {form}")
    rng = np.random.RandomState(n)
    a = np.arange(n, dtype=np.int32)[::-1].copy()
    d, _, _ = _native.rs_draws(rng.get_state(), n)
    got = engine.fisher_yates_apply(d, a)
    rng.shuffle(a)
    np.testing.assert_array_equal(got, a)


@pytest.mark.parametrize("case", [
    dict(n=10000, F=20, seed=0, n_bins=255, max_leaves=31, max_depth=6, msl=5, mcw=2.0, lam=1.0),
    dict(n=30000, F=28, seed=1, n_bins=255, max_leaves=63, max_depth=6, msl=5, mcw=3.0, lam=1.0, nan=0.05),
    dict(n=20000, F=30, seed=2, n_bins=255, max_leaves=63, max_depth=6, msl=5, mcw=3.0, lam=1.0, weights=(0.785, 7.31)),
    dict(n=8000, F=100, seed=3, n_bins=255, max_leaves=63, max_depth=6, msl=5, mcw=3.0, lam=1.0, col=0.7),
    dict(n=40000, F=50, seed=4, n_bins=255, max_leaves=63, max_depth=8, msl=5, mcw=3.0, lam=5.0, nan=0.2, col=0.7, sub=0.5),
    dict(n=3000, F=6, seed=5, n_bins=16, max_leaves=15, max_depth=10, msl=20, mcw=0.0, lam=0.5),
    dict(n=500, F=10, seed=6, n_bins=112, max_leaves=15, max_depth=3, msl=5, mcw=1.0, lam=1.0),
    dict(n=2000, F=4, seed=7, n_bins=64, max_leaves=1, max_depth=6, msl=5, mcw=1.0, lam=1.0),
    dict(n=50, F=3, seed=8, n_bins=8, max_leaves=31, max_depth=6, msl=40, mcw=1.0, lam=1.0),
    dict(n=30000, F=12, seed=9, n_bins=255, max_leaves=63, max_depth=8, msl=5, mcw=1.0, lam=1.0, nan=0.7),
    dict(n=5000, F=5, seed=10, n_bins=64, max_leaves=31, max_depth=1, msl=5, mcw=1.0, lam=1.0),
    dict(n=60000, F=30, seed=11, n_bins=255, max_leaves=255, max_depth=12, msl=2, mcw=0.5, lam=1.0, nan=0.05),
    # n_bins = 256: 257-bin features (uint16 codes, est:2163-2166).
    dict(n=40000, F=30, seed=13, n_bins=256, max_leaves=63, max_depth=6, msl=5, mcw=3.0, lam=1.0),
    dict(n=30000, F=28, seed=14, n_bins=256, max_leaves=63, max_depth=8, msl=5, mcw=1.0, lam=1.0,
         nan=0.1, col=0.8),
    # 1.5M in-bag rows: the 2048-row partition tiles.
    dict(n=2_000_000, F=8, seed=12, n_bins=255, max_leaves=63, max_depth=6, msl=5, mcw=3.0, lam=1.0,
         nan=0.05, sub=0.75, col=1.0),
])
def test_build_tree_lockstep(engine, case):
    _announce(f"lockstep {case}")
    _lockstep_case(engine, **case)


@pytest.mark.gpu
@pytest.mark.parametrize("case", [
    dict(n=40000, F=50, seed=4, n_bins=255, max_leaves=63, max_depth=8, msl=5, mcw=3.0, lam=5.0, nan=0.2, col=0.7, sub=0.5),
    dict(n=3000, F=6, seed=5, n_bins=16, max_leaves=15, max_depth=10, msl=20, mcw=0.0, lam=0.5),
    dict(n=60000, F=30, seed=11, n_bins=255, max_leaves=255, max_depth=12, msl=2, mcw=0.5, lam=1.0, nan=0.05),
])
def test_build_tree_lockstep_moving_every_level(engine, case, monkeypatch):
    """The builder that moves the rows at every level (instead of every
    second level, the default) builds the oracle's trees too."""
    _announce(f"lockstep, rows moved every level {case}")
    monkeypatch.setenv("BSSCL_TEST_PAIR_LEVELS", "0")
    _lockstep_case(engine, **case)


def test_predict_matches_oracle(engine):
    _announce("predict")
    X, y = make_data(20000, 12, seed=9, nan_frac=0.05)
    m = om.OracleGBM(n_estimators=8, max_depth=5, learning_rate=0.1, n_bins=255,
                     class_weight=None, random_state=3).fit(X, y)
    Xb = m.X_bin_
    engine.load_codes(0, Xb)
    for tree in m.trees[:3]:
        np.testing.assert_array_equal(engine.predict_tree(0, len(X), tree), om.predict_tree(Xb, tree))
    F = engine.predict(0, len(X), m._packed, len(m.trees), 0.1)
    np.testing.assert_allclose(F, om.predict_all_trees(Xb, m._packed, len(m.trees), 0.1), rtol=0, atol=1e-12)


def _swap_first_children(packed, t):
    """Tree t of a packed model with nodes 1 and 2 exchanged: the root's right
    child then precedes its left child (same tree, other numbering)."""
    p = {k: np.array(v, copy=True) for k, v in packed.items()}
    a = int(p["offsets"][t])
    i1, i2 = a + 1, a + 2
    for k in ("features", "thresholds", "values", "left", "right"):
        p[k][[i1, i2]] = p[k][[i2, i1]]
    for k in ("left", "right"):
        seg = p[k][a:int(p["offsets"][t + 1])]
        one, two = seg == 1, seg == 2
        seg[one], seg[two] = 2, 1
    return p


def test_predict_kernels_agree(engine, monkeypatch):
    """The LDS-staged ensemble kernel (several tree runs per block) and the
    HBM walk give bit-identical F; a tree numbered with the right child first
    takes the HBM walk and still predicts the oracle's F (est:863-884)."""
    _announce("predict kernels")
    X, y = make_data(30000, 24, seed=21, nan_frac=0.05)
    m = om.OracleGBM(n_estimators=60, max_depth=6, learning_rate=0.1, n_bins=255,
                     class_weight=None, random_state=4).fit(X, y)
    Xb = m.X_bin_
    engine.load_codes(0, Xb)
    n_t = len(m.trees)
    assert int(m._packed["offsets"][n_t]) > 2048  # several runs of whole trees
    want = om.predict_all_trees(Xb, m._packed, n_t, 0.1)
    staged = engine.predict(0, len(X), m._packed, n_t, 0.1)
    monkeypatch.setenv("BSSCL_TEST_PREDICT_GLOBAL", "1")
    walked = engine.predict(0, len(X), m._packed, n_t, 0.1)
    monkeypatch.delenv("BSSCL_TEST_PREDICT_GLOBAL")
    np.testing.assert_array_equal(staged, walked)
    np.testing.assert_allclose(staged, want, rtol=0, atol=1e-12)
    swapped = _swap_first_children(m._packed, 5)
    assert swapped["right"][int(swapped["offsets"][5])] + 1 == swapped["left"][int(swapped["offsets"][5])]
    np.testing.assert_array_equal(engine.predict(0, len(X), swapped, n_t, 0.1), staged)
    print(f"[result] predict kernels: {n_t} trees, {int(m._packed['offsets'][n_t])} nodes over "
          f"{len(X)} rows: staged == HBM walk == renumbered tree", flush=True)


def _fit_case(name):
    if name == "defaults_28":
        # Every parameter at the reference's default: n_bins='auto' resolves
        # to 256 at p = 28 (est:1963-1964), so the continuous columns get 257
        # bins.
        X, y = make_data(30000, 28, seed=15, nan_frac=0.05, nan_cols=list(range(0, 28, 4)))
        return X, y, dict(random_state=0)
    if name == "top_bin_28":
        # Defaults again, and in two columns 60 rows sit exactly at the
        # column's maximum (code 256 of 257) and are all positive: the split
        # at bin 255 (code 256 goes right) is the best one there.
        rng = np.random.default_rng(16)
        X = rng.standard_normal((20000, 28)).astype(np.float32)
        y = (rng.random(20000) < 0.05).astype(np.int64)
        for j in (3, 11):
            idx = rng.choice(20000, 60, replace=False)
            X[idx, j] = X[:, j].max()
            y[idx] = 1
        return X, y, dict(n_estimators=40, random_state=0)
    if name in ("nbins_600", "nbins_2000"):
        # More than 256 bins per feature (uint16 codes, est:2163-2166): two
        # or more 8-bit code tiers per feature, with bagging and NaN columns.
        X, y = make_data(40000, 10, seed=18, nan_frac=0.05, nan_cols=[1, 6])
        nb = 600 if name == "nbins_600" else 2000
        return X, y, dict(n_estimators=12, max_depth=6, n_bins=nb, subsample=0.8,
                          colsample_bytree=0.8, random_state=0)
    if name == "config1":
        rng = np.random.default_rng(0)
        X = rng.standard_normal((10_000, 20), dtype=np.float32)
        w = rng.standard_normal(20)
        y = (rng.random(10_000) < 1 / (1 + np.exp(-(X @ w)))).astype(np.int64)
        params = dict(n_estimators=10, max_depth=6, learning_rate=0.1, n_bins=255,
                      class_weight=None, random_state=0)
    elif name == "scale_pos_weight":
        # scale_pos_weight with objective='binary' (est:2570-2576): class
        # weights 1 and 6, edges from weighted quantiles (est:2114-2124, host
        # branch), 4% positives.
        X, y = make_data(25000, 16, seed=17, nan_frac=0.05, nan_cols=[2, 9])
        y = (np.random.default_rng(7).random(25000) < 0.04).astype(np.int64)
        X[y == 1, :6] += 0.8
        params = dict(n_estimators=12, max_depth=6, n_bins=255, scale_pos_weight=6.0,
                      objective="binary", random_state=0)
    elif name == "confident_400":
        # A long fit on separable data (12% positives, balanced_sqrt): the
        # late rounds' gradients and hessians of most rows are far below
        # the class weight that scales the fixed-point values, and a small
        # min_child_weight lets the trees keep splitting those rows.
        rng = np.random.default_rng(0)
        X = rng.standard_normal((30000, 8)).astype(np.float32)
        y = ((X[:, 0] + 0.5 * X[:, 1]) > 1.3).astype(np.int64)
        params = dict(n_estimators=400, max_depth=6, learning_rate=1.0, n_bins=255,
                      min_child_weight=1e-3, class_weight="balanced_sqrt", random_state=0)
    elif name == "nan_imbalanced":
        X, y = make_data(30000, 30, seed=12, nan_frac=0.05)
        y = (np.random.default_rng(1).random(30000) < 0.03).astype(np.int64)
        X[y == 1, :10] += 1.0
        params = dict(n_estimators=12, max_depth=6, n_bins=255, random_state=0)
    else:
        rng = np.random.default_rng(3)
        X = np.where(rng.random((20000, 40)) < 0.9, 0.0,
                     rng.exponential(1.0, (20000, 40))).astype(np.float32)
        y = (X[:, :8].sum(1) + rng.logistic(size=20000) > 3.0).astype(np.int64)
        params = dict(n_estimators=10, max_depth=6, n_bins=255, random_state=1)
    return X, y, params


@pytest.mark.parametrize("name", ["config1", "nan_imbalanced", "sparse", "defaults_28",
                                  "top_bin_28", "scale_pos_weight", "confident_400",
                                  "nbins_600", "nbins_2000"])
def test_fit_lockstep_and_end_to_end(engine, name):
    """Every round of the oracle's fit, rebuilt by the engine from the same
    gradients, rows and features (lockstep), and the estimator's own tree of
    that round (end to end) equal the oracle's tree, following certified
    gain ties (tests/fitcmp.py).  Then every round's training loss and
    predict_proba match."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    _announce(f"fit {name}")
    X, y, params = _fit_case(name)
    est = HybridHistGBMNumbaV1_0_1(verbose=False, **params).fit(X, y)
    ref, rep = fitcmp.follow_fit(engine, est, X, y, params)
    print(rep.line(name), flush=True)
    assert rep.rounds == ref.n_estimators == len(est.trees)
    fitcmp.assert_fit_equal(ref, est, X)
    if name == "confident_400":
        print(f"[result] confident_400: final training loss {est.train_loss_history_[-1]:.3g}",
              flush=True)
        assert est.train_loss_history_[-1] < 1e-4
    if name in ("nbins_600", "nbins_2000"):
        from bsscl_gbm import estimator as est_mod
        got = est_mod._engine(0).get_codes(0, *X.shape, u16=True)
        np.testing.assert_array_equal(got, ref.X_bin_)
        splits = [t for tr in est.trees for f, t in zip(tr[0][:tr[5]], tr[1][:tr[5]]) if f >= 0]
        past = sum(t > 255 for t in splits)
        print(f"[result] {name}: {est._max_bins} bins, {past} of {len(splits)} splits past "
              f"bin 255", flush=True)
        assert past > 0
    if name in ("defaults_28", "top_bin_28"):
        from bsscl_gbm import estimator as est_mod
        assert est.n_bins == 256 and est._max_bins == 257
        got = est_mod._engine(0).get_codes(0, *X.shape, u16=True)
        np.testing.assert_array_equal(got, ref.X_bin_)
        splits = [(f, t) for tr in est.trees for f, t in zip(tr[0][:tr[5]], tr[1][:tr[5]]) if f >= 0]
        at255 = sum(t == 255 for _, t in splits)
        print(f"[result] {name}: {at255} splits at bin 255 of {len(splits)}", flush=True)
        if name == "top_bin_28":
            assert at255 > 0


def test_fit_fixed_point_scale_from_device_maxima(engine, monkeypatch):
    """A boosting round scales its tree's int64 gradients and hessians from
    the largest |g| and h of the current F, which the previous F update (or
    boost_begin) leaves on the device.  Those maxima equal NumPy's over the
    device's float64 gradients of the same F, at the start and after the
    fit.  On the confident fit, where late rounds' hessians are far below
    the class-weight bound, the device-scaled fit follows the oracle with no
    more certified ties than the bound-scaled one (BSSCL_TEST_BOUND_SCALE=1)."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    _announce("fit confident_400 (160 rounds): device maxima against the bound")
    X, y, params = _fit_case("confident_400")
    params = dict(params, n_estimators=160)
    eng = est_mod._engine(0)
    n = len(y)
    ties = {}
    for mode in ("bound", "device"):
        if mode == "bound":
            monkeypatch.setenv("BSSCL_TEST_BOUND_SCALE", "1")
        else:
            monkeypatch.delenv("BSSCL_TEST_BOUND_SCALE", raising=False)
        est = HybridHistGBMNumbaV1_0_1(verbose=False, **params).fit(X, y)
        # After the fit the engine still holds the run's F and its maxima.
        g, h = eng.boost_grad_hess(n)
        gmax, hmax = eng.boost_grad_hess_max()
        assert gmax == np.max(np.abs(g)) and hmax == np.max(h)
        w0, w1 = est._class_weight_pair(y)
        print(f"[result] confident fit after 160 rounds: max |g| {gmax:.3g}, max h {hmax:.3g} "
              f"(bound: {max(w0, w1):.3g}, {0.25 * max(w0, w1):.3g})", flush=True)
        ref, rep = fitcmp.follow_fit(engine, est, X, y, params, lockstep=False)
        fitcmp.assert_fit_equal(ref, est, X)
        ties[mode] = sum(rep.end_to_end_ties)
        print(rep.line(f"confident_160 {mode}-scaled"), flush=True)
    assert ties["device"] <= ties["bound"]
    # The starting F's maxima (boost_begin), against NumPy's.
    eng.boost_begin(y, 1.0, 3.0, 0.25)
    g, h = eng.boost_grad_hess(n)
    assert eng.boost_grad_hess_max() == (np.max(np.abs(g)), np.max(h))


def test_fit_graph_rounds_match_direct_launches(engine, monkeypatch):
    """Boosting rounds replayed from captured HIP graphs give the trees and
    losses of rounds whose kernels are launched one by one: the rows
    stream's graph (Fisher-Yates, in-bag sort, code gather; the default) and
    the tree stream's (gradients, levels, replay, F update and the readback;
    BSSCL_GRAPHS=1).  Rows and features are bagged, so each round's draws
    reach the rows graph through its device-side address.  Graphs are
    replayed within a fit and across fits, pipelined and not.  At profiling
    level 1 the tree kernels are launched one by one (their timing stamps
    take per-round addresses) and every histogram launch is timed."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    X, y = make_data(60000, 24, seed=21, nan_frac=0.03)
    params = dict(n_estimators=14, max_depth=6, n_bins=255, subsample=0.7,
                  colsample_bytree=0.8, random_state=3)
    eng = est_mod._engine(0)

    def fit(graphs, prof=0, pipeline=True):
        _announce(f"fit BSSCL_GRAPHS={graphs} prof={prof} pipeline={pipeline}")
        if graphs is None:
            monkeypatch.delenv("BSSCL_GRAPHS", raising=False)
        else:
            monkeypatch.setenv("BSSCL_GRAPHS", graphs)
        est = HybridHistGBMNumbaV1_0_1(verbose=False, **params)
        est._pipeline_rounds = pipeline
        eng.set_profiling(prof)
        try:
            st0 = eng.stats()
            est.fit(X, y)
            st = eng.stats()
        finally:
            eng.set_profiling(0)
        d = {k: st[k] - (st0[k] if prof == 0 else 0.0) for k in st}
        print(f"[result] BSSCL_GRAPHS={graphs} prof={prof} pipeline={pipeline}: rows graph "
              f"rounds {d['rows_graph_rounds']:.0f}, tree graph rounds "
              f"{d['tree_graph_rounds']:.0f}, captures {d['graph_captures']:.0f}, "
              f"histogram launches {d['hist_launches']:.0f}", flush=True)
        return est, d

    n = params["n_estimators"]
    ref, d0 = fit("0")
    assert d0["rows_graph_rounds"] == d0["tree_graph_rounds"] == 0
    _, dp0 = fit("0", prof=1)
    # (A fit's first round starts the permutation, outside the rows graph.)
    for graphs, prof, pipeline, rows_min, tree_min in (
            (None, 0, True, n - 1, 0), ("1", 0, True, n - 1, n), ("1", 0, True, n - 1, n),
            ("1", 1, True, n - 1, 0), ("1", 0, False, n - 1, n)):
        got, d = fit(graphs, prof, pipeline)
        mode = (graphs, prof, pipeline)
        assert d["rows_graph_rounds"] >= rows_min, mode
        assert d["tree_graph_rounds"] >= tree_min, mode
        if tree_min == 0:
            assert d["tree_graph_rounds"] == 0, mode
        if prof == 1:
            assert d["hist_launches"] == dp0["hist_launches"] > 0, mode
            assert d["hist_ms"] > 0
        assert got.train_loss_history_ == ref.train_loss_history_, mode
        assert len(got.trees) == len(ref.trees) == n
        for a, b in zip(ref.trees, got.trees):
            nc = a[5]
            assert nc == b[5], mode
            for k in (0, 1, 2, 3, 4, 6):
                np.testing.assert_array_equal(a[k][:nc], b[k][:nc], err_msg=str(mode))
    monkeypatch.delenv("BSSCL_GRAPHS", raising=False)


def test_graph_rounds_after_buffers_grow(engine, monkeypatch):
    """Fits of different sizes in turn (the second grows the engine's
    buffers, so graphs captured before hold stale addresses and must be
    captured again; the third returns to the first size with the larger
    buffers) give with BSSCL_GRAPHS=1 the trees and losses of fits whose
    kernels are launched one by one."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    eng = est_mod._engine(0)
    cases = [make_data(30000, 12, seed=41, nan_frac=0.02), make_data(90000, 20, seed=42),
             make_data(30000, 12, seed=41, nan_frac=0.02)]
    params = dict(n_estimators=8, max_depth=5, n_bins=255, subsample=0.8,
                  colsample_bytree=0.9, random_state=5)
    fits = {}
    for graphs in ("0", "1"):
        monkeypatch.setenv("BSSCL_GRAPHS", graphs)
        for j, (X, y) in enumerate(cases):
            _announce(f"fit {j} ({X.shape[0]} x {X.shape[1]}) BSSCL_GRAPHS={graphs}")
            st0 = eng.stats()
            fits[graphs, j] = HybridHistGBMNumbaV1_0_1(verbose=False, **params).fit(X, y)
            st = eng.stats()
            if graphs == "1":
                assert st["tree_graph_rounds"] - st0["tree_graph_rounds"] >= params["n_estimators"]
    monkeypatch.delenv("BSSCL_GRAPHS", raising=False)
    for j in range(len(cases)):
        ref, got = fits["0", j], fits["1", j]
        assert got.train_loss_history_ == ref.train_loss_history_, j
        for a, b in zip(ref.trees, got.trees):
            nc = a[5]
            assert nc == b[5], j
            for k in (0, 1, 2, 3, 4, 6):
                np.testing.assert_array_equal(a[k][:nc], b[k][:nc], err_msg=str(j))
    print(f"[result] graphs after buffer growth: {len(cases)} fits equal to direct launches",
          flush=True)


def test_fit_planner_counts_same_level_splits(engine, monkeypatch):
    """With min_child_weight >= min_samples_leaf * (largest hessian), every
    split a node can take is kept (est:614-615, 678-683), so the level
    planner also counts the level's other candidates as kept splits ranked
    above a candidate.  A depth-8 fit with 63 leaves then expands far fewer
    nodes, and its trees and losses equal those of the planner that counts
    earlier levels only (BSSCL_TEST_ALL_KEPT=0) and the oracle's."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    X, y = make_data(80000, 24, seed=31, nan_frac=0.02)
    params = dict(n_estimators=8, max_depth=8, n_bins=255, random_state=2, class_weight=None)
    eng = est_mod._engine(0)
    fits, expanded = {}, {}
    for mode in ("1", "0"):
        _announce(f"planner counting same-level splits: BSSCL_TEST_ALL_KEPT={mode}")
        monkeypatch.setenv("BSSCL_TEST_ALL_KEPT", mode)
        est = HybridHistGBMNumbaV1_0_1(verbose=False, **params)
        eng.set_profiling(1)
        try:
            est.fit(X, y)
            st = eng.stats()
        finally:
            eng.set_profiling(0)
        fits[mode] = est
        expanded[mode] = st["nodes_expanded"] / max(st["trees"], 1)
    monkeypatch.delenv("BSSCL_TEST_ALL_KEPT", raising=False)
    print(f"[result] nodes expanded per tree: {expanded['1']:.1f} counting the level's "
          f"splits, {expanded['0']:.1f} without", flush=True)
    a_fit, b_fit = fits["1"], fits["0"]
    assert a_fit.min_child_weight >= a_fit.min_samples_leaf * 0.25
    assert expanded["1"] < expanded["0"]
    assert a_fit.train_loss_history_ == b_fit.train_loss_history_
    for a, b in zip(a_fit.trees, b_fit.trees):
        nc = a[5]
        assert nc == b[5]
        for k in (0, 1, 2, 3, 4, 6):
            np.testing.assert_array_equal(a[k][:nc], b[k][:nc])
    ref, rep = fitcmp.follow_fit(engine, a_fit, X, y, params)
    print(rep.line("planner counting same-level splits"), flush=True)
    fitcmp.assert_fit_equal(ref, a_fit, X)


def test_profiling_counts_agree(engine, monkeypatch):
    """The node-table counts behind the histogram roofline (rows x features
    histogrammed, bytes, nodes expanded), taken by the in-LDS replay kernel,
    equal those the host takes from the node table read back after the
    other replay form, and include every round's root."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    from bsscl_gbm import estimator as est_mod
    X, y, params = _fit_case("nan_imbalanced")
    params = dict(params, n_estimators=6)
    eng = est_mod._engine(0)
    got = {}
    for mode, env in [("lds", {}), ("table", {"BSSCL_TEST_REPLAY_GLOBAL": "1"})]:
        _announce(f"profiling counts, replay {mode}")
        monkeypatch.delenv("BSSCL_TEST_REPLAY_GLOBAL", raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        est = HybridHistGBMNumbaV1_0_1(verbose=False, **params)
        eng.set_profiling(1)
        try:
            est.fit(X, y)
            st = eng.stats()
        finally:
            eng.set_profiling(0)
        got[mode] = {k: st[k] for k in ("hist_row_features", "hist_bytes", "nodes_expanded",
                                        "trees")}
    monkeypatch.delenv("BSSCL_TEST_REPLAY_GLOBAL", raising=False)
    print(f"[result] profiling counts {got['lds']}", flush=True)
    assert got["lds"] == got["table"]
    assert got["lds"]["trees"] == 6
    assert got["lds"]["hist_row_features"] > 0 and got["lds"]["nodes_expanded"] >= 6


def test_fit_device_replay_fallbacks_agree(engine, monkeypatch):
    """The round's device replay (pipelined and not), the host replay
    (forced), the path that regrows a too-small node table, the general
    planner in place of the LDS one, and rows moved at every level instead of
    every second one give identical trees and losses."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    X, y, params = _fit_case("nan_imbalanced")
    params = dict(params, n_estimators=6)
    fits = {}
    hooks = ("BSSCL_TEST_HOST_REPLAY", "BSSCL_TEST_NODE_CAP", "BSSCL_TEST_REPLAY_GLOBAL",
             "BSSCL_TEST_PLAN_GLOBAL", "BSSCL_TEST_PAIR_LEVELS")
    for mode, env in [("device", {}), ("sync", {}), ("host", {"BSSCL_TEST_HOST_REPLAY": "1"}),
                      ("global", {"BSSCL_TEST_REPLAY_GLOBAL": "1"}),
                      ("lds", {"BSSCL_TEST_REPLAY_GLOBAL": "2"}),
                      ("regrow", {"BSSCL_TEST_NODE_CAP": "9"}),
                      ("plan_global", {"BSSCL_TEST_PLAN_GLOBAL": "1"}),
                      ("every_level", {"BSSCL_TEST_PAIR_LEVELS": "0"})]:
        _announce(f"fit replay path {mode}")
        for k in hooks:
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        est = HybridHistGBMNumbaV1_0_1(verbose=False, **params)
        est._pipeline_rounds = mode != "sync"
        fits[mode] = est.fit(X, y)
    for k in hooks:
        monkeypatch.delenv(k, raising=False)
    ref = fits["device"]
    for mode in ("sync", "host", "global", "lds", "regrow", "plan_global", "every_level"):
        got = fits[mode]
        assert got.train_loss_history_ == ref.train_loss_history_, mode
        for a, b in zip(ref.trees, got.trees):
            nc = a[5]
            assert nc == b[5], mode
            for k in (0, 1, 2, 3, 4, 6):
                np.testing.assert_array_equal(a[k][:nc], b[k][:nc], err_msg=mode)
