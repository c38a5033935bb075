"""Pins the oracle (oracle/oracle.c + oracle/model.py) to facts that do not
come from the oracle itself: closed forms, brute force on small inputs,
invariants of the reference's algorithm, and values derived by hand from
the reference's parameter rules.  CPU only."""
import numpy as np
import pytest

from conftest import make_data
from oracle import model as om
import schedule_model as sm


def closed_form_codes(X, edges, bin_counts, nan_bin_id):
    """Code of each value: 0 below e[0], nb-1 at/above e[nb], else
    searchsorted(e[1:nb], v, 'right'); NaN features shifted by +1 with NaN -> 0
    (src/bsscl_gbm/estimator_v1_0_1.py:155-226, 2144-2189)."""
    n, F = X.shape
    has_any = np.any(nan_bin_id >= 0)
    out = np.zeros((n, F), np.int64)
    for j in range(F):
        nb = int(bin_counts[j])
        e = edges[j]
        v = X[:, j].astype(np.float64)
        isn = np.isnan(v)
        if has_any:
            v = np.where(isn, 0.0, v)
        c = np.searchsorted(e[1:nb], v, side="right")
        c = np.where(v < e[0], 0, c)
        c = np.where(v >= e[nb], nb - 1, c)
        if not has_any:
            c = np.where(isn, 0, c)
        if nan_bin_id[j] >= 0:
            c = c + 1
            c = np.where(isn, 0, c)
        out[:, j] = c
    return out


@pytest.mark.parametrize("strategy", ["standard", "hybrid"])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_binning_matches_closed_form(strategy, seed):
    rng = np.random.default_rng(seed)
    n, F = 3000, 9
    X = rng.standard_normal((n, F)).astype(np.float32)
    X[:, 1] = np.round(X[:, 1] * 3)            # few uniques: unique branch
    X[:, 2] = 7.0                              # constant column
    X[rng.random(n) < 0.2, 3] = np.nan         # NaN feature
    X[:, 4] = np.nan                           # all-NaN column
    X[:5, 5] = [np.inf, -np.inf, 1e30, -1e30, 0.0]
    X[:, 6] = rng.exponential(1.0, n) * (rng.random(n) < 0.1)  # mostly zero
    for n_bins in (16, 255, 256, 300, 1000):
        e, bc, nid = om.build_bin_edges(X, n_bins)
        codes = om.bin_features(X, e, bc, nid, strategy)
        want = closed_form_codes(X, e, bc, nid)
        dt = np.uint8 if bc.max() <= 255 else np.uint16
        np.testing.assert_array_equal(codes, want.astype(dt))
        # Prediction-time inputs outside the training range and NaN in a
        # feature that had no NaN during training.
        Xp = X.copy()
        Xp[:50, 0] = np.nan
        Xp[50:60, 7] = 1e9
        np.testing.assert_array_equal(om.bin_features(Xp, e, bc, nid, strategy),
                                      closed_form_codes(Xp, e, bc, nid).astype(dt))


def test_binning_without_nan_model_maps_nan_to_zero():
    X, _ = make_data(500, 4, seed=3)
    e, bc, nid = om.build_bin_edges(X, 255)
    assert (nid < 0).all()
    Xp = X.copy()
    Xp[:10, 2] = np.nan
    codes = om.bin_features(Xp, e, bc, nid, "standard")
    assert (codes[:10, 2] == 0).all()


def test_bin_edges_known_answers():
    X = np.array([[1.0, np.nan], [2.0, 5.0], [3.0, np.nan], [2.0, 5.0]], np.float64)
    e, bc, nid = om.build_bin_edges(X, 255)
    # Column 0: sorted uniques plus e[-1] + 1e-8 (est:2110-2111, 2127).
    np.testing.assert_array_equal(e[0, :4], [1.0, 2.0, 3.0, 3.0 + 1e-8])
    assert bc[0] == 3 and nid[0] == -1
    # Column 1: NaN bin reserved, one numeric value (est:2093-2096, 2130-2133).
    assert nid[1] == 0 and bc[1] == 2
    np.testing.assert_array_equal(e[1, :2], [5.0, 5.0 + 1e-8])
    # Padding repeats the last edge (est:2137-2139).
    assert (e[1, 2:] == e[1, 1]).all()
    # float32 unique branch: e[-1] + 1e-8 rounds back to e[-1].
    X32 = np.array([[1.0], [2.0], [3.0]], np.float32)
    e32, bc32, _ = om.build_bin_edges(X32, 255)
    assert e32[0, 3] == e32[0, 2] == 3.0 and bc32[0] == 3


def test_bin_edges_percentile_branch():
    rng = np.random.default_rng(5)
    col = rng.standard_normal(20000).astype(np.float32)
    e, bc, _ = om.build_bin_edges(col[:, None], 255)
    # n_bins=255 leaves 255 numeric bins for a NaN-free column: 256 quantile
    # points, so 256 codes (est:2108-2113, 2133) and max_bins = 256.
    assert int(bc[0]) == 256
    q = np.linspace(0, 1, 256) * 100
    np.testing.assert_array_equal(e[0, :256], np.unique(np.percentile(col, q)))
    assert e[0, 0] == col.min() and e[0, 255] == col.max()
    assert np.all(np.diff(e[0, :256]) > 0)


def _node_rows(X_bin, tree, rows):
    tf, tt, tv, tl, tr, nc, _ = tree
    per = {0: rows}
    order = [0]
    for node in order:
        if tf[node] >= 0:
            r = per[node]
            m = X_bin[r, tf[node]] <= tt[node]
            per[tl[node]] = r[m]
            per[tr[node]] = r[~m]
            order += [tl[node], tr[node]]
    return per


def brute_best_split(X_bin, g, h, rows, feats, bc, mcw, lam):
    """Direct sums per candidate (no prefix scan), reference tie-break."""
    best = (-1e9, -1, 0)
    Gt, Ht = g[rows].sum(), h[rows].sum()
    for j in feats:
        nb = int(bc[j])
        c = np.minimum(X_bin[rows, j].astype(np.int64), nb - 1)
        for b in range(nb - 1):
            left = c <= b
            GL, HL = g[rows][left].sum(), h[rows][left].sum()
            GR, HR = Gt - GL, Ht - HL
            if HL < mcw or HR < mcw:
                continue
            gain = GL * GL / (HL + lam) + GR * GR / (HR + lam) - Gt * Gt / (Ht + lam)
            if gain > best[0] + 1e-9 * max(1.0, abs(best[0])):
                best = (gain, int(j), b)
    return best


@pytest.mark.parametrize("seed,n_bins", [(0, 32), (1, 32), (2, 600)])
def test_tree_invariants_and_brute_force_splits(seed, n_bins):
    """n_bins = 600 gives uint16 codes and splits past bin 255."""
    rng = np.random.default_rng(seed)
    n, F = 1500, 5
    X, y = make_data(n, F, seed=seed, nan_frac=0.05)
    e, bc, nid = om.build_bin_edges(X, n_bins)
    Xb = om.bin_features(X, e, bc, nid, "standard")
    assert (Xb.dtype == np.uint16) == (n_bins > 255)
    p = 1 / (1 + np.exp(-rng.standard_normal(n)))
    g, h = p - y, p * (1 - p)
    rows = rng.permutation(n)[:1200].astype(np.int64)
    feats = np.array([0, 2, 3, 4], np.int32)
    lam, mcw, msl, ml, md = 1.0, 1.0, 5, 15, 4
    tree, counts, pops = om.build_tree(Xb, g, h, rows, feats, ml, md, msl, mcw, bc,
                                       int(bc.max()), lam, 0.0, trace=True)
    tf, tt, tv, tl, tr, nc, sg = tree
    if n_bins > 256:
        assert np.any(tt[:nc][tf[:nc] >= 0] > 255)
    per = _node_rows(Xb, tree, rows)
    assert set(per) == set(range(nc))
    n_leaves = int(np.sum(tf[:nc] < 0))
    assert n_leaves <= ml
    depth = {0: 0}
    for node in range(nc):
        r = per[node]
        if tf[node] >= 0:
            depth[tl[node]] = depth[tr[node]] = depth[node] + 1
            assert depth[node] < md
            bg, bf, bb = brute_best_split(Xb, g, h, r, feats, bc, mcw, lam)
            assert (bf, bb) == (tf[node], tt[node])
            assert abs(bg - sg[node]) <= 1e-9 * max(1.0, abs(bg))
            assert len(per[tl[node]]) >= msl and len(per[tr[node]]) >= msl
        # Every node keeps its own value -G/(H+lambda) (est:693, 769).
        np.testing.assert_allclose(tv[node], -g[r].sum() / (h[r].sum() + lam), rtol=1e-12, atol=1e-15)
    # The partition trace records the closed-form child sizes in split order.
    split_nodes = [k for k in range(nc) if tf[k] >= 0]
    got = sorted(map(tuple, counts.tolist()))
    want = sorted((len(per[tl[k]]), len(per[tr[k]])) for k in split_nodes)
    assert got == want


@pytest.mark.parametrize("trial", range(12))
def test_tree_matches_level_schedule(trial):
    """The oracle's sequential best-first builder and the engine's
    level-synchronous schedule (tests/schedule_model.py) give the same tree."""
    rng = np.random.default_rng(100 + trial)
    n = int(rng.integers(300, 5000))
    F = int(rng.integers(2, 10))
    X, y = make_data(n, F, seed=trial, nan_frac=0.1 if trial % 3 == 0 else 0.0)
    nb = int(rng.choice([16, 64, 255]))
    e, bc, nid = om.build_bin_edges(X, nb)
    Xb = om.bin_features(X, e, bc, nid, "standard")
    p = 1 / (1 + np.exp(-0.3 * rng.standard_normal(n)))
    w = np.where(y == 1, 1.7, 0.8)
    g, h = w * (p - y), w * p * (1 - p)
    rows = rng.permutation(n)[: int(n * 0.8)].astype(np.int64)
    fs = np.sort(rng.permutation(F)[: max(1, int(F * 0.8))]).astype(np.int32)
    ml = int(rng.choice([3, 15, 31, 63]))
    md = int(rng.choice([2, 4, 6, 8]))
    msl = int(rng.choice([1, 5, 20]))
    mcw = float(rng.choice([0.0, 1.0, 3.0]))
    lam = float(rng.choice([0.5, 1.0, 5.0]))
    ref = om.build_tree(Xb, g, h, rows, fs, ml, md, msl, mcw, bc, int(bc.max()), lam, 0.0)
    got = sm.build(Xb, g, h, rows, fs, ml, md, msl, mcw, bc, lam, 0.0)
    assert ref[5] == got[5]
    k = ref[5]
    for i in (0, 1, 3, 4):
        np.testing.assert_array_equal(ref[i][:k], got[i][:k])
    np.testing.assert_allclose(ref[2][:k], got[2][:k], rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("trial", range(24))
def test_tree_matches_level_schedule_counting_level_splits(trial):
    """With min_child_weight >= min_samples_leaf * max hessian every split
    is kept (est:614-615, 678-683); the schedule that then also counts the
    level's other candidates as kept splits gives the sequential builder's
    tree, and never expands more nodes than the schedule without them."""
    rng = np.random.default_rng(500 + trial)
    n = int(rng.integers(2000, 12000))
    F = int(rng.integers(3, 12))
    X, y = make_data(n, F, seed=50 + trial, nan_frac=0.1 if trial % 2 else 0.0)
    e, bc, nid = om.build_bin_edges(X, 255)
    Xb = om.bin_features(X, e, bc, nid, "standard")
    p = 1 / (1 + np.exp(-0.5 * rng.standard_normal(n)))
    w = np.where(y == 1, float(rng.choice([1.0, 1.4])), 1.0)
    g, h = w * (p - y), w * p * (1 - p)
    rows = rng.permutation(n)[: int(n * 0.75)].astype(np.int64)
    fs = np.sort(rng.permutation(F)[: max(1, int(F * 0.8))]).astype(np.int32)
    ml = int(rng.choice([7, 15, 31, 63]))
    md = int(rng.choice([5, 6, 8, 10]))
    msl = int(rng.choice([1, 5, 10]))
    mcw = msl * float(h.max()) * float(rng.choice([1.0 + 1e-9, 1.5, 3.0]))
    lam = float(rng.choice([1.0, 5.0]))
    ref = om.build_tree(Xb, g, h, rows, fs, ml, md, msl, mcw, bc, int(bc.max()), lam, 0.0)
    st0, st1 = {}, {}
    plain = sm.build(Xb, g, h, rows, fs, ml, md, msl, mcw, bc, lam, 0.0, stats=st0)
    got = sm.build(Xb, g, h, rows, fs, ml, md, msl, mcw, bc, lam, 0.0, stats=st1, all_kept=True)
    assert st1["expanded"] <= st0["expanded"]
    for tree in (plain, got):
        assert ref[5] == tree[5]
        k = ref[5]
        for i in (0, 1, 3, 4):
            np.testing.assert_array_equal(ref[i][:k], tree[i][:k])
        np.testing.assert_allclose(ref[2][:k], tree[2][:k], rtol=1e-9, atol=1e-12)


def test_predict_brute_force():
    X, y = make_data(2000, 6, seed=4)
    m = om.OracleGBM(n_estimators=5, max_depth=4, learning_rate=0.1, n_bins=64,
                     class_weight=None, random_state=0).fit(X, y)
    Xb = m.X_bin_
    F = np.zeros(len(X))
    for tree in m.trees:
        tf, tt, tv, tl, tr, nc, _ = tree
        for i in range(len(X)):
            node = 0
            while tf[node] >= 0:
                node = tl[node] if Xb[i, tf[node]] <= tt[node] else tr[node]
            F[i] += 0.1 * tv[node]
    np.testing.assert_allclose(om.predict_all_trees(Xb, m._packed, 5, 0.1), F, rtol=0, atol=1e-12)
    # Training F is base + the same sums.
    np.testing.assert_allclose(m.F_train_, F + m.base_score_, rtol=0, atol=1e-12)


def test_class_weights_and_base_score_closed_form():
    y = np.array([0] * 90 + [1] * 10)
    m = om.OracleGBM(class_weight="balanced_sqrt")
    w = m._class_weights(y)
    np.testing.assert_allclose(w[0], (100 / (2 * 90)) ** 0.35)
    np.testing.assert_allclose(w[-1], (100 / (2 * 10)) ** 0.35)
    m2 = om.OracleGBM(class_weight="balanced")
    np.testing.assert_allclose(m2._class_weights(y)[-1], 100 / 20)
    assert (om.OracleGBM(class_weight=None)._class_weights(y) == 1).all()
    p0 = (10 * w[-1]) / (90 * w[0] + 10 * w[-1])
    assert abs(np.average(y, weights=w) - p0) < 1e-15


@pytest.mark.parametrize("n,p,want", [
    # (n_sub, F_sel, min_child_weight, max_leaves, lambda, lr, strategy)
    (10_000, 20, (8000, 16, 2.0, 31, 1.0, 0.1, "standard")),
    (1_000_000, 28, (750_000, 22, 3.0, 63, 1.0, 0.08, "hybrid")),
    (284_807, 30, (213_605, 24, 3.0, 63, 1.0, 0.08, "hybrid")),
    (100_000, 100, (75_000, 70, 3.0, 63, 1.0, 0.08, "hybrid")),
    (10_000_000, 50, (5_000_000, 35, 3.0, 63, 5.0, 0.08, "hybrid")),
])
def test_adaptive_parameters_for_benchmark_shapes(n, p, want):
    """Resolved parameters of the five benchmark shapes (est:1925-2029)."""
    m = om.OracleGBM(n_bins=255, learning_rate=0.1 if n == 10_000 else "auto",
                     class_weight=None if n == 10_000 else "balanced_sqrt")
    m._adaptive(np.zeros((n, p), np.float32) if n <= 20_000 else _Shape(n, p))
    got = (max(1, int(n * m.subsample)), max(1, int(p * m.colsample_bytree)),
           m.min_child_weight, m.max_leaves, m.reg_lambda, m.learning_rate,
           m.binning_strategy)
    assert got == want


class _Shape:
    """Stand-in with only .shape; the rules read X only for n <= 20000."""

    def __init__(self, n, p):
        self.shape = (n, p)


# --------------------------------------------------------------------------
# scale_pos_weight: weighted-quantile edges (est:2114-2124), class weights
# (est:2570-2576).
# --------------------------------------------------------------------------

@pytest.mark.parametrize("n", [7, 100, 5001])
def test_weighted_quantiles_equal_weights_are_hazen(n):
    """With equal weights every value sits at position (k + 1/2) / n, which
    is the Hazen plotting position (Hyndman & Fan type 5): NumPy's
    percentile(method='hazen') computes the same quantiles independently.
    Unequal positions (a dropped -w/2, another divisor) fail this; the
    default linear percentile differs from it."""
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n)
    q = np.linspace(0, 1, 33)
    got = om.weighted_quantiles(v, np.full(n, 2.5), q)
    np.testing.assert_allclose(got, np.percentile(v, q * 100, method="hazen"), rtol=0, atol=1e-14)
    assert not np.allclose(got, np.percentile(v, q * 100))


def test_weighted_quantiles_two_values_closed_form():
    """Values a < b with weights wa, wb sit at wa/2/W and (wa + wb/2)/W; q
    between them interpolates linearly, q outside takes the end value."""
    a, b, wa, wb = -1.0, 3.0, 1.0, 5.0
    W = wa + wb
    pa, pb = 0.5 * wa / W, (wa + 0.5 * wb) / W
    q = np.array([0.0, pa, 0.3, 0.5, pb, 1.0])
    want = np.where(q <= pa, a, np.where(q >= pb, b, a + (b - a) * (q - pa) / (pb - pa)))
    got = om.weighted_quantiles(np.array([b, a]), np.array([wb, wa]), q)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-15)


def test_scale_pos_weight_class_weights():
    y = np.array([0] * 90 + [1] * 10)
    m = om.OracleGBM(scale_pos_weight=4.0, class_weight="balanced_sqrt", objective="binary")
    w = m._class_weights(y)
    assert (w[:90] == 1.0).all() and (w[90:] == 4.0).all()
    # With the default objective ('auto') the reference ignores scale_pos_weight
    # (est:2572): the class weights stay balanced_sqrt.
    w_auto = om.OracleGBM(scale_pos_weight=4.0, class_weight="balanced_sqrt")._class_weights(y)
    np.testing.assert_allclose(w_auto[-1], (100 / (2 * 10)) ** 0.35)


def test_estimator_weighted_edges_match_oracle():
    """The estimator's host branch for scale_pos_weight (est:2114-2124) gives
    the oracle's edges and bin counts, with NaN columns and few-valued
    columns mixed in."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    X, y = make_data(6000, 9, seed=21, nan_frac=0.1, nan_cols=[1, 4], dtype=np.float64)
    X[:, 7] = np.round(X[:, 7])  # few distinct values: the sorted-uniques branch
    sw = np.ones(len(y))
    sw[y == 1] = 3.5
    est = HybridHistGBMNumbaV1_0_1(n_bins=64, verbose=False)
    e_est, c_est = est._build_bin_edges_host(X, sample_weight=sw)
    e_ref, c_ref, nan_ref = om.build_bin_edges(X, 64, sample_weight=sw)
    np.testing.assert_array_equal(c_est, c_ref)
    np.testing.assert_array_equal(e_est, e_ref)
    np.testing.assert_array_equal(est._nan_bin_id, nan_ref)
    e_unw, _, _ = om.build_bin_edges(X, 64)
    assert not np.array_equal(e_unw, e_ref)  # the weights move the edges


def test_counting_level_splits_needs_kept_splits():
    """The condition matters: with min_child_weight = 0 and a large
    min_samples_leaf, splits are refused (est:678-683), and a schedule that
    counted the level's other candidates anyway misses a node the sequential
    builder pops within a few hundred random trees."""
    for trial in range(400):
        rng = np.random.default_rng(900 + trial)
        n = int(rng.integers(300, 3000))
        F = int(rng.integers(2, 8))
        X, y = make_data(n, F, seed=trial)
        e, bc, nid = om.build_bin_edges(X, 255)
        Xb = om.bin_features(X, e, bc, nid, "standard")
        p = 1 / (1 + np.exp(-0.5 * rng.standard_normal(n)))
        g, h = p - y, p * (1 - p)
        rows = rng.permutation(n)[: int(n * 0.75)].astype(np.int64)
        fs = np.arange(F, dtype=np.int32)
        ml = int(rng.choice([3, 5, 7, 15]))
        msl = int(rng.choice([100, 200, 400]))
        ref = om.build_tree(Xb, g, h, rows, fs, ml, 8, msl, 0.0, bc, int(bc.max()), 1.0, 0.0)
        try:
            got = sm.build(Xb, g, h, rows, fs, ml, 8, msl, 0.0, bc, 1.0, 0.0, all_kept=True)
        except AssertionError:
            return  # popped a node the schedule did not expand
        if got[5] != ref[5] or not np.array_equal(got[0][:ref[5]], ref[0][:ref[5]]):
            return
    raise AssertionError("no refused split changed the schedule")
