"""The tie-following comparison (tests/treecmp.py) on the CPU: the oracle's
builder plays both sides, with ties planted by forcing its choices.

* A split tie: two identical feature columns give exactly equal gains; the
  "engine" tree takes the second column at the root.
* A pop tie: the root splits rows into two mirror images (g -> -g, same h and
  codes), so both children's best gains agree to rounding; the "engine" tree
  pops them in the other order.
* Not a tie: a worse split forced at the root must fail the comparison, and
  so must a changed leaf value.
"""
import numpy as np
import pytest

import treecmp
from oracle import model as om

PARAMS = dict(max_leaves=9, max_depth=5, min_samples_leaf=5, min_child_weight=0.1,
              reg_lambda=1.0, gamma=0.0)


def _build(X_bin, g, h, bc, **kw):
    rows = np.arange(len(g), dtype=np.int64)
    feats = np.arange(X_bin.shape[1], dtype=np.int32)
    p = PARAMS
    return om.build_tree(X_bin, g, h, rows, feats, p["max_leaves"], p["max_depth"],
                         p["min_samples_leaf"], p["min_child_weight"], bc, int(bc.max()),
                         p["reg_lambda"], p["gamma"], **kw)


def _follow(got, X_bin, g, h, bc):
    rows = np.arange(len(g), dtype=np.int64)
    feats = np.arange(X_bin.shape[1], dtype=np.int32)
    p = PARAMS
    return treecmp.follow(got, X_bin, g, h, rows, feats, p["max_leaves"], p["max_depth"],
                          p["min_samples_leaf"], p["min_child_weight"], bc, int(bc.max()),
                          p["reg_lambda"], p["gamma"])


def _dup_data(seed=0, n=3000):
    rng = np.random.default_rng(seed)
    c = rng.integers(0, 40, (n, 4)).astype(np.uint8)
    c[:, 1] = c[:, 0]
    g = ((c[:, 0] > 20) * 1.5 - 0.75 + (c[:, 2] > 12) * 0.6 - 0.3 * (c[:, 3] < 8)
         + 0.3 * rng.standard_normal(n))
    g -= g.mean()
    h = 0.2 + 0.3 * rng.random(n)
    return c, g, h, np.full(4, 40, np.int32)


def _mirror_data(seed=1, m=1500):
    rng = np.random.default_rng(seed)
    c = rng.integers(0, 32, (m, 4)).astype(np.uint8)
    c[:, 0] = 0
    c2 = c.copy()
    c2[:, 0] = 1
    g1 = 0.1 + 0.2 * rng.random(m) + (c[:, 2] > 15) * 0.8 - (c[:, 3] < 6) * 0.6
    h1 = 0.1 + 0.5 * rng.random(m)
    X_bin = np.vstack([c, c2])
    bc = np.array([2, 32, 32, 32], np.int32)
    return X_bin, np.concatenate([g1, -g1]), np.concatenate([h1, h1]), bc


def test_split_sequence_order():
    X_bin, g, h, bc = _dup_data()
    tree = _build(X_bin, g, h, bc)
    seq = treecmp.split_sequence(tree)
    assert len(seq) == (tree[5] - 1) // 2 > 3
    assert seq[0][0] == 0
    assert treecmp.compare(tree, tree) == "equal"


def test_follow_split_tie():
    X_bin, g, h, bc = _dup_data()
    ref = _build(X_bin, g, h, bc)
    assert ref[0][0] == 0, "the duplicated column should win at the root"
    got = _build(X_bin, g, h, bc, forced={0: (1, int(ref[1][0]))})
    with pytest.raises(AssertionError):
        treecmp.compare(ref, got)
    out = _follow(got, X_bin, g, h, bc)
    assert [t[:3] for t in out.ties] == [("split", 0, 0)]
    assert treecmp.compare(out.tree, got) == "equal"


def test_follow_pop_tie():
    X_bin, g, h, bc = _mirror_data()
    ref = _build(X_bin, g, h, bc)
    seq = treecmp.split_sequence(ref)
    assert seq[0] == (0, 0, 0), "the mirror split should come first"
    first = seq[1][0]
    assert first in (1, 2)
    got = _build(X_bin, g, h, bc, forced_pops={1: 3 - first})
    assert treecmp.split_sequence(got)[1][0] == 3 - first
    out = _follow(got, X_bin, g, h, bc)
    assert out.ties and out.ties[0][:3] == ("pop", 1, 3 - first)
    assert treecmp.compare(out.tree, got) == "equal"


def test_follow_rejects_non_tie():
    X_bin, g, h, bc = _dup_data()
    ref = _build(X_bin, g, h, bc)
    got = _build(X_bin, g, h, bc, forced={0: (2, 20)})
    assert treecmp.split_sequence(got)[0] == (0, 2, 20)
    with pytest.raises(AssertionError, match="gain"):
        _follow(got, X_bin, g, h, bc)
    bad = list(ref)
    bad[2] = ref[2].copy()
    bad[2][ref[5] - 1] += 1e-3
    with pytest.raises(AssertionError):
        _follow(tuple(bad), X_bin, g, h, bc)


def test_forced_split_must_be_candidate():
    X_bin, g, h, bc = _dup_data()
    with pytest.raises(ValueError):
        _build(X_bin, g, h, bc, forced={0: (2, 39)})  # the last bin is no split
