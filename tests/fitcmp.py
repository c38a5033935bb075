"""Whole-fit parity with tie following (test helper).

``follow_fit`` runs the oracle's fit (oracle/model.py) on the data an
estimator was fitted on.  At every round it

* rebuilds the round's tree on the engine from the oracle's own gradients,
  rows and features (lockstep: ``engine.build_tree``), and
* takes the estimator's tree of that round (end to end),

and compares both with the oracle's tree through ``treecmp.follow``.  The
oracle then keeps the end-to-end tree it has rebuilt with the estimator's
choices at certified gain ties, so both fits stay on one trajectory and every
later round, every training loss and ``predict_proba`` stay comparable.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import treecmp
from oracle import model as om

# A tree may contain this many certified ties before the comparison counts
# the case as a failure (the fitted workloads show at most a few per fit).
MAX_TIES_PER_TREE = 8


@dataclass
class FitReport:
    rounds: int = 0
    lockstep_ties: list = field(default_factory=list)     # ties per round
    end_to_end_ties: list = field(default_factory=list)

    def line(self, name):
        return (f"[result] {name}: {self.rounds} rounds, all trees compared; lockstep ties "
                f"{sum(self.lockstep_ties)} (max {max(self.lockstep_ties, default=0)}/tree), "
                f"end-to-end ties {sum(self.end_to_end_ties)} "
                f"(max {max(self.end_to_end_ties, default=0)}/tree)")


def _builder_args(ref, si, fi):
    return (si, fi, ref.max_leaves, ref.max_depth, ref.min_samples_leaf,
            ref.min_child_weight, ref.feature_bin_counts, ref._max_bins,
            ref.reg_lambda, ref.gamma)


def follow_fit(engine, est, X, y, params, lockstep=True):
    """Returns (oracle model, FitReport); raises AssertionError at the first
    difference that is not a certified tie."""
    ref = om.OracleGBM(edge_threads=16, **{k: v for k, v in params.items() if k != "verbose"})
    rep = FitReport()
    multiclass = getattr(est, "_is_multiclass", False)

    def engine_tree(k, m):
        return est.mc_trees[k][m] if multiclass else est.trees[m]

    def check(m, k, g, h, si, fi, tree):
        Xb = ref.X_bin_
        args = _builder_args(ref, si, fi)
        if lockstep:
            if m == 0 and k == 0:
                engine.load_codes(0, Xb)
            got = engine.build_tree(g, h, *args)
            fl = treecmp.follow(got, Xb, g, h, *args, ref=tree)
            rep.lockstep_ties.append(fl.n_ties)
            assert fl.n_ties <= MAX_TIES_PER_TREE, (m, k, fl.ties)
        fe = treecmp.follow(engine_tree(k, m), Xb, g, h, *args, ref=tree)
        rep.end_to_end_ties.append(fe.n_ties)
        assert fe.n_ties <= MAX_TIES_PER_TREE, (m, k, fe.ties)
        rep.rounds = m + 1
        return fe.tree

    if multiclass:
        ref.fit(X, y, tree_hook=lambda m, k, g, h, si, fi, t: check(m, k, g, h, si, fi, t))
    else:
        ref.fit(X, y, tree_hook=lambda m, g, h, si, fi, t: check(m, 0, g, h, si, fi, t))
    return ref, rep


def assert_fit_equal(ref, est, X_eval, loss_rtol=1e-9, proba_atol=1e-6):
    """Fitted attributes, every round's training loss and predict_proba."""
    np.testing.assert_array_equal(est.bin_edges, ref.bin_edges)
    np.testing.assert_array_equal(est.feature_bin_counts, ref.feature_bin_counts)
    if not getattr(est, "_is_multiclass", False):
        assert est.base_score_ == ref.base_score_
        assert len(est.trees) == len(ref.trees)
    np.testing.assert_allclose(est.train_loss_history_, ref.train_loss_history_, rtol=loss_rtol)
    np.testing.assert_allclose(est.predict_proba(X_eval), ref.predict_proba(X_eval),
                               rtol=0, atol=proba_atol)
