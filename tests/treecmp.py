"""Tree comparison for parity tests (test helper).

Trees must be identical -- same node count, features, thresholds and child
ids -- except where the two builders chose between candidates whose gains
differ by at most ``GAIN_TIE_RTOL`` relative (the tolerance for split ties):
the engine sums fixed-point gradients, the reference sums fp64 in row order,
so exact-tie and near-tie candidates may legitimately be ordered differently.
Leaf and internal values must agree within ``VALUE_RTOL``/``VALUE_ATOL``.

``follow`` does not stop at such a tie.  It walks both trees in the order
their splits were made (split s creates nodes 2s+1 and 2s+2, est:686-687),
and at the first difference it recomputes both candidates' gains in fp64 by
direct sums over the node's rows.  A certified tie is then adopted: the
oracle's builder is rerun with the engine's choice forced at that node (a
different split of one node) or at that pop (a different node popped,
est:645-653), and the walk goes on.  Every split, node value and gain of the
whole tree is compared; anything else fails the test.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

GAIN_TIE_RTOL = 1e-7
# Node values are -G/(H+lambda) of fixed-point sums; G of a node can be near
# zero (the root of the first round), so the bar is absolute plus relative.
VALUE_RTOL = 1e-6
VALUE_ATOL = 1e-7


def node_rows(X_bin, tree, rows):
    tf, tt, tv, tl, tr, nc, _ = tree
    per = {0: np.asarray(rows)}
    order = [0]
    for node in order:
        if tf[node] >= 0:
            r = per[node]
            m = X_bin[r, tf[node]] <= tt[node]
            per[int(tl[node])] = r[m]
            per[int(tr[node])] = r[~m]
            order += [int(tl[node]), int(tr[node])]
    return per


def split_gain(X_bin, g, h, rows, feat, b, nb, lam):
    c = np.minimum(X_bin[rows, feat].astype(np.int64), nb - 1)
    left = c <= b
    Gt, Ht = g[rows].sum(), h[rows].sum()
    GL, HL = g[rows][left].sum(), h[rows][left].sum()
    GR, HR = Gt - GL, Ht - HL
    return GL * GL / (HL + lam) + GR * GR / (HR + lam) - Gt * Gt / (Ht + lam)


def split_sequence(tree):
    """[(node, feature, bin)] in the order the builder made the splits."""
    tf, tt, tv, tl, tr, nc, _ = tree
    seq = [None] * ((nc - 1) // 2)
    for v in range(nc):
        if tf[v] >= 0:
            s = (int(tl[v]) - 1) // 2
            assert int(tl[v]) == 2 * s + 1 and int(tr[v]) == 2 * s + 2, \
                f"node {v}: children {tl[v]}, {tr[v]}"
            seq[s] = (v, int(tf[v]), int(tt[v]))
    assert all(x is not None for x in seq), "split ids are not consecutive"
    return seq


def compare(ref, got):
    """Strict: identical splits in identical order, values and gains within
    the bars.  Returns "equal" or raises AssertionError."""
    rs, gs = split_sequence(ref), split_sequence(got)
    assert rs == gs, _first_diff_message(rs, gs)
    _values_equal(ref, got)
    return "equal"


def _first_diff_message(rs, gs):
    for s in range(max(len(rs), len(gs))):
        a = rs[s] if s < len(rs) else None
        b = gs[s] if s < len(gs) else None
        if a != b:
            return f"split {s}: reference {a} vs engine {b}"
    return "equal"


def _values_equal(ref, got):
    rn, gn = ref[5], got[5]
    assert rn == gn, f"node counts {rn} vs {gn}"
    np.testing.assert_array_equal(got[0][:gn], ref[0][:rn])
    np.testing.assert_allclose(got[2][:gn], ref[2][:rn], rtol=VALUE_RTOL, atol=VALUE_ATOL)
    np.testing.assert_allclose(got[6][:gn], ref[6][:rn], rtol=1e-6, atol=1e-6)


@dataclass
class Followed:
    tree: tuple                   # the oracle's tree with the engine's tie choices
    ties: list = field(default_factory=list)   # (kind, split index, node, gain_ref, gain_eng)

    @property
    def n_ties(self):
        return len(self.ties)


def follow(got, X_bin, g, h, rows, feats, max_leaves, max_depth, min_samples_leaf,
           min_child_weight, bin_counts, max_bins, reg_lambda, gamma, ref=None,
           max_ties=64):
    """Compares the engine's tree ``got`` with the oracle's builder on the
    same inputs, following certified gain ties (module docstring).  ``ref``
    is the oracle's unforced tree when the caller already has it.  Returns a
    ``Followed`` whose ``tree`` equals ``got`` within the value bars."""
    from oracle import model as om
    bc = np.asarray(bin_counts)
    args = (rows, feats, max_leaves, max_depth, min_samples_leaf, min_child_weight,
            bc, max_bins, reg_lambda, gamma)
    forced, pops = {}, {}
    out = Followed(ref if ref is not None else om.build_tree(X_bin, g, h, *args))
    gs = split_sequence(got)
    while True:
        rs = split_sequence(out.tree)
        s = next((k for k in range(max(len(rs), len(gs)))
                  if k >= len(rs) or k >= len(gs) or rs[k] != gs[k]), None)
        if s is None:
            _values_equal(out.tree, got)
            return out
        if s >= len(rs) or s >= len(gs):
            raise AssertionError(
                f"one builder stops after {min(len(rs), len(gs))} splits: "
                + _first_diff_message(rs, gs))
        if len(out.ties) >= max_ties:
            raise AssertionError(f"more than {max_ties} ties; last at split {s}")
        (va, fa, ta), (vb, fb, tb) = rs[s], gs[s]
        per = node_rows(X_bin, out.tree, rows)
        ga = split_gain(X_bin, g, h, per[va], fa, ta, int(bc[fa]), reg_lambda)
        gb = split_gain(X_bin, g, h, per[vb], fb, tb, int(bc[fb]), reg_lambda)
        if abs(ga - gb) > GAIN_TIE_RTOL * max(abs(ga), abs(gb), 1e-300):
            raise AssertionError(
                f"split {s}: reference node {va} ({fa},{ta}) gain {ga!r} vs "
                f"engine node {vb} ({fb},{tb}) gain {gb!r}")
        if va == vb:
            assert forced.get(va) != (fb, tb), f"forcing node {va} changed nothing"
            forced[va] = (fb, tb)
            out.ties.append(("split", s, va, ga, gb))
        else:
            assert pops.get(s) != vb, f"forcing pop {s} changed nothing"
            pops[s] = vb
            out.ties.append(("pop", s, vb, ga, gb))
        out.tree = om.build_tree(X_bin, g, h, *args, forced=forced, forced_pops=pops)
