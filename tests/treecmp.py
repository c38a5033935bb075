"""Tree comparison for parity tests (test helper).

Trees must be identical -- same node count, features, thresholds and child
ids -- except where the two builders chose between splits whose gains differ
by at most ``GAIN_TIE_RTOL`` relative (the tolerance for split ties): the
engine sums fixed-point gradients, the reference sums fp64 in row order, so
exact-tie and near-tie candidates may legitimately be ordered differently.
Leaf and internal values must agree within ``VALUE_RTOL``/``VALUE_ATOL``.
"""
from __future__ import annotations

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


def compare(ref, got, X_bin=None, g=None, h=None, rows=None, bin_counts=None,
            lam=None):
    """Returns "equal", or "tie" when the first difference is a choice between
    near-equal gains; raises AssertionError otherwise."""
    rf, rt, rv, rl, rr, rn, rs = ref
    gf, gt, gv, gl, gr, gn, gs = got
    for node in range(min(rn, gn)):
        same = (rf[node] == gf[node] and (rf[node] < 0 or
                (rt[node] == gt[node] and rl[node] == gl[node] and rr[node] == gr[node])))
        if not same:
            if X_bin is None:
                raise AssertionError(f"trees differ at node {node}")
            per = node_rows(X_bin, ref, rows)
            r = per.get(node)
            if r is None or rf[node] < 0 or gf[node] < 0:
                a = rs[node] if rf[node] >= 0 else gs[node]
                raise AssertionError(f"node {node}: split vs leaf (gain {a})")
            ga = split_gain(X_bin, g, h, r, int(rf[node]), int(rt[node]), int(bin_counts[rf[node]]), lam)
            gb = split_gain(X_bin, g, h, r, int(gf[node]), int(gt[node]), int(bin_counts[gf[node]]), lam)
            if abs(ga - gb) <= GAIN_TIE_RTOL * max(abs(ga), abs(gb), 1e-300):
                return "tie"
            raise AssertionError(
                f"node {node}: reference split ({rf[node]},{rt[node]}) gain {ga!r} vs "
                f"engine ({gf[node]},{gt[node]}) gain {gb!r}")
    assert rn == gn, f"node counts {rn} vs {gn}"
    np.testing.assert_allclose(gv[:gn], rv[:rn], rtol=VALUE_RTOL, atol=VALUE_ATOL)
    np.testing.assert_allclose(gs[:gn], rs[:rn], rtol=1e-6, atol=1e-6)
    return "equal"
