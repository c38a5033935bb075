"""Pure-NumPy model of the engine's tree schedule (test helper).

The engine builds a tree level by level -- every node of a depth at once --
and then replays the reference's best-first candidate loop
(src/bsscl_gbm/estimator_v1_0_1.py:641-820) on the computed nodes.  A node is
expanded unless at least max_leaves-1 kept splits u have e(u) > e(v), where
e is the smallest gain on the path from the root.  When every split is
known to be kept (``all_kept``: min_child_weight >= min_samples_leaf times
the largest hessian), the level's other candidates count as kept splits too.
This model implements
that schedule with plain fp64 NumPy so tests can check, on the CPU, that it
yields the same trees as the sequential builder of the oracle.
"""
from __future__ import annotations

import numpy as np


def _hist(codes, g, h, nb):
    c = np.minimum(codes.astype(np.int64), nb - 1)
    return np.bincount(c, weights=g, minlength=nb), np.bincount(c, weights=h, minlength=nb)


def _best_split(X_bin, g, h, rows, feats, bin_counts, mcw, lam):
    best = (-1e9, -1, 0)
    for j in feats:
        nb = int(bin_counts[j])
        if nb < 2:
            continue
        G, H = _hist(X_bin[rows, j], g[rows], h[rows], nb)
        Gt, Ht = G.sum(), H.sum()
        GL = np.cumsum(G)[:-1]
        HL = np.cumsum(H)[:-1]
        GR, HR = Gt - GL, Ht - HL
        ok = ~((HL < mcw) | (HR < mcw))
        gain = (GL * GL / (HL + lam) + GR * GR / (HR + lam)) - Gt * Gt / (Ht + lam)
        gain = np.where(ok, gain, -np.inf)
        b = int(np.argmax(gain))
        if gain[b] > best[0]:
            best = (float(gain[b]), int(j), b)
    return best


def build(X_bin, grad, hess, rows, feats, max_leaves, max_depth, msl, mcw,
          bin_counts, lam, gamma, stats=None, all_kept=False):
    rows = np.asarray(rows, np.int64)
    nodes = []

    def make(rws, depth, parent):
        G, H = float(grad[rws].sum()), float(hess[rws].sum())
        nd = dict(rows=rws, depth=depth, parent=parent, G=G, H=H, feat=-1,
                  bin=0, gain=-1.0, expanded=False, ok=False, kids=None, e=0.0)
        can = len(rws) >= msl and H >= mcw and (parent < 0 or depth < max_depth)
        if can:
            gain, f, b = _best_split(X_bin, grad, hess, rws, feats, bin_counts, mcw, lam)
            if f >= 0:
                nd.update(feat=f, bin=b, gain=gain)
        nodes.append(nd)
        return len(nodes) - 1

    make(rows, 0, -1)
    nodes[0]["e"] = nodes[0]["gain"]
    frontier = [0] if nodes[0]["feat"] >= 0 and nodes[0]["gain"] > gamma else []
    while frontier:
        exp = []
        for v in frontier:
            kept = sum(1 for u in nodes if u["expanded"] and u["ok"] and u["e"] > nodes[v]["e"])
            if all_kept:
                kept += sum(1 for u in frontier if u != v and nodes[u]["e"] > nodes[v]["e"])
            if kept < max_leaves - 1:
                exp.append(v)
        if not exp:
            break
        nxt = []
        for v in exp:
            nd = nodes[v]
            r = nd["rows"]
            go_left = X_bin[r, nd["feat"]] <= nd["bin"]
            L, R = r[go_left], r[~go_left]
            nd["expanded"] = True
            nd["ok"] = len(L) >= msl and len(R) >= msl
            if not nd["ok"]:
                continue
            li = make(L, nd["depth"] + 1, v)
            ri = make(R, nd["depth"] + 1, v)
            nd["kids"] = (li, ri)
            for c in (li, ri):
                nodes[c]["e"] = min(nodes[c]["gain"], nd["e"])
                if nodes[c]["feat"] >= 0 and nodes[c]["gain"] > gamma:
                    nxt.append(c)
        frontier = nxt
    if stats is not None:
        stats["expanded"] = sum(1 for u in nodes if u["expanded"])
    return _replay(nodes, max_leaves, lam, gamma)


def _replay(nodes, max_leaves, lam, gamma):
    M = 2 * max_leaves + 2
    MAX_C = max_leaves + 2
    tf = np.full(M, -1, np.int32)
    tt = np.zeros(M, np.int64)
    tv = np.zeros(M, np.float64)
    tl = np.full(M, -1, np.int32)
    tr = np.full(M, -1, np.int32)
    sg = np.zeros(M, np.float64)
    val = lambda nd: -nd["G"] / (nd["H"] + lam)
    root = nodes[0]
    node_count = 1
    if root["feat"] < 0:
        tv[0] = val(root)
        return tf, tt, tv, tl, tr, node_count, sg
    c_node = [0] * MAX_C
    c_int = [-1] * MAX_C
    c_feat = [-1] * MAX_C
    c_gain = [-1.0] * MAX_C
    c_val = [0.0] * MAX_C
    c_act = [False] * MAX_C
    c_int[0], c_feat[0], c_gain[0], c_val[0], c_act[0] = 0, root["feat"], root["gain"], val(root), True
    n_splits = 0
    while n_splits < max_leaves - 1:
        best_ci, best_gain = -1, gamma
        for ci in range(MAX_C):
            if c_act[ci] and c_feat[ci] >= 0 and c_gain[ci] > best_gain:
                best_gain, best_ci = c_gain[ci], ci
        if best_ci < 0:
            break
        ci = best_ci
        nd = nodes[c_int[ci]]
        cur = c_node[ci]
        assert nd["expanded"], "popped a node the schedule did not expand"
        if not nd["ok"]:
            tf[cur] = -1
            tv[cur] = c_val[ci]
            c_act[ci] = False
            continue
        lid, rid = node_count, node_count + 1
        node_count += 2
        tf[cur], tt[cur], tl[cur], tr[cur] = nd["feat"], nd["bin"], lid, rid
        tv[cur], sg[cur] = c_val[ci], c_gain[ci]
        n_splits += 1
        li, ri = nd["kids"]
        left_small = len(nodes[li]["rows"]) <= len(nodes[ri]["rows"])
        order = [(li, lid), (ri, rid)] if left_small else [(ri, rid), (li, lid)]
        free = [s for s in range(MAX_C) if s != ci and not c_act[s]][:2]
        c_act[ci] = False
        for slot, (ch, cid) in zip(free, order):
            cn = nodes[ch]
            c_node[slot], c_int[slot], c_feat[slot] = cid, ch, cn["feat"]
            c_gain[slot] = cn["gain"] if cn["feat"] >= 0 else -1.0
            c_val[slot], c_act[slot] = val(cn), True
    for ci in range(MAX_C):
        if c_act[ci]:
            tf[c_node[ci]] = -1
            tv[c_node[ci]] = c_val[ci]
    return tf, tt, tv, tl, tr, node_count, sg
