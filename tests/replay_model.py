"""NumPy model of the device replay of the reference's candidate loop
(src/bsscl_gbm/estimator_v1_0_1.py:641-820) on a computed node table, in the
two forms of kernels.hip (test helper):

* ``replay_slots``: the slot loop of k_replay_regs -- pop the active slot
  with the largest key (lowest slot on ties), free it, put a kept split's
  children in the first two free slots other than the popped one;
* ``replay_ordered``: the order form -- with distinct keys, best-first
  search pops nodes in the order of the key vectors
  (min key on the path below depth d, for d = 0, 1, ...) compared
  lexicographically, larger first; the loop's stop rules become a cut of
  that order.  Returns None when two candidates have equal keys (the slot
  loop decides those).

A node table is given as arrays over node ids: key G (the node's best gain,
-inf without a split), left child (-1 when the level loop did not expand
it; the right child is left + 1), kept (its split passed min_samples_leaf)
and left_small (its left child has no more rows than the right one).
"""
from __future__ import annotations

import numpy as np


def replay_slots(G, left, kept, left_small, max_leaves, gamma):
    n = len(G)
    C = max_leaves + 2
    M = 2 * max_leaves + 2
    ro_int = np.full(M, -1, np.int64)
    ro_left = np.full(M, -1, np.int64)
    ro_int[0], ro_left[0] = 0, -1
    node_count, status = 1, 0
    if G[0] == -np.inf:
        return ro_int, ro_left, node_count, status
    g = [-np.inf] * C
    act = [False] * C
    sid = [0] * C
    sint = [0] * C
    g[0], act[0] = G[0], True
    n_splits = 0
    while n_splits < max_leaves - 1:
        best = max(g)
        if not best > gamma:
            break
        ci = min(k for k in range(C) if g[k] == best)
        v, cur = sint[ci], sid[ci]
        if left[v] < 0:
            status = 2
            break
        act[ci], g[ci] = False, -np.inf
        if not kept[v]:
            ro_int[cur], ro_left[cur] = v, -1
            continue
        l = left[v]
        left_id = node_count
        node_count += 2
        n_splits += 1
        free = [k for k in range(C) if k != ci and not act[k]][:2]
        if len(free) < 2:
            status = 3
            break
        s_small, s_large = free
        for k in free:
            is_left = (k == s_small) == bool(left_small[v])
            act[k] = True
            sid[k] = left_id if is_left else left_id + 1
            sint[k] = l if is_left else l + 1
            g[k] = G[l] if is_left else G[l + 1]
        ro_int[cur], ro_left[cur] = v, left_id
    if status == 0:
        for k in range(C):
            if act[k]:
                ro_int[sid[k]], ro_left[sid[k]] = sint[k], -1
    assert n <= len(G)
    return ro_int, ro_left, node_count, status


def replay_ordered(G, left, kept, left_small, max_leaves, gamma):
    G = np.asarray(G, np.float64)
    n = len(G)
    M = 2 * max_leaves + 2
    ro_int = np.full(M, -1, np.int64)
    ro_left = np.full(M, -1, np.int64)
    ro_int[0], ro_left[0] = 0, -1
    if G[0] == -np.inf:
        return ro_int, ro_left, 1, 0
    parent = np.full(n, -1, np.int64)
    for v in range(n):
        if left[v] >= 0:
            parent[left[v]] = parent[left[v] + 1] = v
    # Candidates: every ancestor a kept split with key > gamma, own key > gamma.
    pc = np.zeros(n, bool)
    depth = np.zeros(n, np.int64)
    pc[0] = G[0] > gamma
    for v in range(1, n):  # parents have lower ids
        p = parent[v]
        if p < 0:
            continue
        depth[v] = depth[p] + 1
        pc[v] = pc[p] and kept[p] and G[v] > gamma
    cand = np.nonzero(pc)[0]
    if len(np.unique(G[cand])) != len(cand):
        return None
    code = np.zeros(n, np.int64)
    code[cand] = np.argsort(np.argsort(G[cand]))  # rank, larger key -> larger code
    INF = len(cand)
    D = int(depth.max()) + 1
    keys = {}
    for v in cand:
        comp = [INF] * D
        path = []
        u = v
        while u != 0:
            path.append(u)
            u = parent[u]
        path = path[::-1]  # depths 1 .. depth(v)
        for d in range(depth[v]):
            comp[d] = min(code[x] for x in path[d:])
        keys[v] = tuple(comp)
    order = sorted(cand, key=lambda v: keys[v], reverse=True)
    node_count, K, status = 1, 0, 0
    out = {0: 0}
    for v in order:
        if K == max_leaves - 1:
            break
        if left[v] < 0:
            status = 2
            break
        if not kept[v]:
            ro_int[out[v]], ro_left[out[v]] = v, -1
            continue
        l = left[v]
        lid = 1 + 2 * K
        out[l], out[l + 1] = lid, lid + 1
        ro_int[out[v]], ro_left[out[v]] = v, lid
        ro_int[lid], ro_left[lid] = l, -1
        ro_int[lid + 1], ro_left[lid + 1] = l + 1, -1
        K += 1
        node_count += 2
    return ro_int, ro_left, node_count, status


def random_table(rng, n_levels, p_expand=0.8, p_kept=0.9, p_ninf=0.1, ties=False):
    """A node table numbered as the level planner numbers it: each level's
    expanded nodes get consecutive child pairs after all earlier nodes."""
    G, left, kept, ls = [], [], [], []

    def key():
        if rng.random() < p_ninf:
            return -np.inf
        if ties:
            return float(rng.integers(0, 6))
        return float(rng.normal())

    G.append(key())
    left.append(-1)
    kept.append(bool(rng.random() < p_kept))
    ls.append(bool(rng.random() < 0.5))
    level = [0]
    for _ in range(n_levels):
        nxt = []
        for v in level:
            if rng.random() < p_expand:
                l = len(G)
                left[v] = l
                for _c in range(2):
                    G.append(key())
                    left.append(-1)
                    kept.append(bool(rng.random() < p_kept))
                    ls.append(bool(rng.random() < 0.5))
                nxt += [l, l + 1]
        level = nxt
        if not level:
            break
    return (np.array(G), np.array(left, np.int64), np.array(kept), np.array(ls))
