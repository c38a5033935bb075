"""NumPy model of the device Fisher-Yates (kernels.hip, k_fy_*): position
lists of the steps that choose each position, sorted; chains of first
choosers; a_new from successors.  Test helper only."""
import numpy as np


def fisher_yates_sequential(a, draws):
    """The reference's swap loop: for i = n-1 .. 1, swap a[i], a[j(i)],
    with draws[n-1-i] = j(i)."""
    a = np.array(a, copy=True)
    n = len(a)
    for t in range(n - 1):
        i = n - 1 - t
        j = int(draws[t])
        a[i], a[j] = a[j], a[i]
    return a


def fisher_yates_lists(a_old, draws):
    """Closed form used on the device (see k_fy_* in kernels.hip)."""
    n = len(a_old)
    if n <= 1:
        return np.array(a_old, copy=True)
    steps = np.arange(n - 1, 0, -1)               # k for t = 0 .. n-2
    j = np.asarray(draws, dtype=np.int64)
    choose = j != steps
    k_c, p_c = steps[choose], j[choose]
    order = np.lexsort((k_c, p_c))                # by position, then step
    k_s, p_s = k_c[order], p_c[order]
    head = np.full(n, -1, np.int64)
    first = np.ones(len(p_s), bool)
    first[1:] = p_s[1:] != p_s[:-1]
    head[p_s[first]] = k_s[first]
    nxt = np.full(n, -1, np.int64)
    last = np.ones(len(p_s), bool)
    last[:-1] = p_s[:-1] != p_s[1:]
    nxt[k_s[~last]] = k_s[1:][~last[:-1]] if len(k_s) > 1 else []
    nxt[k_s[last]] = -2 - p_s[last]
    # v(k): follow k -> head[k] while it exists.
    root = np.arange(n)
    for _ in range(64):                           # chains are short; iterate to a fixed point
        h = head[root]
        moved = h >= 0
        if not moved.any():
            break
        root = np.where(moved, h, root)
    else:
        while True:
            h = head[root]
            moved = h >= 0
            if not moved.any():
                break
            root = np.where(moved, h, root)
    v = np.asarray(a_old)[root]
    out = np.empty_like(np.asarray(a_old))
    out[0] = v[0]
    i = np.arange(1, n)
    ji = j[n - 1 - i]
    g = nxt[i]
    res = np.where(g >= 0, v[np.maximum(g, 0)], np.asarray(a_old)[np.maximum(-2 - g, 0)])
    out[1:] = np.where(ji == i, v[1:], res)
    return out


def fisher_yates_sorted_keys(a_old, draws):
    """The sorted form of the device kernels (FyKeysIn and the radix sort,
    k_fy_links, k_fy_final_sorted in fisher_yates.hip): key s is
    (j(s) << 32) | s for every step s >= 1, self steps included, and 0 for
    position 0; a stable sort on the high word; a run's first key gives
    head[p] unless it is p itself (a self step or position 0), when the
    second does; every key's successor in its run gives a_new[k] (v of the
    successor, or a_old[p] without one), with v resolved only at the
    successors."""
    a_old = np.asarray(a_old)
    n = len(a_old)
    if n <= 1:
        return np.array(a_old, copy=True)
    s = np.arange(n, dtype=np.uint64)
    p = np.zeros(n, np.uint64)
    p[1:] = np.asarray(draws, dtype=np.uint64)[n - 1 - np.arange(1, n)]
    keys = (p << np.uint64(32)) | s
    keys = keys[np.argsort(keys >> np.uint64(32), kind="stable")]
    hi = (keys >> np.uint64(32)).astype(np.int64)
    lo = (keys & np.uint64(0xFFFFFFFF)).astype(np.int64)
    nxt_same = np.zeros(n, bool)
    nxt_same[:-1] = hi[1:] == hi[:-1]
    succ = np.full(n, -1, np.int64)
    succ[:-1] = np.where(nxt_same[:-1], lo[1:], -1)
    start = np.ones(n, bool)
    start[1:] = hi[1:] != hi[:-1]
    head = np.full(n, -1, np.int64)  # positions without steps keep -1
    head[hi[start]] = np.where(lo[start] != hi[start], lo[start], succ[start])

    def value(x):
        """v(x): a_old at the end of each x's chain x -> head[x] -> ...,
        resolved only for the positions asked (as k_fy_final_sorted does)."""
        root = np.array(x, dtype=np.int64, copy=True)
        while True:
            h = head[root]
            moved = h >= 0
            if not moved.any():
                break
            root = np.where(moved, h, root)
        return a_old[root]

    out = np.full(n, -12345, dtype=a_old.dtype)
    has = succ >= 0
    res = a_old[hi].copy()
    res[has] = value(succ[has])
    out[lo] = res
    return out
