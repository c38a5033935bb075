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
    """The sorted form of the device kernels (k_fy_keys, k_fy_links,
    k_fy_final_sorted, k_fy_final_self in fisher_yates.hip): step k with
    j(k) != k becomes the key (j(k) << 32) | k, steps with j(k) == k the
    largest key; a stable sort on the high word; run starts give head[];
    each key's successor in its run gives a_new[k], with v resolved only at
    the successors and the self steps."""
    a_old = np.asarray(a_old)
    n = len(a_old)
    if n <= 1:
        return np.array(a_old, copy=True)
    NO = np.uint64(0xFFFFFFFFFFFFFFFF)
    k = np.arange(1, n, dtype=np.uint64)
    p = np.asarray(draws, dtype=np.uint64)[n - 1 - np.arange(1, n)]
    keys = np.where(p != k, (p << np.uint64(32)) | k, NO)
    keys = keys[np.argsort(keys >> np.uint64(32), kind="stable")]
    valid = keys != NO
    hi = (keys >> np.uint64(32)).astype(np.int64)
    lo = (keys & np.uint64(0xFFFFFFFF)).astype(np.int64)
    head = np.full(n, -1, np.int64)
    start = valid.copy()
    start[1:] &= hi[1:] != hi[:-1]
    head[hi[start]] = lo[start]

    def value(x):
        """v(x): a_old at the end of each x's chain x -> head[x] -> ...,
        resolved only for the positions asked (as k_fy_final_* do)."""
        root = np.array(x, dtype=np.int64, copy=True)
        while True:
            h = head[root]
            moved = h >= 0
            if not moved.any():
                break
            root = np.where(moved, h, root)
        return a_old[root]

    out = np.full(n, -12345, dtype=a_old.dtype)
    nxt_same = np.zeros(len(keys), bool)
    nxt_same[:-1] = valid[1:] & (hi[1:] == hi[:-1])
    succ = np.full(len(keys), -1, np.int64)
    succ[:-1] = np.where(nxt_same[:-1], lo[1:], -1)
    idx = np.nonzero(valid)[0]
    has = succ[idx] >= 0
    res = a_old[hi[idx]].copy()
    res[has] = value(succ[idx][has])
    out[lo[idx]] = res
    self_k = np.nonzero(np.concatenate([[True], p == k]))[0]
    out[self_k] = value(self_k)
    return out
