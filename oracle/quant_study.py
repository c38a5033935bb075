"""Which parity bar breaks when per-row gradients are narrower (test
infrastructure: a study on the CPU, not part of the engine).

The engine accumulates histograms as exact int64 sums of per-row fixed-point
values with 62 - ceil(log2 rows) - ceil(log2 max|v|) fractional bits, so a
row keeps about 42 significant bits at 1M rows.  Narrower LDS accumulators
would cost fewer LDS operations but keep fewer bits per row:

  * one packed 64-bit add of (g, h) as two 32-bit fields, flushed every W
    rows: each field must hold W rows' sum, so a row keeps 32 - ceil(log2 W)
    bits including the sign (20 bits for W = 2560, the histogram's tile);
  * 32-bit adds per value, flushed every W rows: the same bits per row, and
    as many LDS adds as the int64 form.

For each boosting round of the oracle's own fit (oracle/model.py), this
study rebuilds the round's tree from g and h rounded to k-bit fixed point
with a per-tree power-of-two scale (max |v| * 2^s < 2^(k-1), as the engine
scales its 64-bit values) and compares it with the fp64 tree by the parity
comparison of the GPU tests (tests/treecmp.py: identical splits except
certified gain ties within 1e-7, node values within 1e-6 relative + 1e-7).
Sums of k-bit values over at most 2^(53-k) rows are exact in fp64, so for
k <= 32 the rebuilt tree is the tree an exact k-bit integer accumulation
gives.

    python oracle/quant_study.py [--rounds R] [--bits 16,20,24,28,32,36]
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import model as om  # noqa: E402
import treecmp  # noqa: E402


def quantise(v, rows, k):
    """v[rows] rounded to k-bit fixed point (sign included) with the
    largest power-of-two scale that keeps every |value| below 2^(k-1)."""
    out = np.zeros_like(v)
    vmax = float(np.max(np.abs(v[rows]))) if len(rows) else 0.0
    if vmax == 0.0:
        return out
    s = (k - 1) - int(np.ceil(np.log2(vmax)))
    while vmax * 2.0 ** s >= 2.0 ** (k - 1):
        s -= 1
    out[rows] = np.rint(v[rows] * 2.0 ** s) * 2.0 ** -s
    return out


def classify(exc):
    msg = str(exc)
    if "gain" in msg:
        return "split"
    if "stops after" in msg or "node counts" in msg:
        return "shape"
    if "tolerance" in msg or "Mismatch" in msg:
        return "value"
    return "other"


def study(name, X, y, params, rounds, bits):
    est = om.OracleGBM(**params)
    stats = {k: {"equal": 0, "ties": 0, "split": 0, "shape": 0, "value": 0, "other": 0,
                 "max_value_rel": 0.0} for k in bits}

    def on_round(m, g, h, rows, feats, tree):
        args = (rows, feats, est.max_leaves, est.max_depth, est.min_samples_leaf,
                est.min_child_weight, est.feature_bin_counts, est._max_bins,
                est.reg_lambda, est.gamma)
        for k in bits:
            gq, hq = quantise(g, rows, k), quantise(h, rows, k)
            got = om.build_tree(est.X_bin_, gq, hq, *args)
            st = stats[k]
            try:
                f = treecmp.follow(got, est.X_bin_, g, h, *args, ref=tree)
                st["equal"] += 1
                st["ties"] += f.n_ties
            except AssertionError as e:
                st[classify(e)] += 1
            if got[5] == tree[5] and np.array_equal(got[0][:got[5]], tree[0][:tree[5]]):
                a, b = got[2][:got[5]], tree[2][:tree[5]]
                rel = np.abs(a - b) / np.maximum(np.abs(b), 1e-300)
                st["max_value_rel"] = max(st["max_value_rel"], float(np.max(rel)))

    t = time.perf_counter()
    est.fit(X, y, max_rounds=rounds, round_callback=on_round)
    dt = time.perf_counter() - t
    print(f"\n{name}: {X.shape[0]} x {X.shape[1]}, {rounds} rounds ({dt:.0f} s)", flush=True)
    print("| bits per row | trees within the bars | of them with certified ties | "
          "split differs beyond a tie | tree shape differs | node value bar broken | "
          "max node value rel. error (same shape) |")
    print("|---|---|---|---|---|---|---|")
    for k in bits:
        st = stats[k]
        print(f"| {k} | {st['equal']}/{rounds} | {st['ties']} | {st['split']} | {st['shape']} | "
              f"{st['value'] + st['other']} | {st['max_value_rel']:.2e} |", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--rounds", type=int, default=10)
    ap.add_argument("--bits", default="16,20,24,28,32,36")
    ap.add_argument("--workloads", default="imbalanced,sparse_hd,dense_1m")
    a = ap.parse_args()
    bits = [int(b) for b in a.bits.split(",")]
    om.build()
    import bench
    for wl in a.workloads.split(","):
        X, y, params = bench.make_workload(wl)
        params = dict(params)
        params.pop("verbose", None)
        study(wl, X, y, params, a.rounds, bits)


if __name__ == "__main__":
    main()
