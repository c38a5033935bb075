"""Fit throughput of the binary histogram-GBM path on one MI355X.

A step is one boosting round of HybridHistGBMNumbaV1_0_1.fit: gradients,
the round's bagging sample, one leaf-wise tree, the F update over all rows
and the training loss.  W rounds run untimed, then K rounds are timed; every
round ends with a stream synchronisation, so wall-clock time over the K
rounds is the device time including host work.

Prints one JSON line with the fit rate (trees/s), the histogram kernel's
roofline (algorithmic bytes per launch over its average execution time,
from the first block's start to the last block's end as the kernel stamps
them, against 8 TB/s HBM), a complete fit with the workload's own
n_estimators (training-only and end-to-end trees/s; the median of three
fits when one takes under half a second), prediction through
that ensemble with its own roofline, and the oracle's CPU rates on a
bounded sample (fit trees/s, histogram rows x features/s, predict rows/s).
The same block is repeated for the 10M x 50 depth-8 workload: its
steady-state rounds, its 500-tree fit, predict_proba of a fresh 10M-row
batch through those 500 trees, and the oracle's first rounds at 10M.
The smaller benchmark shapes (10,000 x 20, 284,807 x 30 imbalanced,
100,000 x 100 sparse) follow as complete fits and predictions under
`workloads`, each with the oracle's rates.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "bsscl-gbm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
METRIC = "fit trees/sec at 1M×28 d6 255 bins; histogram-build HBM GB/s vs peak"


def _progress(msg):
    """Progress on stderr; stdout carries only the JSON line."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def make_workload(name, predict=False):
    """Synthetic inputs of the benchmark shapes (float32 X, int64 y) and the
    estimator parameters each is quoted with."""
    if name == "cpu_plumbing":  # 10,000 x 20, 10 trees, depth 6
        rng = np.random.default_rng(0 if not predict else 100)
        X = rng.standard_normal((10_000, 20), dtype=np.float32)
        w = rng.standard_normal(20)
        y = (rng.random(10_000) < _sigmoid(X @ w)).astype(np.int64)
        params = dict(n_estimators=10, max_depth=6, learning_rate=0.1, class_weight=None)
    elif name == "dense_1m":  # 1,000,000 x 28, 5% NaN, 100 trees, depth 6
        rng = np.random.default_rng(1 if not predict else 101)
        n = 1_000_000
        X = rng.standard_normal((n, 28), dtype=np.float32)
        logit = sum(X[:, 2 * k].astype(np.float64) * X[:, 2 * k + 1] for k in range(5))
        logit = logit + 0.5 * rng.standard_normal(n)
        y = (rng.random(n) < _sigmoid(logit)).astype(np.int64)
        X[rng.random(X.shape) < 0.05] = np.nan
        params = dict(n_estimators=100, max_depth=6)
    elif name == "imbalanced":  # 284,807 x 30, 0.17% positives
        rng = np.random.default_rng(2 if not predict else 102)
        n = 284_807
        sig = np.linspace(2.0, 0.3, 28)
        V = rng.standard_normal((n, 28)) * sig
        t = rng.uniform(0, 172_792, n)
        amt = rng.lognormal(3, 1.5, n)
        y = np.zeros(n, np.int64)
        y[rng.choice(n, 484, replace=False)] = 1
        V[y == 1, :10] += 1.5 * sig[:10]
        X = np.column_stack([t, V, amt]).astype(np.float32)
        params = dict(n_estimators=200, max_depth=6, class_weight="balanced_sqrt")
    elif name == "sparse_hd":  # 100,000 x 100, 90% zeros
        rng = np.random.default_rng(3 if not predict else 103)
        n = 100_000
        X = np.where(rng.random((n, 100)) < 0.9, 0.0, rng.exponential(1.0, (n, 100))).astype(np.float32)
        w = rng.standard_normal(8)
        s = X[:, :8].astype(np.float64) @ w + rng.logistic(size=n)
        y = (s > np.quantile(s, 0.99)).astype(np.int64)
        flip = rng.random(n) < 0.05
        y[flip] = 1 - y[flip]
        params = dict(n_estimators=300, max_depth=6, class_weight="balanced_sqrt")
    elif name == "stress_10m":  # 10,000,000 x 50, 10 columns 70% NaN, depth 8
        rng = np.random.default_rng(4 if not predict else 5)
        n = 10_000_000
        X = rng.standard_normal((n, 50), dtype=np.float32)
        X64 = X[:, :10].astype(np.float64)
        logit = (np.sin(2 * X64[:, 0]) + X64[:, 1] * X64[:, 2] + (X64[:, 3] ** 2 - 1)
                 + np.tanh(X64[:, 4]) + (np.abs(X64[:, 5]) - 0.798) + X64[:, 6] * X64[:, 7]
                 + 0.5 * X64[:, 8] - 0.5 * X64[:, 9])
        del X64
        y = (rng.random(n) < _sigmoid(logit)).astype(np.int64)
        block = X[:, 40:50]
        block[rng.random(block.shape) < 0.7] = np.nan
        X[:, 40:50] = block
        params = dict(n_estimators=500, max_depth=8)
    else:
        raise SystemExit(f"unknown workload {name!r}")
    params.update(n_bins=255, random_state=0, verbose=False)
    return X, y, params


BREAKDOWN_ROUNDS = 5


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` and the file they come
    from: the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary (copy-kernel
    calibrated), or (None, None) when no such summary exists."""
    import glob
    import re
    pat = re.compile(r"^traffic_bytes_per_launch\[%s, %s\]: (\d+)\s*$"
                     % (re.escape(kernel), re.escape(workload)))
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        with open(path) as fh:
            for line in fh:
                m = pat.match(line)
                if m:
                    return int(m.group(1)), os.path.relpath(path, ROOT)
    return None, None


def run_gpu(name, steps, warmup, rounds_only=False):
    """Fits warmup + 2 * steps + BREAKDOWN_ROUNDS rounds.  The timed rounds
    run as the library runs by default: unprofiled, each round's rows-stream
    kernels replayed from a captured HIP graph.  The next `steps` rounds of the same
    fit run at profiling level 1, where the histogram kernel stamps each
    block's start and end on the device's constant-rate clock (no event
    packets between the tree's kernels; the kernels are launched one by
    one), for the kernel's timing; the last rounds time every kernel group
    with HIP events (level 2) for the per-kernel breakdown.  Host times
    (enqueue, waits) are kept at every level and taken over the timed
    rounds."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    X, y, params = make_workload(name)
    n, F = X.shape
    _progress(f"{name}: {n} x {F} generated; fitting")
    marks = {}
    prof0 = warmup + steps

    def hook(m, eng):
        if m == warmup:
            marks["s0"] = est._live_sampler.stats()
            marks["host0"] = eng.stats()
            marks["t0"] = time.perf_counter()
        if m == prof0:
            marks["t1"] = time.perf_counter()
            marks["host1"] = eng.stats()
            marks["s1"] = est._live_sampler.stats()
            eng.set_profiling(1)
        if m == prof0 + steps:
            marks["stats"] = eng.stats()
            eng.set_profiling(2)
        if m == prof0 + steps + BREAKDOWN_ROUNDS:
            marks["breakdown"] = eng.stats()
            eng.set_profiling(0)

    full_params = dict(params)
    params = dict(params, n_estimators=warmup + 2 * steps + BREAKDOWN_ROUNDS)
    est = HybridHistGBMNumbaV1_0_1(**params)
    est._round_hook = hook
    t_fit = time.perf_counter()
    est.fit(X, y)
    t_fit = time.perf_counter() - t_fit
    del est._round_hook
    _progress(f"fit done in {t_fit:.1f} s (binning {est.times['binning']:.0f} ms)")
    elapsed = marks["t1"] - marks["t0"]
    st = marks["stats"]
    host = {k: marks["host1"][k] - marks["host0"][k] for k in marks["host1"]}
    predict, fit_full, full, Xp_sample = None, None, None, None
    if not rounds_only:
        # A complete fit with the workload's own n_estimators: bin edges,
        # binning and every boosting round, from host float32 X.
        t_full, full, n_fits = timed_fit(full_params, X, y)
        fit_full = dict(n_estimators=int(full.n_trees_fitted_), seconds=round(t_full, 4),
                        trees_per_s=round(full.n_trees_fitted_ / t_full, 2),
                        binning_ms=round(full.times["binning"], 1),
                        training_ms=round(full.times["training"], 1), fits=n_fits)
        fit_full["training_trees_per_s"] = round(
            full.n_trees_fitted_ / (full.times["training"] / 1e3), 2)
        _progress(f"full fit: {fit_full}")
        predict, Xp_sample = run_predict(full, name)
    s0, s1 = marks["s0"], marks["s1"]
    sampler = {k: (s1[k] - s0[k]) / max(s1["rounds"] - s0["rounds"], 1)
               for k in ("draw_ms", "gen_ms")}
    return dict(est=est, n=n, F=F, elapsed=elapsed, stats=st, t_fit=t_fit,
                breakdown=marks["breakdown"], sampler=sampler, predict=predict, host=host,
                fit_full=fit_full, params=params, model=full, Xp_sample=Xp_sample,
                data=(X, y, full_params))


CPU_PREDICT_ROWS = 200_000


def run_predict(model, name, repeats=3):
    """predict_proba of a fresh batch of the workload through the model's
    whole ensemble: rows/s end to end (host float32 in, probabilities out,
    the rows streamed through the device in chunks) and per k_predict
    launch over the whole batch resident on the device (kernel execution
    time), with the kernel's
    roofline over the algorithmic bytes n * (F + 16) of device-resident
    codes (one code byte per feature, 8 B of output and 8 B of F per row).
    Returns the line's entry and the batch's first CPU_PREDICT_ROWS rows
    (the CPU baseline's predict sample)."""
    from bsscl_gbm import estimator as est_mod
    Xp, _, _ = make_workload(name, predict=True)
    n, F = Xp.shape
    eng = est_mod._engine(0)
    # End to end: predict_proba from host rows, which streams them through
    # the device in row chunks (one walk launch per chunk).
    model.predict_proba(Xp)  # warm-up
    eng.set_profiling(1)
    t = time.perf_counter()
    for _ in range(repeats):
        model.predict_proba(Xp)
    t_total = (time.perf_counter() - t) / repeats
    st = eng.stats()
    eng.set_profiling(0)
    chunk_launches = max(st["predict_launches"] / repeats, 1.0)
    chunked_walk_s = st["predict_ms"] / 1e3 / repeats
    # The kernel: one walk launch over the whole batch resident on the
    # device (bsscl_bin_features, then bsscl_predict_proba).
    packed = {"features": model._packed_features, "thresholds": model._packed_thresholds,
              "values": model._packed_values, "left": model._packed_left,
              "right": model._packed_right, "offsets": model._tree_offsets}
    with eng.lock:
        eng.bin_features(1, Xp, model.bin_edges, model.feature_bin_counts, model._nan_bin_id)
        eng.predict_proba(1, n, packed, len(model.trees), model.learning_rate,
                          getattr(model, 'base_score_', 0.0))  # warm-up
        eng.set_profiling(1)
        for _ in range(repeats):
            eng.predict_proba(1, n, packed, len(model.trees), model.learning_rate,
                              getattr(model, 'base_score_', 0.0))
        st = eng.stats()
        eng.set_profiling(0)
    kernel_s = st["predict_ms"] / 1e3 / max(st["predict_launches"], 1.0)
    bytes_ = n * (F + 16)
    achieved = bytes_ / kernel_s / 1e9
    _progress(f"predict: {n} rows x {len(model.trees)} trees, kernel {1e3 * kernel_s:.2f} ms, "
              f"end to end {1e3 * t_total:.1f} ms (walk {1e3 * chunked_walk_s:.2f} ms in "
              f"{chunk_launches:.0f} launches)")
    sample = np.ascontiguousarray(Xp[:CPU_PREDICT_ROWS])
    del Xp
    return {
        "rows": n, "trees": len(model.trees),
        "rows_per_s": round(n / kernel_s),
        "rows_per_s_end_to_end": round(n / t_total),
        "end_to_end_walk": {"launches": round(chunk_launches),
                            "ms": round(1e3 * chunked_walk_s, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": "k_predict",
                     "avg_launch_us": round(1e6 * kernel_s, 1), "bytes_per_launch": bytes_},
    }, sample


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def hist_roofline(st, workload):
    hist_s = st["hist_ms"] / 1e3
    achieved = st["hist_bytes"] / hist_s / 1e9 if hist_s > 0 else 0.0
    launches = max(st["hist_launches"], 1.0)
    traffic, source = measured_traffic("k_hist", workload)
    return {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "traffic_source": source,
        "kernel": "k_hist",
        "timing": "kernel execution: first block's start to last block's end, stamped by "
                  "the kernel on the device's constant-rate clock, over as many rounds as "
                  "the timed region, right after it in the same fit (profiling level 1: no "
                  "event packets; the timed rounds themselves run unprofiled)",
        "launches": int(st["hist_launches"]),
        "avg_launch_us": round(1e3 * st["hist_ms"] / launches, 2),
        "bytes_per_launch": round(st["hist_bytes"] / launches),
    }


def cpu_cores():
    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit():
        cores = min(cores, int(omp))
    return cores


def run_cpu_baseline(name, rounds, data=None, model=None, Xp_sample=None):
    """The oracle (C/OpenMP restatement of the reference path, serial where
    the reference is serial) on this host: `rounds` rounds of the workload's
    fit after an untimed first round (training trees/s, and the histogram
    phase's rows x features/s over the same rounds), the time from fit() to
    the first round (bin edges and codes), and the traversal of the GPU
    model's whole ensemble over the first rows of the fresh predict batch
    (predict rows/s; the trees equal the oracle's up to certified ties)."""
    from oracle import model as om
    X, y, params = data if data is not None else make_workload(name)
    cores = cpu_cores()
    _progress(f"cpu baseline: oracle on {name}, {rounds} timed rounds, {cores} threads")
    p = dict(params)
    p.pop("verbose", None)
    m = om.OracleGBM(edge_threads=cores, **p)

    def first_round_done(r, *_):
        if r == 0:
            om.hist_stats(reset=True)

    t0 = time.perf_counter()
    m.fit(X, y, max_rounds=rounds + 1, round_callback=first_round_done)
    binning_s = m.round_times_[0] - t0
    t = np.diff(m.round_times_)[1:]  # first round excluded (page-in)
    hist_s, hist_rf = om.hist_stats()
    out = dict(value=float(len(t) / t.sum()), unit="trees/s", cores=cores,
               cpu_model=cpu_model(), kind="port",
               sample=f"rounds 2-{rounds + 1} of the same {name} fit "
                      f"({X.shape[0]}x{X.shape[1]}), oracle/oracle.c via OracleGBM",
               binning_ms=round(1e3 * binning_s, 1),
               hist_rows_x_features_per_s=round(hist_rf / hist_s) if hist_s > 0 else None)
    if model is not None and Xp_sample is not None:
        k = Xp_sample.shape[0]
        t = time.perf_counter()
        codes = om.bin_features(Xp_sample, model.bin_edges, model.feature_bin_counts,
                                model._nan_bin_id, model.binning_strategy)
        t_bin = time.perf_counter() - t
        packed = {"features": model._packed_features, "thresholds": model._packed_thresholds,
                  "values": model._packed_values, "left": model._packed_left,
                  "right": model._packed_right, "offsets": model._tree_offsets}
        t = time.perf_counter()
        om.predict_all_trees(codes, packed, len(model.trees), model.learning_rate)
        t_walk = time.perf_counter() - t
        out["predict_rows_per_s"] = round(k / t_walk)
        out["predict_rows_per_s_end_to_end"] = round(k / (t_walk + t_bin))
        out["predict_sample"] = (f"first {k} rows of the fresh batch through the GPU fit's "
                                 f"{len(model.trees)} trees, oracle_predict_all_trees "
                                 f"(end to end adds oracle_bin_features)")
    return out


def timed_fit(params, X, y):
    """A complete fit's wall time.  Fits under half a second are repeated
    three times and the median fit is returned (with its own binning and
    training times).  Returns (seconds, fitted estimator, fits run)."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    fits = []
    while True:
        est = HybridHistGBMNumbaV1_0_1(**params)
        t = time.perf_counter()
        est.fit(X, y)
        fits.append((time.perf_counter() - t, est))
        if len(fits) >= 3 or fits[0][0] >= 0.5:
            break
    t, est = sorted(fits, key=lambda f: f[0])[len(fits) // 2]
    return t, est, len(fits)


def run_fit_workload(name, cpu_rounds, cpu):
    """A smaller benchmark shape's complete fit (the workload's own
    n_estimators, from host float32, after one untimed fit of the same data)
    and predict_proba of its fresh batch, with the oracle's rates on this
    host when `cpu`."""
    from bsscl_gbm import HybridHistGBMNumbaV1_0_1
    X, y, params = make_workload(name)
    _progress(f"{name}: {X.shape[0]} x {X.shape[1]}, complete fit")
    HybridHistGBMNumbaV1_0_1(**params).fit(X, y)
    t, est, n_fits = timed_fit(params, X, y)
    n_trees = int(est.n_trees_fitted_)
    out = {
        "config": {"rows": X.shape[0], "features": X.shape[1],
                   "n_estimators": n_trees, "max_depth": params["max_depth"],
                   "class_weight": params.get("class_weight", est.class_weight),
                   "subsample": est.subsample, "colsample_bytree": est.colsample_bytree},
        "fit_end_to_end": {
            "seconds": round(t, 4), "trees_per_s": round(n_trees / t, 2),
            "binning_ms": round(est.times["binning"], 1),
            "training_ms": round(est.times["training"], 1),
            "training_trees_per_s": round(n_trees / (est.times["training"] / 1e3), 2),
            "fits": n_fits},
    }
    out["predict"], sample = run_predict(est, name)
    if cpu:
        out["cpu_baseline"] = run_cpu_baseline(name, cpu_rounds, data=(X, y, params),
                                               model=est, Xp_sample=sample)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="dense_1m")
    ap.add_argument("--cpu-rounds", type=int, default=4)
    ap.add_argument("--also-cpu-rounds", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--rounds-only", action="store_true",
                    help="skip the prediction and the end-to-end fit (profiler runs)")
    ap.add_argument("--also", default="stress_10m",
                    help="workload of the extra rounds-only block ('' for none)")
    ap.add_argument("--also-steps", type=int, default=60)
    ap.add_argument("--fits", default="cpu_plumbing,imbalanced,sparse_hd",
                    help="smaller workloads timed as complete fits and predictions "
                         "('' for none)")
    ap.add_argument("--fits-cpu-rounds", type=int, default=3)
    a = ap.parse_args()
    if a.gpus != 1:
        print(json.dumps({"error": "this engine runs on one GPU; --gpus must be 1 "
                                   "(row sharding across GPUs is not built)"}))
        sys.exit(2)
    r = run_gpu(a.workload, a.steps, a.warmup, a.rounds_only)
    st = r["stats"]
    bd = r["breakdown"]
    trees_per_s = a.steps / r["elapsed"]
    hist_s = st["hist_ms"] / 1e3
    line = {
        "metric": METRIC,
        "value": round(trees_per_s, 3),
        "unit": "trees/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(1e3 * r["elapsed"] / a.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": "synthetic",
        "config": {
            "workload": a.workload,
            "rows": r["n"], "features": r["F"],
            "max_depth": r["params"]["max_depth"], "n_bins": 255,
            "max_leaves": int(r["est"].max_leaves),
            "subsample": r["est"].subsample, "colsample_bytree": r["est"].colsample_bytree,
            "parallelism": "single GPU",
        },
        "roofline": hist_roofline(st, a.workload),
        "hist_rows_x_features_per_s": round(st["hist_row_features"] / hist_s) if hist_s > 0 else None,
        "predict": r["predict"],
        "kernel_ms_per_step": {  # every group timed, rounds after the timed region
            "hist": round(bd["hist_ms"] / BREAKDOWN_ROUNDS, 3),
            "partition": round(bd["part_ms"] / BREAKDOWN_ROUNDS, 3),
            "split": round(bd["split_ms"] / BREAKDOWN_ROUNDS, 3),
        },
        "fit_end_to_end": r["fit_full"],
        "nodes_expanded_per_tree": round(st["nodes_expanded"] / max(st["trees"], 1), 2),
        "timed_rounds_as_graphs": {"rows": int(r["host"]["rows_graph_rounds"]),
                                   "tree": int(r["host"]["tree_graph_rounds"])},
        "host_ms_per_step": {
            "sampler_wait": round(r["host"]["sampler_wait_ms"] / a.steps, 3),
            "round": round(r["host"]["round_ms"] / a.steps, 3),
            "enqueue": round(r["host"]["enqueue_ms"] / a.steps, 3),
            "finish_wait": round(r["host"]["finish_ms"] / a.steps, 3),
            "sampler_draw": round(r["sampler"]["draw_ms"], 3),
            "sampler_gen": round(r["sampler"]["gen_ms"], 3),
        },
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = run_cpu_baseline(a.workload, a.cpu_rounds, data=r["data"],
                                                model=r["model"], Xp_sample=r["Xp_sample"])
    del r
    if a.also and a.also != a.workload:
        r2 = run_gpu(a.also, a.also_steps, a.warmup, rounds_only=a.rounds_only)
        st2 = r2["stats"]
        line[a.also] = {
            "trees_per_s": round(a.also_steps / r2["elapsed"], 3),
            "ms_per_step": round(1e3 * r2["elapsed"] / a.also_steps, 3),
            "steps": a.also_steps,
            "timed_rounds_as_graphs": {"rows": int(r2["host"]["rows_graph_rounds"]),
                                       "tree": int(r2["host"]["tree_graph_rounds"])},
            "config": {"rows": r2["n"], "features": r2["F"],
                       "max_depth": r2["params"]["max_depth"],
                       "max_leaves": int(r2["est"].max_leaves),
                       "subsample": r2["est"].subsample,
                       "colsample_bytree": r2["est"].colsample_bytree},
            "roofline": hist_roofline(st2, a.also),
            "kernel_ms_per_step": {k: round(r2["breakdown"][f"{k}_ms"] / BREAKDOWN_ROUNDS, 3)
                                   for k in ("hist", "part", "split")},
            "host_ms_per_step": {
                "enqueue": round(r2["host"]["enqueue_ms"] / a.also_steps, 3),
                "finish_wait": round(r2["host"]["finish_ms"] / a.also_steps, 3),
                "sampler_wait": round(r2["host"]["sampler_wait_ms"] / a.also_steps, 3),
                "sampler_draw": round(r2["sampler"]["draw_ms"], 3),
            },
            "fit_end_to_end": r2["fit_full"],
            "predict": r2["predict"],
        }
        if not a.no_cpu_baseline:
            line[a.also]["cpu_baseline"] = run_cpu_baseline(
                a.also, a.also_cpu_rounds, data=r2["data"], model=r2["model"],
                Xp_sample=r2["Xp_sample"])
        del r2
    if a.fits and not a.rounds_only:
        line["workloads"] = {
            w: run_fit_workload(w, a.fits_cpu_rounds, not a.no_cpu_baseline)
            for w in a.fits.split(",") if w and w not in (a.workload, a.also)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
