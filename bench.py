#!/usr/bin/env python3
"""Benchmark: hist training rounds/s and batch prediction Mrows/s on one MI355X.

Training: binary logistic on a synthetic 10,500,000 x 28 f32 matrix (21
N(0,1) features and 7 nonlinear products of them), max_bin 256, depth 8,
eta 0.1, depthwise. A step is one boosting iteration (device gradients,
one tree, margin update) with the binned index, labels and margins
resident in HBM. `value` = steps / wall time of the timed steps.

Prediction: a 1,000-tree depth-8 forest over 10,000,000 x 100 f32 rows (2%
NaN), rows resident in HBM; reported beside the training figure.

Rank 0 prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "train rounds/s at 10.5M×28 depth-8 logistic; batch predict Mrows/s (1 GPU)"
HBM_PEAK_GBS = 8000.0
HIST_KERNEL = "hbr_hist_dense8"
# 64-bit LDS integer atomic adds per second over the chip, measured on MI355X
# (no published figure): every CU running a 1,024-thread workgroup of
# conflict-free ds_add_u64 loops reaches 5.7 T lane-ops/s (32-bit adds: 8.4 T)
LDS_ATOMIC_PEAK_T = 5.7
# The prediction walks' bound: the texture path (vector memory address and
# data units) spends at least 16 clocks of a CU on a wave-wide load (64
# lanes; up to 64 clocks as the lanes' cache lines diverge), measured on
# MI355X for 4-, 8- and 16-byte loads alike: 2.4 GHz x 256 CUs / 16.
TEXTURE_PEAK_LOADS = 2.4e9 * 256 / 16


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE passes scaled by a known-size copy),
    with the algorithmic bytes per launch of the run it was measured on."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", f"{kernel}_*hbm_counters.md"))):
        vals = {}
        for line in open(path):
            if ":" in line and line.split(":", 1)[0].strip() in ("traffic_bytes_per_launch",
                                                                    "traffic_algorithmic_bytes_per_launch"):
                k, v = line.split(":", 1)
                vals[k.strip()] = int(v.strip())
        if "traffic_bytes_per_launch" in vals:
            return vals["traffic_bytes_per_launch"], vals.get("traffic_algorithmic_bytes_per_launch"), \
                os.path.relpath(path, ROOT)
    return None, None, None


def cpu_info():
    """The first processor's /proc/cpuinfo fields that name it."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except OSError:
        pass
    return info


def cpu_model():
    return cpu_info().get("model name") or platform.processor()


def cpu_host():
    """What the CPU baselines ran on: the model string, its family / model /
    stepping numbers, the clock and the cores available."""
    i = cpu_info()
    out = {"cpu_model": cpu_model(), "cpu_vendor": i.get("vendor_id"),
           "cpu_family_model_stepping": "/".join(i.get(k, "?") for k in ("cpu family", "model", "stepping")),
           "cpu_mhz": i.get("cpu MHz"), "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    try:
        out["cpu_max_mhz"] = int(open("/sys/devices/system/cpu/cpu0/cpufreq/cpuinfo_max_freq").read()) // 1000
    except (OSError, ValueError):
        pass
    return out


def median_round_s(model, repeats):
    """Median wall time of `repeats` single boosting rounds of an oracle
    model (its first round already run as the warmup)."""
    import statistics
    ts = []
    for _ in range(repeats):
        t = time.perf_counter()
        model.more(1)
        ts.append(time.perf_counter() - t)
    return statistics.median(ts), ts


def cpu_training_baseline(args, x, y):
    """The oracle (a C restatement of the reference's CPU hist path: f64
    chain and blocked sums, depthwise growth) on the same workload: all
    cores on the full matrix, and one thread on a row prefix, each the
    median of `cpu_repeats` rounds after a warmup round."""
    from oracle import oracle as O

    p = O.params(objective=O.OBJ_LOGISTIC, max_depth=8, eta=0.1)
    O.set_threads(args.cpu_threads)
    t = time.time()
    ds = O.Dataset(x, max_bin=256)
    log(f"oracle binning in {time.time() - t:.1f}s (excluded)")
    model = O.Model(ds, y, p, 1)
    med, ts = median_round_s(model, args.cpu_repeats)
    log(f"oracle, {args.cpu_threads} threads: rounds " + ", ".join(f"{v:.2f}" for v in ts) + f" s; median {med:.2f}")
    del model, ds
    rows1 = min(args.cpu_single_rows, x.shape[0])
    ds = O.Dataset(x[:rows1], max_bin=256)
    O.set_threads(1)
    model = O.Model(ds, y[:rows1], p, 1)
    med1, ts1 = median_round_s(model, args.cpu_repeats)
    log(f"oracle, 1 thread, {rows1:,} rows: rounds " + ", ".join(f"{v:.2f}" for v in ts1) + f" s; median {med1:.2f}")
    del model, ds
    O.set_threads(0)
    return {
        "value": round(1 / med, 4), "unit": "rounds/s", "cores": args.cpu_threads, "kind": "port",
        "sample": f"the same {x.shape[0]:,} x 28 matrix, median of {args.cpu_repeats} rounds after one warmup "
                  f"round, {args.cpu_threads} OpenMP threads; C restatement of the reference CPU hist path",
        "single_thread": {
            "value": round(1 / med1, 4), "unit": "rounds/s", "cores": 1, "rows": rows1,
            "value_scaled_to_full_rows": round(rows1 / x.shape[0] / med1, 5),
            "sample": f"the first {rows1:,} rows (binned on their own), median of {args.cpu_repeats} rounds "
                      "after one warmup round; the scaled value assumes time linear in rows",
        },
        **cpu_host(),
    }


def cpu_predict_baseline(args, arrs, xp):
    """The reference's batch walk restated on the host (16 rows in
    lock-step over a breadth-first key-compare arena, 256-row blocks in
    parallel: compact/mod.rs:963-1095, model/predict.rs:203-236): all cores
    and one thread, each the median of `cpu_repeats` runs after a warmup."""
    import statistics

    from oracle import oracle as O

    legs = {}
    for threads, rows in ((args.cpu_threads, min(len(xp), 200_000)), (1, min(len(xp), 20_000))):
        O.set_threads(threads)
        O.predict_margin_lockstep(arrs, xp[:rows])
        ts = []
        for _ in range(args.cpu_repeats):
            t = time.perf_counter()
            O.predict_margin_lockstep(arrs, xp[:rows])
            ts.append(time.perf_counter() - t)
        legs[threads] = (rows, statistics.median(ts))
        log(f"oracle lock-step walk, {threads} threads, {rows:,} rows: median {legs[threads][1]:.3f} s")
    O.set_threads(0)
    (rows, med), (rows1, med1) = legs[args.cpu_threads], legs[1]
    return {
        "value": round(rows / med / 1e6, 4), "unit": "Mrows/s", "cores": args.cpu_threads, "kind": "port",
        "sample": f"first {rows:,} rows, all trees, median of {args.cpu_repeats} runs after a warmup; "
                  "16-row lock-step compact walk",
        "single_thread": {"value": round(rows1 / med1 / 1e6, 5), "unit": "Mrows/s", "cores": 1, "rows": rows1},
        **cpu_host(),
    }


def other_workload(args):
    """Training rounds/s of the regression, multiclass or sparse configuration: the
    matrix binned once (excluded), `warmup` rounds, then `steps` timed
    rounds with the index, labels and margins resident in HBM; the oracle
    times a bounded sample of the same rounds on the host."""
    import numpy as np

    import hessboost_amd as hb
    from hessboost_amd import synthetic

    t = time.time()
    if args.workload == "regression":
        x, y = synthetic.regression_100k(n=100_000, f=32, seed=0)
        params = {"objective": "reg:squarederror", "max_depth": 6, "eta": 0.1, "max_bin": 256}
        dm = hb.DMatrix(x, label=y)
        workload = "squared-error hist training, 100,000 x 32 f32, max_bin 256, max_depth 6, eta 0.1, depthwise"
    elif args.workload == "multiclass":
        x, y = synthetic.multiclass(n=2_000_000, f=50, k=10, seed=0)
        params = {"objective": "multi:softprob", "num_class": 10, "max_depth": 6, "eta": 0.3, "max_bin": 256}
        dm = hb.DMatrix(x, label=y)
        workload = "multiclass softmax hist training, 2,000,000 x 50 f32, 10 classes, max_bin 256, max_depth 6, " \
                   "eta 0.3, depthwise (10 trees per round)"
    else:
        (row_ptr, col, val), y, _ = synthetic.sparse_wide(n=500_000, f=2000, density=0.1, seed=0)
        params = {"objective": "reg:squarederror", "grow_policy": "lossguide", "max_depth": 0, "max_leaves": 255,
                  "eta": 0.3, "max_bin": 64}
        dm = hb.DMatrix((row_ptr, col, val), label=y, n_cols=2000)
        workload = "sparse hist training, 500,000 x 2,000 CSR f32 (90% missing), max_bin 64, lossguide 255 leaves"
    if args.nan_rate > 0 and args.workload != "sparse":
        # missing cells: the masked dense rows (or, with HBROCM_MASKED_ROWS=0, CSR rows)
        x[np.random.default_rng(1).random(x.shape, dtype=np.float32) < args.nan_rate] = np.nan
        dm = hb.DMatrix(x, label=y)
        workload += f", {args.nan_rate:.0%} of cells missing (NaN)"
    log(f"generated {args.workload} data in {time.time() - t:.1f}s")
    eng = dm.engine(params["max_bin"])
    log(f"index: {eng.index_info()}")
    trainer = hb.Trainer(eng, params, y)
    trainer.boost(args.warmup)
    t0 = time.perf_counter()
    trainer.boost(args.steps)
    t1 = time.perf_counter()
    dt = (t1 - t0) / args.steps
    # the kernel breakdown from further rounds with HIP events around every kernel
    extra = max(1, min(args.steps, 10))
    eng.set_profiling(True, "hbr_")
    trainer.boost(extra)
    stats = eng.kernel_stats()
    eng.set_profiling(False)
    kern = {k: round(v[0] / extra, 4) for k, v in sorted(stats.items(), key=lambda kv: -kv[1][0])}
    log(f"{args.steps} rounds in {t1 - t0:.3f}s = {1 / dt:.2f} rounds/s; ms per round by kernel: "
        + ", ".join(f"{k} {v}" for k, v in list(kern.items())[:8]))
    result = {
        "metric": f"train rounds/s ({args.workload})", "value": round(1 / dt, 3), "unit": "rounds/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int64", "data": "synthetic",
        "config": {"workload": workload}, "kernel_ms_per_round": kern,
    }
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        O.set_threads(args.cpu_threads)
        if args.workload == "regression":
            ds = O.Dataset(x, max_bin=256)
            p = O.params(max_depth=6, eta=0.1)
        elif args.workload == "multiclass":
            ds = O.Dataset(x, max_bin=256)
            p = O.params(objective=O.OBJ_SOFTMAX, num_class=10, max_depth=6, eta=0.3)
        else:
            ds = O.Dataset(csr=(row_ptr, col, val), n_cols=2000, max_bin=64)
            p = O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=255, eta=0.3, max_bin=64)
        m = O.Model(ds, y, p, 1)
        med, ts = median_round_s(m, args.cpu_repeats)
        log(f"oracle, {args.cpu_threads} threads: rounds " + ", ".join(f"{v:.2f}" for v in ts) + " s")
        O.set_threads(0)
        result["cpu_baseline"] = {"value": round(1 / med, 4), "unit": "rounds/s", "cores": args.cpu_threads,
                                  "kind": "port",
                                  "sample": f"the same workload, median of {args.cpu_repeats} rounds after one "
                                            "warmup round, oracle", **cpu_host()}
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--rows", type=int, default=10_500_000)
    ap.add_argument("--predict-rows", type=int, default=10_000_000)
    ap.add_argument("--predict-trees", type=int, default=1000)
    ap.add_argument("--predict-steps", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eval-rows", type=int, default=0,
                    help="train with an eval set of this many rows (0: none, the headline workload)")
    ap.add_argument("--no-predict", action="store_true")
    ap.add_argument("--breakdown-steps", type=int, default=5)
    ap.add_argument("--no-kernel-events", action="store_true",
                    help="run the fit without timing events on the histogram kernel")
    ap.add_argument("--hist-sample", type=int, default=5,
                    help="time every N-th histogram launch with HIP events (each timed launch stalls the "
                         "stream around its events; N coprime with the 8 levels of a tree samples every level)")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="first run a device-to-device copy of this many MiB (a known-size kernel for "
                         "scaling hardware byte counters in profiles)")
    ap.add_argument("--cpu-threads", type=int, default=min(16, len(os.sched_getaffinity(0))),
                    help="threads of the all-core CPU baseline (the single-thread one uses 1)")
    ap.add_argument("--cpu-repeats", type=int, default=5,
                    help="timed repeats of each CPU baseline leg (median reported), after one warmup")
    ap.add_argument("--cpu-single-rows", type=int, default=1_050_000,
                    help="rows of the training matrix the single-thread CPU leg trains on")
    ap.add_argument("--fit-rounds", type=int, default=500,
                    help="rounds of the timed full fit on the device, the histogram roofline's window (0: skip)")
    ap.add_argument("--row-engine-rounds", type=int, default=20,
                    help="rounds through the row-engine call sequence of hessboost's device_round (0: skip)")
    ap.add_argument("--workload", choices=("higgs", "regression", "multiclass", "sparse"), default="higgs",
                    help="higgs: the default line; multiclass (2M x 50, 10-class softmax, depth 6) and "
                         "sparse (500k x 2000 CSR, 90%% missing, lossguide 255 leaves): their training "
                         "rounds/s on a line of their own")
    ap.add_argument("--nan-rate", type=float, default=0.0,
                    help="regression and multiclass: this fraction of the cells set missing (NaN)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import hessboost_amd as hb
    from hessboost_amd import synthetic

    if args.workload != "higgs":
        other_workload(args)
        return

    if args.copy_probe_mb > 0:
        nbytes = args.copy_probe_mb << 20
        a_buf, b_buf = hb.DeviceBuffer(nbytes), hb.DeviceBuffer(nbytes)
        for _ in range(3):
            b_buf.copy_from(a_buf)
        log(f"copy probe: 3 device copies of {nbytes} bytes")
        del a_buf, b_buf

    # ---------------- training --------------------------------------------------------
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": 256}
    t = time.time()
    x, y = synthetic.higgs_like(n=args.rows, seed=0)
    log(f"generated {x.shape} in {time.time() - t:.1f}s")
    t = time.time()
    dm = hb.DMatrix(x, label=y)
    cuts = dm.cuts(256)
    t_cuts = time.time() - t
    log(f"cuts (host sketch) in {t_cuts:.1f}s (excluded)")
    # the index binned on the device from the rows already in HBM (timed apart
    # from the rounds), then the same from host rows
    x_dev = hb.DeviceBuffer(x.nbytes)
    x_dev.upload(x)
    hb.Engine.from_dense(x_dev, cuts, 0, n_rows=x.shape[0], n_cols=x.shape[1]).close()  # warm
    t = time.perf_counter()
    eng = hb.Engine.from_dense(x_dev, cuts, 0, n_rows=x.shape[0], n_cols=x.shape[1])
    t_bin = time.perf_counter() - t
    del x_dev
    # from host rows: chunks through the device's pinned staging buffers,
    # which a first call allocates (warm, untimed)
    hb.Engine.from_dense(x[:min(len(x), 3_000_000)], cuts, 0).close()
    t = time.perf_counter()
    hb.Engine.from_dense(x, cuts, 0).close()
    t_bin_host = time.perf_counter() - t
    # binning's algorithmic bytes: the f32 matrix read, u8 rows (stride 32) and columns written
    bin_bytes = x.shape[0] * (x.shape[1] * 4 + 32 + x.shape[1])
    log(f"device binning: {t_bin * 1e3:.1f} ms from HBM ({bin_bytes / t_bin / 1e9:.0f} GB/s), "
        f"{t_bin_host * 1e3:.1f} ms from host rows")
    trainer = hb.Trainer(eng, params, y)
    if args.eval_rows > 0:
        # an evaluation set (the first eval_rows training rows) whose margins
        # take every tree on the device, as training's `evals` do
        trainer.add_eval(hb.DMatrix(x[:args.eval_rows]))
        log(f"eval set: {min(args.eval_rows, x.shape[0]):,} rows")
    trainer.boost(args.warmup)
    log(f"{args.warmup} warmup rounds done")
    t0 = time.perf_counter()
    trainer.boost(args.steps)
    t1 = time.perf_counter()
    elapsed = t1 - t0
    rounds_per_s = args.steps / elapsed
    log(f"{args.steps} rounds in {elapsed:.3f}s = {rounds_per_s:.1f} rounds/s")
    # per-kernel time per round, from a few more rounds with every kernel timed
    breakdown = {}
    if args.breakdown_steps > 0:
        eng.set_profiling(True, "")
        trainer.boost(args.breakdown_steps)
        bstats = eng.kernel_stats()
        eng.set_profiling(False)
        breakdown = {k: round(ms / args.breakdown_steps, 4)
                     for k, (ms, timed, n) in sorted(bstats.items(), key=lambda kv: -kv[1][0])}
        log("ms per round by kernel: " + ", ".join(f"{k} {v}" for k, v in breakdown.items()))
    # the margin walk that also sums the next root's histogram: its
    # algorithmic bytes per row (the 32-byte row read and written back with
    # its pair word, the margin read and written, the label, and the row's
    # original index when the trainer holds the rows in a tree's leaf
    # order), its two 64-bit LDS adds per (row, feature column), over its
    # time per round
    walk_root = None
    walk_kernel = next((k for k in breakdown if k.startswith("hbr_walk_grad_root")), None)
    if walk_kernel and breakdown[walk_kernel]:
        wms = breakdown[walk_kernel]
        reordered = eng.counters()["row_orders"] > 0
        wbytes = x.shape[0] * (32 + 32 + 4 + 4 + 4 + (4 if reordered else 0))
        wach = wbytes / (wms * 1e-3) / 1e9
        # 64-bit LDS adds per row: two per feature column the kernel sums
        # (28 for rows of 25-28 features, else all 32 of the row's bytes)
        wcols = 28 if walk_kernel.endswith("_nf28") else 32
        watom = x.shape[0] * wcols * 2 / (wms * 1e-3) / 1e12
        wtraffic, _, wtraffic_src = measured_traffic(walk_kernel)
        walk_root = {"kernel": walk_kernel, "bound": "hbm", "achieved": round(wach, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(wach / HBM_PEAK_GBS, 4),
                     "avg_launch_ms": round(wms, 4), "algorithmic_bytes_per_launch": wbytes,
                     "traffic": wtraffic, "traffic_source": wtraffic_src,
                     "lds_atomics": {"achieved": round(watom, 3), "peak": LDS_ATOMIC_PEAK_T, "unit": "T lane-ops/s",
                                     "frac": round(watom / LDS_ATOMIC_PEAK_T, 4)}}
    n_trees = len(trainer.trees())

    # ---------------- the configured 500-round fit: the histogram roofline's window --------
    # A fresh trainer on the resident index, every round then the trees
    # downloaded. The dense histogram kernel's launches of the fit are timed
    # by events the runtime records with each sampled dispatch's own begin
    # and end (every hist_sample-th launch, so every level is sampled); the
    # fit is the window of the committed kernel trace's and counters' figures.
    fit_res, hist = None, None
    if args.fit_rounds > 0:
        fit = hb.Trainer(eng, params, y)
        before = eng.counters()
        eng.set_profiling(not args.no_kernel_events, HIST_KERNEL, every=max(1, args.hist_sample))
        t = time.perf_counter()
        fit.boost(args.fit_rounds)
        fit_trees = fit.trees()
        t_fit = time.perf_counter() - t
        stats = eng.kernel_stats()
        after = eng.counters()
        eng.set_profiling(False)
        hist_timed_ms = sum(ms for k, (ms, timed, n) in stats.items() if k.startswith(HIST_KERNEL))
        hist_timed = sum(timed for k, (ms, timed, n) in stats.items() if k.startswith(HIST_KERNEL))
        hist_launches = sum(n for k, (ms, timed, n) in stats.items() if k.startswith(HIST_KERNEL))
        hist_names = sorted(k for k in stats if k.startswith(HIST_KERNEL))
        avg_ms = hist_timed_ms / hist_timed if hist_timed else 0.0
        hist_bytes = after["hist_bytes"] - before["hist_bytes"]
        lds_atomics = (after["hist_rows"] - before["hist_rows"]) * x.shape[1] * 2
        per_launch = hist_bytes / max(1, hist_launches)
        achieved = per_launch / (avg_ms * 1e-3) / 1e9 if avg_ms > 0 else 0.0
        hist = dict(names=hist_names, launches=hist_launches, timed=hist_timed, avg_ms=avg_ms,
                    per_launch=per_launch, achieved=achieved, lds=lds_atomics / max(1, hist_launches),
                    near_ties=after["near_ties"] - before["near_ties"])
        log(f"{args.fit_rounds}-round fit in {t_fit:.2f}s ({len(fit_trees)} trees downloaded); "
            f"{'/'.join(hist_names)} {avg_ms:.4f} ms per launch ({hist_timed} of {hist_launches} launches timed), "
            f"{achieved:.0f} GB/s algorithmic; {hist['near_ties']} nodes the guard could not certify")
        fit_res = {
            "rounds": args.fit_rounds, "s": round(t_fit, 3), "rounds_per_s": round(args.fit_rounds / t_fit, 2),
            "s_with_binning": round(t_fit + t_bin, 3),
            "s_with_sketch_and_binning": round(t_fit + t_bin + t_cuts, 3),
            "near_ties": hist["near_ties"],
            "note": "a fresh trainer on the resident index: every round, then the trees downloaded; "
                    "binning from rows in HBM and the host sketch added in the other keys; near_ties: nodes whose "
                    "fixed-point winner the guard could not certify against the CPU's f64 sums",
        }
        del fit

    # ---------------- hessboost's own route: the row-engine call sequence ------------------
    row_engine = None
    if args.row_engine_rounds > 0:
        from hessboost_amd.rowengine import RowEngineRounds

        eng.set_sums("fixed_point")
        fo, cv = cuts.arrays()
        drv = RowEngineRounds(eng, fo, cv, params)
        m0 = np.full(len(y), np.float32(trainer.base_score()[0]), np.float32)
        c0 = eng.counters()
        drv.device_round(m0, y)
        t = time.perf_counter()
        for _ in range(args.row_engine_rounds):
            drv.device_round(m0, y)
        t_re = time.perf_counter() - t
        c1 = eng.counters()
        row_engine = {
            "value": round(args.row_engine_rounds / t_re, 2), "unit": "rounds/s", "rounds": args.row_engine_rounds,
            "near_ties": c1["near_ties"] - c0["near_ties"], "resolved": c1["near_ties_resolved"] - c0["near_ties_resolved"],
            "note": "the same workload through hessboost's device_round / build_device_staged call sequence on the "
                    "C ABI's row engine (hessboost_amd.rowengine, a Python host of the reference's builder): one "
                    "call per level step, each synchronising; fixed-point sums with near ties resolved on the "
                    "device; after one warmup round",
        }
        log(f"row-engine route: {row_engine['value']} rounds/s over {args.row_engine_rounds} rounds; "
            f"{row_engine['near_ties']} near ties, {row_engine['resolved']} resolved on the device")
    traffic, traffic_alg, traffic_src = measured_traffic(hist["names"][0] if hist and hist["names"] else HIST_KERNEL)

    result = {
        "metric": METRIC,
        "value": round(rounds_per_s, 3),
        "unit": "rounds/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": "synthetic",
        "config": {
            "workload": f"binary logistic hist training, {args.rows:,} x 28 f32 (higgs-like), max_bin 256, "
                        "max_depth 8, eta 0.1, depthwise",
            "rows": args.rows, "features": 28, "max_depth": 8, "max_bin": 256, "trees_grown": n_trees,
            **({"eval_rows": args.eval_rows} if args.eval_rows > 0 else {}),
        },
        "roofline": {
            "kernel": "/".join(hist["names"]) or HIST_KERNEL,
            "window": f"the {args.fit_rounds}-round fit from a fresh trainer: every launch of the kernel "
                      "(histogram levels 1-7 of each tree), every "
                      f"{max(1, args.hist_sample)}-th timed by events on the dispatch's own begin and end",
            "bound": "hbm",
            "achieved": round(hist["achieved"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(hist["achieved"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "traffic_run_algorithmic_bytes": traffic_alg,
            "launches": hist["launches"],
            "timed_launches": hist["timed"],
            "avg_launch_ms": round(hist["avg_ms"], 4),
            "algorithmic_bytes_per_launch": int(hist["per_launch"]),
            # the kernel's other bound: two 64-bit LDS integer adds per (row, feature)
            "lds_atomics": {
                "achieved": round(hist["lds"] / (hist["avg_ms"] * 1e-3) / 1e12, 3) if hist["avg_ms"] > 0 else 0.0,
                "peak": LDS_ATOMIC_PEAK_T,
                "unit": "T lane-ops/s",
                "frac": round(hist["lds"] / (hist["avg_ms"] * 1e-3) / 1e12 / LDS_ATOMIC_PEAK_T, 4)
                if hist["avg_ms"] > 0 else 0.0,
                "per_launch": int(hist["lds"]),
            },
        } if hist else None,
        "kernel_ms_per_round": breakdown,
        **({"walk_root_roofline": walk_root} if walk_root else {}),
        # the index built on the device from the f32 rows (not part of the rounds)
        "binning": {
            "value": round(x.shape[0] / t_bin / 1e6, 1), "unit": "Mrows/s",
            "ms": round(t_bin * 1e3, 2), "ms_from_host_rows": round(t_bin_host * 1e3, 2),
            "host_sketch_s": round(t_cuts, 2),
            "roofline": {"bound": "hbm", "achieved": round(bin_bytes / t_bin / 1e9, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(bin_bytes / t_bin / 1e9 / HBM_PEAK_GBS, 4),
                         "note": "whole engine construction (binning, count scan, syncs) on rows in HBM"},
        },
    }

    if fit_res:
        result["fit"] = fit_res
    if row_engine:
        result["row_engine"] = row_engine
    del eng, trainer

    # ---------------- CPU baseline (oracle, same workload) -----------------------------
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_training_baseline(args, x, y)

    # ---------------- batch prediction ---------------------------------------------------
    if not args.no_predict:
        del x, y, dm, cuts
        n, f = args.predict_rows, 100
        t = time.time()
        trees = synthetic.forest(n_trees=args.predict_trees, depth=8, n_features=f, seed=0)
        xp = synthetic.predict_rows(n=n, f=f, seed=1)
        log(f"generated forest + {xp.shape} rows in {time.time() - t:.1f}s")
        arrs = None
        if not args.no_cpu_baseline:
            from oracle import oracle as O

            arrs = O.forest_arrays(trees)
        booster = hb.Booster(objective="reg:squarederror", base_score=np.zeros(1, np.float32), trees=trees,
                             n_outputs=1, n_features=f)
        forest = hb.Forest(booster.forest_desc(), 1, 0)
        dx = hb.DeviceBuffer(xp.nbytes)
        dx.upload(xp)
        dout = hb.DeviceBuffer(4 * n)
        for _ in range(2):
            forest.predict_margin_device(dx.ptr, n, f, dout.ptr)
        dout.download(np.float32, 1)
        forest.set_profiling(True, "hbr_predict")
        t0 = time.perf_counter()
        for _ in range(args.predict_steps):
            forest.predict_margin_device(dx.ptr, n, f, dout.ptr)
        dout.download(np.float32, 1)
        t1 = time.perf_counter()
        pstats = forest.kernel_stats()
        forest.set_profiling(False)
        mrows = n * args.predict_steps / (t1 - t0) / 1e6
        # from host rows: the same walk with the 4 GB of rows copied in by the
        # call (PCIe), in chunks through pinned staging buffers that the
        # warmup call (over two chunks' worth of rows) allocates; the median
        # of three calls
        forest.predict_margin(xp[:min(n, 700_000)])
        host_times = []
        for _ in range(3):
            t = time.perf_counter()
            forest.predict_margin(xp)
            host_times.append(time.perf_counter() - t)
        t_host = sorted(host_times)[1]
        log(f"predict from host rows: {n / t_host / 1e6:.1f} Mrows/s ({t_host:.3f} s with the copy)")
        pkern = sorted(k for k in pstats if k.startswith("hbr_predict"))
        pms = sum(pstats[k][0] for k in pkern)
        pl = sum(pstats[k][1] for k in pkern)
        pbytes = n * (4 * f + 4)
        launch_s = pms / max(1, pl) * 1e-3
        pach = pbytes / launch_s / 1e9 if pms > 0 else 0.0
        node_steps = n * args.predict_trees * 8
        # wave-wide node loads of the walk that ran: the pair walk loads one
        # record per two levels below the root's (a scalar load) and the
        # leaf's value (depth 8: 4 per tree), the mirror walk one node per
        # level and the leaf (9)
        per_tree = 4 if any("pairs" in k for k in pkern) else 9
        loads = (n + 63) // 64 * args.predict_trees * per_tree
        ptraffic, _, ptraffic_src = measured_traffic(pkern[0] if pkern else "hbr_predict")
        log(f"predict: {mrows:.1f} Mrows/s; kernel {launch_s * 1e3:.2f} ms per launch, {pach:.0f} GB/s")
        pred = {
            "metric": "batch predict Mrows/s", "value": round(mrows, 2), "unit": "Mrows/s",
            "steps": args.predict_steps,
            "from_host_rows": {"value": round(n / t_host / 1e6, 2), "unit": "Mrows/s", "s": round(t_host, 4),
                               "note": "rows in host memory, copied to HBM by the call in chunks through pinned "
                                       "staging buffers, overlapped with the walk; median of 3 calls (the resident "
                                       "rate is value)"},
            "config": {"workload": f"{args.predict_trees}-tree depth-8 forest, {n:,} x {f} f32 rows, 2% NaN"},
            "roofline": {"kernel": "/".join(pkern) or "hbr_predict", "bound": "texture path",
                         "achieved": round(loads / launch_s, 1) if pms else 0.0, "peak": TEXTURE_PEAK_LOADS,
                         "unit": "wave-wide loads/s",
                         "frac": round(loads / launch_s / TEXTURE_PEAK_LOADS, 4) if pms else 0.0,
                         "loads_per_launch": loads, "avg_launch_ms": round(launch_s * 1e3, 4),
                         "node_steps_per_s": round(node_steps / launch_s, 1) if pms else None,
                         "hbm": {"achieved": round(pach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(pach / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": pbytes,
                                 "traffic": ptraffic, "traffic_source": ptraffic_src}},
        }
        if arrs is not None:
            pred["cpu_baseline"] = cpu_predict_baseline(args, arrs, xp)
        result["predict"] = pred
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
