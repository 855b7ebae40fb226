"""Benchmark: fit a 10,000-row x 100-feature table on one MI355X, then predict rows/s against its cache.

Workload (the full-size TabICL v2 classifier architecture with random-init weights from seed 2: e = 128, 3 column
blocks of 8 x 16 heads over 128 inducing points, 3 row blocks, d = 512, 12 in-context layers of 8 x 64 heads,
decoder 1024 -> 10). Synthetic table: X ~ N(0, 1) of 10,000 training + 2,048 test rows x 100 features (seed 3);
10 classes, y = argmax(X W + Gumbel noise) with W ~ N(0, 1) (seed 4). One member, f32 cache, chunks of 256 rows.

* fit_s: the whole fit on the card (column, row and in-context stages; every layer's stored records back on the
  host), wall clock, after one warm-up fit.
* value: a step is one prediction pass of 2,048 test rows through all three stages against the fitted caches,
  inputs already resident in HBM; rows/s. Also batches of 1, 64 and 256 rows, the in-context stage alone, and
  2,048 rows against the same table's cache quantised to i16 and to i8 (fitted again in that format).
* roofline: the dominant kernel, the in-context attention (2,048 queries over 10,000 keys, 8 heads of 64): the timed
  steps run a second time with each of its launches bracketed by HIP events on the library's stream
  (tah_probe_attention), its average launch duration over them. Its f32 products run on the fp16 matrix cores as three fp16 products
  each, so its ceiling is the dense fp16 MFMA peak (2.5 PFLOP/s) over three: 833 TFLOP/s of f32 work.
* budgeted_256mb: 2,048 rows predicted within a 256 MB working-memory budget (sub-batched), as the reference
  quotes it.
* cpu_baseline: the oracle (an unvectorised C restatement of the reference's CPU path) on this host's cores,
  predicting a bounded sample of the same test rows against the same caches; and a bounded fit sample timed on both
  (--cpu-fit-rows 10000: the whole training table).
* regression_head: 2,048 rows x 8 members of 999 predicted quantiles read as distributions on the card (mean,
  variance, median and six quantiles a row, tah_quantile_stats), and a sample of rows through the host statement.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--cpu-fit-rows N] [--rows-only N --kv FMT]
"""
import argparse
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

ROWS, FEATURES, CHUNK, BATCH, CLASSES = 10000, 100, 256, 2048, 10
PEAK_F16_MFMA = 2.5e15  # MI355X dense fp16 matrix FLOP/s
PEAK_SPLIT_F32 = PEAK_F16_MFMA / 3  # f32 work at three fp16 products per f32 product
PEAK_HBM = 8.0e12  # MI355X HBM3E bytes/s
# HBM bytes per launch of the roofline kernel, from rocprofv3 FETCH_SIZE and WRITE_SIZE runs of this bench scaled by
# the counters' reading on its own 1 GiB copies (profiles/attention_f32_2048x10000_memory.md): 58.2 MB read + 17.3 MB
# written
TRAFFIC_BYTES = 75.5e6


def pass_cost(model, n, rows=ROWS, features=FEATURES, kv_bytes=4):
    """Algorithmic cost of one prediction pass of n rows against one member (one problem, one label digit):
    (bytes, flops). Bytes: every in-context layer's stored keys and values read once (plus the per-chunk scales of
    an integer cache), the column cache, the weights at f32, the rows in and the scores out. Flops: the in-context
    attention (4 N d per row and layer), the in-context dense layers, the decoder, the column stage (3 blocks over the
    128 inducing points per feature) and the row stage (3 blocks over T = cls + features tokens)."""
    d, L, e, inds, cls = model.d, model.icl_layers, model.e, model.inds, model.cls
    ff, heads, hd, T, C = 2 * d, model.icl_heads, d // model.icl_heads, cls + features, model.outputs
    chunks = -(-rows // CHUNK)
    kv = L * (2 * rows * d * kv_bytes + (chunks * 8 * d if kv_bytes < 4 else 0))
    col = features * 3 * 2 * e * inds * 4
    # the weights prediction reads: not the inducing points and their blocks (fit only), and of the column and
    # in-context blocks only the query third of the input projection (their keys and values come from the caches)
    def block_floats(b, query_only):
        return sum(a.size // 3 if query_only and k in ("in_w", "in_b") else a.size for k, a in b.t.items())

    weights = 4 * (sum(a.size for k, a in model.t.items() if k != "col_ind")
                   + sum(block_floats(b, True) for b in model.col_a2 + model.icl)
                   + sum(block_floats(b, False) for b in model.row))
    nbytes = kv + col + weights + n * (features + C) * 4
    per_row = (4 * rows * d * L
               + 2 * L * (2 * d * d + 2 * d * ff + heads * 2 * hd * hd)
               + 2 * (ff * d + C * ff)
               + 2 * features * 3 * (6 * e * e + 2 * inds * e)
               + 2 * (2 * T * (8 * e * e + 2 * T * e) + 2 * e * e * T + cls * (6 * e * e + 2 * T * e)))
    return nbytes, n * per_row


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def table(rows, features, classes, seed_x=3, seed_w=4):
    rx = np.random.default_rng(seed_x)
    x = rx.standard_normal((rows, features)).astype(np.float32)
    rw = np.random.default_rng(seed_w)
    w = rw.standard_normal((features, classes))
    g = rw.gumbel(size=(rows, classes))
    y = np.argmax(x.astype(np.float64) @ w + g, axis=1).astype(np.float32)
    return x, y


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (for profiler runs)")
    ap.add_argument("--cpu-fit-rows", type=int, default=2500,
                    help="training rows of the CPU fit sample (10000: the whole table, about a minute of CPU work)")
    ap.add_argument("--rows-only", type=int, default=0,
                    help="profiling: after the fit, only predict this many rows 45 times (5 warm-up) and print the time")
    ap.add_argument("--kv", choices=("f32", "i16", "i8"), default="f32", help="cache format of --rows-only")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); multi-GPU sharding is a design note, not built",
              file=sys.stderr)
        sys.exit(2)

    abi = importlib.import_module("tabicl-anywhere_amd.abi")
    M = importlib.import_module("tabicl-anywhere_amd.model")
    hip = importlib.import_module("tabicl-anywhere_amd.hip")
    dm = importlib.import_module("tabicl-anywhere_amd.devmem")
    fitmod = importlib.import_module("tabicl-anywhere_amd.fit")

    model = M.Model.random(M.FULL_CLASSIFIER, seed=2)
    d, L, heads = model.d, model.icl_layers, model.icl_heads
    x_all, y_all = table(ROWS + BATCH, FEATURES, CLASSES)
    x_train, y_train, x_test = x_all[:ROWS], y_all[:ROWS], x_all[ROWS:]
    gpu = hip.Gpu(0)
    log("device:", gpu.name)
    w = gpu.weights(model)

    if args.rows_only > 0:
        # a profiler's view of one batch size: the fit in the chosen format, then 45 predictions of that many rows
        fmt = {"f32": abi.KV_F32, "i16": abi.KV_I16, "i8": abi.KV_I8}[args.kv]
        n = min(args.rows_only, BATCH)
        fq = fitmod.fit_raw(gpu, w, x_train, y_train, CLASSES, CHUNK, fmt)
        vq = gpu.load(w, fmt, ROWS, CHUNK, fq.layers[0], fq.scales[0])
        vq.set_columns(fq.col_kv, FEATURES, 1)
        xq, oq = dm.DeviceBuffer.of(x_test), dm.DeviceBuffer(BATCH * CLASSES * 4)
        for _ in range(5):
            gpu.predict_dev(w, vq, xq.ptr, n, CLASSES, oq.ptr)
        gpu.sync()
        tq = dm.EventTimer(gpu.stream)
        tq.start()
        for _ in range(40):
            gpu.predict_dev(w, vq, xq.ptr, n, CLASSES, oq.ptr)
        log(f"prediction, {n} rows, {args.kv} cache: {tq.stop() / 40:.4f} ms (45 predictions after the fit)")
        for b in (xq, oq):
            b.free()
        vq.free()
        w.free()
        gpu.close()
        return

    # ---- fit on the card ------------------------------------------------------------------------------------
    fitmod.fit_raw(gpu, w, x_train[:1000], y_train[:1000], CLASSES, CHUNK)  # warm-up (kernels loaded, pool grown)
    t0 = time.perf_counter()
    fitted = fitmod.fit_raw(gpu, w, x_train, y_train, CLASSES, CHUNK, abi.KV_F32)
    fit_s = time.perf_counter() - t0
    log(f"fit {ROWS} x {FEATURES} on the card: {fit_s:.3f} s")

    vm = gpu.load(w, abi.KV_F32, ROWS, CHUNK, fitted.layers[0], fitted.scales[0])
    vm.set_columns(fitted.col_kv, FEATURES, 1)
    x_dev = dm.DeviceBuffer.of(x_test)
    out_dev = dm.DeviceBuffer(BATCH * CLASSES * 4)
    timer = dm.EventTimer(gpu.stream)

    def run(n):
        gpu.predict_dev(w, vm, x_dev.ptr, n, CLASSES, out_dev.ptr)

    # ---- the headline: batches of 2,048 rows --------------------------------------------------------------
    for _ in range(args.warmup):
        run(BATCH)
    gpu.sync()
    dm.synchronize()
    t0 = time.perf_counter()
    timer.start()
    for _ in range(args.steps):
        run(BATCH)
    ev_ms = timer.stop()
    dm.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    # the same steps again with the roofline kernel's launches each bracketed by HIP events on the library's stream
    # (the events cost about 2% of a step, so the headline comes from the pass above)
    gpu.probe_attention(args.steps * L)
    timer.start()
    for _ in range(args.steps):
        run(BATCH)
    probed_ms = timer.stop() / args.steps
    probe_n, probe_ms = gpu.probe_read()
    gpu.probe_attention(0)
    if probe_n != args.steps * L:
        raise RuntimeError(f"expected {args.steps * L} attention launches in the timed steps, the probe saw {probe_n}")
    att_kernel_ms = probe_ms / probe_n
    ms_step = max(ev_ms, wall_ms) / args.steps
    rows_s = BATCH / (ms_step / 1e3)
    log(f"prediction, {BATCH} rows: {ms_step:.3f} ms/step, {rows_s:,.0f} rows/s")

    # ---- other batch sizes -------------------------------------------------------------------------------
    per_batch = {}
    for n in (1, 64, 256):
        for _ in range(2):
            run(n)
        gpu.sync()
        reps = 20
        timer.start()
        for _ in range(reps):
            run(n)
        ms = timer.stop() / reps
        per_batch[str(n)] = round(n / (ms / 1e3), 1)
        log(f"prediction, {n} rows: {ms:.3f} ms, {per_batch[str(n)]:,.0f} rows/s")
    per_batch[str(BATCH)] = round(rows_s, 1)
    # fractions of the roofline at each batch: the pass's algorithmic bytes at 8 TB/s and flops at the split-fp16
    # ceiling, against the measured time (one row is HBM-bound, 64 rows and more MFMA-bound)
    roof_by_batch = {}
    for n_s, rps in per_batch.items():
        n = int(n_s)
        nbytes, flops = pass_cost(model, n)
        t = n / rps
        roof_by_batch[n_s] = {"hbm_frac": round(nbytes / PEAK_HBM / t, 4), "mfma_frac": round(flops / PEAK_SPLIT_F32 / t, 4),
                              "bytes": nbytes, "flops": flops}

    # ---- 2,048 rows under a 256 MB working-memory budget (sub-batched; src/gpu.rs:1452-1468, README.md:99) --------
    old_budget = gpu.work_budget()
    gpu.release()
    gpu.set_work_budget(256 << 20)
    try:
        for _ in range(2):
            run(BATCH)
        gpu.sync()
        timer.start()
        for _ in range(args.steps):
            run(BATCH)
        budget_ms = timer.stop() / args.steps
        budget_peak = gpu.working()[1]
    finally:
        gpu.release()
        gpu.set_work_budget(old_budget)
    budgeted = {"rows": BATCH, "work_budget_bytes": 256 << 20, "ms": round(budget_ms, 4),
                "rows_per_s": round(BATCH / (budget_ms / 1e3), 1), "peak_working_bytes": int(budget_peak)}
    log(f"prediction, {BATCH} rows within a 256 MB working budget: {budget_ms:.3f} ms "
        f"(peak working memory {budget_peak / 2**20:.0f} MiB)")
    if budget_peak > 256 << 20 or gpu.overdrawn():
        raise RuntimeError("the budgeted prediction went over its working-memory budget")

    # one row after flushing the 256 MB MALL (a 1 GiB copy between runs), each cache format: the cold-cache latency
    flush_a, flush_b = dm.DeviceBuffer(1 << 30), dm.DeviceBuffer(1 << 30)
    cold = {}

    def one_row_cold(vmx, label):
        times = []
        for _ in range(7):
            dm.copy(flush_b, flush_a, 1 << 30)
            timer.start()
            gpu.predict_dev(w, vmx, x_dev.ptr, 1, CLASSES, out_dev.ptr)
            times.append(timer.stop())
        cold[label] = round(float(np.median(times)), 4)
        log(f"prediction, 1 row after a MALL flush, {label} cache: {cold[label]:.3f} ms")

    one_row_cold(vm, "f32")

    # ---- the same table with the cache quantised to i16 and to i8 (dequantised inside the kernels) -----------------
    per_cache = {"f32": round(rows_s, 1)}
    for name, fmt in (("i16", abi.KV_I16), ("i8", abi.KV_I8)):
        fq = fitmod.fit_raw(gpu, w, x_train, y_train, CLASSES, CHUNK, fmt)
        vq = gpu.load(w, fmt, ROWS, CHUNK, fq.layers[0], fq.scales[0])
        vq.set_columns(fq.col_kv, FEATURES, 1)
        for _ in range(2):
            gpu.predict_dev(w, vq, x_dev.ptr, BATCH, CLASSES, out_dev.ptr)
        gpu.sync()
        timer.start()
        for _ in range(args.steps):
            gpu.predict_dev(w, vq, x_dev.ptr, BATCH, CLASSES, out_dev.ptr)
        ms = timer.stop() / args.steps
        per_cache[name] = round(BATCH / (ms / 1e3), 1)
        log(f"prediction, {BATCH} rows, {name} cache: {ms:.3f} ms, {per_cache[name]:,.0f} rows/s")
        one_row_cold(vq, name)
        vq.free()
    flush_a.free()
    flush_b.free()

    # ---- the in-context stage alone and its attention kernel ---------------------------------------------------
    rng = np.random.default_rng(5)
    h_dev = dm.DeviceBuffer.of(rng.standard_normal((BATCH, d)).astype(np.float32))
    for _ in range(2):
        gpu.in_context_dev(w, vm, h_dev.ptr, BATCH, CLASSES, out_dev.ptr)
    gpu.sync()
    timer.start()
    for _ in range(args.steps):
        gpu.in_context_dev(w, vm, h_dev.ptr, BATCH, CLASSES, out_dev.ptr)
    icl_ms = timer.stop() / args.steps
    log(f"in-context stage alone, {BATCH} rows: {icl_ms:.3f} ms")
    q_dev = dm.DeviceBuffer.of((rng.standard_normal((BATCH, d)) * 0.1).astype(np.float32))
    att_dev = dm.DeviceBuffer(BATCH * d * 4)
    for l in range(2):
        gpu.attend_resident_dev(vm, l, q_dev.ptr, BATCH, att_dev.ptr)
    gpu.sync()
    reps = 3 * L
    timer.start()
    for i in range(reps):
        gpu.attend_resident_dev(vm, i % L, q_dev.ptr, BATCH, att_dev.ptr)
    att_ms = timer.stop() / reps
    flops = 4.0 * ROWS * d * BATCH  # scores and weighted values: 2 * N * d each, per query
    achieved = flops / (att_kernel_ms / 1e3)
    log(f"attention, {BATCH} queries x {ROWS} keys x {heads} heads: {att_kernel_ms:.4f} ms a launch inside the timed "
        f"steps ({probe_n} launches), {achieved / 1e12:.1f} TFLOP/s; {att_ms:.4f} ms back to back with its merge")

    # ---- the regression head: 2,048 rows x 8 members of 999 predicted quantiles read as distributions --------------
    alphas = np.array([0.025, 0.1, 0.25, 0.75, 0.9, 0.975], np.float32)
    rq, nqv = 8 * BATCH, 999
    q_host = (rng.standard_normal((rq, nqv)) * 3.0 + 1.0).astype(np.float32)
    qq_dev = dm.DeviceBuffer.of(q_host)
    st_dev = dm.DeviceBuffer(rq * (3 + alphas.size) * 4)
    gpu.quantile_stats_dev(qq_dev.ptr, rq, nqv, alphas, st_dev.ptr)
    gpu.sync()
    timer.start()
    for _ in range(3):
        gpu.quantile_stats_dev(qq_dev.ptr, rq, nqv, alphas, st_dev.ptr)
    qs_ms = timer.stop() / 3
    regression = {"rows": rq, "quantiles": nqv, "levels": int(alphas.size), "ms": round(qs_ms, 4),
                  "rows_per_s": round(rq / (qs_ms / 1e3), 1)}
    log(f"regression head, {rq} rows x {nqv} quantiles: {qs_ms:.3f} ms, {regression['rows_per_s']:,.0f} rows/s")
    qq_dev.free()
    st_dev.free()

    # a plain 256 MiB device-to-device copy: the known-size reference that the memory counters of a profile of
    # this run are scaled by (profiles/attention_f32_2048x10000_memory.md)
    cal_a, cal_b = dm.DeviceBuffer(256 << 20), dm.DeviceBuffer(256 << 20)
    dm.copy(cal_b, cal_a, 256 << 20)
    dm.synchronize()
    cal_a.free()
    cal_b.free()

    # ---- CPU baseline: the oracle on bounded samples of the same workload ------------------------------------
    cpu, fit_sample = None, None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc

        threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        orc.set_threads(threads)
        cpu_model = "unknown"
        try:
            with open("/proc/cpuinfo") as fh:
                cpu_model = next((ln.split(":", 1)[1].strip() for ln in fh if ln.startswith("model name")), cpu_model)
        except OSError:
            pass
        sample = 256
        t0 = time.perf_counter()
        want = orc.predict_raw(model, fitted, x_test[:sample])
        secs = time.perf_counter() - t0
        got = gpu.predict(w, vm, x_test[:sample], CLASSES)
        cpu = {"value": round(sample / secs, 2), "unit": "rows/s", "cores": threads, "kind": "port",
               "cpu_model": cpu_model,
               "sample": f"{sample} of the test rows through all three stages against the card-fitted caches (the "
                         f"oracle: an unvectorised scalar C restatement of the reference CPU path, not the "
                         f"reference's SIMD build, {threads} OpenMP threads = the cores this process may use, "
                         f"{secs:.1f} s; largest score difference to the card {np.abs(got - want).max():.1e})"}
        log(f"cpu baseline: {cpu['value']} rows/s on {threads} threads ({cpu_model})")
        fr = min(max(args.cpu_fit_rows, CHUNK), ROWS)
        t0 = time.perf_counter()
        orc.fit_raw(model, x_train[:fr], y_train[:fr], CLASSES, CHUNK)
        cpu_fit = time.perf_counter() - t0
        t0 = time.perf_counter()
        fitmod.fit_raw(gpu, w, x_train[:fr], y_train[:fr], CLASSES, CHUNK)
        gpu_fit = time.perf_counter() - t0
        fit_sample = {"rows": fr, "features": FEATURES, "cpu_s": round(cpu_fit, 3), "gpu_s": round(gpu_fit, 4),
                      "speedup": round(cpu_fit / gpu_fit, 1), "cores": threads, "kind": "port",
                      "note": f"the same {fr:,}-row sample of the training table fitted by the oracle (the "
                              f"unvectorised C restatement of the reference CPU path) and by the card"
                              + ("" if fr == ROWS else "; the column and row stages grow linearly with rows and the "
                                 "in-context stage with rows squared, so the full 10,000-row fit is 4 to 16 times "
                                 "the sample on the CPU (bench.py --cpu-fit-rows 10000 times it whole)")}
        log(f"fit sample {fr} x {FEATURES}: cpu {cpu_fit:.2f} s, card {gpu_fit:.3f} s ({cpu_fit / gpu_fit:.0f}x)")
        tab = importlib.import_module("tabicl-anywhere_amd.table")
        hs = 512
        t0 = time.perf_counter()
        for row in q_host[:hs]:
            dd = tab.QuantileDist(row)
            dd.mean(), dd.variance(), dd.icdf(0.5), [dd.icdf(a) for a in alphas]
        host_s = time.perf_counter() - t0
        regression["host_rows_per_s"] = round(hs / host_s, 1)
        regression["host_sample"] = f"{hs} rows through the host statement (table.QuantileDist, numpy, one thread)"
        log(f"regression head on the host: {regression['host_rows_per_s']:,.0f} rows/s")

    line = {
        "metric": "predicted rows/s at 10k x 100 cache (1/64/2048 rows); % roofline; fit s",
        "value": round(rows_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: N(0,1) table of 10,000 + 2,048 rows x 100 features, 10 classes from argmax of a random "
                "projection plus Gumbel noise; random-init full-size TabICL v2 classifier weights (seed 2); the "
                "caches predicted against are those the card fitted",
        "config": {"workload": "fit 10,000 x 100 on the card, then predict 2,048 test rows through the column, row "
                               "and in-context stages (f32 cache, d=512, 12 layers of 8x64 heads, 10 classes)",
                   "train_rows": ROWS, "features": FEATURES, "chunk": CHUNK, "test_rows": BATCH, "classes": CLASSES,
                   "kv": "f32", "members": 1},
        "rows_per_s_by_batch": per_batch,
        "rows_per_s_by_cache": per_cache,
        "in_context_stage_ms": round(icl_ms, 4),
        "fit_s": round(fit_s, 4),
        "regression_head": regression,
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": round(PEAK_SPLIT_F32 / 1e12, 1),
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_SPLIT_F32, 4), "traffic": TRAFFIC_BYTES,
                     "kernel": "k_attn_split64", "ms_per_launch": round(att_kernel_ms, 4), "launches": probe_n,
                     "ms_back_to_back_with_merge": round(att_ms, 4), "probed_ms_per_step": round(probed_ms, 4),
                     "basis": "algorithmic f32 FLOP (4 x queries x keys x d) per launch / the kernel's average launch "
                              "duration over a second pass of the timed steps (HIP events around each launch on the "
                              "library's stream), against the dense fp16 MFMA peak / 3 (each f32 product is three fp16 "
                              "products)"},
        "step_roofline": {"bound": "mfma", "achieved": round(pass_cost(model, BATCH)[1] / (ms_step / 1e3) / 1e12, 2),
                          "peak": round(PEAK_SPLIT_F32 / 1e12, 1), "unit": "TFLOP/s",
                          "frac": round(pass_cost(model, BATCH)[1] / (ms_step / 1e3) / PEAK_SPLIT_F32, 4),
                          "basis": "algorithmic f32 FLOP of a whole 2,048-row prediction pass (all three stages) / "
                                   "ms_per_step, against the split-fp16 ceiling"},
        "roofline_by_batch": roof_by_batch,
        "one_row_after_mall_flush_ms": cold,
        "one_row_cold_hbm_frac": round(pass_cost(model, 1)[0] / PEAK_HBM / (cold["f32"] / 1e3), 4),
        "budgeted_256mb": budgeted,
        "cpu_baseline": cpu,
        "fit_sample": fit_sample,
    }
    print(json.dumps(line), flush=True)
    for b in (q_dev, att_dev, h_dev, out_dev, x_dev):
        b.free()
    vm.free()
    w.free()
    gpu.close()


if __name__ == "__main__":
    main()
