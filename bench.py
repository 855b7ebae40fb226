"""Benchmark: predicted rows/s on one MI355X against a 10,000-row x 100-feature fitted cache.

Workload: the full-size TabICL v2 classifier architecture (e = 128, 3 column blocks of 8 x 16 heads over 128
inducing points, 3 row blocks, d = 512, 12 in-context layers of 8 heads x 64, decoder 1024 -> 10), random-init
weights from seed 2, a stored f32 cache of 10,000 training rows (chunks of 256, the last of 16) and its column cache
for 100 features. A step is one prediction pass of a batch of 2,048 test rows of 100 features through all three
stages (column, row, in-context + decoder), inputs already resident in HBM. Also reported: rows/s at batches of 1,
64 and 256, the in-context stage alone, the attention kernel's share of the fp32 MFMA roofline (measured with HIP
events on the library's stream), and the oracle (the C restatement of the reference's CPU path) timed on this
host's cores on a bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
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
PEAK_F32_MFMA = 157.3e12  # MI355X dense fp32 matrix FLOP/s
PEAK_HBM = 8.0e12


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def synthetic_cache(rng, layers, d):
    """Stored f32 layers of the exact shape a 10,000-row fit writes (values N(0, 0.5^2))."""
    nbytes = (ROWS // CHUNK) * 8 * d * CHUNK + (8 * d * (ROWS % CHUNK) if ROWS % CHUNK else 0)
    one = (rng.standard_normal(nbytes // 4) * 0.5).astype(np.float32).view(np.uint8)
    return [one.copy() for _ in range(layers)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (for profiler runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); multi-GPU sharding is a design note, not built",
              file=sys.stderr)
        sys.exit(2)

    abi = importlib.import_module("tabicl-anywhere_amd.abi")
    M = importlib.import_module("tabicl-anywhere_amd.model")
    hip = importlib.import_module("tabicl-anywhere_amd.hip")
    dm = importlib.import_module("tabicl-anywhere_amd.devmem")

    rng = np.random.default_rng(3)
    model = M.Model.random(M.FULL_CLASSIFIER, seed=2)
    d, L, heads = model.d, model.icl_layers, model.icl_heads
    layers = synthetic_cache(rng, L, d)
    scales = np.full((L, d), 1.0 / 8.0, np.float32)
    gpu = hip.Gpu(0)
    log("device:", gpu.name)
    w = gpu.weights(model)
    vm = gpu.load(w, abi.KV_F32, ROWS, CHUNK, layers, scales)
    col_kv = (rng.standard_normal((FEATURES, 1, len(model.col_a2), 2, model.e, model.inds)) * 0.5).astype(np.float32)
    vm.set_columns(col_kv, FEATURES, 1)
    x_host = rng.standard_normal((BATCH, FEATURES)).astype(np.float32)
    x_dev = dm.DeviceBuffer.of(x_host)
    h_host = rng.standard_normal((BATCH, d)).astype(np.float32)
    h_dev = dm.DeviceBuffer.of(h_host)
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

    # ---- the in-context stage alone (row representations in, scores out) --------------------------------------
    for _ in range(2):
        gpu.in_context_dev(w, vm, h_dev.ptr, BATCH, CLASSES, out_dev.ptr)
    gpu.sync()
    timer.start()
    for _ in range(args.steps):
        gpu.in_context_dev(w, vm, h_dev.ptr, BATCH, CLASSES, out_dev.ptr)
    icl_ms = timer.stop() / args.steps
    log(f"in-context stage alone, {BATCH} rows: {icl_ms:.3f} ms")

    # ---- the dominant kernel: attention over one stored layer, 2,048 queries ---------------------------------
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
    achieved = flops / (att_ms / 1e3)
    log(f"attention, {BATCH} queries x {ROWS} keys x {heads} heads: {att_ms:.3f} ms, {achieved / 1e12:.1f} TFLOP/s")

    # ---- CPU baseline: the oracle on a bounded sample of the same workload -----------------------------------
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc

        threads = min(16, os.cpu_count() or 1)
        orc.set_threads(threads)
        sample = 512
        planmod = importlib.import_module("tabicl-anywhere_amd.plan")
        fitted = orc.Fitted(ROWS, FEATURES, CLASSES, CHUNK, abi.KV_F32,
                            planmod.Plan([CLASSES], [planmod.Node(None, [], CLASSES, True, list(range(CLASSES)))]),
                            col_kv, [scales], [layers])
        t0 = time.perf_counter()
        orc.predict_raw(model, fitted, x_host[:sample])
        secs = time.perf_counter() - t0
        cpu = {"value": round(sample / secs, 2), "unit": "rows/s", "cores": threads, "kind": "port",
               "sample": f"{sample} test rows through all three stages against the same caches "
                         f"(C restatement of the reference CPU path, {threads} OpenMP threads, {secs:.1f} s)"}
        log(f"cpu baseline: {cpu['value']} rows/s on {threads} threads")

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
        "data": "synthetic: random-init full-size TabICL v2 classifier weights (seed 2), N(0,1) test rows, and random "
                "stored f32 caches of the 10,000-row x 100-feature shape",
        "config": {"workload": "predict 2,048 test rows x 100 features through the column, row and in-context stages "
                               "against a 10,000-row f32 cache (d=512, 12 layers of 8x64 heads, 10 classes)",
                   "train_rows": ROWS, "features": FEATURES, "chunk": CHUNK, "test_rows": BATCH, "classes": CLASSES,
                   "kv": "f32"},
        "rows_per_s_by_batch": per_batch,
        "in_context_stage_ms": round(icl_ms, 4),
        "fit_s": None,
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": PEAK_F32_MFMA / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_F32_MFMA, 4), "traffic": None,
                     "kernel": "k_attn_mfma64 (+ split merge)", "ms_per_launch": round(att_ms, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    for b in (q_dev, att_dev, h_dev, out_dev, x_dev):
        b.free()
    vm.free()
    w.free()
    gpu.close()


if __name__ == "__main__":
    main()
