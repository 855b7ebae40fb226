"""Benchmark: predicted rows/s of the in-context stage on one MI355X.

Workload: the full-size TabICL v2 classifier architecture (d = 512, 12 in-context layers of 8 heads x 64, decoder
1024 -> 10), random-init weights from seed 2, against a stored f32 cache of 10,000 training rows (chunks of 256,
the last of 16). A step is one in-context pass (12 layers + decoder) of a batch of 2,048 test rows, inputs already
resident in HBM. Also reported: rows/s at batches of 1, 64 and 256; the attention kernel's share of the MFMA
roofline (measured with HIP events on the library's stream); and the oracle (the C restatement of the reference's
CPU path) timed on this host's cores on a bounded sample of the same workload.

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

ROWS, CHUNK, BATCH, CLASSES = 10000, 256, 2048, 10
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
    h_host = rng.standard_normal((BATCH, d)).astype(np.float32)
    h_dev = dm.DeviceBuffer.of(h_host)
    out_dev = dm.DeviceBuffer(BATCH * CLASSES * 4)
    timer = dm.EventTimer(gpu.stream)

    def run(n):
        gpu.in_context_dev(w, vm, h_dev.ptr, n, CLASSES, out_dev.ptr)

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
    log(f"in-context stage, {BATCH} rows: {ms_step:.3f} ms/step, {rows_s:,.0f} rows/s")

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
        log(f"in-context stage, {n} rows: {ms:.3f} ms, {per_batch[str(n)]:,.0f} rows/s")
    per_batch[str(BATCH)] = round(rows_s, 1)

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
        sample = 1024
        t0 = time.perf_counter()
        orc.in_context(model, scales, layers, abi.KV_F32, ROWS, CHUNK, h_host[:sample], CLASSES)
        secs = time.perf_counter() - t0
        cpu = {"value": round(sample / secs, 2), "unit": "rows/s", "cores": threads, "kind": "port",
               "sample": f"{sample} test rows through the in-context stage over the same 10,000-row f32 cache "
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
        "data": "synthetic: random-init full-size TabICL v2 classifier weights (seed 2), random row representations "
                "and a random stored f32 cache of the 10,000-row shape",
        "config": {"workload": "in-context stage (12 layers + decoder) of 2,048 test rows over a 10,000-row f32 "
                               "key/value cache, d=512, 8x64 heads, 10 classes",
                   "train_rows": ROWS, "chunk": CHUNK, "test_rows": BATCH, "classes": CLASSES, "kv": "f32"},
        "rows_per_s_by_batch": per_batch,
        "fit_s": None,
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": PEAK_F32_MFMA / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_F32_MFMA, 4), "traffic": None,
                     "kernel": "k_attn_mfma64 (+ split merge)", "ms_per_launch": round(att_ms, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    for b in (q_dev, att_dev, h_dev, out_dev):
        b.free()
    vm.free()
    w.free()
    gpu.close()


if __name__ == "__main__":
    main()
