"""The full-size workloads on the card, each checked against the oracle at the stated tolerances (absolute: 5e-5 for
cached keys/values and raw scores; 1e-5 for probabilities over the same caches), layer by layer where a whole-fit
comparison would span twelve layers of rounding:

* 10,000 x 100, 10 classes, f32, 1 member: the column cache of three feature groups against the oracle's column
  stage over all rows; sampled rows' representations from the card's column cache; every layer's keys and values of
  64 sampled training rows, each layer recomputed from the card's records of the layer before; all 2,048
  predictions against the oracle over the card's caches (scores and probabilities).
* The same table, 8 members (feature orders and class shifts, both normalisations) with i16 and i8 caches: each
  quantised build bit for bit the quantiser applied to the card's f32 build; ensemble probabilities of 2,048 rows,
  128 against the oracle over the same caches; the quantised caches' probabilities against the f32 ones.
* 50,000 x 200 regression table (skewed, categorical and missing cells, preprocessed), 8 members, f32 cache:
  per-layer and representation checks on one member, raw outputs and quantile statistics of 32 sampled rows of
  every member against the oracle.
* 100,000 x 100, 120 classes (label digits [5, 5, 5], a 31-node class tree), i16 cache, then 2,048 predictions with
  a 256 MB working-memory budget: the plan, 32 sampled rows' representations and scores against the oracle over
  the card's caches; the budgeted answers equal the unbudgeted ones.
"""
import sys
import time

import numpy as np
import pytest

import oracle as orc
import prep as P
import workloads as W
from conftest import pkg

abi, hip, M, fit, T = pkg("abi"), pkg("hip"), pkg("model"), pkg("fit"), pkg("table")
planmod = pkg("plan")
pytestmark = pytest.mark.gpu

KV_TOL = 5e-5      # cached keys and values, raw scores
PROBA_TOL = 1e-5   # probabilities from the same caches


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpu():
    g = hip.Gpu(0)
    say("device:", g.name)
    yield g
    g.close()


@pytest.fixture(scope="module")
def clf():
    return M.Model.random(M.FULL_CLASSIFIER, seed=2)


def check_representations(m, col_kv, reps, bases, x, y, sample):
    """Sampled training rows' representations: the oracle's cells from the card's column cache, then its row stage."""
    emb = orc.fit_cells_rows(m, col_kv, bases, x[sample], y[sample])
    want = orc.fit_rows(m, emb)
    err = float(np.abs(reps[sample] - want).max())
    say(f"  representations of {len(sample)} sampled rows: worst {err:.2e}")
    assert err < KV_TOL


def test_config2_fit_and_predict_10k(gpu, clf):
    m = clf
    rows, features, classes, chunk, nt = 10000, 100, 10, 256, 2048
    x_all, y_all = W.classification_table(rows + nt, features, classes)
    x, y, xt = x_all[:rows], y_all[:rows], x_all[rows:]
    say(f"config 2: fit {rows} x {features} on the card (f32), predict {nt}")
    w = gpu.weights(m)
    t0 = time.perf_counter()
    plan, col_kv, reps, h, scales, layers = W.fit_pieces(gpu, w, m, x, y, classes, chunk, abi.KV_F32)
    say(f"  card fit {time.perf_counter() - t0:.2f} s")
    # the column cache of three groups against the oracle's column stage over all rows
    groups = [0, 37, 99]
    t0 = time.perf_counter()
    want_col, _ = orc.fit_columns_of(m, x, y, groups, plan.bases, chunk)
    err = float(np.abs(col_kv[groups] - want_col).max())
    say(f"  column cache of groups {groups}: worst {err:.2e} (oracle {time.perf_counter() - t0:.1f} s)")
    assert err < KV_TOL
    rng = np.random.default_rng(22)
    sample = np.sort(rng.choice(rows, 64, replace=False))
    check_representations(m, col_kv, reps, plan.bases, x, y, sample)
    assert np.abs(scales - np.stack([orc.query_scale(b, rows) for b in m.icl])).max() <= 2e-7 * np.abs(scales).max()
    W.check_layers(m, h[sample], layers, scales, rows, chunk, sample, KV_TOL, say)
    # 2,048 predictions against the fitted caches, every one of them through the oracle
    vm = gpu.load(w, abi.KV_F32, rows, chunk, layers, scales)
    vm.set_columns(col_kv, features, 1)
    got = gpu.predict(w, vm, xt, classes)
    t0 = time.perf_counter()
    want = orc.predict_raw(m, W.fitted_of(plan, col_kv, scales, layers, rows, features, classes, chunk, abi.KV_F32),
                           xt)
    err = float(np.abs(got - want).max())
    p_err = float(np.abs(T.finish_proba(got.astype(np.float64), 1, 0.9)
                         - T.finish_proba(want.astype(np.float64), 1, 0.9)).max())
    say(f"  scores of all {nt} predicted rows: worst {err:.2e}; probabilities worst {p_err:.2e} "
        f"(oracle {time.perf_counter() - t0:.1f} s)")
    assert err < KV_TOL and p_err < PROBA_TOL and np.isfinite(got).all()
    vm.free()
    w.free()


def test_config3_ensemble_i16_i8(gpu, clf):
    m = clf
    rows, features, classes, chunk, nt = 10000, 100, 10, 256, 2048
    x_all, y_all = W.classification_table(rows + nt, features, classes)
    prep, tables = P.Prep.fit(x_all[:rows].astype(np.float64))
    variants = [prep.apply(v, x_all[rows:].astype(np.float64)) for v in range(2)]
    members = P.ensemble(len(prep.keep), classes, 2, 8, 42)
    y = y_all[:rows].astype(np.int64)
    say(f"config 3: {len(members)} members, i16 and i8 caches, {nt} rows")
    w = gpu.weights(m)
    rng = np.random.default_rng(33)
    ts = np.sort(rng.choice(nt, 128, replace=False))
    sums = {fmt: np.zeros((nt, classes)) for fmt in (abi.KV_F32, abi.KV_I16, abi.KV_I8)}
    want_sums = {fmt: np.zeros((len(ts), classes)) for fmt in (abi.KV_I16, abi.KV_I8)}
    for i, mb in enumerate(members):
        xs, ys = T.member_inputs(tables[mb.norm], T.Member(mb.norm, mb.features, mb.classes), y)
        xq = T.member_inputs(variants[mb.norm], T.Member(mb.norm, mb.features, mb.classes))
        f32 = None
        for fmt in (abi.KV_F32, abi.KV_I16, abi.KV_I8):
            f = fit.fit_raw(gpu, w, xs, ys, classes, chunk, fmt)
            if fmt == abi.KV_F32:
                f32 = f
            elif i == 0:
                # the card's quantised build is the quantiser applied to its own f32 build, bit for bit
                for l in range(m.icl_layers):
                    rec = f32.layers[0][l].view(np.float32)
                    want = np.concatenate([orc.pack(rec[2 * m.d * c0:2 * m.d * (c0 + min(chunk, rows - c0))], m.d,
                                                    min(chunk, rows - c0), fmt) for c0 in range(0, rows, chunk)])
                    assert np.array_equal(f.layers[0][l], want), f"member 0, format {fmt}, layer {l}"
            vm = gpu.load(w, fmt, rows, chunk, f.layers[0], f.scales[0])
            vm.set_columns(f.col_kv, features, 1)
            T.add_logits(sums[fmt], gpu.predict(w, vm, xq, classes), T.Member(mb.norm, mb.features, mb.classes))
            vm.free()
            if fmt != abi.KV_F32:
                fo = orc.Fitted(rows, features, classes, chunk, fmt, f.plan, f.col_kv, f.scales, f.layers)
                T.add_logits(want_sums[fmt], orc.predict_raw(m, fo, xq[ts]),
                             T.Member(mb.norm, mb.features, mb.classes))
        say(f"  member {i} fitted and predicted in three formats")
    proba = {fmt: T.finish_proba(s, len(members), 0.9) for fmt, s in sums.items()}
    for fmt, name, bound in ((abi.KV_I16, "i16", 1e-4), (abi.KV_I8, "i8", 1e-2)):
        want = T.finish_proba(want_sums[fmt], len(members), 0.9)
        err = float(np.abs(proba[fmt][ts] - want).max())
        drift = float(np.abs(proba[fmt] - proba[abi.KV_F32]).max())
        say(f"  {name}: probabilities against the oracle over the same caches {err:.2e}; against f32 {drift:.2e}")
        assert err < PROBA_TOL
        assert drift < bound  # the reference's own bounds for its quantised caches (tests/pipeline.rs:137-156)
    w.free()


def test_config4_regression_50k(gpu):
    m = M.Model.random(M.FULL_REGRESSOR, seed=5)
    rows, nt, chunk = 50000, 2048, 256
    x_all, y_all = W.regression_table(rows + nt)
    x, yv, xt = x_all[:rows], y_all[:rows], x_all[rows:]
    say(f"config 4: regression {rows} x {x.shape[1]} (skewed, categorical, 10% missing), 8 members, {nt} rows")
    y32 = yv.astype(np.float32).astype(np.float64)
    ym = float(np.add.accumulate(y32)[-1]) / rows
    ys = float(np.sqrt(np.add.accumulate((y32 - ym) ** 2)[-1] / rows))
    yz = ((y32 - ym) / ys).astype(np.float32)
    prep, tables = P.Prep.fit(x)
    variants = [prep.apply(v, xt) for v in range(2)]
    members = P.ensemble(len(prep.keep), 1, 2, 8, 42)
    w = gpu.weights(m)
    rng = np.random.default_rng(44)
    ts = np.sort(rng.choice(nt, 32, replace=False))
    alphas = np.array([0.05, 0.95])
    out = dict(mean=np.zeros(nt), variance=np.zeros(nt), median=np.zeros(nt), quantiles=np.zeros((nt, 2)))
    for i, mb in enumerate(members):
        xs = np.ascontiguousarray(tables[mb.norm][:, mb.features].astype(np.float32))
        xq = np.ascontiguousarray(variants[mb.norm][:, mb.features].astype(np.float32))
        t0 = time.perf_counter()
        plan, col_kv, reps, h, scales, layers = W.fit_pieces(gpu, w, m, xs, yz, m.outputs, chunk, abi.KV_F32)
        say(f"  member {i}: card fit {time.perf_counter() - t0:.2f} s")
        if i == 0:
            sample = np.sort(rng.choice(rows, 32, replace=False))
            check_representations(m, col_kv, reps, plan.bases, xs, yz, sample)
            W.check_layers(m, h[sample], layers, scales, rows, chunk, sample, KV_TOL, say)
        vm = gpu.load(w, abi.KV_F32, rows, chunk, layers, scales)
        vm.set_columns(col_kv, xs.shape[1], 1)
        q = gpu.predict(w, vm, xq, m.outputs)
        vm.free()
        fo = W.fitted_of(plan, col_kv, scales, layers, rows, xs.shape[1], m.outputs, chunk, abi.KV_F32)
        want = orc.predict_raw(m, fo, xq[ts])
        err = float(np.abs(q[ts] - want).max())
        # the distributions read on the card from its outputs, against the host statement on the oracle's outputs
        st = gpu.quantile_stats(q[ts], alphas.astype(np.float32))
        host = np.array([[d.mean(), d.variance(), d.icdf(0.5)] + [d.icdf(a) for a in alphas]
                         for d in map(T.QuantileDist, want)])
        serr = float(np.abs(st - host).max())
        say(f"  member {i}: raw outputs of 32 sampled rows {err:.2e}, their statistics {serr:.2e}")
        assert err < KV_TOL and serr < KV_TOL
        T.add_regression(out, q, alphas, ym, ys, gpu=gpu)
        del layers
    for k in out:
        out[k] /= len(members)
    assert all(np.isfinite(v).all() for v in out.values())
    q05, q95 = out["quantiles"][:, 0], out["quantiles"][:, 1]
    assert (q05 <= out["median"] + 1e-9).all() and (out["median"] <= q95 + 1e-9).all()
    say(f"  mean of predicted means {out['mean'].mean():.3f} (targets {yv.mean():.3f})")
    w.free()


def test_config5_many_classes_100k(gpu, clf):
    m = clf
    rows, features, classes, chunk, nt = 100000, 100, 120, 256, 2048
    means = W.mixture_table(rows)
    x, y = W.mixture_rows(means, rows, seed=61)
    xt, _ = W.mixture_rows(means, nt, seed=62)
    say(f"config 5: {rows} x {features}, {classes} classes, i16 cache, {nt} rows with a 256 MB budget")
    w = gpu.weights(m)
    t0 = time.perf_counter()
    f = fit.fit_raw(gpu, w, x, y, classes, chunk, abi.KV_I16)
    say(f"  card fit {time.perf_counter() - t0:.2f} s")
    # the plan: three label digits of base 5; a root of 10 groups of 12 classes, each split in two leaves of 6
    assert f.plan.bases == [5, 5, 5] and len(f.nodes) == 31
    assert f.nodes[0].k == 10 and not f.nodes[0].leaf
    assert sorted(n.k for n in f.nodes[1:] if not n.leaf) == [2] * 10
    assert sorted(n.k for n in f.nodes if n.leaf) == [6] * 20
    assert sorted(c for n in f.nodes if n.leaf for c in n.map) == list(range(classes))
    vms = [gpu.load(w, abi.KV_I16, node.rows, chunk, f.layers[i], f.scales[i]) for i, node in enumerate(f.nodes)]
    vms[0].set_columns(f.col_kv, features, f.digits)

    def predict():
        rep = gpu.represent(w, gpu.embed(w, vms[0], xt))
        outs = [gpu.in_context(w, vm, rep, node.k) for vm, node in zip(vms, f.nodes)]
        return planmod.tree_scores(f.nodes, outs, classes), rep

    whole, rep = predict()
    old = gpu.work_budget()
    try:
        gpu.release()
        gpu.set_work_budget(256 << 20)
        budgeted, _ = predict()
        peak = gpu.working()[1]
    finally:
        gpu.set_work_budget(old)
    say(f"  256 MB budget: peak working memory {peak / 2**20:.0f} MiB; largest change {np.abs(budgeted - whole).max():.2e}")
    assert peak <= 256 << 20 and gpu.overdrawn() == 0
    assert np.abs(budgeted - whole).max() < 1e-5
    rng = np.random.default_rng(55)
    ts = np.sort(rng.choice(nt, 32, replace=False))
    fo = orc.Fitted(rows, features, classes, chunk, abi.KV_I16, f.plan, f.col_kv, f.scales, f.layers)
    t0 = time.perf_counter()
    want_rep = orc.represent(m, orc.embed(m, fo, xt[ts]))
    err_rep = float(np.abs(rep[ts] - want_rep).max())
    want = orc.predict_raw(m, fo, xt[ts])
    err = float(np.abs(whole[ts] - want).max())
    say(f"  32 sampled rows: representations {err_rep:.2e}, scores {err:.2e} (oracle {time.perf_counter() - t0:.1f} s)")
    assert err_rep < KV_TOL and err < KV_TOL
    acc = float(np.mean(np.argmax(whole, axis=1) == W.mixture_rows(means, nt, seed=62)[1]))
    say(f"  accuracy on the mixture's test rows {acc:.3f}")
    for vm in vms:
        vm.free()
    w.free()
