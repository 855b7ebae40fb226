"""Whole-table flows around the hot path, shared by the oracle and card tests of the reference's golden tables
(`tests/reference.rs:141-326`): a classifier ensemble from a fixture's own preprocessed tables and member settings,
and a regressor ensemble from raw rows (preprocessing restated in oracle/prep.py). `fit_predict(xs, ys, classes,
xt)` is the member-level work under test: the oracle's or the card's fit followed by prediction."""
import os

import numpy as np

import prep as P
from conftest import GOLDEN, pkg

B, T = pkg("bundle"), pkg("table")

# tests/reference.rs:226-230 and 310-318: 16-bit weights move a probability by at most 7e-4 on these tables and a
# regression answer by at most 0.35% of the targets' spread, so 5e-3 and 1% there; the tiny model runs at full
# precision on both sides (1e-5)
HALF_PROBA = 5e-3
HALF_REGRESSION = 0.01
TINY = 1e-5


def fixture(name: str):
    return B.Bundle.open(os.path.join(GOLDEN, f"{name}.tirs"))


def half_weights(kind: str):
    """The reference's published weights at 16-bit precision (`classifier` or `regressor`), joined from parts."""
    return B.join_parts(os.path.join(GOLDEN, "weights", f"{kind}-v2-half.json"))


def table(fx, name):
    e = fx.entry(name)
    return fx.f64s(name).reshape(e.dims)


def members(fx):
    out = []
    i = 0
    while fx.has(f"member{i}_method"):
        norm = 1 if fx.bytes(f"member{i}_method") == b"power" else 0
        out.append(T.Member(norm, fx.i32s(f"member{i}_features").tolist(), fx.i32s(f"member{i}_classes").tolist()))
        i += 1
    return out


def ensemble_proba(fx, fit_predict):
    """`Classifier::predict_proba` over the fixture's preprocessed tables and member list (`src/table.rs:242-272`,
    temperature 0.9)."""
    y, labels = T.encode_labels(fx.i32s("y_train"))
    classes = len(labels)
    names = {0: "none", 1: "power"}
    train = {v: table(fx, f"train_{names[v]}") for v in (0, 1) if fx.has(f"train_{names[v]}")}
    test = {v: table(fx, f"test_{names[v]}") for v in (0, 1) if fx.has(f"test_{names[v]}")}
    ms = members(fx)
    nt = next(iter(test.values())).shape[0]
    avg = np.zeros((nt, classes))
    for mb in ms:
        xs, ys = T.member_inputs(train[mb.norm], mb, y)
        xt = T.member_inputs(test[mb.norm], mb)
        T.add_logits(avg, fit_predict(xs, ys, classes, xt), mb)
    return T.finish_proba(avg, len(ms), 0.9)


def _seq(a) -> float:
    """A float64 sum left to right (Rust's `iter().sum::<f64>()`)."""
    a = np.asarray(a, np.float64)
    return float(np.add.accumulate(a)[-1]) if a.size else 0.0


def ensemble_regression(fx, n_members: int, outputs: int, fit_predict, gpu=None) -> dict:
    """`fit_regressor` then `Regressor::predict` (`src/table.rs:372-496`) from the fixture's raw rows: targets narrowed
    to float32 and standardised, the table preprocessed (plain and power variants, threshold 4), the ensemble's
    members (seed 42) fitted on the standardised targets, each test row's quantiles read as a distribution, members
    averaged. With `gpu`, the distributions are read on the card (`tah_quantile_stats`)."""
    x, y, xt = table(fx, "x_train"), fx.f64s("y_train"), table(fx, "x_test")
    alphas = fx.f64s("alphas")
    n = len(y)
    y32 = y.astype(np.float32).astype(np.float64)
    ym = _seq(y32) / n
    var = _seq((y32 - ym) * (y32 - ym)) / n
    ys = 1.0 if np.sqrt(var) < 10 * np.finfo(np.float64).eps else float(np.sqrt(var))
    prep, tables = P.Prep.fit(x, (False, True), 4.0)
    ms = P.ensemble(len(prep.keep), 1, 2, n_members, 42)
    yz = ((y32 - ym) / ys).astype(np.float32)
    variants = [prep.apply(v, xt) for v in range(len(prep.power))]
    nt = xt.shape[0]
    out = dict(mean=np.zeros(nt), variance=np.zeros(nt), median=np.zeros(nt), quantiles=np.zeros((nt, len(alphas))))
    for mb in ms:
        xs = np.ascontiguousarray(tables[mb.norm][:, mb.features].astype(np.float32))
        xq = np.ascontiguousarray(variants[mb.norm][:, mb.features].astype(np.float32))
        q = fit_predict(xs, yz, outputs, xq)
        T.add_regression(out, q, alphas, ym, ys, gpu=gpu)
    for k in out:
        out[k] /= len(ms)
    return out


def regression_errors(fx, got: dict, tol: float):
    """Worst difference per output against the fixture, and the bar (`tol` of the targets' spread about 50, the
    variance only at full precision: tests/reference.rs:286-296)."""
    yt = fx.f64s("y_test")
    spread = float(np.sqrt(np.mean((yt - 50.0) ** 2)))
    res = {}
    for kind in ("mean", "variance", "median", "quantiles"):
        want = fx.f64s(kind).reshape(got[kind].shape)
        res[kind] = (float(np.abs(got[kind] - want).max()), kind != "variance" or tol < 1e-3)
    return res, tol * spread


def card_fit_predict(gpu, w, kv_format=None):
    """The member-level work on the card: `fit.fit_raw` then prediction through every in-context problem (the class
    tree's nodes walked on the host for more classes than the model's limit)."""
    hip, fit, abi, planmod = pkg("hip"), pkg("fit"), pkg("abi"), pkg("plan")
    fmt = abi.KV_F32 if kv_format is None else kv_format

    def run(xs, ys, classes, xt):
        f = fit.fit_raw(gpu, w, xs, ys, classes, kv_format=fmt)
        vms = [gpu.load(w, f.kv_format, node.rows, f.chunk, f.layers[i], f.scales[i]) for i, node in enumerate(f.nodes)]
        vms[0].set_columns(f.col_kv, f.features, f.digits)
        if len(vms) == 1 and f.digits == 1:
            out = gpu.predict(w, vms[0], xt, classes)
        else:
            rep = gpu.represent(w, gpu.embed(w, vms[0], xt))
            outs = [gpu.in_context(w, vm, rep, node.k) for vm, node in zip(vms, f.nodes)]
            out = outs[0] if len(outs) == 1 else planmod.tree_scores(f.nodes, outs, classes)
        for vm in vms:
            vm.free()
        return out

    return run
