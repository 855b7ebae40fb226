"""Whole ensembles against the reference's golden probabilities (tests/reference.rs:164-244): tiny-one (1 member),
tiny-table (8 members, both normalisations) and tiny-many (14 classes on a 10-class model: label digits and a class
tree), from the fixtures' own preprocessed tables and member settings, at 1e-5. The oracle runs everywhere; the card
runs them in the gpu-marked test."""
import os

import numpy as np
import pytest

import oracle as orc
from conftest import GOLDEN, pkg

B, T, M, abi = pkg("bundle"), pkg("table"), pkg("model"), pkg("abi")
planmod = pkg("plan")


def members(fx):
    out = []
    i = 0
    while fx.has(f"member{i}_method"):
        norm = 1 if fx.bytes(f"member{i}_method") == b"power" else 0
        out.append(T.Member(norm, fx.i32s(f"member{i}_features").tolist(), fx.i32s(f"member{i}_classes").tolist()))
        i += 1
    return out


def tables(fx, which):
    name = {0: "none", 1: "power"}
    return {v: fx.f64s(f"{which}_{name[v]}").reshape(-1, fx.entry(f"{which}_{name[v]}").dims[1])
            for v in (0, 1) if fx.has(f"{which}_{name[v]}")}


def ensemble_proba(fx, fit_predict):
    y = fx.i32s("y_train")
    classes = int(y.max()) + 1
    train, test = tables(fx, "train"), tables(fx, "test")
    ms = members(fx)
    nt = next(iter(test.values())).shape[0]
    avg = np.zeros((nt, classes))
    for mb in ms:
        xs, ys = T.member_inputs(train[mb.norm], mb, y)
        xt = T.member_inputs(test[mb.norm], mb)
        T.add_logits(avg, fit_predict(xs, ys, classes, xt), mb)
    return T.finish_proba(avg, len(ms), 0.9)


@pytest.mark.parametrize("name", ["tiny-one", "tiny-table", "tiny-many"])
def test_oracle_ensemble_matches_reference(tiny_model, name):
    fx = B.Bundle.open(os.path.join(GOLDEN, f"{name}.tirs"))

    def fit_predict(xs, ys, classes, xt):
        return orc.predict_raw(tiny_model, orc.fit_raw(tiny_model, xs, ys, classes), xt)

    proba = ensemble_proba(fx, fit_predict)
    assert np.abs(proba - fx.f64s("proba").reshape(proba.shape)).max() < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny-one", "tiny-table", "tiny-many"])
def test_card_ensemble_matches_reference(tiny_model, name):
    hip, fit = pkg("hip"), pkg("fit")
    fx = B.Bundle.open(os.path.join(GOLDEN, f"{name}.tirs"))
    gpu = hip.Gpu(0)
    w = gpu.weights(tiny_model)

    def fit_predict(xs, ys, classes, xt):
        f = fit.fit_raw(gpu, w, xs, ys, classes)
        vms = [gpu.load(w, f.kv_format, node.rows, f.chunk, f.layers[i], f.scales[i]) for i, node in enumerate(f.nodes)]
        vms[0].set_columns(f.col_kv, f.features, f.digits)
        if len(vms) == 1:
            return gpu.predict(w, vms[0], xt, classes)
        rep = gpu.represent(w, gpu.embed(w, vms[0], xt))
        outs = [gpu.in_context(w, vm, rep, node.k) for vm, node in zip(vms, f.nodes)]
        return planmod.tree_scores(f.nodes, outs, classes)

    proba = ensemble_proba(fx, fit_predict)
    gpu.close()
    assert np.abs(proba - fx.f64s("proba").reshape(proba.shape)).max() < 1e-5


def test_quantile_dist_closed_forms():
    """QuantileDist on quantiles of a known distribution: the median is the middle quantile, icdf is linear between
    levels and monotone, the tails continue the ends, and mean/variance are the sample moments of the quantiles."""
    q = np.linspace(-3.0, 5.0, 99).astype(np.float32)[::-1].copy()  # unsorted on purpose
    d = T.QuantileDist(q)
    assert np.array_equal(d.q, np.sort(q))
    assert abs(d.icdf(0.5) - 1.0) < 1e-5
    assert abs(d.mean() - 1.0) < 1e-5
    assert abs(d.variance() - np.var(np.sort(q).astype(np.float64), ddof=1)) < 1e-3
    # between levels i/100 and (i+1)/100 the quantile moves linearly
    assert abs(d.icdf(0.105) - (d.q[9] + 0.5 * (d.q[10] - d.q[9]))) < 1e-4
    xs = [d.icdf(a) for a in np.linspace(0.001, 0.999, 200)]
    assert all(b >= a - 1e-6 for a, b in zip(xs, xs[1:]))
    assert d.icdf(0.001) < d.q[0] and d.icdf(0.999) > d.q[-1]
