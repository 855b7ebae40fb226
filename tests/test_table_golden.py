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
    y, labels = T.encode_labels(fx.i32s("y_train"))
    classes = len(labels)
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


def planted_tails(n: int, a: float, b: float, c: float, d: float):
    """Quantiles at levels i/(n+1) whose first k and last k values (k = clamp(n/4, 1, 20)) lie on a ln(level) + b and
    -c ln(1 - level) + d, except that the k-th from either end is moved off its line; the middle is monotone. Returns
    the quantiles and the least-squares slopes of exactly the k end points on each side (np.polyfit in float64): a
    window one point shorter or longer gives another slope."""
    lv = np.arange(1, n + 1, dtype=np.float64) / (n + 1)
    k = max(min(20, n // 4), 1)
    q = np.linspace(a * np.log(lv[k - 1]) + b, -c * np.log(1 - lv[n - k]) + d, n)
    q[:k] = a * np.log(lv[:k]) + b
    q[n - k:] = -c * np.log(1 - lv[n - k:]) + d
    if k > 2:
        q[k - 1] += 0.25 * (q[k - 1] - q[k - 2])
        q[n - k] -= 0.25 * (q[n - k + 1] - q[n - k])
    q = q.astype(np.float32)
    ql = q.astype(np.float64)
    lv32 = (np.arange(1, n + 1, dtype=np.float32) / np.float32(n + 1)).astype(np.float64)
    sl = abs(np.polyfit(np.log(lv32[:k]), ql[:k], 1)[0])
    sr = abs(np.polyfit(np.log(1 - lv32[n - k:]), ql[n - k:], 1)[0])
    return q, (min(max(sl, 0.01), 100.0), min(max(sr, 0.01), 100.0))


TAIL_CASES = [  # n, a, b, c, d
    (999, 2.0, 1.0, 3.0, 40.0),     # k = 20
    (99, 0.5, -3.0, 1.25, 7.0),     # k = 20
    (40, 1.5, 0.0, 0.75, 2.0),      # k = 10: n / 4
    (999, 500.0, 0.0, 1e-4, 0.0),   # slopes clamped to [0.01, 100]
]


@pytest.mark.parametrize("n,a,b,c,d", TAIL_CASES)
def test_quantile_dist_planted_tails(n, a, b, c, d):
    """The exponential tails beyond the first and last level are least-squares lines through exactly the first and
    last k points, pinned at the end quantiles (`src/table.rs:300-316`): icdf far out in either tail follows
    slope * ln(level) from the end point. A wrong window, sign or intercept moves these by far more than the bound."""
    q, (sl, sr) = planted_tails(n, a, b, c, d)
    dist = T.QuantileDist(q)
    lv0, lvn = 1.0 / (n + 1), n / (n + 1)
    for alpha in (1e-5, 1e-4, 0.3 * lv0):
        want = float(q[0]) + sl * (np.log(alpha) - np.log(lv0))
        assert abs(float(dist.icdf(alpha)) - want) < 2e-4 * max(1.0, abs(want)), (alpha, dist.icdf(alpha), want)
    for alpha in (1 - 1e-5, 1 - 1e-4, 1 - 0.3 * (1 - lvn)):
        want = float(q[-1]) - sr * (np.log(1 - alpha) - np.log(1 - lvn))
        assert abs(float(dist.icdf(alpha)) - want) < 2e-4 * max(1.0, abs(want)), (alpha, dist.icdf(alpha), want)


def test_quantile_dist_one_point_tails():
    """Below 8 quantiles k is 1: one point has no spread, the slope falls to its floor 0.01, and the tails leave
    the end quantiles at that slope."""
    q = np.array([1.0, 2.0, 4.0, 8.0, 9.0], np.float32)
    dist = T.QuantileDist(q)
    lv0, lvn = 1.0 / 6.0, 5.0 / 6.0
    assert abs(float(dist.icdf(1e-3)) - (1.0 + 0.01 * (np.log(1e-3) - np.log(lv0)))) < 1e-5
    assert abs(float(dist.icdf(1 - 1e-3)) - (9.0 - 0.01 * (np.log(1e-3) - np.log(1 - lvn)))) < 1e-5
