"""Synthetic tables of the full-size workloads (seeded), and helpers that check a large fit on the card layer by
layer against the oracle from the card's own inputs to each layer, so that no comparison spans more than one
layer's arithmetic:

* 10k x 100: X ~ N(0, 1) (seed 3), 10 classes = argmax(X W + Gumbel) with W ~ N(0, 1) (seed 4) -- the table the
  benchmark predicts against;
* 50k x 200 regression: 150 N(0, 1) columns, 30 log-normal (sigma 1.5), 20 categorical codes 0..11, 10% of cells
  missing at random; target = a seeded random MLP of the filled cells + N(0, 0.1);
* 100k x 100, 120 classes: a seeded 120-component Gaussian mixture, the label is the component;
* 256 + 64 x 10 for the tiny architecture: X ~ N(0, 1) (seed 0), 3 classes = argmax(X W) with W ~ N(0, 1) (seed 1).
"""
import numpy as np

import oracle as orc
from conftest import pkg

abi, fit, planmod = pkg("abi"), pkg("fit"), pkg("plan")


def classification_table(rows, features=100, classes=10, seed_x=3, seed_w=4):
    rx = np.random.default_rng(seed_x)
    x = rx.standard_normal((rows, features)).astype(np.float32)
    rw = np.random.default_rng(seed_w)
    w = rw.standard_normal((features, classes))
    g = rw.gumbel(size=(rows, classes))
    return x, np.argmax(x.astype(np.float64) @ w + g, axis=1).astype(np.float32)


def tiny_table(train=256, test=64, features=10, classes=3, seed_x=0, seed_w=1):
    """(x_train, y_train, x_test) of the tiny workload: labels from the argmax of a seeded random projection."""
    x = np.random.default_rng(seed_x).standard_normal((train + test, features)).astype(np.float32)
    w = np.random.default_rng(seed_w).standard_normal((features, classes))
    y = np.argmax(x.astype(np.float64) @ w, axis=1).astype(np.float32)
    return x[:train], y[:train], x[train:]


def regression_table(rows, seed=7):
    rng = np.random.default_rng(seed)
    x = np.empty((rows, 200))
    x[:, :150] = rng.standard_normal((rows, 150))
    x[:, 150:180] = rng.lognormal(0.0, 1.5, (rows, 30))
    probs = rng.dirichlet(np.ones(12), 20)
    for j in range(20):
        x[:, 180 + j] = rng.choice(12, rows, p=probs[j])
    filled = x.copy()
    filled[:, 150:180] = np.log(filled[:, 150:180])
    w1 = rng.standard_normal((200, 32)) / np.sqrt(200)
    w2 = rng.standard_normal(32) / np.sqrt(32)
    y = np.tanh(filled @ w1) @ w2 * 10.0 + 50.0 + rng.normal(0.0, 0.1, rows)
    x[rng.random(x.shape) < 0.1] = np.nan
    return x, y


def mixture_table(rows, features=100, components=120, seed=6):
    rng = np.random.default_rng(seed)
    means = rng.standard_normal((components, features)) * 1.5
    # the component list fixed by the seed, the rows drawn from it with a seed of their own per use
    return means


def mixture_rows(means, rows, seed):
    rng = np.random.default_rng(seed)
    labels = rng.integers(0, means.shape[0], rows)
    x = (means[labels] + rng.standard_normal((rows, means.shape[1]))).astype(np.float32)
    return x, labels.astype(np.float32)


def record_rows(records, rows, chunk, d, sample):
    """Keys and values [len(sample)][2d] of the given rows from one layer's f32 chunk records."""
    rec = np.asarray(records).view(np.float32)
    out = np.empty((len(sample), 2 * d), np.float32)
    for i, r in enumerate(sample):
        ci, j = divmod(int(r), chunk)
        rc = min(chunk, rows - ci * chunk)
        c = rec[2 * d * chunk * ci:2 * d * chunk * ci + 2 * d * rc].reshape(2, d, rc)
        out[i, :d], out[i, d:] = c[0, :, j], c[1, :, j]
    return out


def check_layers(model, h_sample, layers, scales, rows, chunk, sample, tol, say):
    """Layer by layer for the sampled training rows: the oracle's keys and values from its copy of the rows' state
    against the card's stored f32 records, then the rows through the layer over the card's records (the fit's
    attention over all rows' exact keys and values). Returns the worst key/value difference."""
    h = np.ascontiguousarray(h_sample, np.float32)
    worst = 0.0
    for l in range(model.icl_layers):
        want = orc.kv_rows(model, l, h)
        got = record_rows(layers[l], rows, chunk, model.d, sample)
        err = float(np.abs(got - want).max())
        worst = max(worst, err)
        assert err < tol, f"layer {l}: keys/values differ by {err:.2e}"
        if l + 1 < model.icl_layers:
            h = orc.icl_step(model, l, scales[l], layers[l], abi.KV_F32, rows, chunk, h)
    say(f"  in-context keys/values, {len(sample)} sampled rows x {model.icl_layers} layers: worst {worst:.2e}")
    return worst


def fit_pieces(gpu, w, m, x, y, classes, chunk, kv_format):
    """`fit.fit_raw` for a one-problem member, keeping what the checks need: (plan, col_kv, reps, h, scales,
    layers)."""
    plan = planmod.Plan.new(m.max_classes, y, classes)
    assert len(plan.nodes) == 1
    rows = x.shape[0]
    ind_scales = np.stack([fit.query_scale(b, rows) for b in m.col_a1])
    col_kv, reps = gpu.fit_represent(w, x, y, plan.bases, ind_scales)
    h = reps.copy()
    m.add_y(m.t["icl_y"], np.asarray(plan.nodes[0].y, np.float32), h)
    scales = np.stack([fit.query_scale(b, rows) for b in m.icl]).astype(np.float32)
    layers = []
    gpu.in_context_fit(w, h, scales, kv_format, chunk, lambda l, rec: layers.append(rec.copy()))
    return plan, col_kv, reps, h, scales, layers


def fitted_of(plan, col_kv, scales, layers, rows, features, classes, chunk, kv_format):
    return orc.Fitted(rows, features, classes, chunk, kv_format, plan, col_kv, [scales], [layers])
