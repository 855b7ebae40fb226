"""A whole fit on the card (column, row and in-context stages: fit::Attend's columns, rows and in_context) against
the oracle and the reference's golden caches, including label digits with a class tree and a regression model."""
import os
import sys

import numpy as np
import pytest

import oracle as orc
from conftest import GOLDEN, pkg, to_ours

abi, hip, M, fit, B = pkg("abi"), pkg("hip"), pkg("model"), pkg("fit"), pkg("bundle")
planmod = pkg("plan")
pytestmark = pytest.mark.gpu
TOL = 5e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpu():
    g = hip.Gpu(0)
    yield g
    g.close()


def node_outputs_card(gpu, w, fitted, x):
    """Each class-tree node's raw outputs from the card: the column and row stages, then every node's in-context
    stage (src/predict.rs:661-693 before the walk)."""
    vms = [gpu.load(w, fitted.kv_format, node.rows, fitted.chunk, fitted.layers[i], fitted.scales[i])
           for i, node in enumerate(fitted.nodes)]
    vms[0].set_columns(fitted.col_kv, fitted.features, fitted.digits)
    rep = gpu.represent(w, gpu.embed(w, vms[0], x))
    outs = [gpu.in_context(w, vm, rep, node.k) for vm, node in zip(vms, fitted.nodes)]
    for vm in vms:
        vm.free()
    return outs


def node_outputs_oracle(m, fitted, x):
    rep = orc.represent(m, orc.embed(m, fitted, x))
    return [orc.in_context(m, fitted.scales[ni], fitted.layers[ni], fitted.kv_format, node.rows, fitted.chunk, rep,
                           node.k) for ni, node in enumerate(fitted.nodes)]


def tree_proba(nodes, outs, classes):
    """The class probabilities the tree walk multiplies out (before the reference's 0.9 ln(p + 1e-6) scores)."""
    return (np.exp(planmod.tree_scores(nodes, outs, classes).astype(np.float64) / 0.9) - 1e-6).clip(0.0)


def predict_card(gpu, w, fitted, x):
    """Scores from the card for a fitted member: all three stages for one problem, or the column and row stages
    then each problem's in-context stage and the tree walk (src/predict.rs:661-693)."""
    if len(fitted.nodes) > 1:
        return planmod.tree_scores(fitted.nodes, node_outputs_card(gpu, w, fitted, x), fitted.classes)
    vm = gpu.load(w, fitted.kv_format, fitted.nodes[0].rows, fitted.chunk, fitted.layers[0], fitted.scales[0])
    vm.set_columns(fitted.col_kv, fitted.features, fitted.digits)
    out = gpu.predict(w, vm, x, fitted.classes)
    vm.free()
    return out


def test_fit_tiny_matches_reference(gpu, tiny_model, tiny_raw):
    """Every cached number of the golden tiny fit (tests/reference.rs:42-89) and its scores, fitted on the card."""
    m = tiny_model
    x = tiny_raw.f32s("x_train").reshape(120, 7)
    y = tiny_raw.i32s("y_train").astype(np.float32)
    w = gpu.weights(m)
    f = fit.fit_raw(gpu, w, x, y, 3, chunk=48)
    for b in range(len(m.col_a2)):
        for which, kind in enumerate(["col_k", "col_v"]):
            r = tiny_raw.f32s(f"{kind}{b}").reshape(m.cls + 7, -1)
            for g in range(7):
                want = to_ours(r[g + m.cls], m.col_heads, m.inds, m.e // m.col_heads)
                assert np.abs(f.col_kv[g, 0, b, which] - want).max() < TOL, (kind, b, g)
    d = m.d
    for l in range(m.icl_layers):
        got = f.layers[0][l].view(np.float32)
        for which, kind in enumerate(["icl_k", "icl_v"]):
            want = to_ours(tiny_raw.f32s(f"{kind}{l}"), m.icl_heads, 120, d // m.icl_heads)
            for c0 in range(0, 120, 48):
                rc = min(48, 120 - c0)
                c = got[2 * d * c0:2 * d * (c0 + rc)].reshape(2, d, rc)[which]
                assert np.abs(c - want[:, c0:c0 + rc]).max() < 2.5 * TOL
    scores = predict_card(gpu, w, f, tiny_raw.f32s("x_test").reshape(16, 7))
    assert np.abs(scores - tiny_raw.f32s("logits").reshape(16, 3)).max() < TOL


def compare_fits(got, want, kv_format):
    """Two fits of a small model (two in-context layers) compared whole, at the absolute tolerance."""
    assert got.plan.bases == want.plan.bases and len(got.layers) == len(want.layers)
    err = np.abs(got.col_kv - want.col_kv).max()
    say("  column cache worst", err)
    assert err < TOL, err
    for ni in range(len(want.layers)):
        assert np.abs(got.scales[ni] - want.scales[ni]).max() <= 2e-7 * max(1.0, np.abs(want.scales[ni]).max())
        for l in range(len(want.layers[ni])):
            if kv_format == abi.KV_F32:
                a, b = got.layers[ni][l].view(np.float32), want.layers[ni][l].view(np.float32)
                say(f"  node {ni} layer {l} keys/values worst", np.abs(a - b).max())
                assert np.abs(a - b).max() < TOL, (ni, l)


def test_fit_many_classes_with_label_digits(gpu, tiny_model):
    """14 classes on a 10-class model: label digits [4, 4] in the column stage and a three-node class tree
    (src/fit.rs:159-215, src/predict.rs:661-693), fitted and predicted on the card."""
    m = tiny_model
    rng = np.random.default_rng(14)
    x = rng.standard_normal((200, 6)).astype(np.float32)
    y = (np.arange(200) % 14).astype(np.float32)
    rng.shuffle(y)
    w = gpu.weights(m)
    got = fit.fit_raw(gpu, w, x, y, 14, chunk=32)
    want = orc.fit_raw(m, x, y, 14, chunk=32)
    assert got.plan.bases == [4, 4] and len(got.plan.nodes) == 3
    compare_fits(got, want, abi.KV_F32)
    xt = rng.standard_normal((20, 6)).astype(np.float32)
    # each node's raw scores from the card's caches against the oracle's over its own fit, absolutely; then the
    # probabilities the tree multiplies out at the probability tolerance (the final 0.9 ln(p + 1e-6) scores magnify
    # differences of small probabilities by 1/p, so they are compared as probabilities)
    o_card = node_outputs_card(gpu, w, got, xt)
    o_orc = node_outputs_oracle(m, want, xt)
    err = max(float(np.abs(a - b).max()) for a, b in zip(o_card, o_orc))
    p_err = float(np.abs(tree_proba(got.nodes, o_card, 14) - tree_proba(want.nodes, o_orc, 14)).max())
    say(f"  node scores worst {err:.2e}, tree probabilities worst {p_err:.2e}")
    assert err < TOL and p_err < 1e-5


def test_fit_regression_model(gpu):
    """The regression model: targets embedded as numbers (src/model.rs:193-198), 99 quantile outputs."""
    m = M.Model.load(B.Bundle.open(os.path.join(GOLDEN, "tiny-reg.tirs")))
    rng = np.random.default_rng(99)
    x = rng.standard_normal((90, 5)).astype(np.float32)
    y = rng.standard_normal(90).astype(np.float32)
    w = gpu.weights(m)
    got = fit.fit_raw(gpu, w, x, y, m.outputs, chunk=40)
    want = orc.fit_raw(m, x, y, m.outputs, chunk=40)
    compare_fits(got, want, abi.KV_F32)
    xt = rng.standard_normal((12, 5)).astype(np.float32)
    assert np.abs(predict_card(gpu, w, got, xt) - orc.predict_raw(m, want, xt)).max() < TOL


def test_fit_full_size(gpu):
    """The full-size architecture (3 column blocks over 128 inducing points, 3 row blocks, 12 in-context layers)
    fitted on the card for 700 rows x 16 features: the whole column cache against the oracle's column stage, every
    row's representation, and every layer's keys and values of every row recomputed from the card's own records of
    the layer before; then the i16 fit of the same table is the quantiser applied to the f32 one, bit for bit, and
    predictions from both caches agree with the oracle's over the same caches."""
    import workloads as W

    say("fit full 700 x 16")
    m = M.Model.random(M.FULL_CLASSIFIER, seed=2)
    rng = np.random.default_rng(16)
    rows, features, chunk = 700, 16, 256
    x = rng.standard_normal((rows, features)).astype(np.float32)
    y = np.argmax(x[:, :10] + 0.5 * rng.standard_normal((rows, 10)), axis=1).astype(np.float32)
    w = gpu.weights(m)
    plan, col_kv, reps, h, scales, layers = W.fit_pieces(gpu, w, m, x, y, 10, chunk, abi.KV_F32)
    want_col, emb = orc.fit_columns(m, x, y, plan.bases, chunk)
    err = np.abs(col_kv - want_col).max()
    say("  column cache worst", err)
    assert err < TOL
    err = np.abs(reps - orc.fit_rows(m, orc.fit_cells_rows(m, col_kv, plan.bases, x, y))).max()
    say("  representations worst", err)
    assert err < TOL
    W.check_layers(m, h, layers, scales, rows, chunk, np.arange(rows), TOL, say)
    fq = fit.fit_raw(gpu, w, x, y, 10, chunk=chunk, kv_format=abi.KV_I16)
    for l in range(m.icl_layers):
        rec = layers[l].view(np.float32)
        want = np.concatenate([orc.pack(rec[2 * m.d * c0:2 * m.d * (c0 + min(chunk, rows - c0))], m.d,
                                        min(chunk, rows - c0), abi.KV_I16) for c0 in range(0, rows, chunk)])
        assert np.array_equal(fq.layers[0][l], want), l
    xt = rng.standard_normal((16, 16)).astype(np.float32)
    for fmt, lay in ((abi.KV_F32, layers), (abi.KV_I16, fq.layers[0])):
        fo = W.fitted_of(plan, col_kv, scales, lay, rows, features, 10, chunk, fmt)
        f = fit.Fitted(rows, features, 10, chunk, fmt, plan, col_kv, [scales], [lay])
        a = predict_card(gpu, w, f, xt)
        b = orc.predict_raw(m, fo, xt)
        say(f"  format {fmt}: scores worst", np.abs(a - b).max())
        assert np.abs(a - b).max() < TOL


def test_config1_tiny_random_model(gpu):
    """The smallest workload as specified: the reference's tiny architecture with seeded random weights, 256
    training rows x 10 N(0, 1) features, 3 classes from the argmax of a seeded random projection, f32 cache, one
    member, 64 test rows. The card's fit against the oracle's whole (column cache, scales, every layer's keys and
    values), and all 64 rows' scores and probabilities against the oracle's over its own fit."""
    import workloads as W

    m = M.Model.random(M.TINY_CLASSIFIER, seed=0)
    x, y, xt = W.tiny_table()
    w = gpu.weights(m)
    got = fit.fit_raw(gpu, w, x, y, 3, chunk=256)
    want = orc.fit_raw(m, x, y, 3, chunk=256)
    compare_fits(got, want, abi.KV_F32)
    s_card = predict_card(gpu, w, got, xt)
    s_orc = orc.predict_raw(m, want, xt)
    err = float(np.abs(s_card - s_orc).max())
    T = pkg("table")
    p_err = float(np.abs(T.finish_proba(s_card.astype(np.float64), 1, 0.9)
                         - T.finish_proba(s_orc.astype(np.float64), 1, 0.9)).max())
    say(f"  config 1, 64 rows: scores worst {err:.2e}, probabilities worst {p_err:.2e}")
    assert err < TOL and p_err < 1e-5 and np.isfinite(s_card).all()
    w.free()


@pytest.mark.parametrize("bases", [[5, 5, 5], [3, 4, 2]])
def test_label_digits_on_card_are_single_digit_stages(gpu, tiny_model, bases):
    """The card's label-digit column stage pinned by what the digits mean (src/fit.rs:356-363): digit j of label y
    is (y // prod_{i>j} b_i) % b_j, and each digit's slice of the card's column cache equals the card's one-digit
    stage fitted on those labels; the whole cache also matches the oracle's."""
    m = tiny_model
    rng = np.random.default_rng(7 + sum(bases))
    rows, features = 150, 6
    total = int(np.prod(bases))
    x = rng.standard_normal((rows, features)).astype(np.float32)
    y = rng.integers(0, total, rows)
    w = gpu.weights(m)
    ind_scales = np.stack([fit.query_scale(b, rows) for b in m.col_a1])
    col, _ = gpu.fit_represent(w, x, y.astype(np.float32), bases, ind_scales)
    worst = 0.0
    for j in range(len(bases)):
        yj = (y // int(np.prod(bases[j + 1:], dtype=np.int64))) % bases[j]
        col1, _ = gpu.fit_represent(w, x, yj.astype(np.float32), [bases[j]], ind_scales)
        worst = max(worst, float(np.abs(col[:, j] - col1[:, 0]).max()))
    want, _ = orc.fit_columns(m, x, y.astype(np.float32), bases, 256)
    err = float(np.abs(col - want).max())
    say(f"  digits {bases}: per-digit slices against one-digit stages {worst:.2e}; against the oracle {err:.2e}")
    assert worst == 0.0 and err < TOL
    w.free()
