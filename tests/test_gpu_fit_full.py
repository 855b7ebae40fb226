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


def predict_card(gpu, w, fitted, x):
    """Scores from the card for a fitted member: all three stages for one problem, or the column and row stages
    then each problem's in-context stage and the tree walk (src/predict.rs:661-693)."""
    vms = [gpu.load(w, fitted.kv_format, node.rows, fitted.chunk, fitted.layers[i], fitted.scales[i])
           for i, node in enumerate(fitted.nodes)]
    vms[0].set_columns(fitted.col_kv, fitted.features, fitted.digits)
    if len(vms) == 1:
        return gpu.predict(w, vms[0], x, fitted.classes)
    rep = gpu.represent(w, gpu.embed(w, vms[0], x))
    outs = [gpu.in_context(w, vm, rep, node.k) for vm, node in zip(vms, fitted.nodes)]
    return planmod.tree_scores(fitted.nodes, outs, fitted.classes)


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


def compare_fits(got, want, kv_format, tol_scale=1.0):
    assert got.plan.bases == want.plan.bases and len(got.layers) == len(want.layers)
    err = np.abs(got.col_kv - want.col_kv).max()
    assert err < TOL * tol_scale * max(1.0, np.abs(want.col_kv).max()), err
    for ni in range(len(want.layers)):
        assert np.abs(got.scales[ni] - want.scales[ni]).max() <= 2e-7 * max(1.0, np.abs(want.scales[ni]).max())
        for l in range(len(want.layers[ni])):
            if kv_format == abi.KV_F32:
                a, b = got.layers[ni][l].view(np.float32), want.layers[ni][l].view(np.float32)
                assert np.abs(a - b).max() < TOL * tol_scale * max(1.0, np.abs(b).max()), (ni, l)


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
    s_card = predict_card(gpu, w, got, xt)
    s_orc = orc.predict_raw(m, want, xt)
    assert np.abs(s_card - s_orc).max() < TOL * 10  # through the tree's softmax and log


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


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16])
def test_fit_full_size(gpu, kv_format):
    """The full-size architecture (3 column blocks over 128 inducing points, 3 row blocks, 12 in-context layers)
    fitted on the card for 700 rows x 16 features, against the oracle; then predictions from both caches."""
    say(f"fit full fmt={kv_format}")
    m = M.Model.random(M.FULL_CLASSIFIER, seed=2)
    rng = np.random.default_rng(16)
    x = rng.standard_normal((700, 16)).astype(np.float32)
    y = np.argmax(x[:, :10] + 0.5 * rng.standard_normal((700, 10)), axis=1).astype(np.float32)
    w = gpu.weights(m)
    got = fit.fit_raw(gpu, w, x, y, 10, chunk=256, kv_format=kv_format)
    want = orc.fit_raw(m, x, y, 10, chunk=256, kv_format=kv_format)
    say("  col_kv worst", np.abs(got.col_kv - want.col_kv).max())
    compare_fits(got, want, kv_format, tol_scale=4.0)
    xt = rng.standard_normal((16, 16)).astype(np.float32)
    a = predict_card(gpu, w, got, xt)
    b = orc.predict_raw(m, want, xt)
    tol = TOL if kv_format == abi.KV_F32 else 5e-3
    say("  scores worst", np.abs(a - b).max(), "scale", np.abs(b).max())
    assert np.abs(a - b).max() < tol * max(1.0, np.abs(b).max())
