"""The column and row stages on the card, and prediction from feature rows (AttendCached::rows), against the
oracle and the reference's golden embeddings, representations and scores."""
import sys

import numpy as np
import pytest

import oracle as orc
from conftest import pkg

abi, hip, M = pkg("abi"), pkg("hip"), pkg("model")
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


@pytest.fixture(scope="module")
def full_model():
    return M.Model.random(M.FULL_CLASSIFIER, seed=2)


@pytest.fixture(scope="module")
def full_weights(gpu, full_model):
    return gpu.weights(full_model)


def test_stages_tiny_match_reference(gpu, tiny_model, tiny_raw):
    """embed, represent and all three stages on the card for the golden tiny table (tests/reference.rs:91-116)."""
    say("stages tiny golden")
    m = tiny_model
    x = tiny_raw.f32s("x_train").reshape(120, 7)
    y = tiny_raw.i32s("y_train").astype(np.float32)
    fit = orc.fit_raw(m, x, y, 3, chunk=48)
    xt = tiny_raw.f32s("x_test").reshape(16, 7)
    w = gpu.weights(m)
    vm = gpu.load(w, abi.KV_F32, 120, 48, fit.layers[0], fit.scales[0])
    vm.set_columns(fit.col_kv, 7, 1)
    tok = gpu.embed(w, vm, xt)
    want = tiny_raw.f32s("test_emb").reshape(16, m.cls + 7, m.e)
    assert np.abs(tok - orc.embed(m, fit, xt)).max() < TOL
    assert np.abs(tok[:, m.cls:] - want[:, m.cls:]).max() < TOL
    rep = gpu.represent(w, tok)
    assert np.abs(rep - tiny_raw.f32s("test_rep").reshape(16, m.d)).max() < TOL
    scores = gpu.predict(w, vm, xt, 3)
    assert np.abs(scores - tiny_raw.f32s("logits").reshape(16, 3)).max() < TOL
    card = hip.CardAttend(gpu, w)
    card.hold("", 0, vm)
    assert np.array_equal(card.rows("", xt, 3), scores)


def test_embed_with_label_digits_and_missing_cells(gpu, tiny_model):
    """Several label digits (averaged, src/predict.rs:326-345) and all--100 cells (src/predict.rs:314-316)."""
    m = tiny_model
    rng = np.random.default_rng(5)
    features, digits, n = 6, 2, 40
    col_kv = rng.standard_normal((features, digits, len(m.col_a2), 2, m.e, m.inds)).astype(np.float32)
    x = rng.standard_normal((n, features)).astype(np.float32)
    x[3, :] = -100.0
    x[5, 1:4] = -100.0
    w = gpu.weights(m)
    dummy = [np.zeros(abi.layer_bytes(abi.KV_F32, 8, 8, m.d), np.uint8) for _ in range(m.icl_layers)]
    vm = gpu.load(w, abi.KV_F32, 8, 8, dummy, np.ones((m.icl_layers, m.d), np.float32))
    vm.set_columns(col_kv, features, digits)
    fitted = orc.Fitted(8, features, 3, 8, abi.KV_F32, planmod.Plan([4, 4], []), col_kv, [], [])
    fitted.digits = digits
    got = gpu.embed(w, vm, x)
    want = orc.embed(m, fitted, x)
    assert np.abs(got - want).max() < TOL


@pytest.mark.parametrize("features,n", [(100, 24), (150, 24), (100, 1), (100, 3), (100, 64), (100, 130), (124, 130),
                                        (100, 520), (100, 800), (100, 801), (100, 1030)])
def test_stages_full_size(gpu, full_model, full_weights, features, n):
    """Full-size column stage (3 blocks, 8 x 16 heads, 128 inducing points per group) and row stage (104, 128 or
    154 tokens, RoPE) against the oracle, then all three stages with a stored in-context cache. One row takes the
    single-row routes (the fused column block over its key/value images, the f32 projections and feed-forward);
    from 128 rows the fused column and row blocks, the column stage written into the tokens and each block forming
    the next one's keys and values (130 rows: up to 128 tokens, the row block's largest row); from 512 rows the last
    row block's class-token attention; from 768 rows a prediction's column and row stages as two halves on two
    streams (800 rows: 400 each; 801 rows: 400 and 401); from 1,024 rows the input layer a workgroup per table row."""
    say(f"stages full features={features} n={n}")
    m = full_model
    rng = np.random.default_rng(features + n)
    col_kv = (rng.standard_normal((features, 1, len(m.col_a2), 2, m.e, m.inds)) * 0.5).astype(np.float32)
    rows, chunk = 600, 256
    layers = []
    for _ in range(m.icl_layers):
        parts = [orc.pack((rng.standard_normal(2 * m.d * min(chunk, rows - c0)) * 0.5).astype(np.float32), m.d,
                          min(chunk, rows - c0), abi.KV_F32) for c0 in range(0, rows, chunk)]
        layers.append(np.concatenate(parts))
    scales = np.stack([orc.query_scale(b, rows) for b in m.icl])
    vm = gpu.load(full_weights, abi.KV_F32, rows, chunk, layers, scales)
    vm.set_columns(col_kv, features, 1)
    x = rng.standard_normal((n, features)).astype(np.float32)
    if n > 2:
        x[2, :] = -100.0
    fitted = orc.Fitted(rows, features, 10, chunk, abi.KV_F32, planmod.Plan([10], [planmod.Node(None, [], 10, True, list(range(10)))]),
                        col_kv, [scales], [layers])
    tok = gpu.embed(full_weights, vm, x)
    want_tok = orc.embed(m, fitted, x)
    plain = [r for r in range(n) if r != 2 or n <= 2]
    err = np.abs(tok[plain] - want_tok[plain]).max()
    say("  embed worst", err, "(rows without the -100 sentinel)")
    assert err < TOL
    if n > 2:
        # the sentinel row's cells are -100 and their blocks' layer norms cancel most of their bits: the same
        # arithmetic in another order differs in the last bits of numbers near 100, so that row is compared
        # relative to its size
        rel = (np.abs(tok[2] - want_tok[2]) / np.maximum(1.0, np.abs(want_tok[2]))).max()
        say("  embed, -100 row: worst relative", rel)
        assert rel < TOL
    rep = gpu.represent(full_weights, want_tok)
    want_rep = orc.represent(m, want_tok)
    err = np.abs(rep - want_rep).max()
    say("  represent worst", err)
    assert err < TOL
    scores = gpu.predict(full_weights, vm, x, 10)
    want = orc.predict_raw(m, fitted, x)
    err = np.abs(scores - want).max()
    say("  predict worst", err, "scale", np.abs(want).max())
    assert err < TOL


def test_stages_many_cells(gpu, full_model, full_weights):
    """Many cells (72,000) and tokens (168,000): the column and row stages' dense layers and attention over grids of
    thousands of workgroups, embed and represent against the oracle."""
    say("stages many cells")
    m = full_model
    rng = np.random.default_rng(77)
    features, n = 3, 24000
    col_kv = (rng.standard_normal((features, 1, len(m.col_a2), 2, m.e, m.inds)) * 0.5).astype(np.float32)
    scales = np.stack([orc.query_scale(b, 64) for b in m.icl])
    layers = [orc.pack((rng.standard_normal(2 * m.d * 64) * 0.5).astype(np.float32), m.d, 64, abi.KV_F32)
              for _ in range(m.icl_layers)]
    vm = gpu.load(full_weights, abi.KV_F32, 64, 64, layers, scales)
    vm.set_columns(col_kv, features, 1)
    x = rng.standard_normal((n, features)).astype(np.float32)
    fitted = orc.Fitted(64, features, 10, 64, abi.KV_F32, planmod.Plan([10], [planmod.Node(None, [], 10, True, list(range(10)))]),
                        col_kv, [scales], [layers])
    tok = gpu.embed(full_weights, vm, x)
    want_tok = orc.embed(m, fitted, x)
    err = np.abs(tok - want_tok).max()
    say("  embed worst", err, "scale", np.abs(want_tok).max())
    assert err < TOL
    rep = gpu.represent(full_weights, want_tok)
    want_rep = orc.represent(m, want_tok)
    err = np.abs(rep - want_rep).max()
    say("  represent worst", err)
    assert err < TOL


def test_sub_batches_give_the_same_answers(gpu, tiny_model, tiny_raw):
    """A working-memory budget that forces sub-batches of rows changes no answer beyond rounding
    (tests/card.rs:237-274), and a budget too small for one row is an OutOfMemory error."""
    m = tiny_model
    x = tiny_raw.f32s("x_train").reshape(120, 7)
    y = tiny_raw.i32s("y_train").astype(np.float32)
    fit = orc.fit_raw(m, x, y, 3, chunk=48)
    xt = np.concatenate([tiny_raw.f32s("x_test").reshape(16, 7)] * 8)
    w = gpu.weights(m)
    vm = gpu.load(w, abi.KV_F32, 120, 48, fit.layers[0], fit.scales[0])
    vm.set_columns(fit.col_kv, 7, 1)
    whole = gpu.predict(w, vm, xt, 3)
    old = gpu.work_budget()
    try:
        gpu.release()
        gpu.set_work_budget(64 << 10)
        part = gpu.predict(w, vm, xt, 3)
        assert np.abs(part - whole).max() < 1e-5
        assert gpu.working()[1] <= 64 << 10
        gpu.set_work_budget(4 << 10)
        with pytest.raises(hip.BudgetError):
            gpu.predict(w, vm, xt, 3)
    finally:
        gpu.set_work_budget(old)
