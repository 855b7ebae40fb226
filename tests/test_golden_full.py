"""The reference's own golden tables at the full-size TabICL v2 architecture (its published weights at 16-bit
precision, `docs/weights`, BSD licence in tests/golden/weights) and its regression goldens, as
`tests/reference.rs:149-326` runs them:

* preprocessing (oracle/prep.py) against the fixtures' transformed tables at 1e-6, and the ensemble's members
  against the fixtures' member lists (which also pins the Mersenne Twister: `src/prep.rs:440-446`'s known answers);
* table-b (2 classes, 3 members) and many-a (14 classes: label digits [4, 4] and a 7-node class tree, 2 members) end
  to end at 5e-3 of the reference's full-precision probabilities (`docs_half_*`, `tests/reference.rs:250-262`);
* tiny-reg-a/b (the tiny regressor, 4 and 1 members) at 1e-5 of the targets' spread and reg-a/b (16-bit regressor
  weights) at 1%, which pins the regression target embedding, the 999-quantile decoder and QuantileDist's tails
  (the requested levels 5e-4 and 0.9995 lie beyond the model's).

The oracle runs here on the CPU; the card runs the same flows in the gpu-marked tests."""
import os
import sys

import numpy as np
import pytest

import oracle as orc
import prep as P
import tables as TB
from conftest import GOLDEN, pkg

B, M, T = pkg("bundle"), pkg("model"), pkg("table")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def half_clf():
    return M.Model.load(TB.half_weights("classifier"))


@pytest.fixture(scope="module")
def half_reg():
    return M.Model.load(TB.half_weights("regressor"))


@pytest.fixture(scope="module")
def tiny_reg():
    return M.Model.load(B.Bundle.open(os.path.join(GOLDEN, "tiny-reg.tirs")))


def oracle_fit_predict(model):
    return lambda xs, ys, classes, xt: orc.predict_raw(model, orc.fit_raw(model, xs, ys, classes), xt)


def test_python_random_known_answers():
    """`src/prep.rs:440-446`: random.Random(42)'s first three words and its shuffle of range(10)."""
    r = P.py_random(42)
    assert [r.getrandbits(32) for _ in range(3)] == [2746317213, 478163327, 107420369]
    r = P.py_random(42)
    v = list(range(10))
    r.shuffle(v)
    assert v == [7, 3, 2, 8, 5, 6, 9, 4, 0, 1]


def test_bounded_minimum():
    """`src/prep.rs:448-453`: the minimiser finds a stationary point of a wavy parabola."""
    x = P.minimize_bounded(lambda x: (x - 1.3) ** 2 + 0.1 * np.sin(5.0 * x), -2.0, 4.0, 1.48e-8)
    assert abs(2.0 * (x - 1.3) + 0.5 * np.cos(5.0 * x)) < 1e-5


@pytest.mark.parametrize("name", ["table-b", "many-a", "tiny-table", "tiny-one", "tiny-many"])
def test_preprocessing_matches_reference(name):
    fx = TB.fixture(name)
    x, xt = TB.table(fx, "x_train"), TB.table(fx, "x_test")
    prep, tabs = P.Prep.fit(x)
    for v, meth in enumerate(("none", "power")):
        if not fx.has(f"train_{meth}"):
            continue
        bad_train = np.abs(tabs[v] - TB.table(fx, f"train_{meth}")).max()
        bad_test = np.abs(prep.apply(v, xt) - TB.table(fx, f"test_{meth}")).max()
        say(f"{name} '{meth}': train {bad_train:.2e}, test {bad_test:.2e}")
        assert bad_train < 1e-6 and bad_test < 1e-6
    if fx.has("lambdas"):
        assert np.abs(np.array([c.lam for c in prep.norms[1]]) - fx.f64s("lambdas")).max() < 1e-6
    _, labels = T.encode_labels(fx.i32s("y_train"))
    want = TB.members(fx)
    ours = P.ensemble(len(prep.keep), len(labels), 2, len(want), 42)
    for mb in want:
        assert any(o.norm == mb.norm and o.features == mb.features and o.classes == mb.classes for o in ours)


@pytest.mark.parametrize("name", ["table-b", "many-a"])
def test_oracle_half_weights_tables(half_clf, name):
    fx = TB.fixture(name)
    proba = TB.ensemble_proba(fx, oracle_fit_predict(half_clf))
    bad = np.abs(proba - fx.f64s("proba").reshape(proba.shape)).max()
    say(f"oracle {name} (16-bit weights): worst probability difference {bad:.2e}")
    assert bad < TB.HALF_PROBA


@pytest.mark.parametrize("name,members,half", [("tiny-reg-a", 4, False), ("tiny-reg-b", 1, False),
                                                ("reg-b", 1, True), ("reg-a", 4, True)])
def test_oracle_regression(tiny_reg, half_reg, name, members, half):
    model = half_reg if half else tiny_reg
    fx = TB.fixture(name)
    got = TB.ensemble_regression(fx, members, model.outputs, oracle_fit_predict(model))
    res, bar = TB.regression_errors(fx, got, TB.HALF_REGRESSION if half else TB.TINY)
    for kind, (bad, checked) in res.items():
        say(f"oracle {name} {kind}: worst {bad:.2e} (bar {bar:.2e}{'' if checked else ', not compared'})")
        assert bad < bar or not checked


# ---- the card ----------------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def gpu():
    hip = pkg("hip")
    g = hip.Gpu(0)
    yield g
    g.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["table-b", "many-a"])
def test_card_half_weights_tables(gpu, half_clf, name):
    say(f"card {name}: 16-bit classifier weights")
    w = gpu.weights(half_clf)
    fx = TB.fixture(name)
    proba = TB.ensemble_proba(fx, TB.card_fit_predict(gpu, w))
    bad = np.abs(proba - fx.f64s("proba").reshape(proba.shape)).max()
    say(f"  worst probability difference {bad:.2e}")
    w.free()
    assert bad < TB.HALF_PROBA


@pytest.mark.gpu
@pytest.mark.parametrize("name,members,half", [("tiny-reg-a", 4, False), ("tiny-reg-b", 1, False),
                                                ("reg-b", 1, True), ("reg-a", 4, True)])
def test_card_regression(gpu, tiny_reg, half_reg, name, members, half):
    say(f"card {name}: {members} members")
    model = half_reg if half else tiny_reg
    w = gpu.weights(model)
    fx = TB.fixture(name)
    got = TB.ensemble_regression(fx, members, model.outputs, TB.card_fit_predict(gpu, w), gpu=gpu)
    w.free()
    res, bar = TB.regression_errors(fx, got, TB.HALF_REGRESSION if half else TB.TINY)
    for kind, (bad, checked) in res.items():
        say(f"  {kind}: worst {bad:.2e} (bar {bar:.2e}{'' if checked else ', not compared'})")
        assert bad < bar or not checked
