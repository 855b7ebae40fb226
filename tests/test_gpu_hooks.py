"""The fit hooks one at a time, with the trait's own layouts (`fit::Attend`, src/fit.rs:45-74), and the handle's
`attend_rows`, `calibrate` and `stages` (src/gpu.rs:744-746, 1306-1383), through the C ABI:

* `columns` on a batch of feature groups against the oracle's column stage; `rows` against the oracle's row stage
  on the same cells; `attend_rows` against the oracle's attention over the same keys and values;
* a whole fit driven through the hooks as an unmodified `fit_raw_async` drives them (`fit.fit_raw_hooks`) against
  the one-call fit (`fit.fit_raw`), at the full-size architecture;
* the batch sizes and `attend_fits` follow the working-memory budget; asking for more than the batch allows is an
  OutOfMemory error; the stage counter counts each hook the card took.
"""
import sys

import numpy as np
import pytest

import oracle as orc
from conftest import pkg

abi, hip, M, fit = pkg("abi"), pkg("hip"), pkg("model"), pkg("fit")
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
def full():
    return M.Model.random(M.FULL_CLASSIFIER, seed=2)


def ind_queries(m, rows):
    nb = len(m.col_a1)
    return np.stack([fit.query(b, fit.query_scale(b, rows), m.t["col_ind"].reshape(nb, m.inds, m.e)[i])
                     for i, b in enumerate(m.col_a1)]).astype(np.float32)


def test_columns_and_rows_hooks(gpu, full):
    m = full
    rng = np.random.default_rng(3)
    rows, features = 900, 12
    x = rng.standard_normal((rows, features)).astype(np.float32)
    x[5] = -100.0
    y = rng.integers(0, 10, rows).astype(np.float32)
    w = gpu.weights(m)
    before = gpu.stages
    g0, gn = 3, 5
    cells = fit.input_cells(m, x, y, g0, gn)
    rec = gpu.columns(w, cells, rows, gn, ind_queries(m, rows))
    want_col, want_emb = orc.fit_columns_of(m, x, y, list(range(g0, g0 + gn)), [10], 256)
    err_rec = np.abs(rec - want_col[:, 0]).max()
    err_cells = np.abs(cells.transpose(1, 0, 2) - want_emb)
    err_cells[:, 5] /= 100.0  # the -100 row's cells are near 100: compared relative to their size
    say(f"columns: cache worst {err_rec:.2e}, cells worst {err_cells.max():.2e}")
    assert err_rec < TOL and err_cells.max() < TOL
    # the row stage on cells the oracle made, for a batch of rows
    _, emb = orc.fit_columns(m, x, y, [10], 256)
    sample = [0, 5, 17, 899]
    got = gpu.rows(w, np.ascontiguousarray(emb[:, sample].transpose(1, 0, 2)))
    want = orc.fit_rows(m, np.ascontiguousarray(emb[:, sample]))
    say(f"rows: worst {np.abs(got - want).max():.2e}")
    assert np.abs(got - want).max() < TOL
    assert gpu.stages == before + 2
    w.free()


def test_fit_through_the_hooks_matches_the_one_call_fit(gpu, full):
    m = full
    rng = np.random.default_rng(4)
    rows, features = 1500, 20
    x = rng.standard_normal((rows, features)).astype(np.float32)
    y = np.argmax(x[:, :10] + rng.standard_normal((rows, 10)), axis=1).astype(np.float32)
    w = gpu.weights(m)
    old = gpu.work_budget()
    try:
        # a budget that splits the groups and the rows into several calls
        gpu.release()
        gpu.set_work_budget(96 << 20)
        cb, rb = gpu.column_batch(w, rows), gpu.row_batch(w, features)
        say(f"hooks under 96 MiB: {cb} groups and {rb} rows a call")
        assert 0 < cb < features and 0 < rb < rows
        before = gpu.stages
        a = fit.fit_raw_hooks(gpu, w, x, y, 10)
        calls = -(-features // cb) + -(-rows // rb) + 1
        assert gpu.stages == before + calls
        assert gpu.working()[1] <= 96 << 20
    finally:
        gpu.set_work_budget(old)
    b = fit.fit_raw(gpu, w, x, y, 10)
    err_col = np.abs(a.col_kv - b.col_kv).max()
    err_kv = max(np.abs(la.view(np.float32) - lb.view(np.float32)).max() for la, lb in zip(a.layers[0], b.layers[0]))
    say(f"hooks against the one-call fit: column cache {err_col:.2e}, keys/values {err_kv:.2e}")
    assert err_col < TOL and err_kv < TOL
    w.free()


def test_batches_follow_the_budget(gpu, full):
    m = full
    w = gpu.weights(m)
    old = gpu.work_budget()
    try:
        gpu.release()
        assert gpu.attend_fits(10000, 512) and gpu.column_batch(w, 10000) > 0 and gpu.row_batch(w, 100) > 0
        gpu.set_work_budget(64 << 10)
        assert not gpu.attend_fits(10000, 512)
        assert gpu.column_batch(w, 10000) == 0 and gpu.row_batch(w, 100) == 0
        gpu.set_work_budget(64 << 20)
        n = gpu.column_batch(w, 2000)
        assert n > 0
        cells = np.zeros((2000, n + 1, m.e), np.float32)
        with pytest.raises(hip.BudgetError):
            gpu.columns(w, cells, 2000, n + 1, ind_queries(m, 2000))
    finally:
        gpu.set_work_budget(old)
    w.free()


@pytest.mark.parametrize("nq,n", [(1, 300), (64, 2048), (300, 5000)])
def test_attend_rows(gpu, nq, n):
    d, heads = 512, 8
    rng = np.random.default_rng(nq + n)
    q = (rng.standard_normal((nq, d)) * 0.2).astype(np.float32)
    k = rng.standard_normal((n, d)).astype(np.float32)
    v = rng.standard_normal((n, d)).astype(np.float32)
    got = gpu.attend_rows(q, k, v, d, heads)
    # plain softmax attention in float64
    qh, kh, vh = (a.astype(np.float64).reshape(-1, heads, 64).transpose(1, 0, 2) for a in (q, k, v))
    s = qh @ kh.transpose(0, 2, 1)
    p = np.exp(s - s.max(axis=2, keepdims=True))
    want = ((p / p.sum(axis=2, keepdims=True)) @ vh).transpose(1, 0, 2).reshape(nq, d)
    say(f"attend_rows nq={nq} n={n}: worst {np.abs(got - want).max():.2e}")
    assert np.abs(got - want).max() < TOL


def test_calibrate(gpu):
    rate = gpu.calibrate(50.0)
    say(f"calibrate: {rate / 1e12:.1f} T multiply-adds/s (256 queries over 2,048 keys, host to host)")
    assert rate > 1e11
