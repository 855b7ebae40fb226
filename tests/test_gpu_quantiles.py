"""The regression head on the card (`tah_quantile_stats`): every row of a member's predicted quantiles read as a
distribution, against the host statement of the reference's `QuantileDist` (`src/table.rs:292-346`), which sums
left to right in float32 and sorts by `f32::total_cmp` as the reference does.

Mean, variance, median and every quantile between the first and last level are compared bit for bit. The tails
beyond them go through `ln` (the device's logf against the host's, each within an ulp): the tail slopes regress the
end quantiles on the logs of their levels, whose spread is small, so an ulp in a log moves a tail quantile by up to
about 1e-5 relative; those are compared at the raw-score tolerance, 5e-5."""
import sys

import numpy as np
import pytest

from conftest import pkg

hip, T = pkg("hip"), pkg("table")
pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


ALPHAS = np.array([0.0002, 0.0005, 0.001, 0.0015, 0.01, 0.025, 0.1, 0.25, 0.5, 0.5004, 0.75, 0.9, 0.975, 0.99,
                   0.9985, 0.999, 0.9995, 0.9999], np.float32)


@pytest.fixture(scope="module")
def gpu():
    g = hip.Gpu(0)
    yield g
    g.close()


def host_stats(q, alphas):
    out = np.empty((q.shape[0], 3 + alphas.size), np.float32)
    for r, row in enumerate(q):
        d = T.QuantileDist(row)
        out[r, 0], out[r, 1], out[r, 2] = d.mean(), d.variance(), d.icdf(0.5)
        out[r, 3:] = [d.icdf(a) for a in alphas]
    return out


def rows_of(rng, rows, n):
    q = rng.standard_normal((rows, n)).astype(np.float32) * rng.uniform(0.01, 50.0, (rows, 1)).astype(np.float32)
    q += rng.uniform(-100.0, 100.0, (rows, 1)).astype(np.float32)
    q[0] = 3.25                                     # a constant row (zero variance, flat tails)
    q[1] = np.round(q[1])                           # ties
    q[2, ::3] = 0.0
    q[2, 1::3] = -0.0                               # signed zeros, ordered -0 before +0
    q[3] *= np.float32(1e6)                         # large magnitudes
    q[4] = np.sort(q[4])[::-1]                      # reversed
    if rows > 6:
        q[5, 7] = np.nan                            # a NaN: sorted last by total_cmp, the moments NaN
        q[6, : max(1, n // 4)] = -np.inf            # infinities in the left tail
    return q


@pytest.mark.parametrize("n,rows", [(999, 300), (99, 64), (4, 5), (1024, 9)])
def test_quantile_stats_match_host(gpu, n, rows):
    say(f"quantile stats n={n} rows={rows}")
    rng = np.random.default_rng(n)
    q = rows_of(rng, rows, n)
    got = gpu.quantile_stats(q, ALPHAS)
    want = host_stats(q, ALPHAS)
    lo, hi = np.float32(1) / np.float32(n + 1), np.float32(n) / np.float32(n + 1)
    inner = np.concatenate([[True, True, True], (ALPHAS >= lo) & (ALPHAS <= hi)])
    assert np.array_equal(got[:, inner], want[:, inner], equal_nan=True)
    tail = ~inner
    if tail.any():
        gt, wt = got[:, tail], want[:, tail]
        assert np.array_equal(np.isnan(gt), np.isnan(wt)) and np.array_equal(np.isinf(gt), np.isinf(wt))
        ok = np.isfinite(wt)
        err = np.abs(gt[ok] - wt[ok]) / np.maximum(np.abs(wt[ok]), 1.0)
        say("  tails worst relative", err.max())
        assert err.max() < 5e-5


def test_quantile_stats_no_alphas_and_empty(gpu):
    q = np.random.default_rng(3).standard_normal((7, 999)).astype(np.float32)
    got = gpu.quantile_stats(q, [])
    assert got.shape == (7, 3)
    assert np.array_equal(got, host_stats(q, np.zeros(0, np.float32)))
    assert gpu.quantile_stats(np.zeros((0, 999), np.float32), ALPHAS).shape == (0, 3 + ALPHAS.size)


def test_quantile_stats_rejects_bad_sizes(gpu):
    with pytest.raises(ValueError):
        gpu.quantile_stats(np.zeros((2, 1), np.float32), ALPHAS)  # one quantile a row
    with pytest.raises(ValueError):
        gpu.quantile_stats(np.zeros((2, 1025), np.float32), ALPHAS)  # more than 1,024
    with pytest.raises(ValueError):
        gpu.quantile_stats(np.zeros((2, 99), np.float32), np.full(65, 0.5, np.float32))  # more than 64 levels


def test_add_regression_card_matches_host(gpu):
    """A member's contribution to the averaged regression answer, card against host (float64 sums)."""
    rng = np.random.default_rng(11)
    q = rows_of(rng, 40, 999)
    blank = lambda: {"mean": np.zeros(40), "variance": np.zeros(40), "median": np.zeros(40),
                     "quantiles": np.zeros((40, ALPHAS.size))}
    a, b = blank(), blank()
    T.add_regression(a, q, ALPHAS, 2.5, 0.75, gpu=gpu)
    T.add_regression(b, q, ALPHAS, 2.5, 0.75)
    for k in ("mean", "variance", "median"):
        assert np.array_equal(a[k], b[k], equal_nan=True)
    assert np.allclose(a["quantiles"], b["quantiles"], rtol=5e-5, atol=5e-5, equal_nan=True)


def test_quantile_stats_planted_tails(gpu):
    """The card's tail fits on quantiles planted on known lines (the same closed forms the host statement is pinned
    by in test_table_golden.py): icdf far out in either tail follows the least-squares slope of exactly the k end
    points from the end quantile."""
    from test_table_golden import TAIL_CASES, planted_tails

    for n, a, b, c, d in TAIL_CASES:
        q, (sl, sr) = planted_tails(n, a, b, c, d)
        lv0, lvn = 1.0 / (n + 1), n / (n + 1)
        lo = np.array([1e-5, 1e-4, 0.3 * lv0], np.float32)
        hi = np.array([1 - 1e-5, 1 - 1e-4, 1 - 0.3 * (1 - lvn)], np.float32)
        st = gpu.quantile_stats(q[None, :], np.concatenate([lo, hi]))[0, 3:]
        want = np.concatenate([q[0] + sl * (np.log(lo.astype(np.float64)) - np.log(lv0)),
                               q[-1] - sr * (np.log(1 - hi.astype(np.float64)) - np.log(1 - lvn))])
        err = np.abs(st - want) / np.maximum(1.0, np.abs(want))
        say(f"planted tails n={n}: worst relative {err.max():.2e}")
        assert err.max() < 2e-4
