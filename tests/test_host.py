"""Host-side pieces of the drop-in surface that run without a GPU: the float32 restatement of the query scale and
its elementary functions (checked against the oracle, which is pinned to the reference), and the bundle format."""
import os

import numpy as np

import oracle as orc
from conftest import GOLDEN, pkg

fit, B, M = pkg("fit"), pkg("bundle"), pkg("model")


def test_exp_erf_gelu_match_the_oracle_bit_for_bit():
    x = np.linspace(-30.0, 30.0, 20001, dtype=np.float32)
    l = orc.lib()
    assert np.array_equal(fit.exp1(x), np.array([l.orc_exp1(float(v)) for v in x], np.float32))
    assert np.array_equal(fit.erf1(x), np.array([l.orc_erf1(float(v)) for v in x], np.float32))
    g = x.copy()
    l.orc_gelu(orc.fp(g), g.size)
    assert np.array_equal(fit.gelu(x), g)


def test_query_scale_matches_the_oracle(tiny_model):
    full = M.Model.random(M.FULL_CLASSIFIER, seed=2)
    for m in (tiny_model, full):
        for b in list(m.icl) + list(m.col_a1) + list(m.col_a2):
            for n in (1, 120, 10000, 100000):
                want = orc.query_scale(b, n)
                got = fit.query_scale(b, n)
                # logf may differ by one unit in the last place between libraries
                assert np.abs(got - want).max() <= 2e-7 * max(1.0, np.abs(want).max()), (n,)


def test_bundle_round_trip(tmp_path):
    t = {"a": np.arange(7, dtype=np.float32), "b": np.arange(6, dtype=np.int32).reshape(2, 3),
         "c": np.frombuffer(b"hello", dtype=np.uint8), "d": np.ones((2, 2), np.float16)}
    p = os.path.join(tmp_path, "x.tirs")
    raw = B.write(p, t)
    b = B.Bundle.open(p)
    assert b.bytes("c") == b"hello" and b.i32s("b").tolist() == list(range(6))
    assert b.f32s("d").tolist() == [1.0] * 4
    assert all(e.offset % 64 == 0 for e in b.entries)
    assert raw[:8] == b"TIRSBNDL"
    # the reference's own fixtures parse, and re-writing one reproduces its layout exactly
    g = B.Bundle.open(os.path.join(GOLDEN, "tiny-raw.tirs"))
    again = B.write(None, {e.name: g.array(e.name) for e in g.entries})
    assert again == bytes(g.data)


def test_copy_records_is_an_exact_copy():
    """The fit's record copy (sliced over threads from 4 MiB on) returns the same bytes, in a new array, at sizes
    below, at and above the threshold and not a multiple of the slice count."""
    rng = np.random.default_rng(5)
    for n in (0, 1, 4095, 1 << 22, (1 << 22) + 1, 41_156_608 + 7):
        src = rng.integers(0, 256, n, dtype=np.uint8)
        got = fit.copy_records(src)
        assert got.dtype == np.uint8 and got.shape == src.shape
        assert np.array_equal(got, src)
        if n:
            assert not np.shares_memory(got, src)
