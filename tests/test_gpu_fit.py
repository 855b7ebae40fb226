"""Fitting on the card against the oracle: the quantiser bit for bit, the all-rows attention of a layer, and the
whole in-context stage's key/value cache build (every layer's stored records), at the tiny model (also against the
reference's golden cache) and at the full-size architecture, in all three stored formats."""
import sys

import numpy as np
import pytest

import oracle as orc
from conftest import pkg, to_ours

abi, hip, M = pkg("abi"), pkg("hip"), pkg("model")
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


@pytest.mark.parametrize("kv_format", [abi.KV_I16, abi.KV_I8])
@pytest.mark.parametrize("d,rc", [(512, 256), (512, 16), (16, 48), (16, 1), (8, 37)])
def test_pack_bit_exact(gpu, kv_format, d, rc):
    """The on-card quantiser writes the same bytes as the reference's pack for the same floats."""
    say(f"pack fmt={kv_format} d={d} rc={rc}")
    rng = np.random.default_rng(d * 1000 + rc + kv_format)
    c = (rng.standard_normal((2 * d, rc)) * rng.uniform(1e-3, 30.0, (2 * d, 1))).astype(np.float32)
    c[1] = 0.0
    if rc >= 4:
        big = np.float32(127.0 if kv_format == abi.KV_I8 else 32767.0)
        c[2, :4] = [big, -big, 0.5, -0.5]  # scale 1 exactly: exact ties round away from zero
        c[3, 0] = np.float32(-3.0)
        c[4] = np.linspace(-1.0, 1.0, rc, dtype=np.float32)
    got = gpu.pack(c, d, rc, kv_format)
    want = orc.pack(c, d, rc, kv_format)
    assert got.tobytes() == want.tobytes()
    f = gpu.pack(c, d, rc, abi.KV_F32)
    assert f.view(np.float32).tolist() == c.reshape(-1).tolist()


def kv_rows_to_records(k, v, chunk):
    rows, d = k.shape
    out = []
    for c0 in range(0, rows, chunk):
        rc = min(chunk, rows - c0)
        out.append(np.concatenate([k[c0:c0 + rc].T.reshape(-1), v[c0:c0 + rc].T.reshape(-1)]))
    return np.concatenate(out).astype(np.float32)


@pytest.mark.parametrize("rows,chunk,d,heads", [(300, 48, 512, 8), (2000, 256, 512, 8), (120, 48, 16, 2)])
def test_attend_all_rows(gpu, rows, chunk, d, heads):
    """Attend::attend: every row over all rows of a layer's exact f32 keys and values."""
    say(f"attend rows={rows} chunk={chunk} d={d}")
    rng = np.random.default_rng(rows)
    q = (rng.standard_normal((rows, d)) * 0.2).astype(np.float32)
    kv = kv_rows_to_records(rng.standard_normal((rows, d)).astype(np.float32),
                            rng.standard_normal((rows, d)).astype(np.float32), chunk)
    got = gpu.attend(q, kv, rows, chunk, d, heads)
    want = np.zeros_like(got)
    orc.lib().orc_fit_attend(orc.fp(q), orc.fp(kv), rows, chunk, d, heads, orc.fp(want))
    assert np.abs(got - want).max() < TOL


def gpu_fit_icl(gpu, weights, h, scales, kv_format, chunk):
    layers = []
    gpu.in_context_fit(weights, h, scales, kv_format, chunk, lambda l, rec: layers.append(rec.copy()))
    return layers


def test_in_context_fit_tiny_matches_reference(gpu, tiny_model, tiny_raw):
    """The cache the card builds for the golden tiny table: against the oracle's and the reference's icl_k/icl_v
    (tests/reference.rs:72-89 at 2.5 x 5e-5), and prediction from it against the golden logits."""
    say("in_context fit tiny golden")
    m = tiny_model
    x = tiny_raw.f32s("x_train").reshape(120, 7)
    y = tiny_raw.i32s("y_train").astype(np.float32)
    col_kv, emb = orc.fit_columns(m, x, y, [3], 48)
    reps = orc.fit_rows(m, emb)
    h = reps.copy()
    m.add_y(m.t["icl_y"], y, h)
    scales = np.stack([orc.query_scale(b, 120) for b in m.icl])
    w = gpu.weights(m)
    layers = gpu_fit_icl(gpu, w, h, scales, abi.KV_F32, 48)
    o_scales, o_layers, _ = orc.fit_icl(m, h, 48, abi.KV_F32)
    assert np.array_equal(o_scales, scales)
    d = m.d
    for l in range(m.icl_layers):
        got = layers[l].view(np.float32)
        assert np.abs(got - o_layers[l].view(np.float32)).max() < TOL
        for which, kind in enumerate(["icl_k", "icl_v"]):
            want = to_ours(tiny_raw.f32s(f"{kind}{l}"), m.icl_heads, 120, d // m.icl_heads)
            for c0 in range(0, 120, 48):
                rc = min(48, 120 - c0)
                chunk = got[2 * d * c0:2 * d * (c0 + rc)].reshape(2, d, rc)[which]
                assert np.abs(chunk - want[:, c0:c0 + rc]).max() < 2.5 * TOL, (kind, l)
    fitted = orc.Fitted(120, 7, 3, 48, abi.KV_F32, pkg("plan").Plan.new(m.max_classes, y, 3), col_kv, [scales], [layers])
    rep = orc.represent(m, orc.embed(m, fitted, tiny_raw.f32s("x_test").reshape(16, 7)))
    vm = gpu.load(w, abi.KV_F32, 120, 48, layers, scales)
    logits = gpu.in_context(w, vm, rep, 3)
    assert np.abs(logits - tiny_raw.f32s("logits").reshape(16, 3)).max() < TOL


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16, abi.KV_I8])
def test_in_context_fit_full_size(gpu, full_model, kv_format):
    """The full-size in-context stage fitted on the card (12 layers, d = 512) for 1,500 rows against the oracle:
    f32 keys and values within 5e-5; integer caches with the same scales (to rounding) and codes at most one step
    apart (the f32 inputs differ by rounding, so codes at a rounding tie may differ); predictions from the two
    caches agree within 5e-5 (f32) or 5e-3 (i16/i8)."""
    say(f"in_context fit full fmt={kv_format}")
    m = full_model
    rows, chunk, d = 1500, 256, m.d
    rng = np.random.default_rng(7)
    h = rng.standard_normal((rows, d)).astype(np.float32)
    y = rng.integers(0, 10, rows).astype(np.float32)
    m.add_y(m.t["icl_y"], y, h)
    scales = np.stack([orc.query_scale(b, rows) for b in m.icl])
    w = gpu.weights(m)
    layers = gpu_fit_icl(gpu, w, h, scales, kv_format, chunk)
    o_scales, o_layers, o_f32 = orc.fit_icl(m, h, chunk, kv_format, want_f32=True)
    assert len(layers) == m.icl_layers
    for l in range(m.icl_layers):
        assert layers[l].nbytes == abi.layer_bytes(kv_format, rows, chunk, d)
        if kv_format == abi.KV_F32:
            err = np.abs(layers[l].view(np.float32) - o_layers[l].view(np.float32)).max()
            assert err < TOL, (l, err)
        else:
            full = abi.kv_record(kv_format, d, chunk)
            it = np.int16 if kv_format == abi.KV_I16 else np.int8
            for ci, c0 in enumerate(range(0, rows, chunk)):
                rc = min(chunk, rows - c0)
                a = layers[l][ci * full:ci * full + abi.kv_record(kv_format, d, rc)]
                b = o_layers[l][ci * full:ci * full + abi.kv_record(kv_format, d, rc)]
                sa, sb = a[:8 * d].view(np.float32), b[:8 * d].view(np.float32)
                assert np.abs(sa - sb).max() <= 1e-5 * np.abs(sb).max(), (l, ci)
                ca, cb = a[8 * d:].view(it).astype(np.int32), b[8 * d:].view(it).astype(np.int32)
                assert np.abs(ca - cb).max() <= 1, (l, ci)
    # predictions over the card's cache: the card against the oracle on the same stored records, absolutely
    hq = rng.standard_normal((32, d)).astype(np.float32)
    vm = gpu.load(w, kv_format, rows, chunk, layers, scales)
    got = gpu.in_context(w, vm, hq, 10)
    vm.free()
    same = orc.in_context(m, scales, layers, kv_format, rows, chunk, hq, 10)
    err = float(np.abs(got - same).max())
    say(f"  predictions over the same cache worst {err:.2e}")
    assert err < TOL
    # and over the oracle's own fit of the same rows: two fits whose twelve layers each round differently, so the
    # caches differ by the fit's own rounding (and the integer caches by a code step at ties); their predictions are
    # compared relative to the scores' magnitude, since that drift grows with it
    other = orc.in_context(m, scales, o_layers, kv_format, rows, chunk, hq, 10)
    tol = TOL if kv_format == abi.KV_F32 else 5e-3
    drift = float(np.abs(got - other).max())
    say(f"  predictions over the oracle's fit worst {drift:.2e}, scores up to {np.abs(other).max():.2f}")
    assert drift < tol * max(1.0, np.abs(other).max())


def test_sink_can_stop_the_fit(gpu, tiny_model):
    """A sink that refuses a layer stops the fit with an error, and the device stays usable."""
    m = tiny_model
    w = gpu.weights(m)
    h = np.random.default_rng(0).standard_normal((50, m.d)).astype(np.float32)
    scales = np.stack([orc.query_scale(b, 50) for b in m.icl])
    seen = []

    def sink(l, rec):
        seen.append(l)
        return l == 0

    with pytest.raises(hip.SinkError):
        gpu.in_context_fit(w, h, scales, abi.KV_I8, 16, sink)
    assert seen == [0]
    assert len(gpu_fit_icl(gpu, w, h, scales, abi.KV_I8, 16)) == m.icl_layers
