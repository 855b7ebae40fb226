"""Prediction on the card against the oracle: the in-context attention over stored layers in all three formats,
and the whole in-context stage, at the tiny model (against the reference's golden logits too) and at the full-size
TabICL v2 architecture. Tolerances are the stated ones: attention outputs and raw scores within 5e-5."""
import sys

import numpy as np
import pytest

import oracle as orc
from conftest import pkg

abi, hip, M = pkg("abi"), pkg("hip"), pkg("model")
pytestmark = pytest.mark.gpu

SCORE_TOL = 5e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpu():
    g = hip.Gpu(0)
    say("device:", g.name)
    yield g
    g.close()


@pytest.fixture(scope="module")
def full_model():
    return M.Model.random(M.FULL_CLASSIFIER, seed=2)


@pytest.fixture(scope="module")
def full_weights(gpu, full_model):
    return gpu.weights(full_model)


def random_layers(rng, layers, rows, chunk, d, kv_format, scale=1.0):
    """Stored layers of random keys and values (normal, scaled), packed by the oracle's quantiser."""
    out = []
    for _ in range(layers):
        parts = []
        for c0 in range(0, rows, chunk):
            rc = min(chunk, rows - c0)
            c = (rng.standard_normal(2 * d * rc) * scale).astype(np.float32)
            parts.append(orc.pack(c, d, rc, kv_format))
        out.append(np.concatenate(parts))
    return out


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16, abi.KV_I8])
@pytest.mark.parametrize("rows,chunk", [(10000, 256), (1000, 48), (37, 8), (50, 64)])
@pytest.mark.parametrize("nq", [1, 2, 3, 4, 7, 9, 16, 17, 33, 64, 130])
def test_attention_full_width(gpu, full_model, full_weights, kv_format, rows, chunk, nq):
    """AttendCached::attend at d = 512, 8 heads of 64 over the layer's tiles: f32 up to 16 queries by the few-query
    kernel (16 / 17 the boundary), beyond by the 32-query tiles (33: a second wavefront of queries); i8 the same (its
    chunks' scales copied with each block; chunks of 48 rows: every block begins one), i16 from 2 queries, one by the
    decode kernel; chunks of 8 and 48 rows leave some wavefronts' keys past a block's end."""
    say(f"attention d=512 fmt={kv_format} rows={rows} chunk={chunk} nq={nq}")
    rng = np.random.default_rng(rows * 7 + nq + kv_format)
    d, L = full_model.d, full_model.icl_layers
    layers = random_layers(rng, 1, rows, chunk, d, kv_format, scale=0.5) * L
    scales = np.ones((L, d), np.float32)
    vm = gpu.load(full_weights, kv_format, rows, chunk, layers, scales)
    q = (rng.standard_normal((nq, d)) * 0.3).astype(np.float32)
    got = gpu.attend_resident(vm, 3, q)
    want = orc.attend_records(q, layers[0], kv_format, rows, chunk, d, full_model.icl_heads)
    vm.free()
    err = np.abs(got - want).max()
    say("  worst", err)
    assert err < SCORE_TOL


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16, abi.KV_I8])
@pytest.mark.parametrize("nq", [2048, 1280, 640])
def test_attention_many_queries(gpu, full_model, full_weights, kv_format, nq):
    """Many queries over 3,000 stored rows (47 key blocks), against the oracle: 2,048 (8 tiles of 256 queries x 8
    heads x 4 key ranges of 12 blocks, the last 11), 1,280 (5 tiles x 8 heads x 6 ranges of 8 blocks, the last 7: the
    range count that keeps 240 workgroups in one round, where rounding up would make 7 ranges and 280) and 640 (f32
    and i8: 5 tiles of 128 queries x 8 heads x 6 or 12 ranges; i16: 3 tiles of 256, the last only half live, x 8
    heads x 10 ranges of 5 blocks, the last 2)."""
    say(f"attention {nq} queries fmt={kv_format}")
    rng = np.random.default_rng(nq + kv_format)
    d, L = full_model.d, full_model.icl_layers
    rows, chunk = 3000, 256
    layers = random_layers(rng, 1, rows, chunk, d, kv_format, scale=0.5) * L
    vm = gpu.load(full_weights, kv_format, rows, chunk, layers, np.ones((L, d), np.float32))
    q = (rng.standard_normal((nq, d)) * 0.3).astype(np.float32)
    got = gpu.attend_resident(vm, 5, q)
    want = orc.attend_records(q, layers[0], kv_format, rows, chunk, d, full_model.icl_heads)
    vm.free()
    err = np.abs(got - want).max()
    say("  worst", err)
    assert err < SCORE_TOL


@pytest.mark.parametrize("kv_scale,q_scale", [(2000.0, 1e-4), (1e-3, 300.0), (1.0, 1.0)])
@pytest.mark.parametrize("nq", [96, 5])
def test_attention_magnitudes(gpu, full_model, full_weights, kv_scale, q_scale, nq):
    """Keys, values and queries far from unit size, and heads of different sizes (each head's coordinates scaled by
    4^h): the split-fp16 path's power-of-two scaling keeps f32 accuracy, relative to the outputs' size (96 queries:
    the 32-query kernel; 5: the few-query kernel)."""
    say(f"attention magnitudes kv={kv_scale} q={q_scale} nq={nq}")
    rng = np.random.default_rng(int(kv_scale * 10) + 3)
    d, L, heads = full_model.d, full_model.icl_layers, full_model.icl_heads
    rows, chunk = 3000, 256
    per_dim = np.repeat(4.0 ** (np.arange(heads) - heads // 2), d // heads).astype(np.float32)
    parts = []
    for c0 in range(0, rows, chunk):
        rc = min(chunk, rows - c0)
        kv = rng.standard_normal((2, d, rc)).astype(np.float32) * np.float32(kv_scale)
        kv[0] *= per_dim[:, None]
        kv[1] *= per_dim[:, None]
        parts.append(orc.pack(kv.reshape(-1), d, rc, abi.KV_F32))
    layers = [np.concatenate(parts)] * L
    vm = gpu.load(full_weights, abi.KV_F32, rows, chunk, layers, np.ones((L, d), np.float32))
    q = (rng.standard_normal((nq, d)) * q_scale / per_dim).astype(np.float32)  # scores stay of moderate size
    got = gpu.attend_resident(vm, 0, q)
    want = orc.attend_records(q, layers[0], abi.KV_F32, rows, chunk, d, heads)
    vm.free()
    for h in range(heads):
        sl = slice(h * 64, (h + 1) * 64)
        size = np.abs(want[:, sl]).max()
        err = np.abs(got[:, sl] - want[:, sl]).max()
        say(f"  head {h}: worst {err:.3g} of {size:.3g}")
        assert err <= 2e-5 * size, h


def test_model_bytes(gpu, full_weights):
    """Gpu::model_bytes at 10,000 rows, chunk 256 (157 key blocks of 64 over 40 chunks, 8 heads of 64): each layer held
    once, as tiles in place of its records: f32 as 32 KB split images per (key block, head) with the heads' maxima;
    i16 as 16.5 KB code tiles (each half with its 64 factors) with the heads' maxima; i8 as 16 KB code images with
    768 bytes of scales per (chunk, head); then the query scales. The 16-bit formats stay under the reference's 285 MB resident
    model (README.md:100) with room for nothing else of the layer."""
    def a256(n):
        return (n + 255) // 256 * 256

    tiles = {abi.KV_F32: 32768, abi.KV_I16: 2 * (8192 + 256), abi.KV_I8: 16384}
    tail = {abi.KV_F32: 0, abi.KV_I16: 0, abi.KV_I8: 40 * 8 * 768}
    for fmt in (abi.KV_F32, abi.KV_I16, abi.KV_I8):
        want = 12 * a256(a256(157 * 8 * tiles[fmt]) + 256 + tail[fmt]) + a256(12 * 512 * 4)
        assert hip.VramModel.model_bytes(full_weights, fmt, 10000, 256) == want, fmt
    i16 = hip.VramModel.model_bytes(full_weights, abi.KV_I16, 10000, 256)
    assert i16 <= 260e6 and i16 <= 12 * 20_643_840 * 1.03  # within 3% of the stored i16 records
    assert hip.VramModel.model_bytes(full_weights, abi.KV_F32, 0, 256) == 0


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16, abi.KV_I8])
def test_attention_tiny_width(gpu, tiny_model, kv_format):
    """Head width 8 (the tiny model): the decode kernel at any query count."""
    say(f"attention tiny fmt={kv_format}")
    w = gpu.weights(tiny_model)
    rng = np.random.default_rng(kv_format)
    d, L = tiny_model.d, tiny_model.icl_layers
    for rows, chunk, nq in ((120, 48, 16), (300, 64, 70), (5, 8, 1)):
        layers = random_layers(rng, L, rows, chunk, d, kv_format)
        vm = gpu.load(w, kv_format, rows, chunk, layers, np.ones((L, d), np.float32))
        q = rng.standard_normal((nq, d)).astype(np.float32)
        got = gpu.attend_resident(vm, 1, q)
        want = orc.attend_records(q, layers[1], kv_format, rows, chunk, d, tiny_model.icl_heads)
        vm.free()
        assert np.abs(got - want).max() < SCORE_TOL, (rows, chunk, nq)


def test_stage_tiny_matches_oracle_and_reference(gpu, tiny_model, tiny_raw):
    """AttendCached::stage on the tiny model fitted by the oracle: the raw scores agree with the oracle's and
    with the reference's golden logits (tests/reference.rs:141-148, at TINY = 5e-5)."""
    say("stage tiny golden")
    x = tiny_raw.f32s("x_train").reshape(120, 7)
    y = tiny_raw.i32s("y_train").astype(np.float32)
    fit = orc.fit_raw(tiny_model, x, y, 3, chunk=48)
    rep = orc.represent(tiny_model, orc.embed(tiny_model, fit, tiny_raw.f32s("x_test").reshape(16, 7)))
    w = gpu.weights(tiny_model)
    vm = gpu.load(w, abi.KV_F32, 120, 48, fit.layers[0], fit.scales[0])
    got = gpu.in_context(w, vm, rep, 3)
    want = orc.in_context(tiny_model, fit.scales[0], fit.layers[0], abi.KV_F32, 120, 48, rep, 3)
    assert np.abs(got - want).max() < SCORE_TOL
    assert np.abs(got - tiny_raw.f32s("logits").reshape(16, 3)).max() < SCORE_TOL
    # through the plugin trait
    card = hip.CardAttend(gpu, w)
    assert card.stage("", 0, rep, tiny_model.d, 3) is None  # not held: the CPU streams instead
    card.hold("", 0, vm)
    assert np.array_equal(card.stage("", 0, rep, tiny_model.d, 3), got)


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16, abi.KV_I8])
@pytest.mark.parametrize("nq", [1, 2, 3, 4, 7, 8, 20, 64, 200, 600])
def test_stage_full_size(gpu, full_model, full_weights, kv_format, nq):
    """The whole in-context stage (12 layers of 8 x 64 heads, d = 512, then the decoder) over a stored cache of
    2,000 rows, against the oracle on the same inputs."""
    say(f"stage full fmt={kv_format} nq={nq}")
    rng = np.random.default_rng(100 + nq + kv_format)
    d, L, rows, chunk = full_model.d, full_model.icl_layers, 2000, 256
    layers = random_layers(rng, L, rows, chunk, d, kv_format)
    scales = np.stack([orc.query_scale(b, rows) for b in full_model.icl])
    vm = gpu.load(full_weights, kv_format, rows, chunk, layers, scales)
    h = rng.standard_normal((nq, d)).astype(np.float32)
    got = gpu.in_context(full_weights, vm, h, 10)
    want = orc.in_context(full_model, scales, layers, kv_format, rows, chunk, h, 10)
    vm.free()
    err = np.abs(got - want).max()
    say("  worst", err, "scale", np.abs(want).max())
    assert err < SCORE_TOL


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16, abi.KV_I8])
@pytest.mark.parametrize("nq,rows,checked", [(1024, 3000, 1024), (2048, 10000, 256), (768, 3000, 768), (1280, 3000, 320)])
def test_stage_large_batches_sampled(gpu, full_model, full_weights, kv_format, nq, rows, checked):
    """The whole in-context stage for a large batch (the 8-wavefront attention kernel, few key ranges, the split-K
    dense layers), `checked` of its rows against the oracle on the same inputs (rows are independent): all 1,024 at
    3,000 stored rows, 256 at 10,000; all 768 (the few-row dense kernels, 3 query tiles) and 320 of 1,280 (the split-K
    dense layers over 40 row tiles, 5 query tiles)."""
    say(f"stage large batch fmt={kv_format} nq={nq} rows={rows}")
    rng = np.random.default_rng(nq + rows + kv_format)
    d, L, chunk = full_model.d, full_model.icl_layers, 256
    layers = random_layers(rng, L, rows, chunk, d, kv_format)
    scales = np.stack([orc.query_scale(b, rows) for b in full_model.icl])
    vm = gpu.load(full_weights, kv_format, rows, chunk, layers, scales)
    h = rng.standard_normal((nq, d)).astype(np.float32)
    got = gpu.in_context(full_weights, vm, h, 10)
    sample = np.sort(rng.choice(nq, checked, replace=False))
    want = orc.in_context(full_model, scales, layers, kv_format, rows, chunk, h[sample], 10)
    vm.free()
    err = np.abs(got[sample] - want).max()
    say("  worst", err, "scale", np.abs(want).max())
    assert err < SCORE_TOL and np.isfinite(got).all()
