"""The oracle pinned: against the reference's golden vectors, its known-answer unit tests, and closed forms in
float64 chosen so that a plausible slip (a dropped scale, a wrong index, a transposed operand) fails one of them."""
import math

import numpy as np
import pytest

import oracle as orc
from conftest import pkg, to_ours

abi = pkg("abi")
planmod = pkg("plan")

# tests/reference.rs:143-148: the tiny model at full precision on both sides
TINY = 5e-5


# ---- golden vectors: every stage against upstream PyTorch (tests/reference.rs:42-121, tiny_raw 141-148) -----
@pytest.fixture(scope="module")
def tiny_fit(tiny_model, tiny_raw):
    x = tiny_raw.f32s("x_train").reshape(120, 7)
    y = tiny_raw.i32s("y_train").astype(np.float32)
    # the reference's comparison fits with chunk 48 (tests/reference.rs:48): chunks of 48, 48 and 24 rows
    return orc.fit_raw(tiny_model, x, y, int(y.max()) + 1, chunk=48)


def test_column_cache_matches_reference(tiny_model, tiny_raw, tiny_fit):
    m = tiny_model
    for b in range(len(m.col_a2)):
        for which, kind in enumerate(["col_k", "col_v"]):
            r = tiny_raw.f32s(f"{kind}{b}").reshape(m.cls + 7, -1)
            for g in range(7):
                # the reference's cache has the class-token columns first; ours only the feature groups
                want = to_ours(r[g + m.cls], m.col_heads, m.inds, m.e // m.col_heads)
                got = tiny_fit.col_kv[g, 0, b, which]
                assert np.abs(got - want).max() < TINY, (kind, b, g)


def test_in_context_cache_matches_reference(tiny_model, tiny_raw, tiny_fit):
    d = tiny_model.d
    for l in range(tiny_model.icl_layers):
        got = tiny_fit.layers[0][l].view(np.float32)
        for which, kind in enumerate(["icl_k", "icl_v"]):
            want = to_ours(tiny_raw.f32s(f"{kind}{l}"), tiny_model.icl_heads, 120, d // tiny_model.icl_heads)
            for c0 in range(0, 120, 48):
                rc = min(48, 120 - c0)
                chunk = got[2 * d * c0:2 * d * (c0 + rc)].reshape(2, d, rc)[which]
                assert np.abs(chunk - want[:, c0:c0 + rc]).max() < 2.5 * TINY, (kind, l, c0)


def test_layer_by_layer_cache_matches_reference(tiny_model, tiny_raw):
    """The per-layer pieces the large-fit tests recompute sampled rows with: keys and values of given rows
    (`kv_rows`) and one in-context layer over stored records (`icl_step`), from the reference's own row
    representations, against its golden in-context cache of both layers."""
    m = tiny_model
    d, n = m.d, 120
    y = tiny_raw.i32s("y_train").astype(np.float32)
    h = tiny_raw.f32s("train_rep").reshape(n, d).copy()
    m.add_y(m.t["icl_y"], y, h)
    scales = np.stack([orc.query_scale(b, n) for b in m.icl])
    for l in range(m.icl_layers):
        kv = orc.kv_rows(m, l, h)
        for which, kind in enumerate(["icl_k", "icl_v"]):
            want = to_ours(tiny_raw.f32s(f"{kind}{l}"), m.icl_heads, n, d // m.icl_heads)
            assert np.abs(kv[:, which * d:(which + 1) * d].T - want).max() < 2.5 * TINY, (kind, l)
        # the layer's stored records (f32, chunks of 48) from these keys and values, then every row through it
        rec = np.concatenate([np.ascontiguousarray(np.concatenate([kv[c0:c0 + 48, :d].T, kv[c0:c0 + 48, d:].T]))
                              .astype(np.float32).reshape(-1).view(np.uint8) for c0 in range(0, n, 48)])
        h = orc.icl_step(m, l, scales[l], rec, abi.KV_F32, n, 48, h)


@pytest.mark.parametrize("bases,classes", [([3], 3), ([4, 4], 14)])
def test_column_stage_pieces_agree_with_the_whole(tiny_model, bases, classes):
    """The column stage for a subset of feature groups, and the cells of sampled rows from a fitted column cache,
    are the whole stage's numbers bit for bit (groups are independent; a row's cells depend only on its own inputs
    and its groups' caches), with label digits and a -100 row included."""
    m = tiny_model
    rng = np.random.default_rng(len(bases))
    x = rng.standard_normal((150, 6)).astype(np.float32)
    x[3, :] = -100.0
    y = rng.integers(0, classes, 150).astype(np.float32)
    col, emb = orc.fit_columns(m, x, y, bases, 32)
    col2, emb2 = orc.fit_columns_of(m, x, y, [4, 1], bases, 32)
    assert np.array_equal(col2, col[[4, 1]]) and np.array_equal(emb2, emb[[4, 1]])
    rows = [0, 3, 77, 149]
    assert np.array_equal(orc.fit_cells_rows(m, col, bases, x[rows], y[rows]), emb[:, rows])


@pytest.mark.parametrize("bases", [[5, 5, 5], [3, 4, 2]])
def test_label_digits_are_single_digit_stages(tiny_model, bases):
    """The label-digit column stage (src/fit.rs:356-363) pinned by its meaning rather than its formula: with digits
    b_0..b_{k-1}, digit j of label y is y_j = (y // prod_{i>j} b_i) % b_j (the mixed-radix expansion, most significant
    digit first), and the stage runs each digit as a one-digit stage of its own over the same input cells. So each
    digit's slice of the cache equals a one-digit stage fitted on the labels y_j, and the cells are the digits'
    cells averaged (summed in digit order, times 1/k). A divisor of b_{j+1} alone, a reversed digit order or a
    digit taken before the division fails it from the third digit on."""
    m = tiny_model
    rng = np.random.default_rng(sum(bases))
    total = int(np.prod(bases))
    x = rng.standard_normal((90, 6)).astype(np.float32)
    x[5, :] = -100.0
    y = rng.integers(0, total, 90)
    col, emb = orc.fit_columns(m, x, y.astype(np.float32), bases, 32)
    # the expansion checked against its definition: the digits rebuild the label
    digits = []
    for j in range(len(bases)):
        digits.append((y // int(np.prod(bases[j + 1:], dtype=np.int64))) % bases[j])
    rebuilt = np.zeros_like(y)
    for j, dj in enumerate(digits):
        rebuilt = rebuilt * bases[j] + dj
    assert np.array_equal(rebuilt, y)
    acc = None
    for j, dj in enumerate(digits):
        col1, emb1 = orc.fit_columns(m, x, dj.astype(np.float32), [bases[j]], 32)
        assert np.array_equal(col[:, j], col1[:, 0]), f"digit {j}"
        acc = emb1.copy() if acc is None else (acc + emb1).astype(np.float32)
    assert np.array_equal(emb, (acc * np.float32(1.0 / len(bases))).astype(np.float32))


def test_prediction_stages_match_reference(tiny_model, tiny_raw, tiny_fit):
    m = tiny_model
    xt = tiny_raw.f32s("x_test").reshape(16, 7)
    tok = orc.embed(m, tiny_fit, xt)
    want = tiny_raw.f32s("test_emb").reshape(16, m.cls + 7, m.e)
    assert np.abs(tok[:, m.cls:] - want[:, m.cls:]).max() < TINY
    rep = orc.represent(m, tok)
    assert np.abs(rep - tiny_raw.f32s("test_rep").reshape(16, m.d)).max() < TINY
    logits = orc.predict_raw(m, tiny_fit, xt)
    assert np.abs(logits - tiny_raw.f32s("logits").reshape(16, 3)).max() < TINY
    # the reference's own check that the cached path equals a plain forward pass (tools/dump_raw.py)
    assert np.abs(logits - tiny_raw.f32s("logits_plain").reshape(16, 3)).max() < 1e-4


def test_chunk_size_does_not_change_answers(tiny_model, tiny_raw):
    """tests/pipeline.rs:56-64: any chunk size gives the same scores (to summation order)."""
    x = tiny_raw.f32s("x_train").reshape(120, 7)
    y = tiny_raw.i32s("y_train").astype(np.float32)
    xt = tiny_raw.f32s("x_test").reshape(16, 7)
    a = orc.predict_raw(tiny_model, orc.fit_raw(tiny_model, x, y, 3, chunk=8), xt)
    b = orc.predict_raw(tiny_model, orc.fit_raw(tiny_model, x, y, 3, chunk=256), xt)
    assert np.abs(a - b).max() < 1e-5


# ---- known answers of the elementary functions (src/kern.rs:353-373, 492-499) ---------------------------------
def test_exp_matches_float64():
    l = orc.lib()
    worst = 0.0
    for x in np.arange(-80.0, 80.0, 0.0137, dtype=np.float32):
        a, b = l.orc_exp1(float(x)), math.exp(float(x))
        worst = max(worst, abs(a - b) / b)
    assert worst < 2e-7
    assert l.orc_exp1(-1000.0) == l.orc_exp1(-87.0) and math.isfinite(l.orc_exp1(1000.0))


def test_erf_tanh_gelu_known_answers():
    l = orc.lib()
    for x in np.arange(-6.0, 6.0, 0.0171, dtype=np.float32):
        assert abs(l.orc_erf1(float(x)) - math.erf(float(x))) < 3e-7
        assert abs(l.orc_tanh1(float(x)) - math.tanh(float(x))) < 4e-7
    g = np.array([-10.0, -1.0, 0.0, 0.1, 1.0, 10.0], np.float32)
    l.orc_gelu(orc.fp(g), 6)
    want = [-0.0, -0.15865525, 0.0, 0.0539828, 0.8413447, 10.0]
    assert np.abs(g - want).max() < 1e-6
    assert abs(l.orc_tanh1(-0.5) + 0.46211716) < 1e-6


# ---- layer norm and linear against float64 ------------------------------------------------------------------
def test_layer_norm_and_linear_closed_form():
    rng = np.random.default_rng(0)
    for n in (1, 7, 64, 129):
        x = rng.standard_normal(n).astype(np.float32) * 3 + 1
        w = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        y = np.zeros(n, np.float32)
        orc.lib().orc_layer_norm(orc.fp(x), n, orc.fp(w), orc.fp(b), orc.fp(y))
        x64 = x.astype(np.float64)
        want = (x64 - x64.mean()) / np.sqrt(x64.var() + 1e-5) * w + b
        assert np.abs(y - want).max() < 1e-5
        W = rng.standard_normal((5, n)).astype(np.float32)
        out = np.zeros(5, np.float32)
        orc.lib().orc_linear(orc.fp(W), orc.fp(b[:5] if n >= 5 else np.zeros(5, np.float32)), orc.fp(x), n, 5, orc.fp(out))
        bias = b[:5] if n >= 5 else np.zeros(5)
        assert np.abs(out - (W.astype(np.float64) @ x64 + bias)).max() < 1e-4


# ---- the quantiser, bit for bit (src/fit.rs:549-576) --------------------------------------------------------
def pack_closed_form(c, d, rc, kv_format):
    """Per coordinate row: scale = max|v| / top (1 when the row is all zero); code = round half away from zero of
    v * (1/scale), saturated. Scales first, then the codes."""
    top = np.float32(32767.0 if kv_format == abi.KV_I16 else 127.0)
    rows = c.reshape(2 * d, rc)
    big = np.abs(rows).max(axis=1)
    s = np.where(big > 0, big / top, np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / s).astype(np.float32)
    v = (rows * inv[:, None]).astype(np.float32)
    # round half away from zero, evaluated exactly in float64
    r = np.sign(v) * np.floor(np.abs(v.astype(np.float64)) + 0.5)
    lo, hi = (-32768, 32767) if kv_format == abi.KV_I16 else (-128, 127)
    codes = np.clip(r, lo, hi).astype(np.int16 if kv_format == abi.KV_I16 else np.int8)
    return np.concatenate([s.view(np.uint8), codes.reshape(-1).view(np.uint8)])


@pytest.mark.parametrize("kv_format", [abi.KV_I16, abi.KV_I8])
@pytest.mark.parametrize("rc", [1, 16, 48, 256])
def test_pack_is_the_closed_form(kv_format, rc):
    rng = np.random.default_rng(rc + 10 * kv_format)
    d = 16
    c = (rng.standard_normal((2 * d, rc)) * rng.uniform(0.01, 100, (2 * d, 1))).astype(np.float32)
    c[3] = 0.0                   # an all-zero row keeps scale 1
    c[5, 0] = -np.abs(c[5]).max() - 1.0  # the largest magnitude negative: code -top exactly
    if rc > 2:
        c[7, :3] = [0.5, -0.5, 1.5]  # exact ties at the scale the row gets
        c[7, 3:] = 0.0
        c[7, 0] = 127.0 * 0.5 / 127.0
    got = orc.pack(c, d, rc, kv_format)
    want = pack_closed_form(c, d, rc, kv_format)
    assert got.tobytes() == want.tobytes()


def test_pack_f32_is_the_floats():
    c = np.arange(2 * 4 * 3, dtype=np.float32)
    assert orc.pack(c, 4, 3, abi.KV_F32).view(np.float32).tolist() == c.tolist()


# ---- streaming attention against float64 plain softmax attention ---------------------------------------------
def plain_attention(q, k, v, heads):
    """q [n][d]; k, v [rows][d]; per head softmax(q k^T) v in float64."""
    n, d = q.shape
    hd = d // heads
    out = np.zeros((n, d))
    for h in range(heads):
        s = q[:, h * hd:(h + 1) * hd].astype(np.float64) @ k[:, h * hd:(h + 1) * hd].T.astype(np.float64)
        w = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h * hd:(h + 1) * hd] = (w / w.sum(axis=1, keepdims=True)) @ v[:, h * hd:(h + 1) * hd].astype(np.float64)
    return out


def records_from_rows(k, v, chunk, kv_format):
    rows, d = k.shape
    parts = []
    for c0 in range(0, rows, chunk):
        rc = min(chunk, rows - c0)
        c = np.concatenate([k[c0:c0 + rc].T.reshape(-1), v[c0:c0 + rc].T.reshape(-1)]).astype(np.float32)
        parts.append(orc.pack(c, d, rc, kv_format))
    return np.concatenate(parts)


def dequant_rows(records, kv_format, rows, chunk, d):
    """`layer_rows` (src/predict.rs:590-629): the stored layer widened to floats, [rows][d] keys and values."""
    k = np.zeros((rows, d), np.float32)
    v = np.zeros((rows, d), np.float32)
    full = abi.kv_record(kv_format, d, chunk)
    for ci, c0 in enumerate(range(0, rows, chunk)):
        rc = min(chunk, rows - c0)
        rec = records[ci * full:ci * full + abi.kv_record(kv_format, d, rc)]
        if kv_format == abi.KV_F32:
            allv = rec.view(np.float32).reshape(2 * d, rc)
        else:
            sc = rec[:8 * d].view(np.float32)
            body = rec[8 * d:].view(np.int16 if kv_format == abi.KV_I16 else np.int8).astype(np.float32)
            allv = body.reshape(2 * d, rc) * sc[:, None]
        k[c0:c0 + rc] = allv[:d].T
        v[c0:c0 + rc] = allv[d:].T
    return k, v


@pytest.mark.parametrize("kv_format", [abi.KV_F32, abi.KV_I16, abi.KV_I8])
@pytest.mark.parametrize("rows,chunk,parts", [(37, 8, 1), (300, 64, 3), (256, 256, 1), (1000, 256, 4)])
def test_attend_records_is_plain_attention(kv_format, rows, chunk, parts):
    rng = np.random.default_rng(rows + kv_format)
    d, heads, n = 32, 4, 5
    q = rng.standard_normal((n, d)).astype(np.float32)
    k = rng.standard_normal((rows, d)).astype(np.float32)
    v = rng.standard_normal((rows, d)).astype(np.float32)
    rec = records_from_rows(k, v, chunk, kv_format)
    got = orc.attend_records(q, rec, kv_format, rows, chunk, d, heads, parts)
    kq, vq = dequant_rows(rec, kv_format, rows, chunk, d)
    # what the stored numbers stand for, attended exactly
    assert np.abs(got - plain_attention(q, kq, vq, heads)).max() < 1e-5
    if kv_format == abi.KV_F32:
        assert np.abs(got - plain_attention(q, k, v, heads)).max() < 1e-5


# ---- the class tree and label digits (src/fit.rs:159-215) ----------------------------------------------------
def test_plan_digits_and_tree():
    y = np.arange(120, dtype=np.float32)
    p = planmod.Plan.new(10, y, 120)
    assert p.bases == [5, 5, 5]
    assert len(p.nodes) == 31
    assert [n.k for n in p.nodes[:2]] == [10, 2] and p.nodes[0].map[:2] == [1, 4]
    leaves = [n for n in p.nodes if n.leaf]
    assert len(leaves) == 20 and all(n.k == 6 for n in leaves)
    # every class reached exactly once, through one path
    assert sorted(c for n in leaves for c in n.map) == list(range(120))
    p14 = planmod.Plan.new(10, np.arange(14, dtype=np.float32), 14)
    assert p14.bases == [4, 4] and [n.k for n in p14.nodes] == [2, 7, 7]
    assert planmod.Plan.new(10, np.zeros(5, np.float32), 3).bases == [3]
    t = p.tree(120)
    back = planmod.parse_tree(t, len(p.nodes))
    assert [(n.leaf, n.k, n.map) for n in back] == [(n.leaf, n.k, n.map) for n in p.nodes]


def test_tree_scores_brute_force():
    """Probabilities multiplied down the tree add up to one per row and equal the product along each path."""
    rng = np.random.default_rng(3)
    y = np.repeat(np.arange(14, dtype=np.float32), 2)
    p = planmod.Plan.new(10, y, 14)
    nodes = planmod.parse_tree(p.tree(len(y)), len(p.nodes))
    outs = [rng.standard_normal((4, n.k)).astype(np.float32) for n in nodes]
    s = planmod.tree_scores(nodes, outs, 14)
    probs = np.exp(s / 0.9) - 1e-6
    assert np.abs(probs.sum(axis=1) - 1.0).max() < 1e-4
    sm = lambda o: np.exp((o - o.max()) / 0.9) / np.exp((o - o.max()) / 0.9).sum()
    for r in range(4):
        root = sm(outs[0][r].astype(np.float64))
        for gi, child in enumerate(nodes[0].map):
            leaf = sm(outs[child][r].astype(np.float64))
            for j, cls_ in enumerate(nodes[child].map):
                assert abs(probs[r, cls_] - root[gi] * leaf[j]) < 1e-5


def test_tiny_workload_on_the_cpu_path():
    """The tiny workload (the reference's tiny architecture, seeded weights, 256 x 10 training rows, 3 classes, 64
    test rows) through the CPU path: every score finite, and the same scores (to summation order) at any chunk size
    (tests/pipeline.rs:56-64), the short last chunk included."""
    import workloads as W

    M = pkg("model")
    m = M.Model.random(M.TINY_CLASSIFIER, seed=0)
    x, y, xt = W.tiny_table()
    assert sorted(set(y.astype(int).tolist())) == [0, 1, 2]
    a = orc.predict_raw(m, orc.fit_raw(m, x, y, 3, chunk=256), xt)
    b = orc.predict_raw(m, orc.fit_raw(m, x, y, 3, chunk=48), xt)
    assert a.shape == (64, 3) and np.isfinite(a).all()
    assert np.abs(a - b).max() < 1e-5
