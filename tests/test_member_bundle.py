"""A fitted member as a `.tirs` bundle: the tensors `raw_entries` names (`src/fit.rs:224-241`: meta, tree, col_kv,
n{j}_scale, n{j}_kv{l}) written in that order, read back through `Cache.open` (`src/predict.rs:138-160`) byte for byte,
and predictions from the reopened bundle identical to those from the member in memory -- on the oracle here, on
the card in the gpu-marked test (the stored records go to the card as the bundle holds them)."""
import numpy as np
import pytest

import oracle as orc
from conftest import pkg

B, fit, C, abi = pkg("bundle"), pkg("fit"), pkg("cache"), pkg("abi")


def as_member(of):
    return fit.Fitted(of.rows, of.features, of.classes, of.chunk, of.kv_format, of.plan, of.col_kv, of.scales,
                      of.layers)


@pytest.mark.parametrize("classes,kv_format", [(3, abi.KV_F32), (14, abi.KV_I8)])
def test_member_round_trip(tiny_model, classes, kv_format):
    rng = np.random.default_rng(classes)
    x = rng.standard_normal((130, 6)).astype(np.float32)
    y = (np.arange(130) % classes).astype(np.float32)
    of = orc.fit_raw(tiny_model, x, y, classes, chunk=32, kv_format=kv_format)
    member = as_member(of)
    data = member.write(None, "m1/")
    b = B.Bundle(data)
    assert [(e.name, e.dtype, list(e.dims)) for e in b.entries] == [(n, d, list(s)) for n, d, s in
                                                                     member.raw_entries("m1/")]
    c = C.Cache.open(b, "m1/")
    assert (c.rows, c.features, c.classes, c.chunk, c.kv_format, c.digits) == (130, 6, classes, 32, kv_format,
                                                                               len(of.plan.bases))
    assert [(n.leaf, n.rows, n.k, n.map) for n in c.nodes] == [(n.leaf, n.rows, n.k, n.map) for n in of.nodes]
    assert np.array_equal(c.col_kv(), of.col_kv)
    for i in range(len(of.nodes)):
        assert np.array_equal(c.scales(i), of.scales[i])
        for l, rec in enumerate(c.layers(i, tiny_model.icl_layers)):
            assert rec.dtype == np.uint8 and np.array_equal(rec, of.layers[i][l])
    # the same bundle written again is the same bytes
    assert fit.Fitted(c.rows, c.features, c.classes, c.chunk, c.kv_format, of.plan, c.col_kv(),
                      [c.scales(i) for i in range(len(c.nodes))],
                      [c.layers(i, tiny_model.icl_layers) for i in range(len(c.nodes))]).write(None, "m1/") == data
    # and the oracle predicts the same from it
    xt = rng.standard_normal((9, 6)).astype(np.float32)
    reopened = orc.Fitted(c.rows, c.features, c.classes, c.chunk, c.kv_format, of.plan, c.col_kv(),
                          [c.scales(i) for i in range(len(c.nodes))],
                          [[np.ascontiguousarray(r) for r in c.layers(i, tiny_model.icl_layers)]
                           for i in range(len(c.nodes))])
    assert np.array_equal(orc.predict_raw(tiny_model, reopened, xt), orc.predict_raw(tiny_model, of, xt))


def test_damaged_meta_is_refused(tiny_model):
    data = B.write(None, {"meta": np.array([1, 2, 3], np.int32), "tree": np.zeros(3, np.int32)})
    with pytest.raises(B.BundleError):
        C.Cache.open(B.Bundle(data))


@pytest.mark.gpu
@pytest.mark.parametrize("classes,kv_format", [(10, abi.KV_I16), (14, abi.KV_F32)])
def test_card_member_bundle(classes, kv_format):
    hip, M = pkg("hip"), pkg("model")
    model = M.Model.random(M.FULL_CLASSIFIER, seed=2)
    gpu = hip.Gpu(0)
    w = gpu.weights(model)
    rng = np.random.default_rng(classes + kv_format)
    x = rng.standard_normal((1200, 20)).astype(np.float32)
    y = (np.arange(1200) % classes).astype(np.float32)
    rng.shuffle(y)
    f = fit.fit_raw(gpu, w, x, y, classes, kv_format=kv_format)
    c = C.Cache.open(B.Bundle(f.write(None, "m0/")), "m0/")
    xt = rng.standard_normal((40, 20)).astype(np.float32)

    def scores(vms, nodes):
        rep = gpu.represent(w, gpu.embed(w, vms[0], xt))
        outs = [gpu.in_context(w, vm, rep, node.k) for vm, node in zip(vms, nodes)]
        return outs[0] if len(outs) == 1 else pkg("plan").tree_scores(nodes, outs, classes)

    from_bundle = c.load(gpu, w)
    direct = [gpu.load(w, kv_format, node.rows, f.chunk, f.layers[i], f.scales[i]) for i, node in enumerate(f.nodes)]
    direct[0].set_columns(f.col_kv, f.features, f.digits)
    a, b = scores(from_bundle, c.nodes), scores(direct, f.nodes)
    print(f"member bundle, {classes} classes, format {kv_format}: {len(c.nodes)} problems, identical: "
          f"{np.array_equal(a, b)}", flush=True)
    assert np.array_equal(a, b)
    for vm in from_bundle + direct:
        vm.free()
    w.free()
    gpu.close()
