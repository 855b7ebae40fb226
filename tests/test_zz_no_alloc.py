"""The allocation-free in-context stage (tah_stage_dev_noalloc) against the pooled one (tah_stage_dev) through the C
ABI: two calls in a row, the second with fewer rows, on the full-size TabICL v2 architecture, in all three stored
formats: 256 then 4 rows and 3 then 1 row over a 2,000-row stored cache (the many-query attention and the few-row
decode attention, whose split partials both live in the scratch array), 200 then 40 rows, and 256 then 1 row over a
50,000-row stored cache (the most split partials the scratch array must hold). The outputs must agree within the
stated 5e-5 for raw scores (they run the same kernels on the same inputs), and the working-memory pool must not grow
during the allocation-free calls."""
import ctypes
import sys

import numpy as np
import pytest

import oracle as orc
from conftest import pkg

abi, hip, M, devmem = pkg("abi"), pkg("hip"), pkg("model"), pkg("devmem")
pytestmark = pytest.mark.gpu

SCORE_TOL = 5e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def random_layers(rng, layers, rows, chunk, d, kv_format, scale=0.5):
    out = []
    for _ in range(layers):
        parts = []
        for c0 in range(0, rows, chunk):
            rc = min(chunk, rows - c0)
            parts.append(orc.pack((rng.standard_normal(2 * d * rc) * scale).astype(np.float32), d, rc, kv_format))
        out.append(np.concatenate(parts))
    return out


CASES = [(fmt, 2000, calls) for fmt in (abi.KV_F32, abi.KV_I16, abi.KV_I8) for calls in ((256, 4), (3, 1))]
CASES += [(abi.KV_F32, 2000, (200, 40)), (abi.KV_I8, 50000, (256, 1))]


@pytest.mark.parametrize("kv_format,rows,calls", CASES)
def test_stage_noalloc_matches_pooled(kv_format, rows, calls):
    say(f"stage_noalloc fmt={kv_format}: rows {rows}, calls of {calls[0]} then {calls[1]} queries")
    model = M.Model.random(M.FULL_CLASSIFIER, seed=11)
    rng = np.random.default_rng(17 + kv_format + rows)
    d, L, chunk = model.d, model.icl_layers, 256
    layers = random_layers(rng, L, rows, chunk, d, kv_format)
    scales = (0.125 * (1.0 + 0.1 * rng.standard_normal((L, d)))).astype(np.float32)
    gpu = hip.Gpu(0)
    lib = gpu._l
    w = gpu.weights(model)
    vm = gpu.load(w, kv_format, rows, chunk, layers, scales)
    del layers
    out_n = 10
    top = max(calls)
    h_all = (rng.standard_normal((top, d)) * 0.5).astype(np.float32)
    hbuf = devmem.DeviceBuffer.of(h_all)
    obuf = devmem.DeviceBuffer(top * out_n * 4)
    pooled_out = devmem.DeviceBuffer(top * out_n * 4)
    got = []
    for nq in calls:
        hbuf.upload(h_all[:nq])
        rc = lib.tah_stage_dev_noalloc(gpu._h, w._h, vm._h, ctypes.c_void_p(hbuf.ptr), nq, out_n, ctypes.c_void_p(obuf.ptr))
        gpu._check(rc)
        gpu.sync()
        got.append(obuf.download((nq, out_n)))
        assert gpu.working() == (0, 0), "the allocation-free stage borrowed working memory"
    # the input rows are left as they were (the stage works on its own copy)
    assert np.array_equal(hbuf.download((calls[-1], d)), h_all[:calls[-1]])
    for nq, g in zip(calls, got):
        hbuf.upload(h_all[:nq])
        gpu.in_context_dev(w, vm, hbuf.ptr, nq, out_n, pooled_out.ptr)
        gpu.sync()
        want = pooled_out.download((nq, out_n))
        err = float(np.abs(g - want).max())
        say(f"  nq={nq}: worst difference to the pooled stage {err:.2e}")
        assert np.isfinite(g).all() and err < SCORE_TOL
    # too many rows is refused with a clear error and nothing runs
    rc = lib.tah_stage_dev_noalloc(gpu._h, w._h, vm._h, ctypes.c_void_p(hbuf.ptr), 257, out_n, ctypes.c_void_p(obuf.ptr))
    assert rc == abi.E_ARG and b"at most 256 rows" in lib.tah_last_error(gpu._h)
    vm.free()
    w.free()
    gpu.close()
