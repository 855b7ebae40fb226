"""The drop-in boundary without a GPU: the library builds, loads, and exports every function include/tah.h
declares; the host-side size rules agree with the reference's (Kv::record, raw_entries)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT, pkg

abi = pkg("abi")


def declared():
    text = open(os.path.join(ROOT, "include", "tah.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tah_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert set(declared()) == set(abi.SIGNATURES), "ctypes binding and include/tah.h must list the same functions"


def test_library_exports_every_declared_symbol():
    if not os.path.exists(abi.LIB_PATH):
        pytest.skip("libtah_hip.so not built")
    lib = ctypes.CDLL(abi.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_record_sizes_match_the_reference():
    if not os.path.exists(abi.LIB_PATH):
        pytest.skip("libtah_hip.so not built")
    l = abi.lib()
    # src/fit.rs:123-126 at the full-size model (d = 512) and the tiny one (d = 16)
    for fmt in (abi.KV_F32, abi.KV_I16, abi.KV_I8):
        for d, rc in ((512, 256), (512, 16), (16, 48), (16, 24)):
            assert l.tah_kv_record(fmt, d, rc) == abi.kv_record(fmt, d, rc)
    assert abi.kv_record(abi.KV_F32, 512, 256) == 1 << 20
    # the published per-layer sizes at 10,000 rows, chunk 256: 40 chunks, the last of 16 rows
    assert abi.layer_bytes(abi.KV_F32, 10000, 256, 512) == 40_960_000
    assert abi.layer_bytes(abi.KV_I16, 10000, 256, 512) == 20_643_840
    assert abi.layer_bytes(abi.KV_I8, 10000, 256, 512) == 10_403_840
    assert l.tah_model_bytes(None, abi.KV_F32, 10000, 256) == 0  # no weights, no size
