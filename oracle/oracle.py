"""TEST INFRASTRUCTURE ONLY: Python driver of the oracle (liboracle.so, the C restatement of the reference's CPU
path). Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it, as the checker or the timed
CPU baseline.

`fit_raw` follows `fit_raw_async` (`src/fit.rs:285-752`, CPU path): column stage, row stage, then per in-context
problem the target embedding and the in-context stage. `predict_raw` follows `predict_raw_async`
(`src/predict.rs:638-699`): column stage, row stage, in-context stage per problem, tree walk.
"""
from __future__ import annotations

import ctypes
import importlib
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

abi = importlib.import_module("tabicl-anywhere_amd.abi")
planmod = importlib.import_module("tabicl-anywhere_amd.plan")

LIB_PATH = os.path.join(HERE, "liboracle.so")
F32P = abi.F32P
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        i, f, p, u8pp = ctypes.c_int, ctypes.c_float, F32P, ctypes.POINTER(abi.U8P)
        md = ctypes.POINTER(abi.ModelDesc)
        bp = ctypes.POINTER(abi.Block)
        sig = {
            "orc_exp1": (f, [f]), "orc_erf1": (f, [f]), "orc_tanh1": (f, [f]), "orc_gelu": (None, [p, i]),
            "orc_layer_norm": (None, [p, i, p, p, p]), "orc_linear": (None, [p, p, p, i, i, p]),
            "orc_query_scale": (None, [bp, i, p]), "orc_query": (None, [bp, p, p, p]),
            "orc_feed_forward": (None, [bp, p]), "orc_kv_record": (ctypes.c_size_t, [i, i, i]),
            "orc_pack": (None, [p, i, i, i, abi.U8P]),
            "orc_attend_records": (None, [p, i, abi.U8P, i, i, i, i, i, i, p]),
            "orc_in_context": (None, [md, p, u8pp, i, i, i, p, i, i, p]),
            "orc_fit_columns": (None, [md, p, p, i, i, ctypes.POINTER(ctypes.c_int), i, i, p, p]),
            "orc_fit_rows": (None, [md, p, i, i, p]),
            "orc_fit_icl": (None, [md, p, i, i, i, p, u8pp, p]),
            "orc_fit_attend": (None, [p, p, i, i, i, i, p]),
            "orc_kv_rows": (None, [md, i, p, i, p]),
            "orc_fit_columns_of": (None, [md, p, p, i, i, ctypes.POINTER(ctypes.c_int), i, ctypes.POINTER(ctypes.c_int),
                                          i, i, p, p]),
            "orc_fit_cells_rows": (None, [md, p, ctypes.POINTER(ctypes.c_int), i, p, p, i, i, p]),
            "orc_icl_step": (None, [md, i, p, abi.U8P, i, i, i, p, i]),
            "orc_embed": (None, [md, p, i, p, i, i, p]),
            "orc_represent": (None, [md, p, i, i, p]),
            "orc_set_threads": (None, [i]), "orc_threads": (i, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(l, name)
            fn.restype, fn.argtypes = res, args
        _lib = l
    return _lib


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(F32P)


def u8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(abi.U8P)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


# ---- small pieces, for tests ----------------------------------------------------------------------------------
def pack(c: np.ndarray, d: int, rc: int, kv_format: int) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.float32)
    out = np.zeros(abi.kv_record(kv_format, d, rc), np.uint8)
    lib().orc_pack(fp(c), d, rc, kv_format, u8(out))
    return out


def attend_records(q: np.ndarray, records: np.ndarray, kv_format: int, rows: int, chunk: int, d: int, heads: int,
                   key_parts: int = 1) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    nq = q.shape[0]
    out = np.zeros((nq, d), np.float32)
    lib().orc_attend_records(fp(q), nq, u8(np.ascontiguousarray(records)), kv_format, rows, chunk, d, heads, key_parts, fp(out))
    return out


def query(model, block_index: int, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    b = model.icl[block_index].c_struct()
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    for r in range(x.shape[0]):
        lib().orc_query(ctypes.byref(b), fp(np.ascontiguousarray(scale, dtype=np.float32)),
                        x[r].ctypes.data_as(F32P), out[r].ctypes.data_as(F32P))
    return out


def query_scale(block, n: int) -> np.ndarray:
    b = block.c_struct()
    out = np.zeros(block.d, np.float32)
    lib().orc_query_scale(ctypes.byref(b), int(n), fp(out))
    return out


# ---- a fitted member ------------------------------------------------------------------------------------------
class Fitted:
    """What `fit_raw` writes for one member (`raw_entries`, `src/fit.rs:224-241`), held in memory."""

    def __init__(self, rows, features, classes, chunk, kv_format, plan, col_kv, scales, layers):
        self.rows, self.features, self.classes, self.chunk, self.kv_format = rows, features, classes, chunk, kv_format
        self.plan = plan
        self.digits = len(plan.bases)
        self.col_kv = col_kv          # [features][digits][blocks][2][e][inds]
        self.scales = scales          # per node: [layers][d]
        self.layers = layers          # per node: list of uint8 arrays, one per layer
        self.nodes = planmod.parse_tree(plan.tree(rows), len(plan.nodes))


def _records_array(layers):
    ptrs = (abi.U8P * len(layers))(*[u8(l) for l in layers])
    return ptrs


def fit_columns(model, x, y, bases, chunk):
    rows, features = x.shape
    m = model.desc()
    digits = len(bases)
    col_kv = np.zeros((features, digits, len(model.col_a2), 2, model.e, model.inds), np.float32)
    emb = np.zeros((features, rows, model.e), np.float32)
    b = (ctypes.c_int * digits)(*bases)
    lib().orc_fit_columns(ctypes.byref(m), fp(x), fp(y), rows, features, b, digits, chunk, fp(col_kv), fp(emb))
    return col_kv, emb


def fit_columns_of(model, x, y, groups, bases, chunk):
    """The fit's column stage for the listed feature groups only: col_kv [len(groups)][digits][blocks][2][e][inds]
    and the groups' cells [len(groups)][rows][e]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    rows, features = x.shape
    digits = len(bases)
    col_kv = np.zeros((len(groups), digits, len(model.col_a2), 2, model.e, model.inds), np.float32)
    emb = np.zeros((len(groups), rows, model.e), np.float32)
    gs = (ctypes.c_int * len(groups))(*groups)
    b = (ctypes.c_int * digits)(*bases)
    lib().orc_fit_columns_of(ctypes.byref(model.desc()), fp(x), fp(y), rows, features, gs, len(groups), b, digits,
                             chunk, fp(col_kv), fp(emb))
    return col_kv, emb


def fit_cells_rows(model, col_kv, bases, x, y):
    """The fit's cells [features][n][e] of the given training rows after the column stage, from a fitted column
    cache (col_kv [features][digits][blocks][2][e][inds])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    n, features = x.shape
    emb = np.zeros((features, n, model.e), np.float32)
    b = (ctypes.c_int * len(bases))(*bases)
    lib().orc_fit_cells_rows(ctypes.byref(model.desc()), fp(np.ascontiguousarray(col_kv, dtype=np.float32)), b,
                             len(bases), fp(x), fp(y), n, features, fp(emb))
    return emb


def fit_rows(model, emb):
    features, rows, _ = emb.shape
    reps = np.zeros((rows, model.d), np.float32)
    lib().orc_fit_rows(ctypes.byref(model.desc()), fp(emb), rows, features, fp(reps))
    return reps


def fit_icl(model, h, chunk, kv_format, want_f32=False):
    rows = h.shape[0]
    h = np.ascontiguousarray(h, dtype=np.float32).copy()
    scales = np.zeros((model.icl_layers, model.d), np.float32)
    layers = [np.zeros(abi.layer_bytes(kv_format, rows, chunk, model.d), np.uint8) for _ in range(model.icl_layers)]
    kvf = np.zeros((model.icl_layers, 2 * rows * model.d), np.float32) if want_f32 else None
    lib().orc_fit_icl(ctypes.byref(model.desc()), fp(h), rows, chunk, kv_format, fp(scales), _records_array(layers),
                      fp(kvf) if want_f32 else None)
    return scales, layers, kvf


def fit_raw(model, x, y, classes, chunk=256, kv_format=abi.KV_F32):
    """`fit_raw_async` on the CPU: x [rows][features] f32 (already numeric and normalised), y class indices (or
    standardised targets for regression) as floats."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    rows, features = x.shape
    chunk = max(chunk, 8)
    plan = planmod.Plan.new(model.max_classes, y, classes)
    col_kv, emb = fit_columns(model, x, y, plan.bases, chunk)
    reps = fit_rows(model, emb)
    scales, layers = [], []
    for node in plan.nodes:
        h = reps if node.rows is None else reps[np.array(node.rows, dtype=np.int64)]
        h = np.ascontiguousarray(h, dtype=np.float32).copy()
        model.add_y(model.t["icl_y"], np.array(node.y, np.float32), h)
        s, l, _ = fit_icl(model, h, chunk, kv_format)
        scales.append(s)
        layers.append(l)
    return Fitted(rows, features, classes, chunk, kv_format, plan, col_kv, scales, layers)


def kv_rows(model, layer, h):
    """In-context layer `layer`'s keys and values [n][2d] of given rows h [n][d] (norm1 and the key/value
    projection, `src/fit.rs:627-663`)."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    out = np.zeros((h.shape[0], 2 * model.d), np.float32)
    lib().orc_kv_rows(ctypes.byref(model.desc()), int(layer), fp(h), h.shape[0], fp(out))
    return out


def icl_step(model, layer, scale, records, kv_format, rows, chunk, h):
    """Given rows h [n][d] through one in-context layer over its stored records (a copy is returned)."""
    h = np.ascontiguousarray(h, dtype=np.float32).copy()
    lib().orc_icl_step(ctypes.byref(model.desc()), int(layer), fp(np.ascontiguousarray(scale, dtype=np.float32)),
                       u8(np.ascontiguousarray(records)), int(kv_format), int(rows), int(chunk), fp(h), h.shape[0])
    return h


# ---- prediction ---------------------------------------------------------------------------------------------
def embed(model, fitted, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, features = x.shape
    tokens = model.cls + features
    tok = np.zeros((n, tokens, model.e), np.float32)
    lib().orc_embed(ctypes.byref(model.desc()), fp(fitted.col_kv), fitted.digits, fp(x), n, features, fp(tok))
    return tok


def represent(model, tok):
    n, tokens, _ = tok.shape
    tok = np.ascontiguousarray(tok, dtype=np.float32).copy()
    rep = np.zeros((n, model.d), np.float32)
    lib().orc_represent(ctypes.byref(model.desc()), fp(tok), n, tokens, fp(rep))
    return rep


def in_context(model, scales, layers, kv_format, rows, chunk, h, out_n):
    h = np.ascontiguousarray(h, dtype=np.float32).copy()
    n = h.shape[0]
    out = np.zeros((n, out_n), np.float32)
    lib().orc_in_context(ctypes.byref(model.desc()), fp(np.ascontiguousarray(scales)), _records_array(layers), kv_format,
                         rows, chunk, fp(h), n, out_n, fp(out))
    return out


def predict_raw(model, fitted, x):
    """Scores `[n][classes]` (`predict_raw_async`, `src/predict.rs:638-699`)."""
    tok = embed(model, fitted, x)
    rep = represent(model, tok)
    if len(fitted.nodes) == 1:
        return in_context(model, fitted.scales[0], fitted.layers[0], fitted.kv_format, fitted.rows, fitted.chunk, rep,
                          fitted.classes)
    outs = []
    for ni, node in enumerate(fitted.nodes):
        outs.append(in_context(model, fitted.scales[ni], fitted.layers[ni], fitted.kv_format, node.rows, fitted.chunk,
                               rep, node.k))
    return planmod.tree_scores(fitted.nodes, outs, fitted.classes)
