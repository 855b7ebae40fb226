"""ctypes mirror of include/tah.h: the two descriptor structs, the status codes, and the loader of libtah_hip.so.

The library is built in-tree (`tabicl-anywhere_amd/libtah_hip.so`, see `csrc/Makefile`); importing a function that
needs it raises `LibraryMissing` if it has not been built, never falls back to anything else.
"""
from __future__ import annotations

import ctypes
import os

F32P = ctypes.POINTER(ctypes.c_float)
U8P = ctypes.POINTER(ctypes.c_uint8)

OK, E_ARG, E_BUDGET, E_DEVICE, E_DECLINED, E_SINK = 0, 1, 2, 3, 4, 5
KV_F32, KV_I16, KV_I8 = 0, 1, 2
KV_NAMES = {"f32": KV_F32, "i16": KV_I16, "i8": KV_I8}

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtah_hip.so")


class Block(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("d", "heads", "ff", "ss_hidden")] + [
        (n, F32P) for n in ("n1w", "n1b", "n2w", "n2b", "in_w", "in_b", "out_w", "out_b", "l1w", "l1b", "l2w",
                            "l2b", "b0w", "b0b", "b2w", "b2b", "q0w", "q0b", "q2w", "q2b")]


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("e", "d", "group", "inds", "cls", "max_classes", "col_heads",
                                              "row_heads", "icl_heads", "col_blocks", "row_blocks", "icl_layers",
                                              "dec_hidden", "outputs", "rope_half")] + [
        ("in_w", F32P), ("in_b", F32P), ("col_a1", ctypes.POINTER(Block)), ("col_a2", ctypes.POINTER(Block)),
        ("col_ind", F32P), ("col_y", F32P), ("cls_tokens", F32P), ("row", ctypes.POINTER(Block)),
        ("rope_freqs", F32P), ("out_lnw", F32P), ("out_lnb", F32P), ("icl", ctypes.POINTER(Block)),
        ("icl_y", F32P), ("lnw", F32P), ("lnb", F32P), ("dec0w", F32P), ("dec0b", F32P), ("dec2w", F32P),
        ("dec2b", F32P)]


# int (*tah_layer_sink)(void *ctx, int32_t layer, const uint8_t *records, size_t bytes)
LAYER_SINK = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int32, U8P, ctypes.c_size_t)


def kv_record(kv_format: int, d: int, rc: int) -> int:
    """`Kv::record` (`src/fit.rs:123-126`): bytes of one stored chunk of `rc` rows."""
    w = {KV_F32: 4, KV_I16: 2, KV_I8: 1}[kv_format]
    return 2 * d * rc * w + (0 if kv_format == KV_F32 else 8 * d)


def layer_bytes(kv_format: int, rows: int, chunk: int, d: int) -> int:
    """Bytes of one stored in-context layer (`raw_entries`, `src/fit.rs:233-234`)."""
    return (rows // chunk) * kv_record(kv_format, d, chunk) + (kv_record(kv_format, d, rows % chunk) if rows % chunk else 0)


class LibraryMissing(RuntimeError):
    pass


_lib = None


def lib():
    """The loaded libtah_hip.so (raises `LibraryMissing` if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(f"{LIB_PATH} is not built; run __graft_entry__.build() (or make -C csrc)")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


# every function include/tah.h declares, with its ctypes signature
SIGNATURES = {
    "tah_kv_record": (ctypes.c_size_t, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
    "tah_open": (ctypes.c_int, [ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p)]),
    "tah_close": (None, [ctypes.c_void_p]),
    "tah_last_error": (ctypes.c_char_p, [ctypes.c_void_p]),
    "tah_device_name": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]),
    "tah_set_work_budget": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t]),
    "tah_work_budget": (ctypes.c_size_t, [ctypes.c_void_p]),
    "tah_working": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "tah_overdrawn": (ctypes.c_size_t, [ctypes.c_void_p]),
    "tah_release": (ctypes.c_int, [ctypes.c_void_p]),
    "tah_sync": (ctypes.c_int, [ctypes.c_void_p]),
    "tah_stream": (ctypes.c_void_p, [ctypes.c_void_p]),
    "tah_weights_upload": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ModelDesc), ctypes.POINTER(ctypes.c_void_p)]),
    "tah_weights_bytes": (ctypes.c_size_t, [ctypes.c_void_p]),
    "tah_weights_free": (None, [ctypes.c_void_p]),
    "tah_model_bytes": (ctypes.c_size_t, [ctypes.c_void_p] + [ctypes.c_int32] * 3),
    "tah_model_load": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.POINTER(U8P), F32P, ctypes.POINTER(ctypes.c_void_p)]),
    "tah_model_free": (None, [ctypes.c_void_p]),
    "tah_attend_resident": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, F32P, ctypes.c_int32, F32P]),
    "tah_attend_resident_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                               ctypes.c_int32, ctypes.c_void_p]),
    "tah_stage": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32,
                                 ctypes.c_int32, F32P]),
    "tah_stage_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "tah_stage_dev_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "tah_model_set_columns": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32,
                                             ctypes.c_int32]),
    "tah_columns_bytes": (ctypes.c_size_t, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32]),
    "tah_model_held_bytes": (ctypes.c_size_t, [ctypes.c_void_p]),
    "tah_embed": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32, F32P]),
    "tah_represent": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32, ctypes.c_int32, F32P]),
    "tah_predict_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32,
                                        ctypes.c_int32, F32P]),
    "tah_predict_rows_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    "tah_fit_represent": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, F32P, F32P, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, F32P, F32P, F32P]),
    "tah_pack": (ctypes.c_int, [ctypes.c_void_p, F32P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, U8P]),
    "tah_attend": (ctypes.c_int, [ctypes.c_void_p, F32P, F32P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                  ctypes.c_int32, F32P]),
    "tah_in_context": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32, F32P, ctypes.c_int32,
                                      ctypes.c_int32, LAYER_SINK, ctypes.c_void_p]),
    "tah_column_batch": (ctypes.c_size_t, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32]),
    "tah_columns": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32, ctypes.c_int32, F32P, F32P]),
    "tah_row_batch": (ctypes.c_size_t, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32]),
    "tah_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, F32P, ctypes.c_int32, ctypes.c_int32, F32P]),
    "tah_attend_fits": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32]),
    "tah_attend_rows": (ctypes.c_int, [ctypes.c_void_p, F32P, F32P, F32P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32, F32P]),
    "tah_calibrate": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_double, ctypes.POINTER(ctypes.c_double)]),
    "tah_stages": (ctypes.c_uint64, [ctypes.c_void_p]),
    "tah_probe_attention": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    "tah_probe_read": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int32)]),
    "tah_quantile_stats": (ctypes.c_int, [ctypes.c_void_p, F32P, ctypes.c_int32, ctypes.c_int32, F32P,
                                          ctypes.c_int32, F32P]),
    "tah_quantile_stats_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, F32P,
                                              ctypes.c_int32, ctypes.c_void_p]),
}


def _declare(l) -> None:
    for name, (res, args) in SIGNATURES.items():
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args
