"""The card handle over libtah_hip.so: the Python mirror of the reference's `gpu::Gpu` surface and its two plugin
traits, as the `hip` feature would expose them.

* `Gpu` mirrors `gpu::Gpu` (`src/gpu.rs:725-1019`): `new`, `name`, `set_work_budget`, `work_budget`, `working`,
  `overdrawn`, `release`, `weights` (`GpuWeights::new`), `load` (`VramModel`, from the bundle's stored chunk records
  as they are), `attend_resident` (`src/gpu.rs:2120-2134`) and `in_context` (`src/gpu.rs:2140`).
* `CardAttend` implements `predict::AttendCached` (`src/predict.rs:63-79`): `attend` and `stage` return `None` when
  the card does not hold the problem, and the caller streams on the CPU as usual.

Errors are the reference's: `CardError` ("graphics card: ...", `io::ErrorKind::Other`), `BudgetError`
(`io::ErrorKind::OutOfMemory`), `ValueError` for invalid arguments. Nothing here falls back to another
implementation: without the built library every call raises `abi.LibraryMissing`.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import abi


class CardError(RuntimeError):
    """A failure on the card (the reference's `fail`, `src/gpu.rs:720-722`)."""


class SinkError(RuntimeError):
    """The layer sink of a fit refused a layer."""


class BudgetError(MemoryError):
    """Over the working-memory budget (`io::ErrorKind::OutOfMemory`, `src/gpu.rs:887-889`)."""


def _fp(a: np.ndarray):
    return a.ctypes.data_as(abi.F32P)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _rows_of(a, width: int, what: str) -> np.ndarray:
    """`a` as a contiguous float32 [rows][width] array; anything else is refused before the card reads past it."""
    a = _f32(a)
    if a.ndim != 2 or a.shape[1] != width:
        raise ValueError(f"{what}: expected [rows][{width}] values, got shape {a.shape}")
    return a


def _features_of(vm) -> int:
    f = getattr(vm, "features", 0)
    if not f:
        raise ValueError("the model holds no column cache (VramModel.set_columns)")
    return f


class Gpu:
    """One GPU: its stream, working-memory pool and last error."""

    def __init__(self, ordinal: int = 0):
        self._l = abi.lib()
        h = ctypes.c_void_p()
        rc = self._l.tah_open(int(ordinal), ctypes.byref(h))
        if rc != abi.OK:
            raise CardError(f"graphics card: none found at ordinal {ordinal} (status {rc})")
        self._h = h
        buf = ctypes.create_string_buffer(256)
        self._l.tah_device_name(self._h, buf, 256)
        self.name = buf.value.decode()
        self.software = False

    new = classmethod(lambda cls, ordinal=0: cls(ordinal))

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._l.tah_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int) -> None:
        if rc == abi.OK:
            return
        msg = (self._l.tah_last_error(self._h) or b"").decode()
        if rc == abi.E_BUDGET:
            raise BudgetError(msg)
        if rc == abi.E_ARG:
            raise ValueError(msg)
        if rc == abi.E_DECLINED:
            raise LookupError(msg)
        if rc == abi.E_SINK:
            raise SinkError(msg)
        raise CardError(msg)

    # ---- working memory (Gpu::set_work_budget .. release, src/gpu.rs:975-1019) --------------------------------
    def set_work_budget(self, nbytes: int) -> None:
        self._check(self._l.tah_set_work_budget(self._h, int(nbytes)))

    def work_budget(self) -> int:
        return int(self._l.tah_work_budget(self._h))

    def working(self):
        now, peak = ctypes.c_size_t(), ctypes.c_size_t()
        self._check(self._l.tah_working(self._h, ctypes.byref(now), ctypes.byref(peak)))
        return now.value, peak.value

    def overdrawn(self) -> int:
        return int(self._l.tah_overdrawn(self._h))

    def release(self) -> None:
        self._check(self._l.tah_release(self._h))

    def sync(self) -> None:
        self._check(self._l.tah_sync(self._h))

    @property
    def stream(self) -> int:
        return int(self._l.tah_stream(self._h) or 0)

    # ---- weights and fitted models -----------------------------------------------------------------------------
    def weights(self, model) -> "GpuWeights":
        return GpuWeights(self, model)

    def load(self, weights: "GpuWeights", kv_format: int, rows: int, chunk: int, layers, scales) -> "VramModel":
        return VramModel(self, weights, kv_format, rows, chunk, layers, scales)

    def attend_resident(self, vm: "VramModel", layer: int, q) -> np.ndarray:
        q = _rows_of(q, vm.d, "attend_resident")
        nq = q.shape[0]
        out = np.empty((nq, vm.d), np.float32)
        self._check(self._l.tah_attend_resident(self._h, vm._h, int(layer), _fp(q), nq, _fp(out)))
        return out

    def in_context(self, weights: "GpuWeights", vm: "VramModel", h, out_n: int) -> np.ndarray:
        """The whole in-context stage: row representations `h [n][d]` to the first `out_n` decoder outputs."""
        h = _rows_of(h, vm.d, "in_context")
        nq = h.shape[0]
        out = np.empty((nq, out_n), np.float32)
        self._check(self._l.tah_stage(self._h, weights._h, vm._h, _fp(h), nq, int(out_n), _fp(out)))
        return out

    # ---- the column and row stages, and all three at once (AttendCached::rows) -------------------------------
    def embed(self, weights: "GpuWeights", vm: "VramModel", x) -> np.ndarray:
        """The column stage: x [n][features] to tokens [n][cls + features][e] (`embed`, `src/predict.rs:282-353`)."""
        x = _rows_of(x, _features_of(vm), "embed")
        n = x.shape[0]
        m = weights.model
        tok = np.empty((n, m.cls + vm.features, m.e), np.float32)
        self._check(self._l.tah_embed(self._h, weights._h, vm._h, _fp(x), n, _fp(tok)))
        return tok

    def represent(self, weights: "GpuWeights", tok) -> np.ndarray:
        """The row stage: tokens [n][T][e] to representations [n][d] (`represent`, `src/predict.rs:356-372`)."""
        tok = _f32(tok)
        if tok.ndim != 3 or tok.shape[2] != weights.model.e:
            raise ValueError(f"represent: expected tokens [n][T][{weights.model.e}], got shape {tok.shape}")
        n, T = tok.shape[0], tok.shape[1]
        rep = np.empty((n, weights.model.d), np.float32)
        self._check(self._l.tah_represent(self._h, weights._h, _fp(tok), n, T, _fp(rep)))
        return rep

    def predict(self, weights: "GpuWeights", vm: "VramModel", x, out_n: int) -> np.ndarray:
        """All three stages (`Gpu::predict`, `src/gpu.rs:2146`): x [n][features] to the first out_n outputs."""
        x = _rows_of(x, _features_of(vm), "predict")
        n = x.shape[0]
        out = np.empty((n, out_n), np.float32)
        self._check(self._l.tah_predict_rows(self._h, weights._h, vm._h, _fp(x), n, int(out_n), _fp(out)))
        return out

    def predict_dev(self, weights: "GpuWeights", vm: "VramModel", x_ptr: int, n: int, out_n: int, out_ptr: int) -> None:
        self._check(self._l.tah_predict_rows_dev(self._h, weights._h, vm._h, ctypes.c_void_p(x_ptr), int(n), int(out_n),
                                                 ctypes.c_void_p(out_ptr)))

    # ---- fitting: fit::Attend (src/fit.rs:45-74) ---------------------------------------------------------------
    # the hooks one at a time (Attend::column_batch, columns, row_batch, rows, attend_fits; src/fit.rs:45-74)
    def column_batch(self, weights: "GpuWeights", rows: int) -> int:
        """Feature groups of `rows` cells `columns` takes per call (0: not offered)."""
        return int(self._l.tah_column_batch(self._h, weights._h, int(rows)))

    def columns(self, weights: "GpuWeights", cells, rows: int, groups: int, ind_q) -> np.ndarray:
        """The column stage for `groups` feature groups: `cells` [rows][groups][e] (input layer and target embedding
        applied) is replaced in place by the cells after the stage; returns what col_kv stores for the groups,
        [groups][blocks][2][e][inds]. `ind_q` is each block's inducing-point queries, [blocks][inds][e]."""
        m = weights.model
        if not (isinstance(cells, np.ndarray) and cells.dtype == np.float32 and cells.flags.c_contiguous
                and cells.size == rows * groups * m.e):
            raise ValueError(f"columns: cells must be a contiguous float32 [rows][groups][{m.e}] array")
        ind_q = _f32(ind_q)
        if ind_q.size != len(m.col_a1) * m.inds * m.e:
            raise ValueError(f"columns: ind_q must be [{len(m.col_a1)}][{m.inds}][{m.e}]")
        rec = np.empty((groups, len(m.col_a2), 2, m.e, m.inds), np.float32)
        self._check(self._l.tah_columns(self._h, weights._h, _fp(cells), int(rows), int(groups), _fp(ind_q), _fp(rec)))
        return rec

    def row_batch(self, weights: "GpuWeights", features: int) -> int:
        """Rows of `features` cells `rows` takes per call (0: not offered)."""
        return int(self._l.tah_row_batch(self._h, weights._h, int(features)))

    def rows(self, weights: "GpuWeights", cells) -> np.ndarray:
        """The row stage: cells [n][features][e] to representations [n][d]."""
        m = weights.model
        cells = _f32(cells)
        if cells.ndim != 3 or cells.shape[2] != m.e:
            raise ValueError(f"rows: cells must be [n][features][{m.e}]")
        reps = np.empty((cells.shape[0], m.d), np.float32)
        self._check(self._l.tah_rows(self._h, weights._h, _fp(cells), int(cells.shape[0]), int(cells.shape[1]), _fp(reps)))
        return reps

    def attend_fits(self, rows: int, d: int) -> bool:
        return bool(self._l.tah_attend_fits(self._h, int(rows), int(d)))

    def attend_rows(self, q, k, v, d: int, heads: int) -> np.ndarray:
        """`Gpu::attend_rows`: attention outputs [nq][d] of scaled queries over row-major keys and values [n][d]."""
        q, k, v = _rows_of(q, d, "attend_rows"), _rows_of(k, d, "attend_rows"), _rows_of(v, d, "attend_rows")
        if k.shape != v.shape:
            raise ValueError("attend_rows: keys and values must have the same shape")
        out = np.empty((q.shape[0], d), np.float32)
        self._check(self._l.tah_attend_rows(self._h, _fp(q), _fp(k), _fp(v), q.shape[0], k.shape[0], int(d), int(heads),
                                            _fp(out)))
        return out

    def calibrate(self, ms: float = 100.0) -> float:
        """`Gpu::calibrate`: the card's in-context attention rate in multiply-adds per second."""
        rate = ctypes.c_double()
        self._check(self._l.tah_calibrate(self._h, float(ms), ctypes.byref(rate)))
        return rate.value

    @property
    def stages(self) -> int:
        """Fitting stages the card has done (`Gpu::stages`)."""
        return int(self._l.tah_stages(self._h))

    def probe_attention(self, launches: int) -> None:
        """Bracket each of the next `launches` launches of the many-query attention kernel on this device's stream
        with HIP events (0 disarms). A measurement hook of this library, not of the reference."""
        self._check(self._l.tah_probe_attention(self._h, int(launches)))

    def probe_read(self):
        """(launches recorded since arming or the last read, their summed duration in ms); synchronises."""
        ms, n = ctypes.c_double(), ctypes.c_int32()
        self._check(self._l.tah_probe_read(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return int(n.value), float(ms.value)

    def fit_represent(self, weights: "GpuWeights", x, y, bases, ind_scales):
        """The column and row stages of a fit with the cells kept on the card (`Attend::columns` + `Attend::rows`):
        x [rows][features] normalised, y [rows] class indices or standardised targets, `bases` the label digits'
        bases, ind_scales [col_blocks][e] each block's query scale for the inducing points. Returns
        (col_kv [features][digits][blocks][2][e][inds], reps [rows][d])."""
        m = weights.model
        x, y = _f32(x), _f32(y).reshape(-1)
        if x.ndim != 2 or y.size != x.shape[0]:
            raise ValueError("fit_represent: x must be [rows][features] and y [rows]")
        rows, features = x.shape
        digits = len(bases)
        ind_scales = _f32(ind_scales)
        if ind_scales.size != len(m.col_a1) * m.e:
            raise ValueError(f"fit_represent: ind_scales must be [{len(m.col_a1)}][{m.e}]")
        col_kv = np.empty((features, digits, len(m.col_a2), 2, m.e, m.inds), np.float32)
        reps = np.empty((rows, m.d), np.float32)
        b = (ctypes.c_int32 * digits)(*[int(v) for v in bases])
        self._check(self._l.tah_fit_represent(self._h, weights._h, _fp(x), _fp(y), rows, features, b, digits,
                                              _fp(ind_scales), _fp(col_kv), _fp(reps)))
        return col_kv, reps

    def quantile_stats(self, q, alphas) -> np.ndarray:
        """Per row of a regression member's outputs `q` ([rows][n] predicted quantiles), the row read as a
        distribution (`QuantileDist`, `src/table.rs:292-346`): [rows][3 + len(alphas)] float32 holding the mean, the
        sample variance, the median and the quantiles at `alphas`."""
        q = _f32(q)
        if q.ndim != 2:
            raise ValueError("quantile_stats: q must be [rows][n]")
        a = _f32(np.asarray(alphas, np.float32).reshape(-1))
        out = np.empty((q.shape[0], 3 + a.size), np.float32)
        self._check(self._l.tah_quantile_stats(self._h, _fp(q), int(q.shape[0]), int(q.shape[1]), _fp(a), int(a.size),
                                               _fp(out)))
        return out

    def quantile_stats_dev(self, q_ptr: int, rows: int, n: int, alphas, out_ptr: int) -> None:
        """`quantile_stats` with q ([rows][n]) and the output ([rows][3 + len(alphas)]) in device memory."""
        a = _f32(np.asarray(alphas, np.float32).reshape(-1))
        self._check(self._l.tah_quantile_stats_dev(self._h, ctypes.c_void_p(q_ptr), int(rows), int(n), _fp(a),
                                                   int(a.size), ctypes.c_void_p(out_ptr)))

    def pack(self, c, d: int, rc: int, kv_format: int) -> np.ndarray:
        """One stored chunk record from its f32 keys and values `c` ([2d][rc]), quantised on the card."""
        c = _f32(c).reshape(-1)
        if c.size != 2 * d * rc:
            raise ValueError("pack: c must hold 2 * d * rc floats")
        out = np.empty(abi.kv_record(kv_format, d, rc), np.uint8)
        self._check(self._l.tah_pack(self._h, _fp(c), int(d), int(rc), int(kv_format), out.ctypes.data_as(abi.U8P)))
        return out

    def attend(self, q, kv, rows: int, chunk: int, d: int, heads: int) -> np.ndarray:
        """`Attend::attend`: all rows' attention over the layer's exact f32 keys and values (chunk layout)."""
        q, kv = _f32(q), _f32(kv).reshape(-1)
        if q.size != rows * d or kv.size != 2 * rows * d:
            raise ValueError("attend: q must be [rows][d] and kv 2 * rows * d floats")
        out = np.empty((rows, d), np.float32)
        self._check(self._l.tah_attend(self._h, _fp(q), _fp(kv), int(rows), int(chunk), int(d), int(heads), _fp(out)))
        return out

    def in_context_fit(self, weights: "GpuWeights", h, scales, kv_format: int, chunk: int, sink) -> bool:
        """`Attend::in_context`: fits the in-context stage of one problem on the card. `sink(layer, records)` gets
        each layer's stored records (a uint8 array, valid during the call) in order; returning a true value (or
        raising) stops the fit. Returns True (the card always offers the stage here)."""
        m = weights.model
        h, scales = _rows_of(h, m.d, "in_context_fit"), _f32(scales)
        if scales.size != m.icl_layers * m.d:
            raise ValueError(f"in_context_fit: scales must be [{m.icl_layers}][{m.d}]")
        rows = h.shape[0]
        failure = []

        def call(_ctx, layer, ptr, nbytes):
            try:
                view = np.ctypeslib.as_array(ptr, shape=(nbytes,))
                return 1 if sink(int(layer), view) else 0
            except BaseException as exc:  # surfaced after the call returns
                failure.append(exc)
                return 1

        cb = abi.LAYER_SINK(call)
        rc = self._l.tah_in_context(self._h, weights._h, _fp(h), rows, _fp(scales), int(kv_format), int(chunk), cb, None)
        if failure:
            raise failure[0]
        self._check(rc)
        return True

    # device-pointer forms: inputs already in HBM, work left queued on the handle's stream
    def attend_resident_dev(self, vm: "VramModel", layer: int, q_ptr: int, nq: int, out_ptr: int) -> None:
        self._check(self._l.tah_attend_resident_dev(self._h, vm._h, int(layer), ctypes.c_void_p(q_ptr), int(nq),
                                                    ctypes.c_void_p(out_ptr)))

    def in_context_dev(self, weights: "GpuWeights", vm: "VramModel", h_ptr: int, nq: int, out_n: int, out_ptr: int) -> None:
        self._check(self._l.tah_stage_dev(self._h, weights._h, vm._h, ctypes.c_void_p(h_ptr), int(nq), int(out_n),
                                          ctypes.c_void_p(out_ptr)))


class GpuWeights:
    """A model's weights on the card (`GpuWeights`, `src/gpu.rs:1838-2027`)."""

    def __init__(self, gpu: Gpu, model):
        self.gpu, self.model = gpu, model
        h = ctypes.c_void_p()
        gpu._check(gpu._l.tah_weights_upload(gpu._h, ctypes.byref(model.desc()), ctypes.byref(h)))
        self._h = h

    def bytes(self) -> int:
        return int(self.gpu._l.tah_weights_bytes(self._h))

    def free(self) -> None:
        if getattr(self, "_h", None):
            self.gpu._l.tah_weights_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class VramModel:
    """One fitted in-context problem held on the card (`VramModel`, `src/gpu.rs:2033-2116`): every layer's stored
    chunk records as they are in the bundle (`n{j}_kv{l}`), and the layers' query scales (`n{j}_scale`)."""

    def __init__(self, gpu: Gpu, weights: GpuWeights, kv_format: int, rows: int, chunk: int, layers, scales):
        self.gpu, self.weights = gpu, weights
        self.kv_format, self.rows, self.chunk = int(kv_format), int(rows), int(chunk)
        self.d = weights.model.d
        want = abi.layer_bytes(self.kv_format, self.rows, self.chunk, self.d)
        bufs = [np.ascontiguousarray(l, dtype=np.uint8).reshape(-1) for l in layers]
        if len(bufs) != weights.model.icl_layers or any(b.nbytes != want for b in bufs):
            raise ValueError(f"model: expected {weights.model.icl_layers} layers of {want} bytes")
        ptrs = (abi.U8P * len(bufs))(*[b.ctypes.data_as(abi.U8P) for b in bufs])
        scales = _f32(scales)
        h = ctypes.c_void_p()
        gpu._check(gpu._l.tah_model_load(gpu._h, weights._h, self.kv_format, self.rows, self.chunk, ptrs, _fp(scales),
                                         ctypes.byref(h)))
        self._h = h

    def set_columns(self, col_kv, features: int, digits: int) -> None:
        """Hold the member's column cache too (`col_kv`, [features][digits][blocks][2][e][inds])."""
        m = self.weights.model
        col_kv = _f32(col_kv).reshape(-1)
        if col_kv.size != features * digits * len(m.col_a2) * 2 * m.e * m.inds:
            raise ValueError("set_columns: col_kv has the wrong size")
        self.gpu._check(self.gpu._l.tah_model_set_columns(self.gpu._h, self._h, self.weights._h, _fp(col_kv),
                                                          int(features), int(digits)))
        self.features, self.digits = int(features), int(digits)

    def bytes(self) -> int:
        """Card bytes this problem holds now: its layers as loaded, plus its column cache and the column blocks'
        key/value images once `set_columns` has run."""
        return int(self.gpu._l.tah_model_held_bytes(self._h)) if getattr(self, "_h", None) else 0

    @staticmethod
    def columns_bytes(weights: "GpuWeights", features: int, digits: int) -> int:
        """Card bytes `set_columns` adds: the column cache and the column blocks' key/value images made from it."""
        return int(abi.lib().tah_columns_bytes(weights._h, int(features), int(digits)))

    @staticmethod
    def model_bytes(weights: "GpuWeights", kv_format: int, rows: int, chunk: int) -> int:
        """Card bytes a problem of `rows` stored rows takes once loaded (`Gpu::model_bytes`, src/gpu.rs:2064-2068):
        the records as stored, plus for head width 64 the split-fp16 tile images the card makes of them."""
        return int(abi.lib().tah_model_bytes(weights._h, kv_format, rows, chunk))

    def free(self) -> None:
        if getattr(self, "_h", None):
            self.gpu._l.tah_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class CardAttend:
    """`predict::AttendCached` over problems held on the card, keyed by `(prefix, node)`."""

    def __init__(self, gpu: Gpu, weights: GpuWeights):
        self.gpu, self.weights = gpu, weights
        self.models: dict = {}

    def hold(self, prefix: str, node: int, vm: VramModel) -> None:
        self.models[(prefix, node)] = vm

    def attend(self, prefix: str, node: int, layer: int, q, d: int, heads: int):
        vm = self.models.get((prefix, node))
        if vm is None or d != vm.d:
            return None
        return self.gpu.attend_resident(vm, layer, q)

    def stage(self, prefix: str, node: int, h, d: int, out_n: int):
        vm = self.models.get((prefix, node))
        if vm is None or d != vm.d:
            return None
        return self.gpu.in_context(self.weights, vm, h, out_n)

    def rows(self, prefix: str, x, out_n: int):
        vm = self.models.get((prefix, 0))
        if vm is None or not getattr(vm, "features", 0) or vm.digits != 1:
            return None
        return self.gpu.predict(self.weights, vm, x, out_n)
