"""Fitting on the card: the reference's `fit_raw_async` (`src/fit.rs:285-752`) with every stage handed to the
accelerator, as its `fit::Attend` hooks allow (`columns`, `rows`, `in_context`).

The host keeps the reference's host-side work: the label-digit plan and class tree (`Plan`, `src/fit.rs:159-215`),
each block's query scale (`Block::query_scale`, `src/nn.rs:97-107`, restated here in float32 with the reference's
own exp and erf polynomials, `src/kern.rs:185-253`), gathering each in-context problem's rows and adding the
target's embedding (`src/fit.rs:577-585`). The card does the column and row stages (`tah_fit_represent`) and each
problem's in-context stage (`tah_in_context`), which hands back every layer's stored chunk records.
"""
from __future__ import annotations

import os
import threading
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field

import numpy as np

from . import abi
from .bundle import write as bundle_write
from .plan import Plan, parse_tree

F = np.float32

# A layer's records (41 MB at 10,000 rows in f32) are copied out of the card's staging buffer before the sink returns,
# and a fresh array's pages fault in on first touch: one thread took 4.1 ms a layer, longer than the card's own work
# on the next layer, which it holds up. Eight slices on as many threads (numpy releases the interpreter for the copy).
_COPY_THREADS = max(1, min(8, os.cpu_count() or 1))
_COPY_MIN = 1 << 22  # smaller records are copied on the calling thread
_copy_pool = None
_copy_lock = threading.Lock()


def copy_records(rec: np.ndarray) -> np.ndarray:
    """A copy of a layer's records (a 1-D array), sliced over a few threads when large."""
    global _copy_pool
    out = np.empty_like(rec)
    n = rec.size
    if _COPY_THREADS == 1 or n < _COPY_MIN:
        np.copyto(out, rec)
        return out
    with _copy_lock:
        if _copy_pool is None:
            _copy_pool = ThreadPoolExecutor(_COPY_THREADS, thread_name_prefix="tah-records")
    step = -(-n // _COPY_THREADS)
    parts = [(i, min(n, i + step)) for i in range(0, n, step)]
    for f in [_copy_pool.submit(np.copyto, out[a:b], rec[a:b]) for a, b in parts]:
        f.result()
    return out


def exp1(x: np.ndarray) -> np.ndarray:
    """`kern::exp1` (`src/kern.rs:185-206`) in float32."""
    x = np.clip(np.asarray(x, F), F(-87.0), F(88.0))
    n = np.floor(x * F(1.44269504088896340736) + F(0.5))
    r = (x - n * F(0.6933594)) - n * F(-2.1219444e-4)
    p = F(1.0) / F(5040.0)
    for c in (F(1.0) / F(720.0), F(1.0) / F(120.0), F(1.0) / F(24.0), F(1.0) / F(6.0), F(0.5), F(1.0), F(1.0)):
        p = p * r + c
    two = ((n.astype(np.int32) + 127) << 23).astype(np.int32).view(F)
    return (p * two).astype(F)


def erf1(x: np.ndarray) -> np.ndarray:
    """`kern::erf1` (`src/kern.rs:227-253`): Abramowitz and Stegun 7.1.26 away from zero, a series near it."""
    x = np.asarray(x, F)
    a = np.abs(x)
    t = F(1.0) / (F(1.0) + F(0.3275911) * a)
    p = F(1.0614054)
    for c in (F(-1.4531521), F(1.4214138), F(-0.28449674), F(0.2548296)):
        p = p * t + c
    far = np.copysign(F(1.0) - p * t * exp1(-a * a), x)
    x2 = x * x
    q = F(-1.0) / F(1320.0)
    for c in (F(1.0) / F(216.0), F(-1.0) / F(42.0), F(0.1), F(-1.0) / F(3.0), F(1.0)):
        q = q * x2 + c
    near = q * x * F(1.12837916709551257390)
    return np.where(a < F(0.5), near, far).astype(F)


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, F)
    return (F(0.5) * x * (F(1.0) + erf1(x * F(0.70710678118654752440)))).astype(F)


def tanh1(x: np.ndarray) -> np.ndarray:
    """`kern::tanh1` (`src/kern.rs:263-268`): tanh through one exponential, in float32."""
    e = exp1(F(2.0) * np.clip(np.asarray(x, F), F(-10.0), F(10.0)))
    return ((e - F(1.0)) / (e + F(1.0))).astype(F)


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    """`kern::layer_norm` (`src/kern.rs:326-347`) over the last axis: mean, then biased variance, eps 1e-5."""
    x = np.asarray(x, F)
    mean = (x.sum(axis=-1, keepdims=True, dtype=F) / F(x.shape[-1])).astype(F)
    c = (x - mean).astype(F)
    var = ((c * c).sum(axis=-1, keepdims=True, dtype=F) / F(x.shape[-1])).astype(F)
    return (c * (F(1.0) / np.sqrt(var + F(1e-5))) * w + b).astype(F)


def query(block, scale: np.ndarray, x: np.ndarray) -> np.ndarray:
    """`nn::query` (`src/nn.rs:130-152`) for rows x [n][d]: the scaled query projection of norm1(x), modulated per
    head by the block's query MLP when it has one."""
    t = block.t
    d, hd = block.d, block.hd
    q = (layer_norm(x, t["n1w"], t["n1b"]) @ t["in_w"].reshape(3 * d, d)[:d].T + t["in_b"][:d]).astype(F)
    scale = np.asarray(scale, F)
    if block.ss_hidden == 0:
        return (q * scale).astype(F)
    qh = q.reshape(-1, block.heads, hd)
    hid = gelu(qh @ t["q0w"].reshape(block.ss_hidden, hd).T + t["q0b"])
    mm = (hid @ t["q2w"].reshape(hd, block.ss_hidden).T + t["q2b"]).astype(F)
    return (qh * (scale.reshape(block.heads, hd) * (F(1.0) + tanh1(mm)))).reshape(q.shape).astype(F)


def query_scale(block, n: int) -> np.ndarray:
    """`Block::query_scale` (`src/nn.rs:97-107`): what every query of the block is multiplied by with n keys."""
    inv = F(1.0) / np.sqrt(F(block.hd))
    if block.ss_hidden == 0:
        return np.full(block.d, inv, F)
    logn = np.log(F(max(n, 1)))
    hid = gelu(block.t["b0w"] * logn + block.t["b0b"])
    w2 = block.t["b2w"].reshape(block.d, block.ss_hidden)
    # each row's sum left to right in float32, as the reference's matvec rows (accumulate is sequential)
    s = np.add.accumulate((w2 * hid[None, :]).astype(F), axis=1, dtype=F)[:, -1]
    out = (s + block.t["b2b"]).astype(F)
    return (out * inv).astype(F)


def input_cells(m, x: np.ndarray, y: np.ndarray, g0: int, gn: int) -> np.ndarray:
    """The training cells of feature groups g0.. g0 + gn, [rows][gn][e], as `fit_raw_async` builds them for the column
    hook (`src/fit.rs:430-447`): each group's values one, two and four places to the right (`group_values`), the
    input layer (a cell whose values are all -100 stays -100), then the target's embedding (`Model::add_y`)."""
    rows, features = x.shape
    e, group = m.e, m.group
    w_in, b_in = m.t["in_w"].reshape(e, group), m.t["in_b"]
    cells = np.empty((rows, gn, e), F)
    for gi in range(gn):
        vals = x[:, [(g0 + gi + (1 << k)) % features for k in range(group)]]
        c = (vals @ w_in.T + b_in).astype(F)
        c[np.all(vals == F(-100.0), axis=1)] = F(-100.0)
        cells[:, gi] = c
    table = m.t["col_y"]
    if m.max_classes > 0:
        cells += table.reshape(-1, e)[y.astype(np.intp)][:, None, :]
    else:
        tw = table.reshape(2, e)
        cells += (tw[0][None, :] * y[:, None] + tw[1][None, :])[:, None, :]
    return cells


def fit_raw_hooks(gpu, weights, x, y, classes: int, chunk: int = 256, kv_format: int = abi.KV_F32) -> "Fitted":
    """`fit_raw_async` (`src/fit.rs:285-752`) exactly as the reference drives an accelerator through `fit::Attend`:
    the host builds each batch of feature groups' cells and the inducing points' queries, the card's `columns`
    takes as many groups per call as `column_batch` allows, the host regroups the cells by feature, the card's
    `rows` takes `row_batch` rows per call, and `in_context` fits every problem. The reference offers the column
    hook for one label digit only; more digits go through `fit_raw` (the whole column stage on the card)."""
    m = weights.model
    x = np.ascontiguousarray(x, F)
    y = np.ascontiguousarray(y, F)
    rows, features = x.shape
    chunk = max(int(chunk), 8)
    plan = Plan.new(m.max_classes, y, classes)
    if len(plan.bases) != 1:
        raise ValueError("fit_raw_hooks: the column hook takes one label digit; use fit_raw for more")
    e, nb = m.e, len(m.col_a2)
    ind_q = np.stack([query(b, query_scale(b, rows), m.t["col_ind"].reshape(nb, m.inds, e)[i])
                      for i, b in enumerate(m.col_a1)]).astype(F)
    col_batch = gpu.column_batch(weights, rows)
    row_batch = gpu.row_batch(weights, features)
    if col_batch == 0 or row_batch == 0:
        raise ValueError("fit_raw_hooks: the card does not offer the column or row stage at this size")
    emb = np.empty((features, rows, e), F)  # the cells by feature group, as the reference keeps them between stages
    col_kv = np.empty((features, 1, nb, 2, e, m.inds), F)
    for g0 in range(0, features, col_batch):
        gn = min(col_batch, features - g0)
        cells = input_cells(m, x, y, g0, gn)
        col_kv[g0:g0 + gn, 0] = gpu.columns(weights, cells, rows, gn, ind_q)
        emb[g0:g0 + gn] = cells.transpose(1, 0, 2)
    reps = np.empty((rows, m.d), F)
    for r0 in range(0, rows, row_batch):
        rn = min(row_batch, rows - r0)
        reps[r0:r0 + rn] = gpu.rows(weights, np.ascontiguousarray(emb[:, r0:r0 + rn].transpose(1, 0, 2)))
    fitted = Fitted(rows, features, classes, chunk, kv_format, plan, col_kv)
    for node in plan.nodes:
        h = reps.copy() if node.rows is None else reps[np.asarray(node.rows, np.int64)]
        m.add_y(m.t["icl_y"], np.asarray(node.y, F), h)
        scales = np.stack([query_scale(b, rows if node.rows is None else len(node.rows)) for b in m.icl]).astype(F)
        layers = []
        gpu.in_context_fit(weights, h, scales, kv_format, chunk, lambda l, rec: layers.append(copy_records(rec)))
        fitted.scales.append(scales)
        fitted.layers.append(layers)
    return fitted


@dataclass
class Fitted:
    """One fitted member, as `raw_entries` (`src/fit.rs:224-241`) names its tensors: `meta`, `tree`, `col_kv`,
    and per in-context problem `n{j}_scale` and `n{j}_kv{l}`."""
    rows: int
    features: int
    classes: int
    chunk: int
    kv_format: int
    plan: Plan
    col_kv: np.ndarray
    scales: list = field(default_factory=list)
    layers: list = field(default_factory=list)

    @property
    def digits(self) -> int:
        return len(self.plan.bases)

    @property
    def nodes(self):
        return parse_tree(self.plan.tree(self.rows), len(self.plan.nodes))

    def meta(self) -> np.ndarray:
        return np.array([self.rows, self.features, self.classes, self.chunk, self.kv_format, self.digits,
                         len(self.plan.nodes)], np.int32)

    def raw_entries(self, prefix: str = "") -> list:
        """The member's tensors as `raw_entries` declares them (`src/fit.rs:224-241`), in that order: `(name, dtype,
        dims)` of meta, tree, col_kv, then per problem its query scales and every layer's stored records."""
        tree = self.plan.tree(self.rows)
        out = [(f"{prefix}meta", "int32", [7]), (f"{prefix}tree", "int32", [len(tree)]),
               (f"{prefix}col_kv", "float32", list(self.col_kv.shape))]
        for ni, layers in enumerate(self.layers):
            out.append((f"{prefix}n{ni}_scale", "float32", list(np.shape(self.scales[ni]))))
            out += [(f"{prefix}n{ni}_kv{l}", "uint8", [int(rec.size)]) for l, rec in enumerate(layers)]
        return out

    def tensors(self, prefix: str = "") -> dict:
        """name -> array, in `raw_entries` order, for `bundle.write`."""
        t = {f"{prefix}meta": self.meta(), f"{prefix}tree": np.asarray(self.plan.tree(self.rows), np.int32),
             f"{prefix}col_kv": np.ascontiguousarray(self.col_kv, F)}
        for ni, layers in enumerate(self.layers):
            t[f"{prefix}n{ni}_scale"] = np.ascontiguousarray(self.scales[ni], F)
            for l, rec in enumerate(layers):
                t[f"{prefix}n{ni}_kv{l}"] = np.ascontiguousarray(rec, np.uint8)
        return t

    def write(self, path=None, prefix: str = "") -> bytes:
        """The member as a `.tirs` bundle (the bytes; also written to `path` if given)."""
        return bundle_write(path, self.tensors(prefix))


def fit_raw(gpu, weights, x, y, classes: int, chunk: int = 256, kv_format: int = abi.KV_F32) -> Fitted:
    """Fit one table that is already numeric and normalised (`x [rows][features]`, `y` class indices or
    standardised targets) with every stage on the card."""
    m = weights.model
    x = np.ascontiguousarray(x, F)
    y = np.ascontiguousarray(y, F)
    rows, features = x.shape
    chunk = max(int(chunk), 8)
    plan = Plan.new(m.max_classes, y, classes)
    digits = len(plan.bases)
    ind_scales = np.stack([query_scale(b, rows) for b in m.col_a1]).astype(F)
    col_kv, reps = gpu.fit_represent(weights, x, y, plan.bases, ind_scales)
    fitted = Fitted(rows, features, classes, chunk, kv_format, plan, col_kv)
    for node in plan.nodes:
        n_rows = rows if node.rows is None else len(node.rows)
        if node.rows is not None:
            h = reps[np.asarray(node.rows, np.int64)]  # a copy
        elif len(plan.nodes) == 1:
            h = reps  # no other problem reads the representations
        else:
            h = reps.copy()
        m.add_y(m.t["icl_y"], np.asarray(node.y, F), h)
        scales = np.stack([query_scale(b, n_rows) for b in m.icl]).astype(F)
        layers = []
        gpu.in_context_fit(weights, h, scales, kv_format, chunk, lambda l, rec: layers.append(copy_records(rec)))
        fitted.scales.append(scales)
        fitted.layers.append(layers)
    return fitted
