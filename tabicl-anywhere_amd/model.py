"""The network's weights as the card takes them: a `tah_model_desc` (include/tah.h) over numpy float32 arrays.

`Model.load(bundle)` follows the reference's `Model::load` (`src/model.rs:202-272`): it reads `config.json`, refuses
any variant other than the TabICL v2 layout the kernels implement, loads every block (`Block::load`,
`src/model.rs:52-98`; absent layer-norm biases become zeros), and turns the two target encoders into per-class tables
(`class_table`, `src/model.rs:164-177`). `Model.random(config, seed)` makes weights of the same architecture from a
seed, for the synthetic full-size workloads.
"""
from __future__ import annotations

import ctypes
import json

import numpy as np

from . import abi
from .bundle import Bundle

# src/model.rs:203-219: the only variant implemented
REQUIRED = {
    "col_feature_group": "same",
    "col_affine": False,
    "col_target_aware": True,
    "col_ssmax": "qassmax-mlp-elementwise",
    "icl_ssmax": "qassmax-mlp-elementwise",
    "row_rope_interleaved": False,
    "norm_first": True,
    "activation": "gelu",
}

# The published TabICL v2 classifier's sizes (its config.json), the architecture of the full-size workloads.
FULL_CLASSIFIER = {
    "max_classes": 10, "num_quantiles": 999, "embed_dim": 128, "col_num_blocks": 3, "col_nhead": 8,
    "col_num_inds": 128, "col_affine": False, "col_feature_group": "same", "col_feature_group_size": 3,
    "col_target_aware": True, "col_ssmax": "qassmax-mlp-elementwise", "row_num_blocks": 3, "row_nhead": 8,
    "row_num_cls": 4, "row_rope_base": 100000, "row_rope_interleaved": False, "icl_num_blocks": 12, "icl_nhead": 8,
    "icl_ssmax": "qassmax-mlp-elementwise", "ff_factor": 2, "dropout": 0.0, "activation": "gelu", "norm_first": True,
    "bias_free_ln": False, "recompute": False,
}
FULL_REGRESSOR = dict(FULL_CLASSIFIER, max_classes=0, bias_free_ln=True)
# The reference's tiny test architecture (tools/make_tiny.py:15-41): embedding 8, two blocks in each stage, two heads,
# 8 inducing points, 2 class tokens (d = 16), 99 quantiles.
TINY_CLASSIFIER = dict(FULL_CLASSIFIER, num_quantiles=99, embed_dim=8, col_num_blocks=2, col_nhead=2, col_num_inds=8,
                       row_num_blocks=2, row_nhead=2, row_num_cls=2, icl_num_blocks=2, icl_nhead=2)


class ModelError(ValueError):
    pass


def class_table(w: np.ndarray, b: np.ndarray, classes: int) -> np.ndarray:
    """`src/model.rs:164-177`: rows `w[:, c] + b` per class; for regression (classes 0) `[weight][bias]`."""
    out = b.shape[0]
    w = w.reshape(out, -1)
    if classes == 0:
        return np.ascontiguousarray(np.concatenate([w.reshape(-1), b]).astype(np.float32))
    return np.ascontiguousarray((w[:, :classes].T + b[None, :]).astype(np.float32))


class Block:
    """One pre-norm attention block's tensors (`src/model.rs:27-98`)."""

    FIELDS = ("n1w", "n1b", "n2w", "n2b", "in_w", "in_b", "out_w", "out_b", "l1w", "l1b", "l2w", "l2b",
              "b0w", "b0b", "b2w", "b2b", "q0w", "q0b", "q2w", "q2b")

    def __init__(self, d: int, heads: int, t: dict):
        self.d, self.heads = d, heads
        self.t = {k: np.ascontiguousarray(v, dtype=np.float32).reshape(-1) for k, v in t.items() if v is not None}
        self.ff = self.t["l1b"].shape[0]
        self.ss_hidden = self.t["b0b"].shape[0] if "b0b" in self.t else 0

    @property
    def hd(self) -> int:
        return self.d // self.heads

    @classmethod
    def load(cls, b: Bundle, p: str, heads: int) -> "Block":
        g = lambda n: b.f32s(f"{p}.{n}")
        n1w = g("norm1.weight")
        d = n1w.shape[0]
        opt = lambda n: g(n) if b.has(f"{p}.{n}") else np.zeros(d, np.float32)
        t = dict(n1w=n1w, n1b=opt("norm1.bias"), n2w=g("norm2.weight"), n2b=opt("norm2.bias"),
                 in_w=g("attn.in_proj_weight"), in_b=g("attn.in_proj_bias"), out_w=g("attn.out_proj.weight"),
                 out_b=g("attn.out_proj.bias"), l1w=g("linear1.weight"), l1b=g("linear1.bias"),
                 l2w=g("linear2.weight"), l2b=g("linear2.bias"))
        if b.has(f"{p}.attn.ssmax_layer.base_mlp.0.weight"):
            s = lambda n: g(f"attn.ssmax_layer.{n}")
            t.update(b0w=s("base_mlp.0.weight"), b0b=s("base_mlp.0.bias"), b2w=s("base_mlp.2.weight"),
                     b2b=s("base_mlp.2.bias"), q0w=s("query_mlp.0.weight"), q0b=s("query_mlp.0.bias"),
                     q2w=s("query_mlp.2.weight"), q2b=s("query_mlp.2.bias"))
        return cls(d, heads, t)

    def c_struct(self) -> abi.Block:
        s = abi.Block(self.d, self.heads, self.ff, self.ss_hidden)
        for f in self.FIELDS:
            a = self.t.get(f)
            setattr(s, f, a.ctypes.data_as(abi.F32P) if a is not None else None)
        return s


class Model:
    """The weights and sizes of one TabICL v2 network (`src/model.rs:110-143`)."""

    def __init__(self, cfg: dict, t: dict, col_a1, col_a2, row, icl):
        self.cfg = cfg
        self.t = {k: np.ascontiguousarray(v, dtype=np.float32).reshape(-1) for k, v in t.items()}
        self.col_a1, self.col_a2, self.row, self.icl = col_a1, col_a2, row, icl
        self.e = self.t["in_b"].shape[0]
        self.d = self.t["lnw"].shape[0]
        self.group = int(cfg["col_feature_group_size"])
        self.inds = int(cfg["col_num_inds"])
        self.cls = int(cfg["row_num_cls"])
        self.max_classes = int(cfg["max_classes"])
        self.col_heads, self.row_heads, self.icl_heads = int(cfg["col_nhead"]), int(cfg["row_nhead"]), int(cfg["icl_nhead"])
        self.icl_layers = len(icl)
        self.dec_hidden = self.t["dec0b"].shape[0]
        self.outputs = self.t["dec2b"].shape[0]
        self._desc = None

    # ---- construction ---------------------------------------------------------------------------------------
    @classmethod
    def load(cls, b: Bundle) -> "Model":
        cfg = json.loads(b.bytes("config.json").decode("utf-8"))
        for k, v in REQUIRED.items():
            got = cfg.get(k, "(missing)")
            if got != v:
                raise ModelError(f"unsupported checkpoint: {k} is {got}, this crate implements {v}")
        mc = int(cfg["max_classes"])
        e = b.f32s("col_embedder.in_linear.bias").shape[0]
        col_a1, col_a2, inds = [], [], []
        for i in range(int(cfg["col_num_blocks"])):
            p = f"col_embedder.tf_col.blocks.{i}"
            col_a1.append(Block.load(b, f"{p}.multihead_attn1", int(cfg["col_nhead"])))
            col_a2.append(Block.load(b, f"{p}.multihead_attn2", int(cfg["col_nhead"])))
            inds.append(b.f32s(f"{p}.ind_vectors"))
        row = [Block.load(b, f"row_interactor.tf_row.blocks.{i}", int(cfg["row_nhead"])) for i in range(int(cfg["row_num_blocks"]))]
        icl = [Block.load(b, f"icl_predictor.tf_icl.blocks.{i}", int(cfg["icl_nhead"])) for i in range(int(cfg["icl_num_blocks"]))]
        lnw = b.f32s("icl_predictor.ln.weight")
        d = lnw.shape[0]
        cls_ = int(cfg["row_num_cls"])
        t = dict(
            in_w=b.f32s("col_embedder.in_linear.weight"), in_b=b.f32s("col_embedder.in_linear.bias"),
            col_ind=np.concatenate(inds),
            col_y=class_table(b.f32s("col_embedder.y_encoder.weight"), b.f32s("col_embedder.y_encoder.bias"), mc),
            cls_tokens=b.f32s("row_interactor.cls_tokens"), rope_freqs=b.f32s("row_interactor.tf_row.rope.freqs"),
            out_lnw=b.f32s("row_interactor.out_ln.weight"),
            out_lnb=b.f32s("row_interactor.out_ln.bias") if b.has("row_interactor.out_ln.bias") else np.zeros(e, np.float32),
            icl_y=class_table(b.f32s("icl_predictor.y_encoder.weight"), b.f32s("icl_predictor.y_encoder.bias"), mc),
            lnw=lnw, lnb=b.f32s("icl_predictor.ln.bias") if b.has("icl_predictor.ln.bias") else np.zeros(d, np.float32),
            dec0w=b.f32s("icl_predictor.decoder.0.weight"), dec0b=b.f32s("icl_predictor.decoder.0.bias"),
            dec2w=b.f32s("icl_predictor.decoder.2.weight"), dec2b=b.f32s("icl_predictor.decoder.2.bias"),
        )
        assert cls_ * e == d
        return cls(cfg, t, col_a1, col_a2, row, icl)

    @classmethod
    def random(cls, cfg: dict, seed: int) -> "Model":
        """Seeded random-init weights of the architecture `cfg` (PyTorch-like uniform fan-in init, then every
        parameter moved off special values by N(0, 0.1) noise the way the reference's tools/make_tiny.py does, so
        no layer norm sits at exactly 1 and 0). RoPE frequencies are the usual `base^(-2i/hd)`."""
        rng = np.random.default_rng(seed)
        e = int(cfg["embed_dim"])
        cls_ = int(cfg["row_num_cls"])
        d = e * cls_
        ff = int(cfg["ff_factor"])
        mc = int(cfg["max_classes"])
        group = int(cfg["col_feature_group_size"])
        inds = int(cfg["col_num_inds"])
        nq = int(cfg["num_quantiles"])
        bias_free = bool(cfg.get("bias_free_ln", False))

        def lin(o, i):
            bound = 1.0 / np.sqrt(i)
            w = rng.uniform(-bound, bound, (o, i)) + 0.1 * rng.standard_normal((o, i)) * bound
            b = rng.uniform(-bound, bound, o) + 0.1 * rng.standard_normal(o) * bound
            return w.astype(np.float32), b.astype(np.float32)

        def ln(n):
            return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32), (0.1 * rng.standard_normal(n)).astype(np.float32)

        def block(width, heads, ss):
            hd = width // heads
            n1w, n1b = ln(width)
            n2w, n2b = ln(width)
            if bias_free:
                n1b = np.zeros(width, np.float32)
                n2b = np.zeros(width, np.float32)
            in_w, in_b = lin(3 * width, width)
            out_w, out_b = lin(width, width)
            l1w, l1b = lin(width * ff, width)
            l2w, l2b = lin(width, width * ff)
            t = dict(n1w=n1w, n1b=n1b, n2w=n2w, n2b=n2b, in_w=in_w, in_b=in_b, out_w=out_w, out_b=out_b,
                     l1w=l1w, l1b=l1b, l2w=l2w, l2b=l2b)
            if ss:
                b0w, b0b = lin(64, 1)
                b2w, b2b = lin(width, 64)
                q0w, q0b = lin(64, hd)
                q2w, q2b = lin(hd, 64)
                t.update(b0w=b0w, b0b=b0b, b2w=b2w, b2b=b2b, q0w=q0w, q0b=q0b, q2w=q2w, q2b=q2b)
            return Block(width, heads, t)

        col_a1, col_a2, ind = [], [], []
        for _ in range(int(cfg["col_num_blocks"])):
            col_a1.append(block(e, int(cfg["col_nhead"]), True))
            col_a2.append(block(e, int(cfg["col_nhead"]), False))
            ind.append(rng.standard_normal((inds, e)).astype(np.float32))
        row = [block(e, int(cfg["row_nhead"]), False) for _ in range(int(cfg["row_num_blocks"]))]
        icl = [block(d, int(cfg["icl_nhead"]), True) for _ in range(int(cfg["icl_num_blocks"]))]
        hd_row = e // int(cfg["row_nhead"])
        base = float(cfg["row_rope_base"])
        freqs = (base ** (-(2.0 * np.arange(hd_row // 2)) / hd_row)).astype(np.float32)
        in_w, in_b = lin(e, group)
        yin = max(mc, 1)
        cy_w, cy_b = lin(e, yin)
        iy_w, iy_b = lin(d, yin)
        lnw, lnb = ln(d)
        olw, olb = ln(e)
        if bias_free:
            lnb = np.zeros(d, np.float32)
            olb = np.zeros(e, np.float32)
        dec0w, dec0b = lin(2 * d, d)
        outputs = mc if mc > 0 else nq
        dec2w, dec2b = lin(outputs, 2 * d)
        t = dict(in_w=in_w, in_b=in_b, col_ind=np.concatenate(ind), col_y=class_table(cy_w, cy_b, mc),
                 cls_tokens=rng.standard_normal((cls_, e)).astype(np.float32), rope_freqs=freqs,
                 out_lnw=olw, out_lnb=olb, icl_y=class_table(iy_w, iy_b, mc), lnw=lnw, lnb=lnb,
                 dec0w=dec0w, dec0b=dec0b, dec2w=dec2w, dec2b=dec2b)
        return cls(dict(cfg), t, col_a1, col_a2, row, icl)

    # ---- the C view -----------------------------------------------------------------------------------------
    def desc(self) -> abi.ModelDesc:
        """The `tah_model_desc` over this model's arrays (kept alive by this object)."""
        if self._desc is not None:
            return self._desc
        arr = lambda blocks: (abi.Block * len(blocks))(*[b.c_struct() for b in blocks])
        self._a1, self._a2, self._row, self._icl = arr(self.col_a1), arr(self.col_a2), arr(self.row), arr(self.icl)
        p = lambda k: self.t[k].ctypes.data_as(abi.F32P)
        m = abi.ModelDesc()
        m.e, m.d, m.group, m.inds, m.cls, m.max_classes = self.e, self.d, self.group, self.inds, self.cls, self.max_classes
        m.col_heads, m.row_heads, m.icl_heads = self.col_heads, self.row_heads, self.icl_heads
        m.col_blocks, m.row_blocks, m.icl_layers = len(self.col_a2), len(self.row), self.icl_layers
        m.dec_hidden, m.outputs, m.rope_half = self.dec_hidden, self.outputs, self.t["rope_freqs"].shape[0]
        m.in_w, m.in_b = p("in_w"), p("in_b")
        m.col_a1 = ctypes.cast(self._a1, ctypes.POINTER(abi.Block))
        m.col_a2 = ctypes.cast(self._a2, ctypes.POINTER(abi.Block))
        m.col_ind, m.col_y, m.cls_tokens = p("col_ind"), p("col_y"), p("cls_tokens")
        m.row = ctypes.cast(self._row, ctypes.POINTER(abi.Block))
        m.rope_freqs, m.out_lnw, m.out_lnb = p("rope_freqs"), p("out_lnw"), p("out_lnb")
        m.icl = ctypes.cast(self._icl, ctypes.POINTER(abi.Block))
        m.icl_y, m.lnw, m.lnb = p("icl_y"), p("lnw"), p("lnb")
        m.dec0w, m.dec0b, m.dec2w, m.dec2b = p("dec0w"), p("dec0b"), p("dec2w"), p("dec2b")
        self._desc = m
        return m

    def add_y(self, table: np.ndarray, y: np.ndarray, cells: np.ndarray) -> None:
        """`Model::add_y` (`src/model.rs:188-200`) for many rows: `cells [rows][w] += embedding(y)`."""
        w = cells.shape[-1]
        # in blocks of rows, so that the gathered embeddings stay small and cached instead of a fresh array as
        # large as the cells
        if self.max_classes > 0:
            tw, idx = table.reshape(-1, w), y.reshape(-1).astype(np.intp)
            for i in range(0, len(cells), 512):
                cells[i:i + 512] += tw[idx[i:i + 512]]
        else:
            tw, yv = table.reshape(2, w), y.reshape(-1).astype(np.float32)
            for i in range(0, len(cells), 512):
                cells[i:i + 512] += tw[0][None, :] * yv[i:i + 512, None] + tw[1][None, :]
