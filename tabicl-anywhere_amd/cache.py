"""A fitted member read from its bundle, and put on the card as stored.

`Cache.open(bundle, prefix)` follows `Cache::open` (`src/predict.rs:138-160`): the member's `meta` (rows, features,
classes, chunk, key/value format, label digits, problems) and its class tree. The layers' stored records
(`n{j}_kv{l}`), the query scales (`n{j}_scale`) and the column cache (`col_kv`) stay in the bundle's bytes; `load`
hands those bytes to the card as they are (`tah_model_load`, `tah_model_set_columns`), one `VramModel` per
in-context problem, with no re-layout on the host (compare the reference's `layer_rows`, `src/predict.rs:590-629`).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .bundle import Bundle, BundleError
from .plan import parse_tree


@dataclass
class Cache:
    bundle: Bundle
    prefix: str
    rows: int
    features: int
    classes: int
    chunk: int
    kv_format: int
    digits: int
    nodes: list

    @classmethod
    def open(cls, bundle: Bundle, prefix: str = "") -> "Cache":
        meta = bundle.i32s(f"{prefix}meta")
        if meta.size != 7 or np.any(meta < 0) or meta[4] > 2:
            raise BundleError(f"{prefix}meta: not a fitted member's description")
        tree = bundle.i32s(f"{prefix}tree")
        nodes = parse_tree(tree, int(meta[6]))
        return cls(bundle, prefix, int(meta[0]), int(meta[1]), int(meta[2]), int(meta[3]), int(meta[4]), int(meta[5]),
                   nodes)

    def col_kv(self) -> np.ndarray:
        return self.bundle.array(f"{self.prefix}col_kv")

    def scales(self, node: int) -> np.ndarray:
        return self.bundle.array(f"{self.prefix}n{node}_scale")

    def layers(self, node: int, count: int) -> list:
        """The stored records of problem `node`'s layers, as views of the bundle's bytes."""
        return [self.bundle.raw(f"{self.prefix}n{node}_kv{l}") for l in range(count)]

    def load(self, gpu, weights) -> list:
        """Every in-context problem of the member on the card (`VramModel`s, in node order), the first holding the
        member's column cache too."""
        m = weights.model
        vms = [gpu.load(weights, self.kv_format, node.rows, self.chunk, self.layers(i, m.icl_layers), self.scales(i))
               for i, node in enumerate(self.nodes)]
        vms[0].set_columns(self.col_kv(), self.features, self.digits)
        return vms
