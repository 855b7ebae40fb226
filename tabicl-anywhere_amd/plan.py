"""Label digits and the class tree: how a table with more classes than the model's native limit is split into
in-context problems. Host-side integer work, bit-exact with the reference.

* `Plan.new` / `Plan._grow` follow `Plan::new` and `Plan::grow` (`src/fit.rs:159-215`): balanced mixed-radix
  bases for the column stage's label digits, and a tree whose inner nodes tell groups of classes apart and whose
  leaves tell the classes of one group apart.
* `Plan.tree` is the stored integer form (`src/fit.rs:217-220`), `parse_tree` its reader (`Cache::open`,
  `src/predict.rs:138-160`).
* `tree_scores` is the prediction-side walk (`src/predict.rs:663-693`): per-node softmax at temperature 0.9,
  probabilities multiplied down the tree, back to scores as `0.9 * ln(p + 1e-6)`.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np


@dataclass
class Node:
    """An in-context problem of the plan. `rows` indexes the training table (None stands for the whole table in its
    own order); `y` holds one target per row in this problem's numbering (a group number at an inner node, a
    within-leaf class number at a leaf); `k` is how many decoder outputs the problem's prediction keeps; `map` sends
    output j to a class (leaf) or to the index of the child problem for group j (inner)."""
    rows: list | None
    y: list
    k: int
    leaf: bool
    map: list = field(default_factory=list)


@dataclass
class Plan:
    bases: list
    nodes: list

    @classmethod
    def new(cls, max_classes: int, y, classes: int) -> "Plan":
        y = [float(v) for v in y]
        mx = max_classes
        if mx == 0 or classes <= mx:
            return cls([max(classes, 1)], [Node(None, list(y), classes, True, list(range(classes)))])
        digits = math.ceil(math.log(classes) / math.log(mx))
        k = min(math.ceil(classes ** (1.0 / digits)), mx)
        bases = [k] * digits
        product = k ** digits
        for i in range(len(bases)):
            if product >= classes:
                break
            if bases[i] < mx:
                product = product // bases[i] * (bases[i] + 1)
                bases[i] += 1
        nodes: list = []
        cls._grow(mx, y, list(range(len(y))), nodes)
        return cls(bases, nodes)

    @staticmethod
    def _grow(mx: int, y, rows, nodes) -> int:
        classes = sorted({int(y[r]) for r in rows})
        at = len(nodes)
        local = {c: i for i, c in enumerate(classes)}
        if len(classes) <= mx:
            nodes.append(Node(list(rows), [float(local[int(y[r])]) for r in rows], len(classes), True, list(classes)))
            return at
        groups = min(-(-len(classes) // mx), mx)
        group_of = [0] * len(classes)
        pos, left = 0, len(classes)
        for g in range(groups):
            size = -(-left // (groups - g))
            for i in range(pos, pos + size):
                group_of[i] = g
            pos += size
            left -= size
        ys = [float(group_of[local[int(y[r])]]) for r in rows]
        nodes.append(Node(list(rows), list(ys), groups, False, []))
        for g in range(groups):
            sub = [r for r, yg in zip(rows, ys) if int(yg) == g]
            child = Plan._grow(mx, y, sub, nodes)
            nodes[at].map.append(child)
        return at

    def tree(self, total_rows: int) -> list:
        out = []
        for n in self.nodes:
            out += [int(n.leaf), total_rows if n.rows is None else len(n.rows), n.k] + [int(v) for v in n.map]
        return out


@dataclass
class NodeInfo:
    leaf: bool
    rows: int
    k: int
    map: list


def parse_tree(tree, n_nodes: int) -> list:
    nodes, at = [], 0
    for _ in range(n_nodes):
        k = int(tree[at + 2])
        nodes.append(NodeInfo(tree[at] != 0, int(tree[at + 1]), k, [int(v) for v in tree[at + 3:at + 3 + k]]))
        at += 3 + k
    return nodes


def tree_scores(nodes, per_node_out, classes: int) -> np.ndarray:
    """Scores `[n][classes]` from each node's raw outputs `[n][k]` (float32, as the reference computes them)."""
    n = per_node_out[0].shape[0]
    probs = []
    for ni, p in enumerate(per_node_out):
        p = np.array(p, dtype=np.float32).reshape(n, nodes[ni].k)
        top = p.max(axis=1, keepdims=True)
        p = np.exp((p - top) / np.float32(0.9)).astype(np.float32)
        p = (p / p.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
        probs.append(p)
    out = np.zeros((n, classes), np.float32)

    def walk(ni, r, weight):
        node = nodes[ni]
        for j, target in enumerate(node.map):
            if node.leaf:
                out[r, target] += np.float32(weight * probs[ni][r, j])
            else:
                walk(target, r, np.float32(weight * probs[ni][r, j]))

    for r in range(n):
        walk(0, r, np.float32(1.0))
    return (np.float32(0.9) * np.log(out + np.float32(1e-6))).astype(np.float32)
