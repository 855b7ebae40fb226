"""The table-level host work around the path (the caller side of the hot path), restated from the reference's
`src/table.rs` so that a whole ensemble's answer can be checked end to end:

* `member_inputs`: a member's view of a preprocessed table, its feature order and class relabelling
  (`src/table.rs:136-147`, `src/table.rs:245-256`);
* `add_logits`: the members' raw scores summed in float64 in class order (`logit_sums`, `src/table.rs:242-272`);
* `finish_proba`: temperature softmax over the sum (`src/table.rs:70-78`);
* `QuantileDist` and `add_regression`: a regression member's 999 (or 99) quantile outputs read as a distribution,
  and the members' means, variances, medians and quantiles averaged (`src/table.rs:292-346`, `src/table.rs:457-496`).

Preprocessing itself (`src/prep.rs`) stays out of this build: tables arrive already normalised.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Member:
    norm: int        # which normalisation variant of the table
    features: list   # feature order
    classes: list    # class relabelling: member sees class c as classes[c]


def encode_labels(labels):
    """Arbitrary integer labels to class indices `0..classes` in increasing label order, and the sorted distinct
    labels that map them back (`encode_labels`, `src/table.rs:42-48`)."""
    labels = np.asarray(labels, np.int64).reshape(-1)
    classes = np.unique(labels)
    return np.searchsorted(classes, labels).astype(np.int64), classes


def member_inputs(table: np.ndarray, m: Member, y=None):
    """`xs[r][j] = table[r][features[j]]` as float32, and `ys[r] = classes[y[r]]` (`src/table.rs:136-147`)."""
    xs = np.ascontiguousarray(np.asarray(table, np.float64)[:, m.features].astype(np.float32))
    if y is None:
        return xs
    return xs, np.array([m.classes[int(c)] for c in y], np.float32)


def add_logits(avg: np.ndarray, logits: np.ndarray, m: Member) -> None:
    """`avg[r][c] += logits[r][classes[c]]` in float64 (`src/table.rs:265-269`)."""
    avg += np.asarray(logits, np.float32)[:, np.asarray(m.classes, np.int64)].astype(np.float64)


def finish_proba(sums: np.ndarray, members: int, temperature: float) -> np.ndarray:
    """`src/table.rs:70-78`: softmax of the summed scores at `members * temperature`, in float64."""
    inv = 1.0 / (members * temperature)
    out = np.exp((sums - sums.max(axis=1, keepdims=True)) * inv)
    return out / out.sum(axis=1, keepdims=True)


def _seq_sum(a) -> np.float32:
    """A float32 sum left to right, the order of Rust's `iter().sum::<f32>()`."""
    a = np.asarray(a, np.float32)
    return np.add.accumulate(a, dtype=np.float32)[-1] if a.size else np.float32(0.0)


def _total_sort(q) -> np.ndarray:
    """Sorted by the total order of float32 (`f32::total_cmp`: -0 before +0, NaNs by sign at the ends)."""
    q = np.asarray(q, np.float32)
    u = q.view(np.uint32)
    key = u ^ np.where(u >> 31 != 0, np.uint32(0xFFFFFFFF), np.uint32(0x80000000))
    return q[np.argsort(key, kind="stable")]


class QuantileDist:
    """`src/table.rs:292-346`: sorted quantiles at levels i/(n+1), linear between them, exponential tails fitted by
    least squares to the first and last k = clamp(n/4, 1, 20) points, all in float32 with the reference's left-to-right
    sums."""

    def __init__(self, q):
        f = np.float32
        q = _total_sort(q)
        n = q.size
        self.q = q
        self.levels = (np.arange(1, n + 1, dtype=f) / f(n + 1)).astype(f)
        k = max(min(20, n // 4), 1)

        def slope(xs, ys):
            mx = f(_seq_sum(xs) / f(k))
            my = f(_seq_sum(ys) / f(k))
            cov = f(_seq_sum((xs - mx) * (ys - my)) / f(k))
            var = f(_seq_sum((xs - mx) * (xs - mx)) / f(k))
            return f(min(max(abs(cov / max(var, f(1e-6))), f(0.01)), f(100.0)))

        ln_l = np.log(np.maximum(self.levels[:k], f(1e-6))).astype(f)
        ln_r = np.log(np.maximum(f(1.0) - self.levels[n - k:], f(1e-6))).astype(f)
        bl, br = slope(ln_l, q[:k]), slope(ln_r, q[n - k:])
        self.tail_l = (bl, f(q[0] - bl * np.log(max(self.levels[0], f(1e-6)))))
        self.tail_r = (f(-br), f(q[n - 1] + br * np.log(f(1.0) - min(self.levels[n - 1], f(1.0 - 1e-6)))))

    def mean(self) -> np.float32:
        return np.float32(_seq_sum(self.q) / np.float32(self.q.size))

    def variance(self) -> np.float32:
        m = self.mean()
        return np.float32(_seq_sum((self.q - m) * (self.q - m)) / np.float32(self.q.size - 1))

    def icdf(self, alpha) -> np.float32:
        f = np.float32
        alpha = f(alpha)
        n = self.q.size
        lv = self.levels
        if alpha < lv[0]:
            return f(self.tail_l[0] * np.log(max(alpha, f(1e-6))) + self.tail_l[1])
        if alpha > lv[n - 1]:
            return f(self.tail_r[0] * np.log(max(f(1.0) - alpha, f(1e-6))) + self.tail_r[1])
        if alpha >= lv[n - 1]:
            return self.q[n - 1]
        i = int(np.searchsorted(lv[:n - 1], alpha, side="right"))
        i = min(max(i - 1, 0), n - 2)
        t = f(min(max((alpha - lv[i]) / max(lv[i + 1] - lv[i], f(1e-6)), f(0.0)), f(1.0)))
        return f(self.q[i] + t * (self.q[i + 1] - self.q[i]))


def add_regression(out: dict, outputs: np.ndarray, alphas, target_mean: float, target_scale: float,
                   gpu=None) -> None:
    """One member's contribution to `Regression` (`src/table.rs:472-490`): per row, the quantile distribution's
    mean, variance, median and quantiles at `alphas`, mapped back to the target's units, added in float64. With a
    card (`hip.Gpu`), the rows are read as distributions there (`tah_quantile_stats`), all at once."""
    if gpu is not None:
        st = gpu.quantile_stats(outputs, alphas).astype(np.float64) * target_scale + target_mean
        out["mean"] += st[:, 0]
        out["variance"] += st[:, 1]
        out["median"] += st[:, 2]
        out["quantiles"] += st[:, 3:]
        return
    back = lambda v: float(v) * target_scale + target_mean
    for r, row in enumerate(np.asarray(outputs, np.float32)):
        d = QuantileDist(row)
        out["mean"][r] += back(d.mean())
        out["variance"][r] += back(d.variance())
        out["median"][r] += back(d.icdf(0.5))
        for a, alpha in enumerate(alphas):
            out["quantiles"][r, a] += back(d.icdf(alpha))
