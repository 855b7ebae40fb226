"""TEST INFRASTRUCTURE ONLY: the reference's table preprocessing and ensemble layout (`src/prep.rs`), restated in
float64 numpy so that the golden tables' raw inputs (x_train, x_test) can be turned into what the hot path takes.
Only tests/ use it, to prepare inputs for the card and for the oracle alike and to check the preprocessing itself
against the fixtures' own transformed tables (`train_none`, `train_power`, `test_*`, `lambdas`) at 1e-6, as
`tests/reference.rs:149-181` does.

The steps follow the reference's, because the numbers must agree:
* missing cells take the column's training mean; columns with one distinct value are dropped (`Prep::fit`,
  `src/prep.rs:393-435`);
* standardise, clip to +-100; for the power variant a Yeo-Johnson transform with the maximum-likelihood exponent
  (bounded Brent search, `src/prep.rs:158-295`) and a second standardisation; then outliers beyond 4 deviations
  (estimated twice) pulled in logarithmically (`ColNorm::fit`, `src/prep.rs:330-371`);
* the ensemble's feature orders and class shifts come from Python's own `random.Random` (Mersenne Twister), which
  the reference reimplements bit for bit (`PyRandom`, `src/prep.rs:17-85`) to match its upstream's member list.
"""
from __future__ import annotations

import math
import random
from dataclasses import dataclass, field

import numpy as np

EPS = np.finfo(np.float64).eps
TINY = np.finfo(np.float64).tiny
HUGE = np.finfo(np.float64).max


# ---- Python's random, as the reference's PyRandom --------------------------------------------------------------
def py_random(seed: int) -> random.Random:
    """`PyRandom::new(seed)` is Python's `random.Random(seed)`; `below(n)` is its `randrange(n)` and `shuffle` its
    `shuffle` (`src/prep.rs:17-85`)."""
    return random.Random(seed)


def latin_orders(n: int, seed: int) -> list:
    """The rows of a random Latin square of side n, as column orders (`latin_orders`, `src/prep.rs:88-108`)."""
    rng = py_random(seed)
    symbols = list(range(n))
    picks = []
    while len(symbols) > 1:
        picks.append(symbols.pop(rng.randrange(len(symbols))))
    square = [symbols]
    for sym in reversed(picks):
        square.append(list(square[0]))
        for i, row in enumerate(square):
            row.insert(i, sym)
    rng.shuffle(square)
    cols = [[row[c] for row in square] for c in range(n)]
    rng.shuffle(cols)
    return cols


@dataclass
class Member:
    norm: int
    features: list
    classes: list


def ensemble(n_features: int, n_classes: int, n_norms: int, n_estimators: int, seed: int) -> list:
    """The members (`ensemble`, `src/prep.rs:120-137`): feature orders from the Latin square (identity for one
    member), every circular class shift, the (order, shift) pairs shuffled, each with every normalisation in turn."""
    if n_estimators == 1:
        feats = [list(range(n_features))]
        classes = [list(range(n_classes))]
    else:
        feats = latin_orders(n_features, seed)
        classes = [[(c + n_classes - i) % n_classes for c in range(n_classes)] for i in range(n_classes)]
    configs = [(f, c) for f in range(len(feats)) for c in range(len(classes))]
    py_random(seed).shuffle(configs)
    out = []
    for f, c in configs:
        for norm in range(n_norms):
            if len(out) == n_estimators:
                return out
            out.append(Member(norm, list(feats[f]), list(classes[c])))
    return out


# ---- the Yeo-Johnson power transform ---------------------------------------------------------------------------
def yeo_johnson(x, lam: float) -> np.ndarray:
    """`yeo_johnson` (`src/prep.rs:151-166`), elementwise."""
    x = np.asarray(x, np.float64)
    out = np.empty_like(x)
    pos = x >= 0
    if abs(lam) < EPS:
        out[pos] = np.log1p(x[pos])
    else:
        out[pos] = np.expm1(lam * np.log1p(x[pos])) / lam
    neg = ~pos
    if abs(lam - 2.0) > EPS:
        out[neg] = -np.expm1((2.0 - lam) * np.log1p(-x[neg])) / (2.0 - lam)
    else:
        out[neg] = -np.log1p(-x[neg])
    return out


def minimize_bounded(f, a: float, b: float, xtol: float) -> float:
    """The bounded Brent minimiser (golden section with parabolic steps, SciPy's `fminbound`), step for step as
    `minimize_bounded` (`src/prep.rs:170-256`), at most 500 steps."""
    sqrt_eps = math.sqrt(2.2e-16)
    golden = 0.5 * (3.0 - math.sqrt(5.0))
    fulc = a + golden * (b - a)
    nfc = xf = fulc
    rat = e = 0.0
    fx = f(xf)
    ffulc = fnfc = fx
    xm = 0.5 * (a + b)
    tol1 = sqrt_eps * abs(xf) + xtol / 3.0
    tol2 = 2.0 * tol1
    sign = lambda v: 1.0 if v > 0 else (-1.0 if v < 0 else 0.0)
    for _ in range(500):
        if abs(xf - xm) <= tol2 - 0.5 * (b - a):
            break
        use_golden = True
        if abs(e) > tol1:
            use_golden = False
            r = (xf - nfc) * (fx - ffulc)
            q = (xf - fulc) * (fx - fnfc)
            p = (xf - fulc) * q - (xf - nfc) * r
            q = 2.0 * (q - r)
            if q > 0.0:
                p = -p
            q = abs(q)
            r = e
            e = rat
            if abs(p) < abs(0.5 * q * r) and q * (a - xf) < p < q * (b - xf):
                rat = p / q
                x = xf + rat
                if x - a < tol2 or b - x < tol2:
                    rat = tol1 * (sign(xm - xf) + (1.0 if xm - xf == 0.0 else 0.0))
            else:
                use_golden = True
        if use_golden:
            e = (a - xf) if xf >= xm else (b - xf)
            rat = golden * e
        x = xf + (sign(rat) + (1.0 if rat == 0.0 else 0.0)) * max(abs(rat), tol1)
        fu = f(x)
        if fu <= fx:
            if x >= xf:
                a = xf
            else:
                b = xf
            fulc, ffulc = nfc, fnfc
            nfc, fnfc = xf, fx
            xf, fx = x, fu
        else:
            if x < xf:
                a = x
            else:
                b = x
            if fu <= fnfc or nfc == xf:
                fulc, ffulc = nfc, fnfc
                nfc, fnfc = x, fu
            elif fu <= ffulc or fulc == xf or fulc == nfc:
                fulc, ffulc = x, fu
        xm = 0.5 * (a + b)
        tol1 = sqrt_eps * abs(xf) + xtol / 3.0
        tol2 = 2.0 * tol1
    return xf


def _var(x, m, ddof: int) -> float:
    return float(np.sum((x - m) * (x - m)) / (len(x) - ddof))


def yeo_johnson_lambda(x) -> float:
    """The exponent that makes x look most normal (maximum likelihood) over the range where the transform cannot
    overflow (`yeo_johnson_lambda`, `src/prep.rs:260-292`)."""
    x = np.asarray(x, np.float64)
    if np.all(x == 0.0):
        return 1.0
    big = float(np.max(np.abs(x)))
    log1p_max = math.log1p(20.0 * big)
    log_eps = math.log(EPS)
    lb = (math.log(TINY) - log_eps) / 2.0 / log1p_max
    ub = (math.log(HUGE) + log_eps) / 2.0 / log1p_max
    if np.all(x < 0.0):
        lb, ub = 2.0 - ub, 2.0 - lb
    elif np.any(x < 0.0):
        lb, ub = max(2.0 - ub, lb), min(2.0 - lb, ub)
    n = float(len(x))
    jac = float(np.sum(np.sign(x) * np.log1p(np.abs(x))))

    def neg_llf(lam):
        y = yeo_johnson(x, lam)
        s = _var(y, float(np.mean(y)), 0)
        logvar = math.log(s) if s >= TINY else -math.inf
        llf = -n / 2.0 * logvar + (lam - 1.0) * jac
        return math.inf if (math.isinf(llf) or math.isnan(llf)) else -llf

    return minimize_bounded(neg_llf, lb, ub, 1.48e-8)


def _is_constant(var: float, mean: float, n: int) -> bool:
    """scikit-learn's "constant to floating point" test (`src/prep.rs:295-299`)."""
    return var <= n * EPS * var + (n * mean * EPS) ** 2


@dataclass
class ColNorm:
    """What one normalisation variant keeps of one column (`ColNorm`, `src/prep.rs:302-315`)."""
    mean: float = 0.0
    scale: float = 1.0
    lam: float = 1.0
    pmean: float = 0.0
    pscale: float = 1.0
    lower: float = 0.0
    upper: float = 0.0

    @classmethod
    def fit(cls, col: np.ndarray, power: bool, threshold: float):
        """Learn from the column's (imputed) training values; returns the norm and the transformed values."""
        n = len(col)
        c = cls()
        c.mean = float(np.mean(col))
        c.scale = math.sqrt(_var(col, c.mean, 0)) + 1e-6
        col = np.clip((col - c.mean) / c.scale, -100.0, 100.0)
        if power:
            m = float(np.mean(col))
            if not _is_constant(_var(col, m, 0), m, n):
                c.lam = yeo_johnson_lambda(col)
                col = yeo_johnson(col, c.lam)
            c.pmean = float(np.mean(col))
            v = _var(col, c.pmean, 0)
            c.pscale = 1.0 if _is_constant(v, c.pmean, n) else math.sqrt(v)
            col = (col - c.pmean) / c.pscale
        ddof = 1 if n > 1 else 0
        m = float(np.mean(col))
        s = max(math.sqrt(_var(col, m, ddof)), 1e-6)
        lo, hi = m - threshold * s, m + threshold * s
        kept = col[~((col < lo) | (col > hi))]
        m = float(np.mean(kept)) if len(kept) else math.nan
        s = math.sqrt(_var(kept, m, ddof)) if len(kept) > ddof else math.nan
        s = 1e-6 if math.isnan(s) else max(s, 1e-6)  # f64::max takes the number over a NaN
        c.lower = m - threshold * s
        c.upper = m + threshold * s
        return c, c.squash(col)

    def squash(self, x) -> np.ndarray:
        """Pull values beyond the bounds in logarithmically (`ColNorm::squash`)."""
        x = np.maximum(-np.log1p(np.abs(x)) + self.lower, x)
        return np.minimum(np.log1p(np.abs(x)) + self.upper, x)

    def apply(self, x, power: bool) -> np.ndarray:
        v = np.clip((np.asarray(x, np.float64) - self.mean) / self.scale, -100.0, 100.0)
        if power:
            v = (yeo_johnson(v, self.lam) - self.pmean) / self.pscale
        return self.squash(v)


@dataclass
class Prep:
    """The fitted preprocessing of a table (`Prep`, `src/prep.rs:378-445`)."""
    n_in: int = 0
    impute: list = field(default_factory=list)
    keep: list = field(default_factory=list)
    power: list = field(default_factory=list)
    norms: list = field(default_factory=list)

    @classmethod
    def fit(cls, x, power=(False, True), threshold: float = 4.0):
        """From a raw training table x [n][h] (NaN for missing): the preprocessing, and per variant the
        transformed training table [n][kept]."""
        x = np.asarray(x, np.float64)
        n, h = x.shape
        p = cls(n_in=h, power=list(power))
        cols = []
        for j in range(h):
            col = x[:, j].copy()
            seen = col[~np.isnan(col)]
            fill = float(np.mean(seen)) if len(seen) else 0.0
            col[np.isnan(col)] = fill
            p.impute.append(fill)
            if n <= 1 or np.any(col != col[0]):
                p.keep.append(j)
                cols.append(col)
        if not p.keep:
            p.keep.append(0)
            cols.append(np.full(n, p.impute[0]))
        tables = []
        for pw in power:
            t = np.empty((n, len(cols)))
            norms = []
            for j, col in enumerate(cols):
                c, v = ColNorm.fit(col.copy(), pw, threshold)
                norms.append(c)
                t[:, j] = v
            p.norms.append(norms)
            tables.append(t)
        return p, tables

    def apply(self, v: int, x) -> np.ndarray:
        """Raw rows x [n][h] through variant v: [n][kept]."""
        x = np.asarray(x, np.float64)
        out = np.empty((x.shape[0], len(self.keep)))
        for j, src in enumerate(self.keep):
            col = np.where(np.isnan(x[:, src]), self.impute[src], x[:, src])
            out[:, j] = self.norms[v][j].apply(col, self.power[v])
        return out
