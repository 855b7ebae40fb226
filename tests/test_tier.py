"""The VRAM tier's bookkeeping (`tier.py`: `VramTier`, `src/gpu.rs:2485-2701`, over `warm::Ledger`,
`src/warm.rs:28-118`) on the host, with a stand-in card: least-recently-used admission within the overall and the
tenants' budgets, problems in use outliving their eviction, a problem too big for its tenant never loaded, loads
on a thread of their own, and card failures answered by the CPU and counted. (tests/card.rs:237-346 runs the same
rules against a card; tests/test_gpu_tier.py does here.)"""
import threading
import time

import numpy as np
import pytest

from conftest import pkg

hip, tier = pkg("hip"), pkg("tier")


def test_ledger_lru_within_budgets():
    L = tier.Ledger()
    ready = lambda v: v != "busy"
    assert L.admit(("a", "m", "p", 0), 40, "a0", 100, 60, ready) == (True, [])
    assert L.admit(("b", "m", "p", 0), 40, "b0", 100, 60, ready) == (True, [])
    L.get(("a", "m", "p", 0))  # a0 used last: b0 is now the oldest
    # over the overall budget: the least recently used of anyone's goes
    assert L.admit(("c", "m", "p", 0), 30, "c0", 100, 60, ready) == (True, ["b0"])
    # over the tenant's share: a's own oldest goes, not c's
    assert L.admit(("a", "m", "p", 1), 30, "a1", 100, 60, ready) == (True, ["a0"])
    assert L.held("a") == (60, 30)
    # larger than a tenant's budget: refused, nothing removed
    assert L.admit(("d", "m", "p", 0), 61, "d0", 100, 60, ready) == (False, [])
    # nothing may go: refused
    L.set(("c", "m", "p", 0), "busy")
    L.set(("a", "m", "p", 1), "busy")
    assert L.admit(("e", "m", "p", 0), 50, "e0", 100, 60, ready) == (False, [])
    assert sorted(L.evict("a")) == ["busy"] and L.held("a") == (30, 0)


class FakeVM:
    def __init__(self, card):
        self.card, self.d, self.freed = card, 8, False
        card.loaded += 1

    def set_columns(self, col_kv, features, digits):
        self.features, self.digits = features, digits

    def free(self):
        assert not self.freed
        self.freed = True
        self.card.freed += 1


class FakeCard:
    def __init__(self, fail=False, delay=0.0):
        self.loaded = self.freed = 0
        self.fail, self.delay = fail, delay

    def load(self, weights, kv_format, rows, chunk, layers, scales):
        time.sleep(self.delay)
        return FakeVM(self)

    def predict(self, weights, vm, x, out_n):
        if self.fail:
            raise hip.CardError("graphics card: lost")
        assert not vm.freed
        return np.full((len(x), out_n), 7.0, np.float32)


class Node:
    def __init__(self, rows):
        self.rows = rows


class Member:
    def __init__(self, nbytes):
        self.nodes, self.kv_format, self.chunk, self.digits, self.features = [Node(10)], 0, 4, 1, 3
        self.layers, self.scales, self.col_kv = [[b""]], [np.zeros(1, np.float32)], np.zeros(1, np.float32)
        self.nbytes = nbytes


class FakeTier(tier.VramTier):
    @staticmethod
    def problem_bytes(f, weights, node):
        return f.nbytes


def test_preload_evict_and_budgets():
    card = FakeCard()
    t = FakeTier(card, 100, 60)
    big, small = {"m0/": Member(70)}, {"m0/": Member(40)}
    assert not t.preload("carol", "a", big, None, "m0/", 0)  # over the tenant's budget: never loaded
    assert card.loaded == 0 and t.on_card("carol") == (0, 0)
    assert t.preload("alice", "a", small, None, "m0/", 0) and t.preload("bob", "a", small, None, "m0/", 0)
    assert t.on_card("alice") == (80, 40) and t.ready("alice") == 40
    assert t.preload("alice", "a", small, None, "m0/", 0)  # already resident (and now the most recently used)
    # a third tenant's load makes room: the least recently used ready problem (bob's) goes
    assert t.preload("dave", "a", small, None, "m0/", 0)
    assert t.on_card("bob") == (80, 0) and t.on_card("alice") == (80, 40) and card.freed == 1
    t.evict("alice")
    t.evict("dave")
    assert t.on_card("x") == (0, 0) and card.freed == card.loaded == 3


def test_in_use_problem_outlives_its_eviction():
    card = FakeCard()
    t = FakeTier(card, 100, 100)
    h = t.handle("alice", "a", {"m0/": Member(60)}, None)
    h.wait = True
    started, release = threading.Event(), threading.Event()
    slow = card.predict

    def predict(weights, vm, x, out_n):
        started.set()
        release.wait(5)
        return slow(weights, vm, x, out_n)

    card.predict = predict
    out = {}
    th = threading.Thread(target=lambda: out.setdefault("y", h.rows("m0/", np.zeros((2, 3)), 4)))
    th.start()
    assert started.wait(5)
    t.evict("alice")
    # released by the tier, but the prediction still runs on it: still on the card, and its room is promised
    assert t.held("alice") == (0, 0) and t.on_card("alice") == (60, 60) and card.freed == 0
    assert not t.preload("bob", "a", {"m0/": Member(60)}, None, "m0/", 0)
    release.set()
    th.join(5)
    assert out["y"].shape == (2, 4) and card.freed == 1 and t.on_card("alice") == (0, 0)


def test_background_load_then_card_answers():
    card = FakeCard(delay=0.05)
    t = FakeTier(card, 100, 100)
    h = t.handle("alice", "a", {"m0/": Member(30)}, None)
    assert h.rows("m0/", np.zeros((1, 3)), 2) is None  # not resident yet: the CPU answers, the load starts
    assert h.rows("m0/", np.zeros((1, 3)), 2) is None  # still loading: no second load
    for _ in range(100):
        if t.ready("alice"):
            break
        time.sleep(0.01)
    assert card.loaded == 1 and np.all(h.rows("m0/", np.zeros((1, 3)), 2) == 7.0)


def test_card_failure_is_answered_by_the_cpu():
    card = FakeCard(fail=True)
    t = FakeTier(card, 100, 100)
    h = t.handle("alice", "a", {"m0/": Member(30)}, None)
    h.wait = True
    assert h.rows("m0/", np.zeros((1, 3)), 2) is None
    assert t.fallbacks == 1 and "lost" in t.last_error()
