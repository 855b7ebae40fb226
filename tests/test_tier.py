"""The VRAM tier's rules (`tier.py`, the part of the reference's `VramTier`, `src/gpu.rs:2485-2701`) on the host, with
a stand-in card: least-recently-used removal within the overall and the tenants' budgets, problems in use outliving
their removal, uploads in flight never removed, a problem too big for its tenant never uploaded, uploads on a thread
of their own, and card failures (of any kind) answered by the CPU and counted. (tests/card.rs:237-346 runs the same
rules against a card; tests/test_gpu_tier.py does here.)"""
import threading
import time

import numpy as np
import pytest

from conftest import pkg

hip, tier = pkg("hip"), pkg("tier")


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


def test_least_recently_used_within_budgets():
    card = FakeCard()
    t = FakeTier(card, 100, 60)
    m = lambda n: {"m0/": Member(n)}
    assert t.preload("a", "x", m(40), None, "m0/", 0) and t.preload("b", "x", m(40), None, "m0/", 0)
    assert t.preload("a", "x", m(40), None, "m0/", 0)  # a used last: b is now the oldest
    # over the overall budget: the oldest of anyone's goes
    assert t.preload("c", "x", m(30), None, "m0/", 0)
    assert t.held("b") == (70, 0) and card.freed == 1
    # over the tenant's share (40 + 30 > 60): a's own oldest goes, not c's
    assert t.preload("a", "y", m(30), None, "m0/", 0)
    assert t.held("a") == (60, 30) and t.held("c") == (60, 30) and card.freed == 2
    # larger than a tenant's budget: refused for good, nothing removed
    assert not t.preload("d", "x", m(61), None, "m0/", 0)
    assert not t.preload("d", "x", m(61), None, "m0/", 0)
    assert t.held("d") == (60, 0) and card.freed == 2
    # removing one model of a tenant leaves its others
    assert t.preload("a", "z", m(20), None, "m0/", 0)
    t.evict("a", "y")
    assert t.held("a") == (50, 20) and t.ready("a") == 20


def test_upload_in_flight_is_never_removed():
    card = FakeCard(delay=0.3)
    t = FakeTier(card, 100, 100)
    h = t.handle("a", "x", {"m0/": Member(70)}, None)
    assert h.rows("m0/", np.zeros((1, 3)), 2) is None  # its upload starts on a thread of its own
    # 70 listed and uploading: a newcomer of 40 finds nothing it may remove
    assert not t.preload("b", "x", {"m0/": Member(40)}, None, "m0/", 0)
    t.evict("a")  # removed while uploading: freed as soon as the upload ends
    assert t.held("a") == (0, 0) and t.on_card("a") == (70, 70)
    for _ in range(100):
        if card.freed:
            break
        time.sleep(0.01)
    assert card.loaded == card.freed == 1 and t.on_card("a") == (0, 0)


def test_any_card_error_goes_to_the_cpu():
    card = FakeCard()
    t = FakeTier(card, 100, 100)
    h = t.handle("a", "x", {"m0/": Member(30)}, None)
    h.wait = True

    def refuse(weights, vm, x, out_n):
        raise ValueError("attention: too many queries for one launch")

    card.predict = refuse
    assert h.rows("m0/", np.zeros((1, 3)), 2) is None
    assert t.fallbacks == 1 and "too many" in t.last_error()
