"""The VRAM tier against the card (the reference's tests/card.rs:277-346 restated): two tenants predicting at
once from different threads while a third thread keeps evicting one of them, every answer the card gives equal to
the card's direct prediction and the bytes on the card within both budgets all the while; everything released at
the end; and a model larger than its tenant's budget never put on the card."""
import sys
import threading
import time

import numpy as np
import pytest

from conftest import pkg

hip, fit, tier = pkg("hip"), pkg("fit"), pkg("tier")
pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def setup(tiny_model):
    gpu = hip.Gpu(0)
    w = gpu.weights(tiny_model)
    rng = np.random.default_rng(21)
    x = rng.standard_normal((120, 5)).astype(np.float32)
    y = rng.integers(0, 3, 120).astype(np.float32)
    f = fit.fit_raw(gpu, w, x, y, 3)
    xt = rng.standard_normal((17, 5)).astype(np.float32)
    vm = gpu.load(w, f.kv_format, f.rows, f.chunk, f.layers[0], f.scales[0])
    vm.set_columns(f.col_kv, f.features, f.digits)
    want = gpu.predict(w, vm, xt, 3)
    vm.free()
    yield gpu, w, {"m0/": f}, xt, want
    gpu.close()


def test_tenants_at_once_and_eviction_in_flight(setup):
    gpu, w, members, xt, want = setup
    say("tier: two tenants, evictions in flight")
    one = tier.VramTier.problem_bytes(members["m0/"], w, 0)
    t = tier.VramTier(gpu, 2 * one, one)
    assert t.preload("alice", "a", members, w, "m0/", 0) and t.preload("bob", "a", members, w, "m0/", 0)
    assert t.on_card("alice") == (2 * one, one)
    stop = threading.Event()
    counts, errors = {}, []

    def run(who):
        h = t.handle(who, "a", members, w)
        n = 0
        for _ in range(6):
            got = h.rows("m0/", xt, 3)
            if got is not None:
                n += 1
                if np.abs(got - want).max() != 0.0:
                    errors.append(f"{who}: wrong answer")
            all_, mine = t.on_card(who)
            if all_ > 2 * one or mine > one:
                errors.append(f"{who}: over budget on the card")
        counts[who] = n

    def evicter():
        while not stop.is_set():
            t.evict("alice")
            time.sleep(0.003)

    ev = threading.Thread(target=evicter)
    ev.start()
    runs = [threading.Thread(target=run, args=(who,)) for who in ("alice", "bob")]
    for r in runs:
        r.start()
    for r in runs:
        r.join(60)
    stop.set()
    ev.join(10)
    say("  answered on the card: alice", counts.get("alice"), "of 6 (evicted all the while), bob", counts.get("bob"))
    assert not errors, errors
    assert counts["bob"] > 0
    assert t.fallbacks == 0, t.last_error()
    time.sleep(0.5)  # loads alice's predictions started may still be finishing
    t.evict("alice")
    t.evict("bob")
    assert t.on_card("alice") == (0, 0)
    assert gpu.overdrawn() == 0


def test_model_larger_than_tenant_budget_stays_off_the_card(setup):
    gpu, w, members, xt, want = setup
    t = tier.VramTier(gpu, 1 << 30, 1 << 10)
    assert not t.preload("carol", "a", members, w, "m0/", 0)
    h = t.handle("carol", "a", members, w)
    for _ in range(3):
        assert h.rows("m0/", xt, 3) is None  # the CPU answers, every time
    assert t.on_card("carol") == (0, 0) and t.fallbacks == 0


def test_tier_counts_what_the_card_holds(setup):
    """The tier's byte figures are what the loaded problems really hold on the card: their layers, the column cache
    and the column blocks' key/value images (`VramModel.bytes`, read from the library after loading)."""
    gpu, w, members, xt, want = setup
    one = tier.VramTier.problem_bytes(members["m0/"], w, 0)
    t = tier.VramTier(gpu, 4 * one, 2 * one)
    assert t.preload("dave", "a", members, w, "m0/", 0) and t.preload("erin", "a", members, w, "m0/", 0)
    held = [r.vm.bytes() for r in t._map.values() if r.vm is not None]
    say(f"  tier: {one} bytes a problem by its estimate; held {held}")
    assert held == [one, one]
    assert t.on_card("dave") == (sum(held), one)
    t.evict("dave")
    t.evict("erin")
    assert t.on_card("dave") == (0, 0)
