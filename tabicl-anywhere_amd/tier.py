"""Graphics memory shared by many tenants: the VRAM tier (`VramTier`, `src/gpu.rs:2485-2701`), with the bookkeeping of
the in-memory tier's ledger (`warm::Ledger`, `src/warm.rs:28-118`).

Every resident problem belongs to one tenant and one model; each tenant has a byte budget within the overall one;
the least recently used ready entry makes room (the tenant's own while it would be over its share, anyone's
otherwise); an entry in use is not released until the prediction using it has finished. The budgets are hard
limits on what is really on the card: a load starts only when the bytes of everything loaded and not yet released,
evicted or not, leave room for it; otherwise that prediction (and only that one) is answered by the CPU (`None`
from the handle). A problem larger than its tenant's budget is never loaded. A card that fails a prediction does
not fail it either: the CPU answers, and the tier counts it (`fallbacks`) and keeps the reason (`last_error`).

What the card holds at worst: `budget` of fitted problems, plus the card's working-memory budget
(`Gpu.set_work_budget`), plus each set of weights in use.
"""
from __future__ import annotations

import threading

from . import hip

LOADING, TOO_BIG = "loading", "too big"


class Ledger:
    """`warm::Ledger`: entries by key (tenant, model, prefix, node) with their bytes and a use clock."""

    def __init__(self):
        self.entries: dict = {}  # key -> [value, bytes, clock]
        self.bytes = 0
        self.by_tenant: dict = {}
        self.clock = 0

    def get(self, key):
        """The entry's value, marked as just used (`src/warm.rs:43-50`)."""
        self.clock += 1
        e = self.entries.get(key)
        if e is None:
            return None
        e[2] = self.clock
        return e[0]

    def set(self, key, value) -> None:
        self.entries[key][0] = value

    def remove(self, key):
        e = self.entries.pop(key, None)
        if e is None:
            return None
        self.bytes -= e[1]
        self.by_tenant[key[0]] = self.by_tenant.get(key[0], 0) - e[1]
        return e[0]

    def admit(self, key, nbytes: int, value, budget: int, tenant_budget: int, may_go):
        """Hold `value` under `key`, first making room within both budgets (`src/warm.rs:61-89`): while the tenant
        would be over its share its own least recently used entry goes, otherwise the least recently used of
        anyone's; only entries `may_go` allows are removed. Returns (admitted, removed values)."""
        out = []
        if nbytes > min(tenant_budget, budget):
            return False, out
        while True:
            mine = self.by_tenant.get(key[0], 0)
            over_tenant = mine + nbytes > tenant_budget
            if not over_tenant and self.bytes + nbytes <= budget:
                break
            victims = [(e[2], k) for k, e in self.entries.items() if (not over_tenant or k[0] == key[0]) and may_go(e[0])]
            if not victims:
                return False, out
            out.append(self.remove(min(victims)[1]))
        self.clock += 1
        self.bytes += nbytes
        self.by_tenant[key[0]] = self.by_tenant.get(key[0], 0) + nbytes
        if key in self.entries:
            out.append(self.remove(key))
        self.entries[key] = [value, nbytes, self.clock]
        return True, out

    def contains(self, key) -> bool:
        return key in self.entries

    def evict(self, tenant: str, model=None) -> list:
        keys = [k for k in self.entries if k[0] == tenant and (model is None or k[1] == model)]
        return [self.remove(k) for k in keys]

    def items(self):
        return [(k, e[0], e[1]) for k, e in self.entries.items()]

    def held(self, tenant: str):
        return self.bytes, self.by_tenant.get(tenant, 0)


class _Resident:
    """A loaded problem: freed on the card once it has been released by the tier and no prediction uses it."""

    def __init__(self, tier: "VramTier", tenant: str, nbytes: int, vm):
        self.tier, self.tenant, self.nbytes, self.vm = tier, tenant, nbytes, vm
        self.uses = 0
        self.released = False

    def release(self) -> None:  # called with the tier's lock held
        self.released = True
        self._maybe_free()

    def _maybe_free(self) -> None:
        if self.released and self.uses == 0 and self.vm is not None:
            self.vm.free()
            self.vm = None
            self.tier._live_give(self.tenant, self.nbytes)


class VramTier:
    """`VramTier` (`src/gpu.rs:2496-2611`) over `hip.Gpu`."""

    def __init__(self, gpu: hip.Gpu, budget: int, tenant_budget: int):
        self.gpu = gpu
        self.budget = int(budget)
        self.tenant_budget = min(int(tenant_budget), self.budget)
        self._state = Ledger()
        self._live_bytes = 0
        self._live_by_tenant: dict = {}
        self._lock = threading.RLock()
        self.fallbacks = 0
        self._last_error = None

    # ---- what is held ------------------------------------------------------------------------------------------
    def held(self, tenant: str):
        """Bytes of graphics memory the tier holds now, in all and by `tenant` (problems being loaded included)."""
        with self._lock:
            return self._state.held(tenant)

    def ready(self, tenant: str) -> int:
        """Bytes of `tenant`'s problems that are loaded and ready."""
        with self._lock:
            return sum(n for k, v, n in self._state.items() if k[0] == tenant and isinstance(v, _Resident))

    def on_card(self, tenant: str):
        """Bytes of fitted problems really on the card now, in all and of `tenant`: what the tier holds plus
        anything evicted that a prediction is still using. Never more than the budgets."""
        with self._lock:
            return self._live_bytes, self._live_by_tenant.get(tenant, 0)

    def last_error(self):
        """Why the card last failed a prediction (which the CPU then answered), if it ever did."""
        return self._last_error

    def evict(self, tenant: str, model=None) -> None:
        """Release everything `tenant` holds (for `model` only, if given); problems in use by a prediction are
        freed when it finishes."""
        with self._lock:
            for v in self._state.evict(tenant, model):
                if isinstance(v, _Resident):
                    v.release()

    def handle(self, tenant: str, model: str, members: dict, weights: hip.GpuWeights) -> "TierAttend":
        """One tenant's use of the tier for one fitted model (`members`: prefix -> `fit.Fitted`), to answer
        predictions in place of the CPU where it can."""
        return TierAttend(self, tenant, model, members, weights)

    def preload(self, tenant: str, model: str, members: dict, weights: hip.GpuWeights, prefix: str, node: int) -> bool:
        """Load problem `node` of member `prefix` now. True if it is resident afterwards; False if the budgets do
        not allow it (now, or ever)."""
        key = (tenant, model, prefix, int(node))
        with self._lock:
            if isinstance(self._state.get(key), _Resident):
                return True
        nbytes = self._claim(key, members[prefix], weights, node)
        if nbytes is None:
            return False
        return self._finish(key, nbytes, members[prefix], weights, node)

    # ---- loading -----------------------------------------------------------------------------------------------
    @staticmethod
    def problem_bytes(f, weights: hip.GpuWeights, node: int) -> int:
        """Card bytes of problem `node` of the fitted member `f` once loaded: its records and their images, plus
        the column cache for a member with one problem and one label digit (`Gpu::model_bytes`,
        `src/gpu.rs:2063-2068`)."""
        rows = f.nodes[node].rows
        n = hip.VramModel.model_bytes(weights, f.kv_format, rows, f.chunk)
        if len(f.nodes) == 1 and f.digits == 1:
            n += f.col_kv.size * 4
        return n

    def _claim(self, key, f, weights, node):
        """Take a place for a problem and count its bytes before anything is uploaded (`src/gpu.rs:2553-2585`).
        None if there is no room within the budgets."""
        nbytes = self.problem_bytes(f, weights, node)
        with self._lock:
            s = self._state
            if s.contains(key):
                return None
            ok, gone = s.admit(key, nbytes, LOADING, self.budget, self.tenant_budget,
                               lambda v: isinstance(v, _Resident))
            for v in gone:
                if isinstance(v, _Resident):
                    v.release()
            if not ok:
                if nbytes > self.tenant_budget:
                    s.admit(key, 0, TOO_BIG, self.budget, self.tenant_budget, lambda v: False)
                return None
            mine = self._live_by_tenant.get(key[0], 0)
            if self._live_bytes + nbytes > self.budget or mine + nbytes > self.tenant_budget:
                # the room is promised to problems still in use: not this time
                s.remove(key)
                return None
            self._live_bytes += nbytes
            self._live_by_tenant[key[0]] = mine + nbytes
            return nbytes

    def _live_give(self, tenant: str, nbytes: int) -> None:
        self._live_bytes -= nbytes
        self._live_by_tenant[tenant] = self._live_by_tenant.get(tenant, 0) - nbytes

    def _finish(self, key, nbytes, f, weights, node) -> bool:
        """Upload a claimed problem and make it ready, unless it was evicted meanwhile (`src/gpu.rs:2588-2611`)."""
        try:
            vm = self.gpu.load(weights, f.kv_format, f.nodes[node].rows, f.chunk, f.layers[node], f.scales[node])
            if len(f.nodes) == 1 and f.digits == 1:
                vm.set_columns(f.col_kv, f.features, f.digits)
        except Exception as e:  # noqa: BLE001 -- the card's failure is recorded and the CPU answers
            with self._lock:
                if self._state.get(key) == LOADING:
                    self._state.remove(key)
                self._live_give(key[0], nbytes)
                self._last_error = str(e)
            return False
        with self._lock:
            res = _Resident(self, key[0], nbytes, vm)
            v = self._state.get(key)
            if v == LOADING:
                self._state.set(key, res)
                return True
            res.release()  # evicted while loading
            return isinstance(v, _Resident)

    def _resident(self, key, f, weights, node, wait: bool):
        """The problem if it is resident (its use counted); otherwise start loading it (once) and say no for now.
        The load runs on a thread of its own (on the calling thread with `wait`)."""
        with self._lock:
            v = self._state.get(key)
            if isinstance(v, _Resident):
                v.uses += 1
                return v
            if v is not None:
                return None
        nbytes = self._claim(key, f, weights, node)
        if nbytes is None:
            return None
        if wait:
            self._finish(key, nbytes, f, weights, node)
            with self._lock:
                v = self._state.get(key)
                if isinstance(v, _Resident):
                    v.uses += 1
                    return v
            return None
        threading.Thread(target=self._finish, args=(key, nbytes, f, weights, node), daemon=True).start()
        return None

    def _done(self, res: _Resident) -> None:
        with self._lock:
            res.uses -= 1
            res._maybe_free()


class TierAttend:
    """`predict::AttendCached` over the tier (`VramHandle`, `src/gpu.rs:2614-2701`): `attend`, `stage` and `rows`
    answer on the card when the problem is resident, else return None (the CPU answers) after starting its
    load. `wait` loads on the calling thread instead, so the first prediction already uses the card."""

    def __init__(self, tier: VramTier, tenant: str, model: str, members: dict, weights: hip.GpuWeights,
                 wait: bool = False):
        self.tier, self.tenant, self.model, self.members, self.weights = tier, tenant, model, members, weights
        self.wait = wait

    def _use(self, prefix: str, node: int, run):
        f = self.members.get(prefix)
        if f is None or node >= len(f.nodes):
            return None
        res = self.tier._resident((self.tenant, self.model, prefix, int(node)), f, self.weights, node, self.wait)
        if res is None:
            return None
        try:
            return run(res.vm, f)
        except (hip.CardError, hip.BudgetError) as e:
            with self.tier._lock:
                self.tier.fallbacks += 1
                self.tier._last_error = str(e)
            return None
        finally:
            self.tier._done(res)

    def attend(self, prefix: str, node: int, layer: int, q, d: int, heads: int):
        return self._use(prefix, node, lambda vm, f: self.tier.gpu.attend_resident(vm, layer, q) if d == vm.d else None)

    def stage(self, prefix: str, node: int, h, d: int, out_n: int):
        return self._use(prefix, node, lambda vm, f: self.tier.gpu.in_context(self.weights, vm, h, out_n)
                         if d == vm.d else None)

    def rows(self, prefix: str, x, out_n: int):
        def run(vm, f):
            if not getattr(vm, "features", 0) or vm.digits != 1:
                return None
            return self.tier.gpu.predict(self.weights, vm, x, out_n)
        return self._use(prefix, 0, run)
