"""Fitted problems of many tenants sharing one card's memory, with the CPU answering whatever the card cannot.

This plays the part of the reference's `VramTier` (`src/gpu.rs:2485-2701`) and follows its observable rules:

* each problem belongs to a tenant; the card holds at most `budget` bytes of problems in all and `tenant_budget`
  of one tenant's;
* making room removes the problems used longest ago: the tenant's own while the newcomer would put it over its
  share, anyone's otherwise; a problem still being uploaded is never removed;
* a problem that a prediction is using stays on the card until that prediction ends, even once removed, and its
  bytes still count, so the budgets bound what is really on the card at every moment;
* a problem larger than its tenant's budget is never uploaded;
* a prediction the card cannot serve (not resident yet, no room, or the card failed) is left to the CPU: the
  handle returns None; card failures are counted (`fallbacks`) and the last one is kept (`last_error`).

The design is this module's own. One ordered map holds every listed problem, most recently used last. Two ledgers
count bytes: `listed` (what the map holds: uploads in flight and ready problems) decides what to remove, and
`resident` (listed plus removed-but-still-in-use) is the hard cap a new upload must fit under. Predictions take a
lease on a problem; the lease's end frees a removed problem.
"""
from __future__ import annotations

import threading
from collections import OrderedDict
from contextlib import contextmanager

from . import hip

UPLOADING, READY, REFUSED = "uploading", "ready", "refused"


class Residency:
    """One problem's presence on the card."""

    __slots__ = ("tenant", "nbytes", "state", "vm", "leases", "listed")

    def __init__(self, tenant: str, nbytes: int, state: str):
        self.tenant, self.nbytes, self.state = tenant, nbytes, state
        self.vm = None
        self.leases = 0      # predictions using it now
        self.listed = True   # still in the tier's map (a removed one lives on while leased)


class _Bytes:
    """Bytes counted overall and per tenant."""

    def __init__(self):
        self.total = 0
        self.of: dict = {}

    def add(self, tenant: str, n: int) -> None:
        self.total += n
        self.of[tenant] = self.of.get(tenant, 0) + n

    def tenant(self, tenant: str) -> int:
        return self.of.get(tenant, 0)


class VramTier:
    """Problems of many tenants on one `hip.Gpu`, within an overall and a per-tenant byte budget."""

    def __init__(self, gpu: hip.Gpu, budget: int, tenant_budget: int):
        self.gpu = gpu
        self.budget = int(budget)
        self.tenant_budget = min(int(tenant_budget), self.budget)
        self._map: "OrderedDict[tuple, Residency]" = OrderedDict()  # (tenant, model, prefix, node) -> residency
        self._listed = _Bytes()
        self._resident = _Bytes()
        self._mu = threading.RLock()
        self.fallbacks = 0
        self._failure = None

    # ---- what is held ------------------------------------------------------------------------------------------
    def held(self, tenant: str):
        """Bytes the tier lists now (uploads in flight included), overall and of `tenant`."""
        with self._mu:
            return self._listed.total, self._listed.tenant(tenant)

    def ready(self, tenant: str) -> int:
        """Bytes of `tenant`'s problems that are uploaded and usable."""
        with self._mu:
            return sum(r.nbytes for k, r in self._map.items() if k[0] == tenant and r.state == READY)

    def on_card(self, tenant: str):
        """Bytes of problems physically on the card, overall and of `tenant`: everything listed plus removed
        problems a prediction still uses. Never above the budgets."""
        with self._mu:
            return self._resident.total, self._resident.tenant(tenant)

    def last_error(self):
        """The message of the card's most recent failure (that prediction went to the CPU), or None."""
        return self._failure

    # ---- removing ----------------------------------------------------------------------------------------------
    def _unlist(self, key) -> None:
        """Take a problem out of the map (lock held); free it now unless a prediction holds a lease on it."""
        r = self._map.pop(key)
        r.listed = False
        if r.state == REFUSED:
            return
        self._listed.add(r.tenant, -r.nbytes)
        self._free_if_idle(r)

    def _free_if_idle(self, r: Residency) -> None:
        if r.listed or r.leases or r.state == UPLOADING:
            return  # an upload in flight is freed by the uploader when it sees the problem was removed
        if r.vm is not None:
            r.vm.free()
            r.vm = None
        self._resident.add(r.tenant, -r.nbytes)
        r.nbytes = 0

    def evict(self, tenant: str, model=None) -> None:
        """Remove everything `tenant` holds (of `model` only, if given). Problems in use are freed when their
        predictions end; uploads in flight when they finish."""
        with self._mu:
            for key in [k for k in self._map if k[0] == tenant and (model is None or k[1] == model)]:
                self._unlist(key)

    # ---- admitting ---------------------------------------------------------------------------------------------
    @staticmethod
    def problem_bytes(f, weights: hip.GpuWeights, node: int) -> int:
        """Card bytes of problem `node` of the fitted member `f` once loaded (`Gpu::model_bytes`,
        `src/gpu.rs:2063-2068`): its layers as the card holds them, plus the column cache and the column blocks'
        key/value images when the member is one problem of one label digit (then prediction runs all three stages on
        the card). The same figure the loaded problem reports (`VramModel.bytes`)."""
        n = hip.VramModel.model_bytes(weights, f.kv_format, f.nodes[node].rows, f.chunk)
        if len(f.nodes) == 1 and f.digits == 1:
            n += hip.VramModel.columns_bytes(weights, f.features, f.digits)
        return n

    def _room_for(self, tenant: str, nbytes: int) -> bool:
        """Remove ready problems, least recently used first, until `nbytes` more of `tenant` fit the listed budgets
        (lock held). False, with nothing removed past what was needed, if no removable problem is left."""
        while True:
            over_share = self._listed.tenant(tenant) + nbytes > self.tenant_budget
            if not over_share and self._listed.total + nbytes <= self.budget:
                return True
            victim = next((k for k, r in self._map.items()
                           if r.state == READY and (not over_share or k[0] == tenant)), None)
            if victim is None:
                return False
            self._unlist(victim)

    def _reserve(self, key, nbytes: int) -> Residency | None:
        """List a problem as uploading, its bytes counted in both ledgers, or say why not by returning None (lock
        held): already listed (uploading, ready or refused), too big for its tenant, or no room."""
        tenant = key[0]
        if key in self._map:
            return None
        if nbytes > self.tenant_budget:
            self._map[key] = Residency(tenant, nbytes, REFUSED)  # remembered: never tried again
            return None
        if not self._room_for(tenant, nbytes):
            return None
        if (self._resident.total + nbytes > self.budget
                or self._resident.tenant(tenant) + nbytes > self.tenant_budget):
            return None  # removed problems still in use hold the room
        r = Residency(tenant, nbytes, UPLOADING)
        self._map[key] = r
        self._listed.add(tenant, nbytes)
        self._resident.add(tenant, nbytes)
        return r

    def _upload(self, key, r: Residency, f, weights, node) -> None:
        """Put a reserved problem on the card; a failure gives its bytes back and is remembered."""
        vm = None
        try:
            vm = self.gpu.load(weights, f.kv_format, f.nodes[node].rows, f.chunk, f.layers[node], f.scales[node])
            if len(f.nodes) == 1 and f.digits == 1:
                vm.set_columns(f.col_kv, f.features, f.digits)
            failure = None
        except Exception as e:  # noqa: BLE001 -- the card's failure: the CPU answers
            failure = e
            if vm is not None:
                vm.free()
                vm = None
        with self._mu:
            r.vm = vm
            r.state = READY
            if failure is not None:
                self._failure = str(failure)
                if r.listed:
                    self._map.pop(key)
                    r.listed = False
                    self._listed.add(r.tenant, -r.nbytes)
            self._free_if_idle(r)  # removed while uploading (or failed): freed now

    def preload(self, tenant: str, model: str, members: dict, weights: hip.GpuWeights, prefix: str, node: int) -> bool:
        """Upload problem `node` of member `prefix` now, on this thread. True if it is resident afterwards."""
        key = (tenant, model, prefix, int(node))
        f = members[prefix]
        with self._mu:
            r = self._map.get(key)
            if r is not None:
                self._map.move_to_end(key)
                return r.state == READY
            r = self._reserve(key, self.problem_bytes(f, weights, node))
        if r is None:
            return False
        self._upload(key, r, f, weights, node)
        with self._mu:
            return r.listed and r.state == READY and r.vm is not None

    @contextmanager
    def _lease(self, key, f, weights, node, wait: bool):
        """The problem's card model for the duration of a prediction, or None (then the CPU answers): a problem not
        yet listed is reserved and uploaded, on this thread with `wait`, else on a thread of its own."""
        mine = None  # a reservation this call made and uploads itself
        with self._mu:
            r = self._map.get(key)
            if r is not None:
                self._map.move_to_end(key)
            else:
                r = self._reserve(key, self.problem_bytes(f, weights, node))
                if r is not None and wait:
                    mine = r
                elif r is not None:
                    threading.Thread(target=self._upload, args=(key, r, f, weights, node), daemon=True).start()
        if mine is not None:
            self._upload(key, mine, f, weights, node)
        with self._mu:
            usable = r is not None and r.listed and r.state == READY and r.vm is not None
            if usable:
                r.leases += 1
        if not usable:
            yield None
            return
        try:
            yield r.vm
        finally:
            with self._mu:
                r.leases -= 1
                self._free_if_idle(r)

    def handle(self, tenant: str, model: str, members: dict, weights: hip.GpuWeights) -> "TierAttend":
        """One tenant's use of the tier for one fitted model (`members`: prefix -> `fit.Fitted`)."""
        return TierAttend(self, tenant, model, members, weights)


class TierAttend:
    """`predict::AttendCached` over the tier: `attend`, `stage` and `rows` answer on the card when the problem is
    resident, and otherwise return None (the CPU answers) after starting its upload. With `wait` the upload runs on
    the calling thread, so the first prediction already uses the card."""

    def __init__(self, tier: VramTier, tenant: str, model: str, members: dict, weights: hip.GpuWeights,
                 wait: bool = False):
        self.tier, self.tenant, self.model, self.members, self.weights = tier, tenant, model, members, weights
        self.wait = wait

    def _on_card(self, prefix: str, node: int, work):
        f = self.members.get(prefix)
        if f is None or node >= len(f.nodes):
            return None
        key = (self.tenant, self.model, prefix, int(node))
        with self.tier._lease(key, f, self.weights, node, self.wait) as vm:
            if vm is None:
                return None
            try:
                return work(vm)
            except Exception as e:  # noqa: BLE001 -- any failure on the card: counted, and the CPU answers
                with self.tier._mu:
                    self.tier.fallbacks += 1
                    self.tier._failure = str(e)
                return None

    def attend(self, prefix: str, node: int, layer: int, q, d: int, heads: int):
        return self._on_card(prefix, node, lambda vm: self.tier.gpu.attend_resident(vm, layer, q) if d == vm.d else None)

    def stage(self, prefix: str, node: int, h, d: int, out_n: int):
        return self._on_card(prefix, node, lambda vm: self.tier.gpu.in_context(self.weights, vm, h, out_n)
                             if d == vm.d else None)

    def rows(self, prefix: str, x, out_n: int):
        def work(vm):
            if not getattr(vm, "features", 0) or vm.digits != 1:
                return None
            return self.tier.gpu.predict(self.weights, vm, x, out_n)
        return self._on_card(prefix, 0, work)
