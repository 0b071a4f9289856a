"""CPU restatement of the streamed-expert cache and copy-ahead policy.

Test infrastructure only (tests/ use it as the oracle; the product never
imports it).  It restates, per routing event of a streamed layer:

* the HBM slot cache: a lookup of a resident (layer, expert) reuses its slot
  and makes it most recent; a miss takes an empty slot (lowest index), else
  the least recently used slot (ExpertGpuCache::acquireSlot,
  src/compute/cuda_backend.cpp:322-363).  Eviction sweeps follow the host LRU's
  evictOne (src/storage/lru_cache.h:184-199): from the least recent end, a
  softly boosted entry spends one protection and survives, the first other
  entry goes; a speculatively inserted entry evicted before any lookup used it
  counts as wasted (:190).  Slots the current call already holds are never
  taken (the device pipeline still reads them); a demand lookup that finds no
  unprotected victim takes the least recent unheld slot anyway, a copy-ahead
  gives up (insert fails, lru_cache.h:108-113).
* the routing history (Scheduler::onLayerRouterDone,
  src/engine/scheduler.cpp:240-262): the layer's winner-overlap EMA
  ema = a*|cur & last|/max(|cur|,|last|) + (1-a)*ema, then last = cur;
  with the popularity predictor, heat = alpha + (1-alpha)*heat per routed
  expert and a one-sweep boost of the hottest (:279-292, lru_cache.h:137-143).
* the guesses for layer+1 (predictNextLayerExperts, :180-219): the previous
  token's selection at layer+1, else this layer's selection; the popularity
  fill adds nothing because it stops at the size of that list (:195,207);
  dropped when layer+1's overlap EMA is below the floor (:303-306); none at
  all past the last layer (:293-294).
* the router-probability mode (setRouterPrefetch, :148-156; :320-352), from
  the winners' routing weights: extra_depth more guesses from this token's
  winners not yet guessed, by descending weight (after the gate); with
  prob_resident a running per-layer maximum weight, and a resident winner with
  weight >= 0.9 x that maximum and two earlier lookups is pinned (lru_.pin:
  never evicted; here a demand lookup with only pinned candidates left takes
  the least recent of them).

The order of one call is the reference's (moeLayer reports the routing before
its expert loop, glm_forward.cpp:548 before :564/:623): the routing-history
update, then the demand lookups in rank order, then copy-aheads of the guesses.
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field


@dataclass
class Options:
    prefetch: bool = True
    ema_predictor: bool = False
    ema_alpha: float = 0.1
    overlap_floor: float = 0.5
    overlap_alpha: float = 0.5
    extra_depth: int = 0
    prob_resident: bool = False


COUNTERS = ("lookups", "hits", "misses", "pred_staged", "pred_consumed", "pred_wasted",
            "pred_resident", "copies", "pinned")

# Slots one call may hold: its k winners plus up to 2k copy-aheads.
MAX_HELD = 24


def _f32(v: float) -> float:
    """Round to IEEE single, as the C++ policy keeps its EMAs in float."""
    import struct
    return struct.unpack("f", struct.pack("f", v))[0]


@dataclass
class StreamPolicy:
    slots: int
    opt: Options = field(default_factory=Options)

    def __post_init__(self):
        self.key = [None] * self.slots          # (layer, expert) per slot
        self.recency: OrderedDict = OrderedDict()  # slot -> None, oldest first
        self.protect = [0] * self.slots
        self.staged = [False] * self.slots
        self.used = [False] * self.slots
        self.pinned = [False] * self.slots
        self.access: dict[tuple[int, int], int] = {}
        self.max_prob: dict[int, float] = {}
        self.last_topk: dict[int, list[int]] = {}
        self.overlap: dict[int, float] = {}
        self.heat: dict[tuple[int, int], float] = {}
        self.n = dict.fromkeys(COUNTERS, 0)

    def find(self, key):
        for s, k in enumerate(self.key):
            if k == key:
                return s
        return -1

    def _touch(self, s):
        self.recency.pop(s, None)
        self.recency[s] = None

    def _victim(self, held, must):
        for s in range(self.slots):
            if self.key[s] is None and s not in held:
                return s
        for s in list(self.recency):          # least recent first
            if s in held or self.pinned[s]:
                continue
            if self.protect[s] > 0:
                self.protect[s] -= 1
                continue
            return s
        if must:
            for s in self.recency:
                if s not in held and not self.pinned[s]:
                    return s
            for s in self.recency:
                if s not in held:
                    return s
        return -1

    def _place(self, s, key, staged):
        if self.key[s] is not None and self.staged[s] and not self.used[s]:
            self.n["pred_wasted"] += 1
        self.key[s] = key
        self.protect[s] = 0
        self.pinned[s] = False
        self.staged[s] = staged
        self.used[s] = not staged
        self._touch(s)

    def lookup(self, layer, expert, held):
        """Demand lookup: (slot, needs_copy)."""
        self.n["lookups"] += 1
        self.access[(layer, expert)] = self.access.get((layer, expert), 0) + 1
        s = self.find((layer, expert))
        if s >= 0:
            self.n["hits"] += 1
            if self.staged[s] and not self.used[s]:
                self.n["pred_consumed"] += 1
            self.used[s] = True
            self._touch(s)
            return s, False
        self.n["misses"] += 1
        s = self._victim(held, True)
        self._place(s, (layer, expert), False)
        self.n["copies"] += 1
        return s, True

    def boost(self, key, cycles=1):
        s = self.find(key)
        if s >= 0:
            self.protect[s] = max(self.protect[s], cycles)
            self._touch(s)

    def pin(self, key):
        s = self.find(key)
        if s >= 0 and not self.pinned[s]:
            self.pinned[s] = True
            self.n["pinned"] += 1

    def route_done(self, layer, topk, probs=None, has_next=True, next_streamed=True):
        o = self.opt
        cur = list(topk)
        last = self.last_topk.get(layer, [])
        ema = self.overlap.get(layer, 0.0)
        if last and cur:
            common = sum(1 for e in cur if e in last)
            frac = _f32(common / max(len(last), len(cur)))
            oa = _f32(o.overlap_alpha)
            ema = _f32(_f32(oa * frac) + _f32(_f32(1.0 - oa) * ema))
        self.overlap[layer] = ema
        self.last_topk[layer] = cur
        if o.prob_resident and probs is not None:
            self.max_prob[layer] = max([self.max_prob.get(layer, 0.0)] + [_f32(p) for p in probs])
        if o.ema_predictor:
            a = _f32(o.ema_alpha if 0.0 < o.ema_alpha <= 1.0 else 0.1)
            best, best_heat = None, -1.0
            for e in cur:
                h = self.heat.get((layer, e), 0.0)
                h = _f32(a + _f32(_f32(1.0 - a) * h))
                self.heat[(layer, e)] = h
                if h > best_heat:
                    best, best_heat = e, h
            if best is not None:
                self.boost((layer, best), 1)
        if not has_next:
            return []
        guess = list(self.last_topk.get(layer + 1) or cur)
        if self.overlap.get(layer + 1, 0.0) < _f32(o.overlap_floor):
            guess = []
        if o.extra_depth > 0 and probs is not None:
            cand = [r for r in range(len(cur)) if _f32(probs[r]) > 0.0 and cur[r] not in guess]
            cand.sort(key=lambda r: -_f32(probs[r]))  # stable: ties in rank order
            guess += [cur[r] for r in cand[:o.extra_depth]]
        if o.prob_resident and probs is not None:
            mx = self.max_prob.get(layer, 0.0)
            if mx > 0.0:
                bar = _f32(_f32(0.9) * mx)
                for e, p in zip(cur, probs):
                    if _f32(p) >= bar and self.access.get((layer, e), 0) >= 2:
                        self.pin((layer, e))
        if not o.prefetch or not next_streamed:
            return []
        return guess

    def stage(self, layer, expert, held):
        """Copy-ahead: slot to copy into, or -1 (resident or nothing evictable)."""
        if self.find((layer, expert)) >= 0:
            self.n["pred_resident"] += 1
            return -1
        s = self._victim(held, False)
        if s < 0:
            return -1
        self._place(s, (layer, expert), True)
        self.n["pred_staged"] += 1
        self.n["copies"] += 1
        return s

    def call(self, layer, topk, next_layer, probs=None, n_experts=1 << 30):
        """One streamed layer call; next_layer: 0 none, 1 streamed, 2 HBM-resident
        (True / False read as 1 / 0).  Returns ([(slot, copy)], [(expert, slot)])."""
        nl = int(next_layer)
        guess = self.route_done(layer, topk, probs, nl != 0, nl == 1)
        held, looked = [], []
        for e in topk:
            s, c = self.lookup(layer, e, held)
            held.append(s)
            looked.append((s, c))
        staged = []
        for e in guess:
            if e < 0 or e >= n_experts or len(held) >= MAX_HELD:
                continue
            s = self.stage(layer + 1, e, held)
            if s < 0:
                continue
            held.append(s)
            staged.append((e, s))
        return looked, staged
