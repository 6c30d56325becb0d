"""Expert placement of the host-CPU hybrid, restated in pure Python — test infrastructure only.

Imported by tests/ as the checker of the product's placement service (libmoert's moert_placement_* and the hybrid
model); never by the product package. It restates the reference's simulator for the configuration its fixtures pin:
tools/moe_sim.py `Sim(policy="lfu_cpu", protocol="token", token_barreira=True)` (Sim 113-465) and, for steps of
m positions, qual-runs/A2-MULTIPOS-SIM-20261103/multipos.py `SimM.layer_m` (50-102) with the union of a layer's
experts in order of first appearance (`primeira_aparicao`, multipos.py:124-127). In the barrier mode the counts do
not depend on time, so the cost model of the simulator is left out; only its decisions are restated.

Pinned by: the reference's fixtures rust/moe-rt/tests/fixtures/a1_sim_token_barreira.json (64 cases, steps of one
position) and a2_sim_passo_barreira.json (123 cases, steps of 1..8 positions), copied under tests/golden/, and the
golden Freq scores of rust/moe-rt/src/cache.rs:368-383.
"""
from __future__ import annotations

import heapq
import math

HALF_LIFE = 128.0  # tokens (moe_sim.py HALF_LIFE; cache.rs HALF_LIFE)
FIELDS = ("needed", "hits", "cpu", "copies_bg", "dropped", "copies_deferred")


class Freq:
    """Decayed frequency per key (moe_sim.py Sim.touch_freq / Sim.score, 152-160; cache.rs Freq 60-87): log2 of the
    value and the step of its last update; a touch adds 1 to the value decayed with a half-life of HALF_LIFE tokens
    (HALF_LIFE * layers steps); score = log2 v + step / (HALF_LIFE * layers), which orders keys as their values
    decayed to a common instant."""

    def __init__(self, layers):
        self.per = HALF_LIFE * layers
        self.f = {}

    def touch(self, key, step):
        lv, s0 = self.f.get(key, (-math.inf, step))
        v = 2.0 ** (lv - (step - s0) / self.per) if lv > -math.inf else 0.0
        self.f[key] = (math.log2(v + 1.0), step)

    def score(self, key):
        lv, s0 = self.f.get(key, (-math.inf, 0))
        return lv + s0 / self.per

    def clear(self):
        self.f.clear()


def first_appearance(ids):
    """Union of the experts of one layer over the positions of a step ([m][k], position-major), in order of first
    appearance, with the number of requests of each (multipos.py:124-127)."""
    es, ns = [], []
    for pos in ids:
        for e in pos:
            e = int(e)
            if e in es:
                ns[es.index(e)] += 1
            else:
                es.append(e)
                ns.append(1)
    return es, ns


class D1Sim:
    """The token protocol with the barrier (the deterministic TokenBarrier mode) and LFU admission.

    State: resident keys, keys whose copy is queued (`inflight`), an eviction heap of (score, version, key) entries
    with lazy deletion, the token's table (the resident keys published when the token starts), and copies deferred
    until the layer of their victim has passed. Keys are (layer, expert) pairs.
    `mutant` plants one mistake (for tests that show what the fixtures detect): "no_defer" (every copy starts at
    once), "lru" (evict the least recently used key, no admission test), "touch_after" (the layer's requests are
    counted into the frequency after its decisions), "no_backlog" (the backlog never refuses)."""

    def __init__(self, layers, experts, top_k, slots, backlog, mutant=None):
        self.L, self.E, self.k, self.cap, self.backlog = layers, experts, top_k, slots, backlog
        self.mutant = mutant
        self.freq = Freq(layers)
        self.resident = {}
        self.inflight = {}  # key -> True while its copy is deferred, False once queued
        self.heap = []
        self.version = {}
        self.lru = {}  # key -> step of its last use (the "lru" mutant's priority)
        self.table = frozenset()
        self.deferred = []  # (victim layer, key)
        self.cur_layer = 0
        self.step = 0
        self.stats = {f: 0 for f in FIELDS}
        self.stats["tokens"] = 0

    # -- eviction heap (moe_sim.py prio / push / victim / make_room, 162-236)
    def prio(self, key):
        return self.lru.get(key, -1) if self.mutant == "lru" else self.freq.score(key)

    def push(self, key):
        v = self.version.get(key, 0) + 1
        self.version[key] = v
        heapq.heappush(self.heap, (self.prio(key), v, key))

    def victim(self, pinned):
        held, found = [], None
        while self.heap:
            prio, v, key = heapq.heappop(self.heap)
            if key not in self.resident or self.version.get(key) != v:
                continue
            if key in pinned:
                held.append((prio, v, key))
                continue
            found = (prio, key)
            break
        for item in held:
            heapq.heappush(self.heap, item)
        if found:
            heapq.heappush(self.heap, (found[0], self.version[found[1]], found[1]))
        return found

    def make_room(self, pinned, candidate_prio):
        """(room, evicted key or None): a slot is free, or the weakest resident outside this layer's keys is evicted
        when its priority is below the candidate's."""
        if len(self.resident) + len(self.inflight) < self.cap:
            return True, None
        vic = self.victim(pinned)
        if vic is None or (candidate_prio is not None and vic[0] >= candidate_prio):
            return False, None
        del self.resident[vic[1]]
        return True, vic[1]

    # -- token protocol (moe_sim.py begin_token 188-199, admit_bg 250-285, release_deferred 425-436)
    def begin_token(self):
        assert not self.deferred, "a deferred copy did not start in the previous token"
        for key in list(self.inflight):  # the barrier: every copy of the previous token has landed
            del self.inflight[key]
            self.resident[key] = None
            self.push(key)
        self.table = frozenset(self.resident)

    def release_deferred(self, layer):
        rest = []
        for v, key in self.deferred:
            if v == layer:
                self.inflight[key] = False
            else:
                rest.append((v, key))
        self.deferred = rest

    def admit(self, key, pinned):
        full = self.mutant != "no_backlog" and len(self.inflight) >= self.backlog
        if self.cap == 0 or full:
            self.stats["dropped"] += 1
            return
        ok, vic = self.make_room(pinned, None if self.mutant == "lru" else self.prio(key))
        if not ok:
            self.stats["dropped"] += 1
            return
        if vic is not None and vic[0] >= self.cur_layer and self.mutant != "no_defer":
            # the GPU may still read the victim's slot at its layer in this token: the copy waits for that layer
            self.inflight[key] = True
            self.deferred.append((vic[0], key))
            self.stats["copies_deferred"] += 1
        else:
            self.inflight[key] = False
        self.stats["copies_bg"] += 1

    def layer(self, l, es, ns, m):
        """One layer of a step of m positions: es the union of its experts (first appearance), ns their requests."""
        self.cur_layer = l
        if l == 0:
            self.begin_token()
        if l > 0:
            self.release_deferred(l - 1)  # the doorbell of l: the GPU has passed the experts of l - 1
        keys = [(l, int(e)) for e in es]
        pinned = set(keys)
        if self.mutant != "touch_after":
            for key, n in zip(keys, ns):
                for _ in range(n):
                    self.freq.touch(key, self.step)
        adm = []
        for key, n in zip(keys, ns):
            self.stats["needed"] += n
            if key in self.table:
                if key in self.resident:  # a victim of a later layer is still read in this token
                    self.lru[key] = self.step
                    self.push(key)
                self.stats["hits"] += n
                continue
            self.stats["cpu"] += n
            if key in self.inflight:
                continue
            adm.append(key)
        if self.mutant == "touch_after":
            for key, n in zip(keys, ns):
                for _ in range(n):
                    self.freq.touch(key, self.step)
        for key in adm:
            self.admit(key, pinned)
        if l == self.L - 1:
            self.release_deferred(l)  # the doorbell of the token's end
        self.step += m

    def run_step(self, ids):
        """One step of m positions: ids[l][p] = the top-k experts of position p at layer l."""
        m = len(ids[0])
        for l in range(self.L):
            es, ns = first_appearance(ids[l])
            self.layer(l, es, ns, m)
        self.stats["tokens"] += m

    def counts(self):
        return {f: self.stats[f] for f in FIELDS}


def replay_tokens(layers, experts, top_k, slots, backlog, routing, mutant=None):
    """A run of single-position steps: routing[t][l] = the top-k experts of token t at layer l (the a1 fixtures)."""
    s = D1Sim(layers, experts, top_k, slots, backlog, mutant)
    for t in range(len(routing)):
        s.run_step([[routing[t][l]] for l in range(layers)])
    return s.counts()


def replay_steps(layers, experts, top_k, slots, backlog, routing, steps, mutant=None):
    """A run in steps of steps[i] positions: routing[pos][l] = the top-k experts (the a2 fixtures)."""
    s = D1Sim(layers, experts, top_k, slots, backlog, mutant)
    pos = 0
    for m in steps:
        s.run_step([[routing[p][l] for p in range(pos, pos + m)] for l in range(layers)])
        pos += m
    assert pos == len(routing)
    return s.counts()
