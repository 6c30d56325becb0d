"""Expert placement of the host-CPU hybrid (host only): the product's state machine (moert_placement_*, moert_freq_*)
and the oracle's restatement of the reference simulator (oracle/placement.py), both against the reference's own
fixtures (rust/moe-rt/tests/fixtures/a1_sim_token_barreira.json, 64 cases of one-position steps, and
a2_sim_passo_barreira.json, 123 cases of 1..8-position steps; copied to tests/golden/) and the golden Freq scores of
rust/moe-rt/src/cache.rs:368-383."""
import json
import math
import os

import numpy as np
import pytest

import moert
import placement as P

HERE = os.path.dirname(os.path.abspath(__file__))
A1 = json.load(open(os.path.join(HERE, "golden", "a1_sim_token_barreira.json")))
A2 = json.load(open(os.path.join(HERE, "golden", "a2_sim_passo_barreira.json")))
# product counter names -> the fixtures' names
NAMES = {"needed": "needed", "hits": "hits", "cpu": "cpu", "copies": "copies_bg", "dropped": "dropped",
         "deferred": "copies_deferred"}

TOUCHES = [(0, 0), (0, 1), (1, 4), (2, 8), (3, 0), (3, 2), (5, 4), (100, 0), (400, 1), (401, 1), (1000, 2), (1500, 8)]
GOLDEN = [(0, 1.6795384259222959), (1, 2.35640533956035), (2, 2.824937203935159), (4, 1.007821901389905),
          (8, 3.9997256579758678)]


def test_freq_gives_the_simulators_scores():
    """cache.rs:368-383: L = 3, 4 experts (key = layer * 4 + expert), the same touches; -inf for a key never
    touched, and after clear. Both the product and the oracle."""
    f, o = moert.Freq(12, 3), P.Freq(3)
    for step, key in TOUCHES:
        f.touch(key, step)
        o.touch(key, step)
    for key, v in GOLDEN:
        assert abs(f.score(key) - v) < 1e-12, key
        assert abs(o.score(key) - v) < 1e-12, key
    assert f.score(3) == -math.inf and o.score(3) == -math.inf
    f.clear()
    assert f.score(8) == -math.inf


def test_freq_closed_forms():
    """A key touched n times at one step has value n (score log2 n + step/per); one half-life (128 tokens = 128 * L
    steps) later a touch gives n/2 + 1; the product refuses a step that goes back."""
    f = moert.Freq(4, 2)
    for _ in range(6):
        f.touch(1, 10)
    assert abs(f.score(1) - (math.log2(6) + 10 / 256)) < 1e-12
    f.touch(1, 10 + 256)
    assert abs(f.score(1) - (math.log2(4.0) + 266 / 256)) < 1e-12
    with pytest.raises(moert.MoertError):
        f.touch(1, 5)


def _case_ids(c, steps):
    """Fixture routing[pos][l] -> per step, ids [layers][m][k]."""
    r = np.asarray(c["routing"], np.int32)  # [pos, L, k]
    pos = 0
    for m in steps:
        yield np.ascontiguousarray(r[pos:pos + m].transpose(1, 0, 2))
        pos += m


def _product(c, steps):
    p = moert.Placement(c["layers"], c["experts"], c["topk"], c["slots"], c["backlog"])
    for ids in _case_ids(c, steps):
        p.step(ids)
    got = p.counters()
    p.close()
    return {NAMES[k]: v for k, v in got.items()}


@pytest.mark.parametrize("c", A1["casos"], ids=lambda c: f"a1-{c['caso']}")
def test_a1_fixture_oracle_and_product(c):
    steps = [1] * c["tokens"]
    want = c["esperado"]
    assert P.replay_tokens(c["layers"], c["experts"], c["topk"], c["slots"], c["backlog"], c["routing"]) == want
    assert _product(c, steps) == want


@pytest.mark.parametrize("c", A2["casos"], ids=lambda c: f"a2-{c['caso']}-{c['tipo']}")
def test_a2_fixture_oracle_and_product(c):
    want = c["esperado"]
    assert P.replay_steps(c["layers"], c["experts"], c["topk"], c["slots"], c["backlog"], c["routing"],
                          c["passos"]) == want
    assert _product(c, c["passos"]) == want


@pytest.mark.parametrize("mutant", ["no_defer", "lru", "touch_after", "no_backlog"])
def test_fixtures_detect_planted_mistakes_in_the_oracle(mutant):
    """Each planted mistake (copies never held, LRU without the admission test, the frequency counted after the
    decisions, no backlog bound) changes the counts of several fixture cases."""
    bad = sum(P.replay_tokens(c["layers"], c["experts"], c["topk"], c["slots"], c["backlog"], c["routing"], mutant)
              != c["esperado"] for c in A1["casos"])
    bad += sum(P.replay_steps(c["layers"], c["experts"], c["topk"], c["slots"], c["backlog"], c["routing"],
                              c["passos"], mutant) != c["esperado"] for c in A2["casos"])
    assert bad >= 10, (mutant, bad)


@pytest.mark.parametrize("seed", range(12))
def test_product_equals_the_oracle_on_fresh_traces(seed):
    """Traces beyond the fixtures (more layers and experts, larger pools, long runs for the decay): the product's
    six counters equal the oracle's, step by step, and the published table holds exactly the resident keys."""
    rng = np.random.default_rng(1000 + seed)
    L, E = int(rng.integers(2, 7)), int(rng.choice([4, 8, 16, 40]))
    k = int(rng.integers(1, min(8, E) + 1))
    slots = int(rng.integers(0, L * E + 1))
    backlog = int(rng.choice([0, 1, 3, 8, 64]))
    T = int(rng.integers(50, 400))
    pop = rng.dirichlet(np.full(E, 0.3), size=L)
    routing = [[list(rng.choice(E, size=k, replace=False, p=pop[l])) for l in range(L)] for _ in range(T)]
    steps = []
    while sum(steps) < T:
        steps.append(int(min(rng.choice([1, 1, 2, 3, 5, 8]), T - sum(steps))))
    sim = P.D1Sim(L, E, k, slots, backlog)
    p = moert.Placement(L, E, k, slots, backlog)
    pos = 0
    for m in steps:
        ids = np.asarray([[routing[q][l] for q in range(pos, pos + m)] for l in range(L)], np.int32)
        sim.run_step(ids.tolist())
        p.step(ids)
        got = {NAMES[a]: b for a, b in p.counters().items()}
        assert got == sim.counts(), (seed, pos)
        pos += m
    table = p.table()
    # the next token's table: the resident keys and every copy of the last token (landed at the barrier)
    assert sorted(np.flatnonzero(table >= 0)) == sorted(l * E + e for (l, e) in list(sim.resident) + list(sim.inflight))
    assert len(set(table[table >= 0])) == int((table >= 0).sum()) <= slots
    p.close()


def test_refusals():
    with pytest.raises(moert.MoertError):
        moert.Placement(2, 4, 5, 2, 1)  # top_k > experts
    with pytest.raises(moert.MoertError):
        moert.Placement(2, 4, 2, 9, 1)  # more slots than experts
    p = moert.Placement(2, 4, 2, 3, 1)
    with pytest.raises(moert.MoertError, match="twice"):
        p.step(np.array([[[1, 1]], [[0, 2]]]))
    with pytest.raises(moert.MoertError):
        p.step(np.array([[[1, 4]], [[0, 2]]]))
    p.step(np.array([[[1, 3]], [[0, 2]]]))
    assert p.counters() == {"needed": 4, "hits": 0, "cpu": 4, "copies": 1, "dropped": 3, "deferred": 0}
