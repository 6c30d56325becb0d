"""Host-CPU hybrid through the C ABI (moert_model_create_hybrid): every step's logits equal the resident model's
within 1e-2 while the host computes the experts outside the token's table, and the placement counters equal the
oracle's restatement of the reference simulator (oracle/placement.py) replayed over the routes the hybrid model
took (the reference's check of its D1 engine against the simulator, rust/moe-rt/tests/fixtures/
a1_sim_token_barreira.json)."""
import numpy as np
import pytest

import moert
import placement as P

pytestmark = pytest.mark.gpu

TINY8 = dict(hidden=256, inter=128, layers=3, heads=4, kv_heads=2, head_dim=64, vocab=97, experts=8, top_k=2)
NAMES = {"needed": "needed", "hits": "hits", "cpu": "cpu", "copies": "copies_bg", "dropped": "dropped",
         "deferred": "copies_deferred"}
TOL = 1e-2


def say(msg):
    print(f"[case] {msg}", flush=True)


def _run(res, hy, toks, label):
    """Both models over the same forced tokens: the largest logit difference per step, and the hybrid's routes
    [steps][layers][k]."""
    diffs, routes = [], []
    for t, tok in enumerate(toks):
        lg, ids, w, am = res.step(int(tok))
        hlg, hids, hw, ham = hy.step(int(tok))
        diffs.append(float(np.abs(hlg - lg).max()))
        routes.append(np.asarray(hids).reshape(-1, hy.cfg.top_k))
        assert diffs[-1] <= TOL, (label, t, diffs[-1])
    return np.array(diffs), np.array(routes)


def _oracle_counts(cfg, slots, backlog, routes):
    return P.replay_tokens(cfg.layers, cfg.experts, cfg.top_k, slots, backlog,
                           [[list(map(int, routes[t, l])) for l in range(cfg.layers)] for t in range(len(routes))])


@pytest.mark.parametrize("wdtype", [moert.Q4_0, moert.Q8_0])
@pytest.mark.parametrize("slots,backlog", [(0, 4), (1, 1), (3, 2), (6, 4), (6, 0), (24, 4)])
def test_hybrid_equals_resident_and_counts_like_the_simulator(gpu, wdtype, slots, backlog):
    """Pools from none (every expert on the host) to all 24 experts, backlogs 0..4: logits within 1e-2 of the
    resident model at every step, counters (needed, hits, cpu, copies, dropped, deferred) equal to the simulator's
    over the hybrid's routes, per-token counters adding up to them."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=13, wdtype=wdtype, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    res = moert.GpuModel(m, 64, attn_splits=4)
    say(f"hybrid dtype={wdtype} slots={slots} backlog={backlog}")
    hy = moert.GpuModel(m, 64, attn_splits=4, hybrid=(slots, backlog, 4))
    toks = np.random.default_rng(77).integers(0, cfg.vocab, 48)
    diffs, routes = _run(res, hy, toks, f"slots={slots}")
    got = {NAMES[k]: v for k, v in hy.cache_counters().items() if k in NAMES}
    want = _oracle_counts(cfg, slots, backlog, routes)
    assert got == want
    assert got["cpu"] > 0 or slots == 24
    counts = hy.cache_token_counts(0, len(toks), words=4)
    assert counts[:, :, 0].sum() == got["hits"] and counts[:, :, 1].sum() == got["copies_bg"]
    assert counts[:, :, 2].sum() == got["dropped"] and counts[:, :, 3].sum() == got["cpu"]
    say(f"hybrid slots={slots}: max logit diff {diffs.max():.2e}, {got}")
    res.close()
    hy.close()


def test_hybrid_generate_and_clear(gpu):
    """generate() drives the same host-side steps: its tokens equal step-by-step greedy decoding of the hybrid
    model; cache_clear empties the pool and zeroes the counters, after which a run counts as from a fresh model."""
    cfg = moert.Config(**TINY8)
    m = moert.SynthModel(cfg, seed=21, wdtype=moert.Q4_0, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)
    hy = moert.GpuModel(m, 64, attn_splits=4, hybrid=(5, 2, 2))
    prompt = [3, 9, 27]
    out = hy.generate(prompt, 12)
    c1 = hy.cache_counters()
    hy.cache_clear()
    assert hy.cache_counters()["needed"] == 0
    hy.reset()
    toks, nxt = [], None
    for i in range(len(prompt) + 11):
        tok = prompt[i] if i < len(prompt) else nxt
        _, _, _, nxt = hy.step(int(tok))
        if i >= len(prompt) - 1:
            toks.append(nxt)
    assert list(out) == toks
    assert hy.cache_counters() == c1
    hy.close()


def test_hybrid_granite_3b_q4_0_quarter_pool(gpu, granite_3b_q4):
    """The expert-cache workload's shape (3B, Q4_0, Zipf routing) with a pool of 25% of the experts and the
    reference's default backlog 4: 48 forced steps within 1e-2 of the resident model, counters equal to the
    simulator's."""
    cfg, m = granite_3b_q4
    toks = np.random.default_rng(512).integers(0, cfg.vocab, 48)
    res = moert.GpuModel(m, 128, attn_splits=64)
    hy = moert.GpuModel(m, 128, attn_splits=64, hybrid=(320, 4, 16))
    say("hybrid 3b q4_0 320 slots")
    diffs, routes = _run(res, hy, toks, "3b")
    got = {NAMES[k]: v for k, v in hy.cache_counters().items() if k in NAMES}
    assert got == _oracle_counts(cfg, 320, 4, routes)
    say(f"hybrid 3b: max logit diff {diffs.max():.2e}, {got}")
    res.close()
    hy.close()
